"""The C-ABI library loads and exports every function the headers in include/ declare (CPU
only: nothing is computed)."""
import ctypes
import os
import re

import pytest

import ggml_mi355x as mx

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


# include/ggml-mi355x.h is the ggml-typed public API: it is implemented by the ggml adapter
# (ggml-rocket_amd/ggml/ggml-mi355x.cpp), which builds only against a host's ggml headers, so it
# is checked against that source here rather than against libmi355x.so
GGML_FACING = "ggml-mi355x.h"
ADAPTER = os.path.join(ROOT, "ggml-rocket_amd", "ggml", "ggml-mi355x.cpp")


def declared_functions(headers=None):
    names = []
    for h in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if not h.endswith(".h") or (headers is None and h == GGML_FACING) or (headers and h not in headers):
            continue
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = "\n".join(l for l in text.splitlines() if not l.lstrip().startswith("#"))
        for m in re.finditer(r"(?:MI355X_API|GGML_BACKEND_API)\s+[^;{(]*?\b(\w+)\s*\(", text):
            names.append(m.group(1))
    return names


def test_headers_declare_entry_points():
    names = declared_functions()
    assert len(names) >= 30, names
    assert "mi355x_gemm" in names and "mi355x_backend_graph_compute" in names


def test_library_exports_every_declared_symbol():
    L = mx.lib()
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert not missing, missing


def test_library_path_is_in_tree():
    assert os.path.dirname(os.path.abspath(mx.LIB_PATH)).startswith(ROOT)
    assert isinstance(mx.lib(), ctypes.CDLL)


def test_ggml_adapter_defines_the_public_api():
    """Every function of the ggml-facing header (the reference's ggml-rocket.h:23-91 under this
    backend's name) is defined in the adapter, which also carries the loader entry."""
    names = declared_functions([GGML_FACING])
    assert set(names) == {"ggml_backend_mi355x_init", "ggml_backend_is_mi355x", "ggml_backend_mi355x_set_n_threads",
                          "ggml_backend_mi355x_moe_stats", "ggml_backend_mi355x_route_ops",
                          "ggml_backend_mi355x_cpu_fallbacks", "ggml_backend_mi355x_reg"}, names
    src = open(ADAPTER).read()
    for n in names:
        assert re.search(r"^\S.*\b" + n + r"\s*\([^;]*\)\s*\{", src, flags=re.M), n
    assert "GGML_BACKEND_DL_IMPL(" in src
    # every host-layer call the adapter makes is exported by the core library
    L = mx.lib()
    used = set(re.findall(r"\b(mi355x_backend_\w+)\s*\(", src))
    assert used and all(hasattr(L, n) for n in used), sorted(n for n in used if not hasattr(L, n))


def test_q4k_x_layout_argument_checks():
    """The expert-stack layout Q4_K_X: the same byte count as Q4_K for whole 32-row groups, no size
    otherwise; its pack rejects partial groups, K off the 256-value blocks and in-place use before
    touching the device (argument checks only: no GPU needed)."""
    import ctypes
    import ggml_mi355x as mx
    L = mx.lib()
    assert mx.weight_bytes(mx.Q4_K_X, 64, 512) == mx.weight_bytes(mx.Q4_K, 64, 512) == 64 * 2 * 144
    assert mx.weight_bytes(mx.Q4_K_X, 33, 512) == -1
    assert mx.weight_bytes(mx.Q4_K_X, 64, 320) == -1
    buf_a = ctypes.create_string_buffer(64 * 2 * 144 + 16)
    buf_b = ctypes.create_string_buffer(64 * 2 * 144 + 16)
    a, b = ctypes.addressof(buf_a) + (-ctypes.addressof(buf_a)) % 16, ctypes.addressof(buf_b) + (-ctypes.addressof(buf_b)) % 16
    assert L.mi355x_weight_pack(mx.Q4_K_X, ctypes.c_void_p(a), 33, 512, ctypes.c_void_p(b), None) == mx.E_ARG
    assert L.mi355x_weight_pack(mx.Q4_K_X, ctypes.c_void_p(a), 64, 320, ctypes.c_void_p(b), None) == mx.E_ARG
    assert L.mi355x_weight_pack(mx.Q4_K_X, ctypes.c_void_p(a), 64, 512, ctypes.c_void_p(a), None) == mx.E_ARG


@pytest.mark.parametrize("x,base,bs", [("Q8_0_X", "Q8_0", 34), ("MXFP4_X", "MXFP4", 17), ("Q6_K_X", "Q6_K", 210 / 8)])
def test_x32_layout_argument_checks(x, base, bs):
    """Q8_0_X, MXFP4_X and Q6_K_X: the ggml byte count for whole 32-row groups of whole blocks
    (bs: bytes per 32 values), no size otherwise; the pack rejects partial groups, partial blocks
    and in-place use before touching the device (argument checks only: no GPU needed)."""
    import ctypes
    import ggml_mi355x as mx
    L = mx.lib()
    xt, bt = getattr(mx, x), getattr(mx, base)
    assert mx.weight_bytes(xt, 64, 512) == mx.weight_bytes(bt, 64, 512) == int(64 * 16 * bs)
    assert mx.weight_bytes(xt, 33, 512) == -1
    assert mx.weight_bytes(xt, 64, 48) == -1
    buf_a = ctypes.create_string_buffer(int(64 * 16 * bs) + 16)
    buf_b = ctypes.create_string_buffer(int(64 * 16 * bs) + 16)
    a, b = ctypes.addressof(buf_a) + (-ctypes.addressof(buf_a)) % 16, ctypes.addressof(buf_b) + (-ctypes.addressof(buf_b)) % 16
    assert L.mi355x_weight_pack(xt, ctypes.c_void_p(a), 33, 512, ctypes.c_void_p(b), None) == mx.E_ARG
    assert L.mi355x_weight_pack(xt, ctypes.c_void_p(a), 64, 48, ctypes.c_void_p(b), None) == mx.E_ARG
    assert L.mi355x_weight_pack(xt, ctypes.c_void_p(a), 64, 512, ctypes.c_void_p(a), None) == mx.E_ARG


def test_mul_mat_id_regrouped_layout_limits():
    """mi355x_mul_mat_id takes the regrouped expert layouts for experts of whole 32-row groups
    whose N * K fits 2^31 (the kernel's 32-bit offsets inside an expert), and refuses the rest
    before touching the device (argument checks only: no GPU needed)."""
    import ctypes
    import ggml_mi355x as mx
    L = mx.lib()
    fake = ctypes.c_void_p(1 << 20)   # 16-byte aligned, never dereferenced on these paths
    for x in ("Q4_K_X", "Q8_0_X", "Q6_K_X", "MXFP4_X"):
        for N, K in [(48, 4096), (1 << 16, (1 << 15) + 256)]:
            a = mx.MoeArgs(getattr(mx, x), fake, 8, N, K, fake, 1, K, K, fake, 2, 1, 2, 4, fake, N, 2 * N)
            ws = L.mi355x_mul_mat_id_workspace(ctypes.byref(a))
            assert L.mi355x_mul_mat_id(ctypes.byref(a), fake, ws, None, None) == mx.E_ARG, (x, N, K)


def test_mul_mat_workspace_sizes_the_decode_first_weight():
    """mi355x_mul_mat_workspace_for makes room for the tiled fp16 weight where the decode-first
    form runs (Q6_K / Q5_K / MXFP4 at M >= 512; Q4_0 at M >= 1024, or at M >= 512 with N >= K;
    Q8_0 at M >= 1024, and at M 512 only where N >= K, N * K > 2^24 and the all-DMA kernel's
    128 x 256 tiles leave part of the chip idle, or with K off the 256-value blocks where N >= K)
    and elsewhere sizes the pack and the in-GEMM decode's split partials only (host-side sizing:
    no GPU needed)."""
    import ggml_mi355x as mx
    L = mx.lib()
    for wt, M, N, K, first in [(mx.Q6_K, 512, 1024, 3072, True), (mx.Q6_K, 128, 1024, 3072, False),
                               (mx.Q8_0, 512, 3072, 1024, False), (mx.Q8_0, 512, 1024, 3072, False),
                               (mx.Q8_0, 512, 8192, 3072, True), (mx.Q8_0, 512, 14336, 4096, False),
                               (mx.Q8_0, 512, 3072, 1088, True),
                               (mx.Q8_0, 1024, 1024, 3072, True), (mx.Q4_K, 2048, 1024, 3072, False),
                               (mx.Q4_K, 512, 6144, 4096, True), (mx.Q4_K, 512, 28672, 4096, False),
                               (mx.Q5_K, 512, 1024, 3072, True), (mx.MXFP4, 512, 1024, 3072, True),
                               (mx.Q4_0, 512, 1024, 3072, False), (mx.Q4_0, 512, 3072, 1024, True)]:
        pack = int(L.mi355x_mul_mat_workspace(M, K))
        poff = (pack + 255) // 256 * 256
        arr = (mx.GemmOut * 1)()
        arr[0] = mx.GemmOut(0, N, 0, N, 0, N)
        part_f16t = int(L.mi355x_gemm_workspace(mx.F16_T, M, K, arr, 1))
        part_own = int(L.mi355x_gemm_workspace(wt, M, K, arr, 1))
        ws = int(L.mi355x_mul_mat_workspace_for(wt, N, K, M))
        assert L.mi355x_mul_mat_decode_first(wt, M, N, K) == int(first)
        if first:
            assert ws == poff + (mx.weight_bytes(mx.F16_T, N, K) + 255) // 256 * 256 + part_f16t, (wt, M, N, K)
        else:
            assert ws == (poff + part_own if part_own else pack), (wt, M, N, K)


def test_host_memory_matches_meminfo():
    """The ggml device reports host memory (MemAvailable / MemTotal), as
    ggml_backend_rocket_device_get_memory does (ggml-rocket.cpp:7277-7293), through the host
    layer's mi355x_backend_get_host_memory; the adapter's device slot calls it."""
    L = mx.lib()
    mx._bind_host(L)
    fr, tot = ctypes.c_size_t(0), ctypes.c_size_t(0)
    L.mi355x_backend_get_host_memory(ctypes.byref(fr), ctypes.byref(tot))
    info = {}
    for line in open("/proc/meminfo"):
        k, v = line.split(":", 1)
        info[k] = int(v.split()[0]) * 1024
    assert tot.value == info["MemTotal"]
    assert 0 < fr.value <= tot.value
    # MemAvailable moves between the two reads; it is the same order of magnitude
    assert abs(fr.value - info["MemAvailable"]) < max(info["MemAvailable"] // 4, 1 << 30)
    src = open(ADAPTER).read()
    body = src[src.index("void device_get_memory("):]
    body = body[:body.index("}")]
    assert "mi355x_backend_get_host_memory(" in body


def test_strict_abi_turns_an_unchecked_version_into_an_error(tmp_path):
    """The adapter's version guard, preprocessed on its own: versions 2 and 3 pass; another
    version warns, and is a compile error under MI355X_STRICT_ABI, which `make ggml STRICT_ABI=1`
    defines (the reference's GGML_ROCKET_STRICT_ABI, ggml-rocket.cpp:7216-7225)."""
    import subprocess
    src = open(ADAPTER).read()
    a = src.index("#if GGML_BACKEND_API_VERSION != 2")
    lines = src[a:].splitlines(keepends=True)
    depth, guard = 0, []
    for l in lines:
        t = l.strip()
        if t.startswith("#if"):
            depth += 1
        elif t.startswith("#endif"):
            depth -= 1
        guard.append(l)
        if depth == 0:
            break
    f = tmp_path / "guard.c"
    f.write_text("".join(guard) + "int x;\n")

    def cc(*defs):
        return subprocess.run(["gcc", "-fsyntax-only", *defs, str(f)], capture_output=True, text=True)

    for v in ("2", "3"):
        r = cc(f"-DGGML_BACKEND_API_VERSION={v}", "-DMI355X_STRICT_ABI")
        assert r.returncode == 0 and "warning" not in r.stderr, r.stderr
    r = cc("-DGGML_BACKEND_API_VERSION=4")
    assert r.returncode == 0 and "warning" in r.stderr
    r = cc("-DGGML_BACKEND_API_VERSION=4", "-DMI355X_STRICT_ABI")
    assert r.returncode != 0 and "error" in r.stderr
    mk = open(os.path.join(ROOT, "ggml-rocket_amd", "Makefile")).read()
    assert "-DMI355X_STRICT_ABI" in mk and "$(ADAPTER_DEFS)" in mk
