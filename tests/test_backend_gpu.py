"""The reference's device gates through the plugin boundary (graph_compute on host tensors):
test-rocket-matmul.cpp, test-rocket-fa.cpp and test-rocket-moe.cpp, each op asserted on its
route with zero CPU fallbacks (a fallback computes the golden's own fp64 arithmetic, so the
numbers alone would pass on a device that computed nothing; test-common.h:140-177)."""
import numpy as np
import pytest

import ggml_mi355x as mx
from oracle import oracle as O
from bars import compare, worst_col_cos, worst_row_cos, amp_for
from fa_cases import REFERENCE_CASES, fill_case, causal_mask, SCALED, QRANGE

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def be(torch_cuda):
    b = mx.Backend()
    yield b
    b.free()


class Mark:
    def __init__(self, be, route=None):
        self.be, self.route = be, route
        self.ops, self.fb = be.route_ops(route), be.cpu_fallbacks()

    def check(self, label):
        ops = self.be.route_ops(self.route) - self.ops
        fb = self.be.cpu_fallbacks() - self.fb
        print(f"  {label}: {ops} op(s) on route {self.route or '(any)'}, {fb} CPU fallback(s)")
        assert ops > 0 and fb == 0, label


def run_mul_mat(be, wtype, K, N, M, Wpayload, X, name=None):
    g = mx.Graph()
    W = g.new_tensor(wtype, [K, N], name)
    Xt = g.new_tensor(mx.F32, [K, M])
    g.set(W, Wpayload)
    g.set(Xt, X)
    d = g.mul_mat(W, Xt)
    assert be.compute([d]) == mx.STATUS_SUCCESS
    return g.get(d, np.float32, (M, N))


def bars(ref, got, M, N, label):
    r = compare(ref, got)
    wc = worst_col_cos(ref.reshape(M, N), got.reshape(M, N))
    print(f"{label}: nbad={r['nbad']} range_err={r['range_err']:.3g} worst_col={wc:.6f}")
    assert r["nbad"] == 0 and r["nonfinite"] == 0 and wc >= 0.999 and r["range_err"] <= 1e-2, label


@pytest.mark.parametrize("K,N,M", [(64, 32, 8), (384, 256, 256), (3840, 4096, 512), (64, 64, 7),
                                   (384, 256, 130), (3840, 4096, 250)])
def test_matmul_f16_shapes(be, K, N, M):
    Wf = O.fill_uniform((N, K), 101 + K, 1.0)
    Xf = O.fill_uniform((M, K), 202 + M, amp_for(K, 1.0))
    W16 = O.f32_to_f16_bits(Wf)
    ref = O.mul_mat(O.F16, W16, Xf, N, K)
    mk = Mark(be)
    got = run_mul_mat(be, mx.F16, K, N, M, W16, Xf, f"blk.shape.{K}.{N}.weight")
    mk.check("F16 shape")
    bars(ref, got, M, N, f"F16 K={K} N={N} M={M}")


def test_outlier_row(be):
    K, N, M = 256, 64, 8
    i = np.arange(K * N)
    Wf = ((((i * 7) % 13) - 6) * 0.05).astype(np.float32).reshape(N, K)
    j = np.arange(K * M)
    Xf = ((((j * 5) % 11) - 5) * 0.02).astype(np.float32).reshape(M, K)
    Xf[3] = ((np.arange(K) % 7) - 3) * 300.0
    W16 = O.f32_to_f16_bits(Wf)
    ref = O.mul_mat(O.F16, W16, Xf, N, K)
    mk = Mark(be)
    got = run_mul_mat(be, mx.F16, K, N, M, W16, Xf)
    mk.check("outlier")
    small = np.delete(np.arange(M), 3)
    assert np.isfinite(got).all()
    assert (np.abs(got[small] - ref[small]) / (np.abs(ref[small]) + 1e-6)).max() < 0.05


def test_same_name_new_bytes(be):
    """test-rocket-matmul.cpp:223-257: the weight cache keys on content, not on the name."""
    K, N, M = 1024, 256, 256
    idx = np.arange(K * N, dtype=np.uint64)
    W1 = ((((idx * 2654435761) >> 20) % 201).astype(np.int64) - 100).astype(np.float32).reshape(N, K) / 400.0
    W2 = ((((idx * 40503 + 17) >> 6) % 201).astype(np.int64) - 100).astype(np.float32).reshape(N, K) / 400.0
    Xf = ((np.arange(K * M) * 31 % 97) - 48).astype(np.float32).reshape(M, K) / 100.0
    for Wf in (W1, W2):
        W16 = O.f32_to_f16_bits(Wf)
        ref = O.mul_mat(O.F16, W16, Xf, N, K)
        got = run_mul_mat(be, mx.F16, K, N, M, W16, Xf, "blk.0.reloaded.weight")
        assert np.abs(got - ref).max() / np.abs(ref).max() < 1e-2


@pytest.mark.parametrize("Ns", [(4096, 4096), (4096, 2048, 2048)])
def test_fused_groups(be, Ns):
    K, M = 3840, 128
    Xf = O.fill_uniform((M, K), 303, amp_for(K, 1.0))
    g = mx.Graph()
    X = g.new_tensor(mx.F32, [K, M])
    g.set(X, Xf)
    nodes, refs = [], []
    for i, N in enumerate(Ns):
        W16 = O.f32_to_f16_bits(O.fill_uniform((N, K), 404 + i, 1.0))
        W = g.new_tensor(mx.F16, [K, N], f"blk.fused.{len(Ns)}.{i}.weight")
        g.set(W, W16)
        nodes.append(g.mul_mat(W, X))
        refs.append(O.mul_mat(O.F16, W16, Xf, N, K))
    f0 = be.route_ops("fused") + be.route_ops("fused-resident")
    fb0 = be.cpu_fallbacks()
    assert be.compute(nodes) == mx.STATUS_SUCCESS
    assert be.route_ops("fused") + be.route_ops("fused-resident") - f0 == len(Ns)
    assert be.cpu_fallbacks() == fb0
    for d, ref, N in zip(nodes, refs, Ns):
        bars(ref, g.get(d, np.float32, (M, N)), M, N, f"fused N={N}")


@pytest.mark.parametrize("K,N,M,wtype", [(256, 128, 64, O.Q8_0), (3840, 256, 128, O.Q8_0), (256, 128, 64, O.Q4_K),
                                         (3840, 256, 128, O.Q4_K), (512, 256, 128, O.Q6_K),
                                         (2880, 256, 128, O.MXFP4), (2880, 256, 128, O.Q4_0),
                                         (3840, 256, 128, O.Q5_K),
                                         # M 512: the mt route's decode-first form (Q6_K; Q8_0 with N >= K)
                                         (512, 256, 512, O.Q6_K), (512, 768, 512, O.Q8_0),
                                         (512, 256, 512, O.Q5_K), (512, 256, 512, O.MXFP4),
                                         (512, 512, 512, O.Q4_K), (512, 512, 512, O.Q4_0)])
@pytest.mark.parametrize("resident", [0, 1])
def test_matmul_quant(be, K, N, M, wtype, resident):
    i = np.arange(N * K, dtype=np.float32)
    Wf = (np.sin(i * np.float32(0.013)) * np.float32(0.5)).astype(np.float32).reshape(N, K)
    Xf = O.fill_uniform((M, K), 505 + K, amp_for(K, 0.61))
    Q = O.quantize(wtype, Wf)
    ref = O.mul_mat(wtype, Q, Xf, N, K)
    be.set_quant_resident(resident)
    route = "prepacked-q" if resident else "mt"
    mk = Mark(be, route)
    got = run_mul_mat(be, wtype, K, N, M, Q, Xf, f"blk.q.{wtype}.{K}.{resident}.weight")
    mk.check(f"quant {route}")
    be.set_quant_resident(-1)
    r = compare(ref, got)
    assert r["nbad"] == 0 and r["range_err"] <= 1e-2


def test_matmul_f32_and_bf16_weights(be):
    K, N, M = 512, 256, 64
    Wf = O.fill_normal((N, K), 31, 0.0, 0.05)
    Xf = O.fill_normal((M, K), 32)
    for wt in (mx.F32, mx.BF16):
        if wt == mx.F32:
            payload, Wq = Wf, Wf
        else:
            bits = (Wf.view(np.uint32) >> 16).astype(np.uint16)
            payload, Wq = bits, (bits.astype(np.uint32) << 16).view(np.float32)
        ref = (Xf.astype(np.float64) @ Wq.astype(np.float64).T)
        mk = Mark(be, "prepacked")
        got = run_mul_mat(be, wt, K, N, M, payload, Xf, f"blk.w{wt}.weight")
        mk.check(f"type {wt}")
        assert compare(ref, got)["range_err"] <= 1e-2


@pytest.mark.parametrize("case", REFERENCE_CASES, ids=[c[0] for c in REFERENCE_CASES])
def test_flash_attn_cases(be, case):
    name, D, T, H, KV, HK, kind, tol = case
    Q, K, V, M = fill_case(D, T, H, KV, HK, kind)
    K16, V16, M16 = O.f32_to_f16_bits(K), O.f32_to_f16_bits(V), O.f32_to_f16_bits(M)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    want = O.flash_attn(Q, K16, V16, M16, scale, q_mode=1 if kind in (SCALED, QRANGE) else 0)
    g = mx.Graph()
    q = g.new_tensor(mx.F32, [D, T, H])
    k = g.new_tensor(mx.F16, [D, KV, HK])
    v = g.new_tensor(mx.F16, [D, KV, HK])
    m = g.new_tensor(mx.F16, [KV, T])
    g.set(q, Q), g.set(k, K16), g.set(v, V16), g.set(m, M16)
    o = g.flash_attn_ext(q, k, v, m, scale)
    # every case, the two range constructions included, runs on the device here: the scores
    # never leave fp32 and a Q row past fp16 range is rescaled (the reference falls back)
    mk = Mark(be, "fa")
    assert be.compute([o]) == mx.STATUS_SUCCESS
    mk.check(name)
    got = g.get(o, np.float32, (T, H, D))
    err = float(np.abs(got.astype(np.float64) - want).max())
    print(f"{name}: max abs err {err:.3g} (tol {tol})")
    assert np.isfinite(got).all() and err <= tol


def test_flash_attn_mla_graph(be):
    """FLASH_ATTN_EXT with keys of 192 and values of 128 through graph_compute: dst takes its
    row width from V (ne0 = dv), the device kernel runs, causal mask at n_kv 1024."""
    D, DV, T, H, KV, HK = 192, 128, 128, 16, 1024, 2
    Q = O.fill_normal((H, T, D), 960)
    K16 = O.f32_to_f16_bits(O.fill_normal((HK, KV, D), 961))
    V16 = O.f32_to_f16_bits(O.fill_normal((HK, KV, DV), 962))
    M16 = O.f32_to_f16_bits(causal_mask(T, KV))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    want = O.flash_attn(Q, K16, V16, M16, scale)
    g = mx.Graph()
    q = g.new_tensor(mx.F32, [D, T, H])
    k = g.new_tensor(mx.F16, [D, KV, HK])
    v = g.new_tensor(mx.F16, [DV, KV, HK])
    m = g.new_tensor(mx.F16, [KV, T])
    g.set(q, Q), g.set(k, K16), g.set(v, V16), g.set(m, M16)
    o = g.flash_attn_ext(q, k, v, m, scale)
    mk = Mark(be, "fa")
    assert be.compute([o]) == mx.STATUS_SUCCESS
    mk.check("mla")
    got = g.get(o, np.float32, (T, H, DV))
    r = compare(want, got)
    print(f"MLA graph: {r}")
    assert r["nonfinite"] == 0 and r["max_abs"] <= 2e-2 and r["range_err"] <= 1e-2


def test_flash_attn_absorbed_mla_graph(be):
    """The absorbed MLA's FLASH_ATTN_EXT through graph_compute: keys of 576, values of 512 as a view
    of the keys' first 512 dims (the latent cache read twice), 16 query heads on one KV head, causal
    at n_kv 1024; claimed and run on the device (the two-GEMM path), no CPU fallback."""
    D, DV, T, H, KV, HK = 576, 512, 96, 16, 1024, 1
    Q = O.fill_normal((H, T, D), 970)
    K16 = O.f32_to_f16_bits(O.fill_normal((HK, KV, D), 971))
    V16 = np.ascontiguousarray(K16[:, :, :DV])
    M16 = O.f32_to_f16_bits(causal_mask(T, KV))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    want = O.flash_attn(Q, K16, V16, M16, scale)
    g = mx.Graph()
    q = g.new_tensor(mx.F32, [D, T, H])
    k = g.new_tensor(mx.F16, [D, KV, HK])
    v = g.permute_view(k, [DV, KV, HK, 1], [2, k.nb[1], k.nb[2], k.nb[3]])
    m = g.new_tensor(mx.F16, [KV, T])
    g.set(q, Q), g.set(k, K16), g.set(m, M16)
    o = g.flash_attn_ext(q, k, v, m, scale)
    mk = Mark(be, "fa")
    assert be.compute([o]) == mx.STATUS_SUCCESS
    mk.check("absorbed mla")
    got = g.get(o, np.float32, (T, H, DV))
    r = compare(want, got)
    print(f"absorbed MLA graph: {r}")
    assert r["nonfinite"] == 0 and r["max_abs"] <= 2e-2 and r["range_err"] <= 1e-2


def _moe_graph(g, wt, K, N, E, ne11, U, T, payload, X, ids, name):
    a = g.new_tensor(wt, [K, N, E], name)
    b = g.new_tensor(mx.F32, [K, ne11, T])
    idt = g.new_tensor(mx.I32, [U, T])
    g.set(a, payload), g.set(b, X), g.set(idt, ids)
    return g.mul_mat_id(a, b, idt)


def _moe_ids(T, U, E):
    t = np.arange(T)[:, None]
    s = np.arange(U)[None, :]
    return ((t * 3 + s * 7 + t // 5) % (E - 1)).astype(np.int32)


def _moe_input(T, ne11, K):
    X = O.fill_uniform((T, ne11, K), 2000 + K, 0.25)
    X[..., (np.arange(K) % 97) == 13] *= 20.0
    return X


@pytest.mark.parametrize("K,N,E,ne11,U,T,wt,floor,native", [
    (256, 128, 8, 1, 2, 64, O.F16, 0.9999, False), (256, 128, 8, 2, 2, 64, O.F16, 0.9999, False),
    (256, 128, 8, 1, 2, 66, O.F16, 0.9999, False), (256, 128, 16, 1, 4, 96, O.F16, 0.9999, False),
    (1024, 128, 8, 1, 2, 64, O.Q4_K, 0.999, True), (1152, 128, 8, 2, 2, 64, O.Q8_0, 0.999, True)])
def test_moe_cases(be, K, N, E, ne11, U, T, wt, floor, native):
    W = np.stack([O.fill_uniform((N, K), 1000 + e, 0.3) for e in range(E)])
    P = O.f32_to_f16_bits(W) if wt == O.F16 else O.quantize(wt, W)
    X = _moe_input(T, ne11, K)
    ids = _moe_ids(T, U, E)
    g = mx.Graph()
    d = _moe_graph(g, wt, K, N, E, ne11, U, T, P, X, ids, f"blk.{K}.{wt}.{ne11}.{T}.ffn_gate_exps.weight")
    res0, _ = be.moe_stats()
    mk = Mark(be, "moe")
    assert be.compute([d]) == mx.STATUS_SUCCESS
    mk.check("moe")
    res1, _ = be.moe_stats()
    assert res1 - res0 == E            # the named stack was ingested into the HBM expert cache
    ref = O.mul_mat_id(wt, P, K, N, E, X, ne11, ids)
    got = g.get(d, np.float32, (T, U, N))
    r = compare(ref, got)
    R = T * U
    part = 1.0 - 10.0 * (1.0 - floor)
    assert r["nbad"] == 0 and r["cos"] >= floor
    assert worst_row_cos(ref.reshape(R, N), got.reshape(R, N)) >= part
    assert worst_col_cos(ref.reshape(R, N), got.reshape(R, N)) >= part


def test_moe_one_ingest_serves_every_m(be):
    """test-rocket-moe.cpp:299-361: one named weight at 64/130/96/258 tokens, ingested once."""
    K, N, E, U = 1024, 128, 8, 2
    W = np.stack([O.fill_uniform((N, K), 5000 + e, 0.3) for e in range(E)])
    P = O.quantize(O.Q4_K, W)
    res0, _ = be.moe_stats()
    for T in (64, 130, 96, 258):
        X = _moe_input(T, 1, K)
        ids = _moe_ids(T, U, E)
        g = mx.Graph()
        d = _moe_graph(g, O.Q4_K, K, N, E, 1, U, T, P, X, ids, "blk.99.ffn_up_exps.weight")
        mk = Mark(be, "moe")
        assert be.compute([d]) == mx.STATUS_SUCCESS
        mk.check(f"cross-M T={T}")
        ref = O.mul_mat_id(O.Q4_K, P, K, N, E, X, 1, ids)
        assert compare(ref, g.get(d, np.float32, (T, U, N)))["cos"] >= 0.999
    res1, _ = be.moe_stats()
    assert 0 < res1 - res0 <= E


def test_injected_device_failure_falls_back(be):
    """A device failure degrades the op to the CPU, counted, with a correct result; the next
    op runs on the device again."""
    K, N, M = 512, 128, 64
    W16 = O.f32_to_f16_bits(O.fill_uniform((N, K), 71, 1.0))
    Xf = O.fill_uniform((M, K), 72, amp_for(K, 1.0))
    ref = O.mul_mat(O.F16, W16, Xf, N, K)
    fb0 = be.cpu_fallbacks()
    be.inject_faults("gemm", 1)
    got = run_mul_mat(be, mx.F16, K, N, M, W16, Xf, "blk.inject.weight")
    assert be.cpu_fallbacks() - fb0 == 1
    assert compare(ref, got)["range_err"] <= 1e-5
    mk = Mark(be)
    got2 = run_mul_mat(be, mx.F16, K, N, M, W16, Xf, "blk.inject.weight")
    mk.check("after the injected failure")
    bars(ref, got2, M, N, "device again")


def test_repacked_weight_computes_from_registered_bytes(be):
    """test-rocket-internals.cpp:564-655 and API.md:280-314 on the device: a Q4_K weight whose
    tensor bytes are ggml-cpu's repacked copy (here: bytes no decoder would accept as the weight)
    computes from its registered original bytes; unregistered, the split fails before any route
    reads the repacked layout, also when a view node of the weight comes first."""
    K, N, M = 512, 256, 512
    W = O.fill_normal((N, K), 960, 0.0, 0.02)
    Q = O.quantize(O.Q4_K, W)
    Xf = O.fill_normal((M, K), 961)
    ref = O.mul_mat(O.Q4_K, Q, Xf, N, K)
    g = mx.Graph()
    Wt = g._new(mx.Q4_K, [K, N], name="blk.r.ffn_down.weight",
                data=np.full(Q.nbytes, 0x5A, dtype=np.uint8))          # the "repacked" copy
    Wt.buffer_kind = mx.BUF_REPACK
    Xt = g.new_tensor(mx.F32, [K, M])
    g.set(Xt, Xf)
    d = g.mul_mat(Wt, Xt)
    other = g.new_tensor(mx.F32, [64, 64], "x")
    try:
        mx.register_weight_source(Wt, Q)
        assert mx.supports_op(d)
        mk = Mark(be)
        assert be.compute([d]) == mx.STATUS_SUCCESS
        mk.check("repacked weight, registered source")
        got = g.get(d, np.float32, (M, N))
        assert Wt.buffer_kind == mx.BUF_REPACK and Wt.data == g.keep[0].ctypes.data   # restored
        bars(ref, got, M, N, "repacked Q4_K from registered bytes")
        mx.register_weight_source(Wt, None)
        mx.register_weight_source(other, np.zeros(64 * 64, dtype=np.float32))   # registry not empty
        view = g.permute_view(Wt, [K, N // 2, 1, 1], [Wt.nb[0], Wt.nb[1], Wt.nb[1] * N, Wt.nb[1] * N])
        assert be.compute([view, d]) == mx.STATUS_FAILED
    finally:
        mx.register_weight_source(Wt, None)
        mx.register_weight_source(other, None)
