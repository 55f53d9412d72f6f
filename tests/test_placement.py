"""The placement gate (CPU only): every CHECK of test-rocket-placement.cpp on this backend's
supports_op / offload_op, with the RK3588 expectations of the reference except where the
MI355X route is wider or narrower; each such row says why.

Knob-dependent modes run in a child process with their environment (knobs are read once per
process), as the reference forks a child per mode.
"""
import json
import os
import subprocess
import sys

import pytest

import ggml_mi355x as mx
from placement_probes import (mm_supported, mm_computed_w_supported, add_offloaded, mm_offloaded,
                              fa_supported, PREC_F32, PREC_BF16, PREC_F16, PREC_Q8)

HERE = os.path.dirname(os.path.abspath(__file__))
K, N, M, MQ = 256, 128, 256, 512

CASES = [
    ("F16 leaf weight, valid shape -> offload", True, lambda: mm_supported(K, N, M, mx.F16)),
    ("F32 leaf weight, valid shape -> offload", True, lambda: mm_supported(K, N, M, mx.F32)),
    ("BF16 leaf weight -> offload (converted to fp16)", True, lambda: mm_supported(K, N, M, mx.BF16)),
    ("Q8_0 leaf, M >= quant floor -> offload", True, lambda: mm_supported(K, N, MQ, mx.Q8_0)),
    ("Q4_K leaf, M >= quant floor -> offload", True, lambda: mm_supported(K, N, MQ, mx.Q4_K)),
    ("Q6_K leaf, M >= quant floor -> offload", True, lambda: mm_supported(K, N, MQ, mx.Q6_K)),
    ("Q4_0 leaf, M >= quant floor -> offload", True, lambda: mm_supported(K, N, MQ, mx.Q4_0)),
    ("Q5_K leaf, M >= quant floor -> offload", True, lambda: mm_supported(K, N, MQ, mx.Q5_K)),
    # MXFP4 (gpt-oss): the reference claims it for its MoE route; decoded exactly to fp16 here,
    # so MUL_MAT takes it as it takes the other quant types
    ("MXFP4 leaf, M >= quant floor -> offload", True, lambda: mm_supported(K, N, MQ, mx.MXFP4)),
    ("MXFP4 leaf, M(256) < quant floor -> CPU", False, lambda: mm_supported(K, N, M, mx.MXFP4)),
    ("Q4_K leaf, M(256) < quant floor -> CPU", False, lambda: mm_supported(K, N, M, mx.Q4_K)),
    ("K%32 != 0 (K=80) -> CPU", False, lambda: mm_supported(80, N, M, mx.F16)),
    ("N%16 != 0 (N=70) -> CPU", False, lambda: mm_supported(K, 70, M, mx.F16)),
    ("N=112 (N%16 == 0) -> offload", True, lambda: mm_supported(K, 112, M, mx.F16)),
    ("K<64 (K=32) -> CPU", False, lambda: mm_supported(32, N, M, mx.F16)),
    ("N<64 (N=48) -> CPU", False, lambda: mm_supported(K, 48, M, mx.F16)),
    ("M=1 decode GEMV -> CPU", False, lambda: mm_supported(K, N, 1, mx.F16)),
    ("computed (non-leaf) src0 -> CPU", False, lambda: mm_computed_w_supported(K, N, M)),
    ("offload_op: valid GEMM -> offload", True, lambda: mm_offloaded(K, N, M)),
    ("offload_op: ADD -> CPU", False, lambda: add_offloaded(K, M)),
    # The accumulator declaration: the reference's NPU route writes an fp16 C, so it declines
    # F32 / BF16 (ggml-rocket.cpp:7372-7380). This device accumulates in fp32 and writes F32,
    # which meets both declarations.
    ("acc F32 declared -> offload (fp32 accumulation here)", True, lambda: mm_supported(K, N, M, mx.F16, 0, PREC_F32)),
    ("acc BF16 declared -> offload (fp32 accumulation here)", True, lambda: mm_supported(K, N, M, mx.F16, 0, PREC_BF16)),
    ("acc F16 declared -> offload", True, lambda: mm_supported(K, N, M, mx.F16, 0, PREC_F16)),
    ("src1 F32 declared -> CPU (the activation is converted to fp16)", False,
     lambda: mm_supported(K, N, M, mx.F16, 3, PREC_F32)),
    ("src1 BF16 declared -> CPU", False, lambda: mm_supported(K, N, M, mx.F16, 3, PREC_BF16)),
    ("src1 F16 declared -> offload", True, lambda: mm_supported(K, N, M, mx.F16, 3, PREC_F16)),
    ("src1 Q8 declared -> offload", True, lambda: mm_supported(K, N, M, mx.F16, 3, PREC_Q8)),
    ("128x128 F32 leaf -> offload", True, lambda: mm_supported(128, 128, M, mx.F32)),
    ("same, SRC0_IS_HADAMARD hint -> CPU", False, lambda: mm_supported(128, 128, M, mx.F32, 1, 1)),
    ("FA: F16 KV, n_tokens >= min_t, n_kv >= min_kv -> offload", True,
     lambda: fa_supported(64, 256, 8, 1024, 2, mx.F16, 0.0)),
    ("FA: acc F32 declared -> offload (read, not enforced)", True,
     lambda: fa_supported(64, 256, 8, 1024, 2, mx.F16, 0.0, PREC_F32)),
    ("FA: decode (n_tokens=1 < min_t) -> CPU", False, lambda: fa_supported(64, 1, 8, 1024, 2, mx.F16, 0.0)),
    ("FA: short context (n_kv=512 < min_kv) -> CPU", False, lambda: fa_supported(64, 256, 8, 512, 2, mx.F16, 0.0)),
    ("FA: head_dim%32 != 0 (48) -> CPU", False, lambda: fa_supported(48, 256, 8, 1024, 2, mx.F16, 0.0)),
    ("FA: K/V not F16 -> CPU", False, lambda: fa_supported(64, 256, 8, 1024, 2, mx.F32, 0.0)),
    ("FA: ALiBi (max_bias > 0) -> CPU", False, lambda: fa_supported(64, 256, 8, 1024, 2, mx.F16, 8.0)),
    # The fused kernel takes dk and dv up to 256 (zero-padded onto the 64/64, 128/128, 192/128 and
    # 256/256 builds), the two-GEMM path dk % 32 / dv % 8 up to 1024; the reference takes any
    # dk%32 / dv%16 (ggml-rocket.cpp:7740-7760), so only head dims past 1024 are narrower.
    ("FA: head_dim 128 -> offload", True, lambda: fa_supported(128, 512, 32, 4096, 8, mx.F16, 0.0)),
    ("FA: head_dim 96 -> offload (padded to 128)", True, lambda: fa_supported(96, 256, 8, 1024, 2, mx.F16, 0.0)),
    ("FA: head_dim 32 -> offload (padded to 64)", True, lambda: fa_supported(32, 256, 8, 1024, 2, mx.F16, 0.0)),
    ("FA: dk 192 / dv 128 (MLA) -> offload", True, lambda: fa_supported(192, 256, 8, 1024, 2, mx.F16, 0.0, 0, 128)),
    ("FA: dk 160 / dv 80 -> offload (padded to 192 / 128)", True, lambda: fa_supported(160, 256, 8, 1024, 2, mx.F16, 0.0, 0, 80)),
    ("FA: dk 128 / dv 64 -> offload (dv padded to 128)", True, lambda: fa_supported(128, 256, 8, 1024, 2, mx.F16, 0.0, 0, 64)),
    ("FA: dk 192 / dv 192 -> offload (padded to 256)", True, lambda: fa_supported(192, 256, 8, 1024, 2, mx.F16, 0.0)),
    ("FA: head_dim 256 (Gemma) -> offload", True, lambda: fa_supported(256, 256, 8, 1024, 2, mx.F16, 0.0)),
    ("FA: dk 576 / dv 512 (absorbed MLA) -> offload (two-GEMM path)", True, lambda: fa_supported(576, 256, 8, 1024, 1, mx.F16, 0.0, 0, 512)),
    ("FA: head_dim 288 -> offload (two-GEMM path)", True, lambda: fa_supported(288, 256, 8, 1024, 2, mx.F16, 0.0)),
    ("FA: head_dim 1056 -> CPU (> 1024)", False, lambda: fa_supported(1056, 256, 8, 1024, 2, mx.F16, 0.0)),
    # Narrower: a quantized type without a device decoder is declined (the reference takes any
    # type with a ggml to_float, 7452-7455).
    # a type with neither a device decoder nor a registered host one (the plugin registers
    # ggml's to_float for every quantized type; this process registers none)
    ("Q4_1 leaf -> CPU (no decoder)", False, lambda: mm_supported(K, N, MQ, 3)),
    ("Q2_K leaf -> CPU (no decoder)", False, lambda: mm_supported(K, N, MQ, 10)),
]


@pytest.mark.parametrize("label,want,fn", CASES, ids=[c[0] for c in CASES])
def test_placement(label, want, fn):
    assert fn() == want, label


def test_supports_buft():
    """ggml-rocket.cpp:7795-7797: host buffers and CPU_REPACK (whose weights are claimed only
    through registered original bytes)."""
    assert mx.host().mi355x_backend_supports_buft(mx.BUF_HOST)
    assert mx.host().mi355x_backend_supports_buft(mx.BUF_REPACK)
    assert not mx.host().mi355x_backend_supports_buft(mx.BUF_OTHER)


def _repacked_q4k(g, name="blk.0.ffn_down.weight"):
    """A Q4_K weight in a CPU_REPACK buffer: its own bytes (the repacked copy) differ from the
    original bytes a host would register."""
    import numpy as np
    nb = K // 256 * 144 * N
    W = g._new(mx.Q4_K, [K, N], name=name, data=np.full(nb, 0x5A, dtype=np.uint8))
    W.buffer_kind = mx.BUF_REPACK
    orig = np.random.default_rng(7).integers(0, 256, nb, dtype=np.uint8)
    return W, orig


def test_repacked_weight_sources():
    """test-rocket-internals.cpp:564-655: a repacked weight is claimed only through its
    registered original bytes; name and size must match; unregistering declines it again; the
    weight key is the same in placement and in compute."""
    import ctypes
    g = mx.Graph()
    W, orig = _repacked_q4k(g)
    X = g.new_tensor(mx.F32, [K, MQ])
    mm = g.mul_mat(W, X)
    try:
        assert not mx.supports_op(mm), "an unregistered repacked weight's MUL_MAT is declined"
        mx.register_weight_source(W, orig)
        assert mx.supports_op(mm), "a registered weight's MUL_MAT is claimed"
        k_place = mx.weight_key(W)
        repacked, kind = W.data, W.buffer_kind
        W.data, W.buffer_kind = orig.ctypes.data, mx.BUF_HOST      # what graph_compute does
        k_compute = mx.weight_key(W)
        W.data, W.buffer_kind = repacked, kind
        assert k_place and k_place == k_compute, "one key in placement and in compute"
        W.name = b"blk.1.ffn_down.weight"
        assert not mx.supports_op(mm), "a renamed tensor does not use the old registration"
        W.name = b"blk.0.ffn_down.weight"
        assert mx.supports_op(mm)
        mx.register_weight_source(W, orig[:-1])
        assert not mx.supports_op(mm), "a registration of another size is not used"
        mx.register_weight_source(W, orig)
        half = g.permute_view(W, [K, N // 2, 1, 1], [W.nb[0], W.nb[1], W.nb[1] * (N // 2), W.nb[1] * (N // 2)],
                              offset=W.nb[1] * (N // 2))
        assert mx.supports_op(g.mul_mat(half, X)) is False   # a view is not a leaf weight
        mx.register_weight_source(W, None)
        assert not mx.supports_op(mm), "unregistered: declined again"
    finally:
        mx.register_weight_source(W, None)


def _child(mode, env):
    e = {k: v for k, v in os.environ.items() if not k.startswith(("MI355X_", "ROCKET_"))}
    e.update(env)
    r = subprocess.run([sys.executable, os.path.join(HERE, "placement_probes.py"), mode], env=e,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout.strip().splitlines()[-1])


@pytest.mark.parametrize("mode,env", [("auto", {}), ("budget", {"MI355X_MOE_CACHE_MB": "1"}),
                                      ("off", {"MI355X_MOE": "0"}), ("forced", {"MI355X_MOE": "1"}),
                                      ("prec_quant", {"ROCKET_INT8": "1", "ROCKET_INT4": "1"}),
                                      ("host_decoder", {"MI355X_MOE": "1"})])
def test_moe_and_knob_modes(mode, env):
    bad = [row for row in _child(mode, env) if row[1] != row[2]]
    assert not bad, bad


def test_reference_knob_spelling_is_honoured():
    """A ROCKET_* knob means what it means for the reference (MOE=0 under its own name)."""
    bad = [row for row in _child("off", {"ROCKET_MOE": "0"}) if row[1] != row[2]]
    assert not bad, bad


def test_moe_charge_all_source():
    """Same budget, same four stacks in one buffer: charging the mapped source admits fewer
    (test-rocket-placement.cpp:302-372, 527-538)."""
    n_default = _child("src_admitted", {})
    n_all_src = _child("src_admitted", {"MI355X_MOE_CHARGE_ALL_SOURCE": "1"})
    assert n_all_src < n_default, (n_default, n_all_src)
