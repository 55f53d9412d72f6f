"""One Llama-3-8B-shape prefill layer through the plugin boundary, at its real sizes.

The headline workload's exact integrated path: named Q4_K host weights (quantized by the oracle
from N(0, 0.02)), M = 512 tokens, d 4096, FFN 14336, 32 query / 8 KV heads of 128, handed to
mi355x_backend_graph_compute in the splits the ggml scheduler forms for one layer:
{Q, K, V} (a fused group), {FLASH_ATTN_EXT causal at n_kv 2048, O} (O reads the attention's dst
through a view), {gate, up} (a fused group) and {down} (K = 14336). It runs under both
QUANT_RESIDENT routes (1: weights decoded once to resident fp16, "fused-resident" /
"prepacked-q"; 0: Q4_K blocks decoded in the GEMM on every call, "fused" / "mt"), each op
asserted on its route with zero CPU fallbacks (test-common.h:140-177,
test-rocket-matmul.cpp:259-366), and 48 sampled token rows of every op are checked against the
oracle: the fp64 GEMM of the same Q4_K bytes, and the double attention over the Q the device
produced (so the attention check isolates FLASH_ATTN_EXT from the Q projection's rounding).
Bars: no bad element (|d| >= 0.5 and rel >= 0.05), max|d|/max|ref| <= 1e-2, worst-column
cosine >= 0.999 (GEMM); max abs <= 2e-2 and max|d|/max|ref| <= 1e-2 (attention).
"""
import ctypes
import math

import numpy as np
import pytest

import ggml_mi355x as mx
from oracle import oracle as O
from bars import compare, worst_col_cos

pytestmark = pytest.mark.gpu

D, FFN, NH, NKV, HD, T, CTX = 4096, 14336, 32, 8, 128, 512, 2048
SHAPES = {"q": (D, D), "k": (NKV * HD, D), "v": (NKV * HD, D), "o": (D, D),
          "gate": (FFN, D), "up": (FFN, D), "down": (D, FFN)}
ROWS = np.sort(np.random.default_rng(77).choice(T, 48, replace=False))


@pytest.fixture(scope="module")
def layer(torch_cuda):
    w = {name: O.quantize(O.Q4_K, O.fill_normal((N, K), 0x5EED0000 + 0x500 + i, 0.0, 0.02))
         for i, (name, (N, K)) in enumerate(SHAPES.items())}
    x = O.fill_normal((T, D), 0x5EED0508)
    act = O.fill_normal((T, FFN), 0x5EED0509)
    kc = O.f32_to_f16_bits(O.fill_normal((CTX, NKV, HD), 0x5EED050A))    # cache [n_ctx][HK][D]
    vc = O.f32_to_f16_bits(O.fill_normal((CTX, NKV, HD), 0x5EED050B))
    j, t = np.arange(CTX)[None, :], np.arange(T)[:, None]
    mask = O.f32_to_f16_bits(np.where(j > CTX - T + t, -np.inf, 0.0).astype(np.float32))
    return w, x, act, kc, vc, mask


def _graph(w, x, act, kc, vc, mask):
    g = mx.Graph()
    W = {n: g.new_tensor(mx.Q4_K, [K, N], f"blk.0.{n}.weight") for n, (N, K) in SHAPES.items()}
    for n in W:
        g.set(W[n], w[n])
    X = g.new_tensor(mx.F32, [D, T])
    A = g.new_tensor(mx.F32, [FFN, T])
    KC = g.new_tensor(mx.F16, [HD, NKV, CTX], "cache_k_l0")
    VC = g.new_tensor(mx.F16, [HD, NKV, CTX], "cache_v_l0")
    MK = g.new_tensor(mx.F16, [CTX, T])
    g.set(X, x), g.set(A, act), g.set(KC, kc), g.set(VC, vc), g.set(MK, mask)
    mm = {n: g.mul_mat(W[n], A if n == "down" else X) for n in ("q", "k", "v", "gate", "up", "down")}
    # Q [D, T] viewed as [HD, T, NH] (llama.cpp's permute of its [HD, NH, T] projection)
    qv = g.permute_view(mm["q"], [HD, T, NH, 1], [4, D * 4, HD * 4, D * 4 * T])
    kv = g.permute_view(KC, [HD, CTX, NKV, 1], [2, NKV * HD * 2, HD * 2, NKV * HD * 2 * CTX])
    vv = g.permute_view(VC, [HD, CTX, NKV, 1], [2, NKV * HD * 2, HD * 2, NKV * HD * 2 * CTX])
    fa = g.flash_attn_ext(qv, kv, vv, MK, 1.0 / math.sqrt(HD))          # dst [HD, NH, T]
    fa2d = g.permute_view(fa, [D, T, 1, 1], [4, D * 4, D * 4 * T, D * 4 * T])
    mm["o"] = g.mul_mat(W["o"], fa2d)
    splits = [[mm["q"], mm["k"], mm["v"]], [fa, fa2d, mm["o"]], [mm["gate"], mm["up"]], [mm["down"]]]
    return g, mm, fa, splits


def _check_gemm(label, ref, got):
    r = compare(ref, got)
    wc = worst_col_cos(ref, got)
    print(f"  {label}: nbad={r['nbad']} range_err={r['range_err']:.3g} worst_col={wc:.6f}", flush=True)
    assert r["nbad"] == 0 and r["nonfinite"] == 0 and r["range_err"] <= 1e-2 and wc >= 0.999, label


@pytest.mark.parametrize("resident", [1, 0])
def test_8b_layer_through_graph_compute(layer, resident):
    w, x, act, kc, vc, mask = layer
    be = mx.Backend()
    be.set_quant_resident(resident)
    g, mm, fa, splits = _graph(w, x, act, kc, vc, mask)
    print(f"8B layer, QUANT_RESIDENT={resident}", flush=True)
    for nodes in splits:
        assert be.compute(nodes) == mx.STATUS_SUCCESS
    routes = {r: be.route_ops(r) for r in ("fused-resident", "prepacked-q", "fused", "mt", "fa", "prepacked")}
    print(f"  routes {routes}, CPU fallbacks {be.cpu_fallbacks()}", flush=True)
    assert be.cpu_fallbacks() == 0
    if resident:
        assert routes["fused-resident"] == 5 and routes["prepacked-q"] == 2 and routes["fa"] == 1
    else:
        assert routes["fused"] == 5 and routes["mt"] == 2 and routes["fa"] == 1
    assert be.route_ops() == 8
    hs = be.host_stats()
    print(f"  host stats {hs}", flush=True)
    assert hs["fa_mirror_hits"] == 1 and hs["calls"] == 4 and hs["copyback_redone"] == 0

    got = {n: g.get(t, np.float32, (T, SHAPES[n][0])) for n, t in mm.items()}
    for n in ("q", "k", "v", "gate", "up"):
        N, K = SHAPES[n]
        _check_gemm(f"{n} [{N} x {K}]", O.mul_mat(O.Q4_K, w[n], x[ROWS], N, K), got[n][ROWS])
    N, K = SHAPES["down"]
    _check_gemm(f"down [{N} x {K}]", O.mul_mat(O.Q4_K, w["down"], act[ROWS], N, K), got["down"][ROWS])

    # attention over the device's own Q, for the sampled query tokens
    attn = g.get(fa, np.float32, (T, NH, HD))
    q_dev = got["q"].reshape(T, NH, HD)
    qh = np.ascontiguousarray(q_dev[ROWS].transpose(1, 0, 2))          # [H][48][D]
    kh = np.ascontiguousarray(kc.reshape(CTX, NKV, HD).transpose(1, 0, 2))
    vh = np.ascontiguousarray(vc.reshape(CTX, NKV, HD).transpose(1, 0, 2))
    want = O.flash_attn(qh, kh, vh, np.ascontiguousarray(mask.reshape(T, CTX)[ROWS]),
                        float(1.0 / math.sqrt(HD)))
    r = compare(want, attn[ROWS])
    print(f"  FLASH_ATTN_EXT n_kv {CTX}: max_abs={r['max_abs']:.3g} range_err={r['range_err']:.3g}", flush=True)
    assert r["nonfinite"] == 0 and r["max_abs"] <= 2e-2 and r["range_err"] <= 1e-2

    # O over the attention the device wrote to host memory
    N, K = SHAPES["o"]
    _check_gemm(f"o [{N} x {K}]", O.mul_mat(O.Q4_K, w["o"], attn.reshape(T, D)[ROWS], N, K), got["o"][ROWS])
    be.free()
