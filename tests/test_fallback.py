"""The degraded paths (CPU): what graph_compute computes when a device job fails. Faults are
forced from the host (inject_faults), so no kernel is launched and these run without a GPU.

The reference's counterparts: the FLASH_ATTN_EXT fallback to the full-precision reference
(ggml-rocket.cpp:5627-5639 -> rocket_fa_ref_f32, 5392-5442) and the MUL_MAT_ID fallback to the
CPU per expert (6927-6939), each counted in cpu_fallbacks (ggml-rocket.h:78-88); the breaker
cases of test-rocket-internals.cpp:535-561 on the "fa" and "moe" groups. The operands are the
strided views llama.cpp hands over: Q a permute of its [D, H, T] projection, K and V a slice of
a longer KV cache laid out [n_ctx][HK][D].
"""
import numpy as np
import pytest

import ggml_mi355x as mx
from oracle import oracle as O
from bars import compare


def _fa_graph(g, D, DV, T, H, KV, HK, n_ctx, seed, causal=True):
    """Q, K, V and mask as llama.cpp lays them out; returns the tensors and the oracle's dense
    operands (q [H][T][D] F32, k/v [HK][KV][D] fp16 bits, mask [T][KV] fp16 bits)."""
    q_tok = O.fill_normal((T, H, D), seed)                       # [T][H][D]
    k_ctx = O.f32_to_f16_bits(O.fill_normal((n_ctx, HK, D), seed + 1))
    v_ctx = O.f32_to_f16_bits(O.fill_normal((n_ctx, HK, DV), seed + 2))
    j, t = np.arange(KV)[None, :], np.arange(T)[:, None]
    mask = np.where(j > KV - T + t, -np.inf, 0.0).astype(np.float32) if causal else np.zeros((T, KV), np.float32)
    m16 = O.f32_to_f16_bits(mask)

    qb = g.new_tensor(mx.F32, [D, H, T], "q_proj")
    g.set(qb, q_tok)
    q = g.permute_view(qb, [D, T, H, 1], [4, 4 * D * H, 4 * D, 4 * D * H * T])
    kb = g.new_tensor(mx.F16, [D, HK, n_ctx], "cache_k_l0")
    vb = g.new_tensor(mx.F16, [DV, HK, n_ctx], "cache_v_l0")
    g.set(kb, k_ctx), g.set(vb, v_ctx)
    k = g.permute_view(kb, [D, KV, HK, 1], [2, 2 * D * HK, 2 * D, 2 * D * HK * n_ctx])
    v = g.permute_view(vb, [DV, KV, HK, 1], [2, 2 * DV * HK, 2 * DV, 2 * DV * HK * n_ctx])
    m = g.new_tensor(mx.F16, [KV, T])
    g.set(m, m16)
    dense = (np.ascontiguousarray(q_tok.transpose(1, 0, 2)),
             np.ascontiguousarray(k_ctx[:KV].transpose(1, 0, 2)),
             np.ascontiguousarray(v_ctx[:KV].transpose(1, 0, 2)), m16)
    return q, k, v, m, dense


@pytest.mark.parametrize("D,DV,T,H,KV,HK,n_ctx,softcap", [
    (128, 128, 48, 8, 160, 2, 256, 0.0),     # GQA 4:1, KV a slice of a longer cache
    (64, 64, 33, 4, 96, 4, 96, 30.0),        # ragged T, soft-capped, no GQA
    (192, 128, 32, 4, 128, 1, 200, 0.0),     # MLA widths (dk 192, dv 128)
])
def test_flash_attn_fallback_matches_oracle(D, DV, T, H, KV, HK, n_ctx, softcap):
    be = mx.Backend()
    g = mx.Graph()
    q, k, v, m, (Qd, Kd, Vd, Md) = _fa_graph(g, D, DV, T, H, KV, HK, n_ctx, 4100 + D + T)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    o = g.flash_attn_ext(q, k, v, m, scale, softcap=softcap)
    be.inject_faults("fa", 1)
    assert be.compute([o]) == mx.STATUS_SUCCESS
    assert be.cpu_fallbacks() == 1 and be.route_ops("fa") == 1
    assert be.route_stats("fa") == (1, 1, 0)
    got = g.get(o, np.float32, (T, H, DV))
    # the fallback is the full-precision reference: Q kept F32 (q_mode 1), double arithmetic
    want = O.flash_attn(Qd, Kd, Vd, Md, scale, softcap=softcap, q_mode=1)
    assert np.abs(got.astype(np.float64) - want).max() <= 1e-5 * max(1.0, np.abs(want).max())
    be.free()


def test_flash_attn_fallback_fully_masked_rows_are_zero():
    """Rows whose every key is masked are written as zeros (ggml-rocket.cpp:5395-5397)."""
    be = mx.Backend()
    g = mx.Graph()
    D, T, H, KV, HK = 64, 16, 2, 64, 1
    q, k, v, m, (Qd, Kd, Vd, Md) = _fa_graph(g, D, D, T, H, KV, HK, KV, 4242, causal=False)
    mask = np.zeros((T, KV), np.float32)
    mask[3, :] = -np.inf
    mask[7, 10:] = -np.inf
    g.set(m, O.f32_to_f16_bits(mask))
    o = g.flash_attn_ext(q, k, v, m, 0.125)
    be.inject_faults("fa", 1)
    assert be.compute([o]) == mx.STATUS_SUCCESS and be.cpu_fallbacks() == 1
    got = g.get(o, np.float32, (T, H, D))
    assert np.all(got[3] == 0.0)
    want = O.flash_attn(Qd, Kd, Vd, O.f32_to_f16_bits(mask), 0.125, q_mode=1)
    assert np.abs(got.astype(np.float64) - want).max() <= 1e-5 * np.abs(want).max()
    be.free()


def _moe(g, wt, K, N, E, ne11, U, T, seed, name):
    W = O.fill_normal((E, N, K), seed, 0.0, 0.05)
    P = O.f32_to_f16_bits(W) if wt == O.F16 else O.quantize(wt, W)
    X = O.fill_normal((T, ne11, K), seed + 1)
    logits = O.fill_normal((T, E), seed + 2)
    ids = np.argsort(-logits, axis=1, kind="stable")[:, :U].astype(np.int32)
    a = g.new_tensor(wt, [K, N, E], name)
    b = g.new_tensor(mx.F32, [K, ne11, T])
    idt = g.new_tensor(mx.I32, [U, T])
    g.set(a, P), g.set(b, X), g.set(idt, ids)
    return g.mul_mat_id(a, b, idt), O.mul_mat_id(wt, P, K, N, E, X, ne11, ids)


@pytest.mark.parametrize("wt,ne11", [(O.Q4_K, 1), (O.Q4_K, 4), (O.F16, 1), (O.Q8_0, 4)])
def test_mul_mat_id_fallback_matches_oracle(wt, ne11):
    """Both ne11 forms (one activation row per token, or one per slot)."""
    be = mx.Backend()
    g = mx.Graph()
    K, N, E, U, T = 512, 96, 8, 4, 24
    d, want = _moe(g, wt, K, N, E, ne11, U, T, 7000 + wt + ne11, f"blk.0.ffn_up_exps.{wt}.{ne11}.weight")
    be.inject_faults("moe", 1)
    assert be.compute([d]) == mx.STATUS_SUCCESS
    assert be.cpu_fallbacks() == 1 and be.route_ops("moe") == 1
    # a CPU run counts no expert as resident or streamed
    assert be.moe_stats() == (0, 0)
    got = g.get(d, np.float32, (T, U, N))
    r = compare(want, got)
    assert r["nbad"] == 0 and r["range_err"] <= 1e-6
    be.free()


def test_open_breaker_serves_fa_and_moe_from_the_cpu():
    """Three device failures in a row rest the group's route: the next calls run on the CPU
    without a device attempt, with the same results."""
    be = mx.Backend()
    g = mx.Graph()
    q, k, v, m, (Qd, Kd, Vd, Md) = _fa_graph(g, 64, 64, 16, 4, 64, 2, 64, 4300)
    o = g.flash_attn_ext(q, k, v, m, 0.125)
    d, want = _moe(g, O.Q4_K, 256, 64, 4, 1, 2, 16, 4400, "blk.1.ffn_gate_exps.weight")
    be.inject_faults("fa", 3)
    be.inject_faults("moe", 3)
    for i in range(5):
        assert be.compute([o, d]) == mx.STATUS_SUCCESS
    assert be.route_stats("fa") == (3, 3, 2)
    assert be.route_stats("moe") == (3, 3, 2)
    assert be.cpu_fallbacks() == 10
    want_o = O.flash_attn(Qd, Kd, Vd, Md, 0.125, q_mode=1)
    assert np.abs(g.get(o, np.float32, (16, 4, 64)) - want_o).max() <= 1e-5 * np.abs(want_o).max()
    assert compare(want, g.get(d, np.float32, (16, 2, 64)))["range_err"] <= 1e-6
    be.free()
