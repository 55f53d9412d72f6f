"""The plugin path fed from a GGUF file: a tiny random-init llama model (2 layers, d 256, FFN
512, 4 query / 2 KV heads of 64) written by llama3_gguf.py, its weights handed to
graph_compute as views of the memory-mapped file under their GGUF names, as a host's ggml hands
a mapped model over. One layer's ops at 512 tokens (fused Q/K/V, FLASH_ATTN_EXT causal at n_kv
1024 with O, fused gate/up, down) are checked against the oracle on the same file bytes with the
layer test's bars, routes asserted with no CPU fallback; then bench.py's GGUF-driven host path
runs the whole 2048-token prefill over the file."""
import argparse
import ctypes
import math

import numpy as np
import pytest

import ggml_mi355x as mx
import gguf_io as G
import llama3_gguf as L
from oracle import oracle as O
from bars import compare, worst_col_cos

pytestmark = pytest.mark.gpu

T, CTX = 512, 1024


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    p = str(tmp_path_factory.mktemp("gguf") / "tiny.gguf")
    L.write_llama3(p, layers=2, d=256, ffn=512, heads=4, kv_heads=2, vocab=1024)
    return p


def _check(label, ref, got):
    r = compare(ref, got)
    wc = worst_col_cos(ref, got)
    print(f"  {label}: nbad={r['nbad']} range_err={r['range_err']:.3g} worst_col={wc:.6f}", flush=True)
    assert r["nbad"] == 0 and r["nonfinite"] == 0 and r["range_err"] <= 1e-2 and wc >= 0.999, label


def test_layer_from_gguf(torch_cuda, model):
    r = G.Reader(model)
    d, ffn = r.kv["llama.embedding_length"], r.kv["llama.feed_forward_length"]
    nh, nkv = r.kv["llama.attention.head_count"], r.kv["llama.attention.head_count_kv"]
    hd = d // nh
    names = {"q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output", "gate": "ffn_gate",
             "up": "ffn_up", "down": "ffn_down"}
    g = mx.Graph()
    W, shp = {}, {}
    for n, gn in names.items():
        tn = f"blk.1.{gn}.weight"
        t, ne, _, _ = r.tensors[tn]
        assert t == mx.Q4_K
        W[n] = g._new(t, ne, name=tn, data=r.data(tn))
        shp[n] = (ne[1], ne[0])
    x = O.fill_normal((T, d), 0x5EED0601)
    act = O.fill_normal((T, ffn), 0x5EED0602)
    kc = O.f32_to_f16_bits(O.fill_normal((CTX, nkv, hd), 0x5EED0603))
    vc = O.f32_to_f16_bits(O.fill_normal((CTX, nkv, hd), 0x5EED0604))
    j, t_ = np.arange(CTX)[None, :], np.arange(T)[:, None]
    mask = O.f32_to_f16_bits(np.where(j > CTX - T + t_, -np.inf, 0.0).astype(np.float32))
    X = g.new_tensor(mx.F32, [d, T]); A = g.new_tensor(mx.F32, [ffn, T])
    KC = g.new_tensor(mx.F16, [hd, nkv, CTX], "cache_k_l1"); VC = g.new_tensor(mx.F16, [hd, nkv, CTX], "cache_v_l1")
    MK = g.new_tensor(mx.F16, [CTX, T])
    for tt, a in ((X, x), (A, act), (KC, kc), (VC, vc), (MK, mask)):
        g.set(tt, a)
    mm = {n: g.mul_mat(W[n], A if n == "down" else X) for n in ("q", "k", "v", "gate", "up", "down")}
    qv = g.permute_view(mm["q"], [hd, T, nh, 1], [4, d * 4, hd * 4, d * 4 * T])
    kv = g.permute_view(KC, [hd, CTX, nkv, 1], [2, nkv * hd * 2, hd * 2, nkv * hd * 2 * CTX])
    vv = g.permute_view(VC, [hd, CTX, nkv, 1], [2, nkv * hd * 2, hd * 2, nkv * hd * 2 * CTX])
    fa = g.flash_attn_ext(qv, kv, vv, MK, 1.0 / math.sqrt(hd))
    fa2d = g.permute_view(fa, [d, T, 1, 1], [4, d * 4, d * 4 * T, d * 4 * T])
    mm["o"] = g.mul_mat(W["o"], fa2d)
    be = mx.Backend()
    be.set_quant_resident(1)
    for nodes in ([mm["q"], mm["k"], mm["v"]], [fa, fa2d, mm["o"]], [mm["gate"], mm["up"]], [mm["down"]]):
        assert be.compute(nodes) == mx.STATUS_SUCCESS
    assert be.cpu_fallbacks() == 0
    assert be.route_ops("fused-resident") == 5 and be.route_ops("prepacked-q") == 2 and be.route_ops("fa") == 1
    rows = np.sort(np.random.default_rng(3).choice(T, 48, replace=False))
    got = {n: g.get(tt, np.float32, (T, shp[n][0])) for n, tt in mm.items()}
    for n in ("q", "k", "v", "gate", "up", "down"):
        N, K = shp[n]
        src = act if n == "down" else x
        _check(f"{n} [{N} x {K}]", O.mul_mat(O.Q4_K, np.array(r.data(f'blk.1.{names[n]}.weight')), src[rows], N, K),
               got[n][rows])
    attn = g.get(fa, np.float32, (T, nh, hd))
    qh = np.ascontiguousarray(got["q"].reshape(T, nh, hd)[rows].transpose(1, 0, 2))
    kh = np.ascontiguousarray(kc.reshape(CTX, nkv, hd).transpose(1, 0, 2))
    vh = np.ascontiguousarray(vc.reshape(CTX, nkv, hd).transpose(1, 0, 2))
    want = O.flash_attn(qh, kh, vh, np.ascontiguousarray(mask.reshape(T, CTX)[rows]), float(1.0 / math.sqrt(hd)))
    ra = compare(want, attn[rows])
    assert ra["nonfinite"] == 0 and ra["max_abs"] <= 2e-2 and ra["range_err"] <= 1e-2
    N, K = shp["o"]
    _check("o", O.mul_mat(O.Q4_K, np.array(r.data("blk.1.attn_output.weight")), attn.reshape(T, d)[rows], N, K),
           got["o"][rows])
    be.free()


def test_bench_host_path_from_gguf(torch_cuda, model):
    import bench
    out = bench.host_path(argparse.Namespace(layers=2, gguf=model, fa_min_kv=1024))
    print(out, flush=True)
    assert out["cpu_fallbacks"] == 0 and out["value"] > 0
    assert out["config"]["d_model"] == 256 and out["config"]["layers"] == 2
    # three passes (cache fill, timed, per-call split) x 4 micro-batches x 2 layers: Q/K/V and
    # gate/up fused (5 ops), O and down (2); FLASH_ATTN_EXT in the 3 micro-batches with
    # n_kv >= 1024, whose O reads the attention's device copy
    r = out["routes"]
    assert r["fused-resident"] == 3 * 4 * 2 * 5 and r["prepacked-q"] == 3 * 4 * 2 * 2 and r["fa"] == 3 * 3 * 2
    assert out["fa_mirror_hits"] == 3 * 2 and sum(c["MB_up"] + c["MB_down"] for c in out["per_call"].values()) > 0
