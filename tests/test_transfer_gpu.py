"""The host-buffer copy pipeline of graph_compute on the device.

Operands go up through pinned upload slots on the compute stream; results come back through
pinned download slots on a copy stream, queued behind the kernels that produce them and
delivered while later ops of the same call run. These tests pin the rules that keep that
invisible to the host: a FLASH_ATTN_EXT result is read from its device copy by a later MUL_MAT
only while no other node of the call writes over its host bytes and no later attention replaced
it; an op that reads host bytes a queued result has yet to write waits for them; a result that
cannot be copied back is recomputed on the CPU together with every op queued after it; every
dst is written when graph_compute returns. Also: a buffer that grows frees its old bytes in
stream order (nothing waits on other streams), and freeing a backend returns its HBM.
Oracle: the fp64 GEMM and the double attention of oracle.c; bars as in test_backend_gpu.py.
"""
import ctypes
import math

import numpy as np
import pytest

import ggml_mi355x as mx
from oracle import oracle as O
from bars import compare, worst_col_cos, amp_for

pytestmark = pytest.mark.gpu

HD, NH, NKV, T, KV = 128, 2, 1, 64, 256
D = HD * NH


def _w(g, N, K, seed, name):
    W16 = O.f32_to_f16_bits(O.fill_uniform((N, K), seed, 1.0))
    W = g.new_tensor(mx.F16, [K, N], name)
    g.set(W, W16)
    return W, W16


def _attn_inputs(seed):
    q = O.fill_normal((NH, T, HD), seed)
    k = O.f32_to_f16_bits(O.fill_normal((NKV, KV, HD), seed + 1))
    v = O.f32_to_f16_bits(O.fill_normal((NKV, KV, HD), seed + 2))
    j, t = np.arange(KV)[None, :], np.arange(T)[:, None]
    m = O.f32_to_f16_bits(np.where(j > KV - T + t, -np.inf, 0.0).astype(np.float32))
    return q, k, v, m


def _fa(g, q, k, v, m, buf):
    """FLASH_ATTN_EXT over host inputs, its dst [HD, NH, T] in the host bytes `buf`."""
    Q = g.new_tensor(mx.F32, [HD, T, NH])
    K = g.new_tensor(mx.F16, [HD, KV, NKV])
    V = g.new_tensor(mx.F16, [HD, KV, NKV])
    M = g.new_tensor(mx.F16, [KV, T])
    g.set(Q, q), g.set(K, k), g.set(V, v), g.set(M, m)
    fa = g._new(mx.F32, [HD, NH, T], op=mx.OP_FLASH_ATTN_EXT, srcs=(Q, K, V, M), data=buf)
    ctypes.memmove(ctypes.addressof(fa.op_params), (ctypes.c_float * 3)(1.0 / math.sqrt(HD), 0.0, 0.0), 12)
    fa2d = g.permute_view(fa, [D, T, 1, 1], [4, D * 4, D * 4 * T, D * 4 * T])
    return fa, fa2d


def _attn_ref(q, k, v, m, q_mode=0):
    """[T][NH * HD], the layout of the attention's dst (q_mode 1: Q kept in F32, as the CPU
    fallback reads it)"""
    o = O.flash_attn(q, k, v, m.reshape(T, KV), float(1.0 / math.sqrt(HD)), q_mode=q_mode)   # [T][NH][HD]
    return o.reshape(T, D)


def _gemm_ok(label, ref, got):
    r = compare(ref, got)
    wc = worst_col_cos(ref, got)
    print(f"  {label}: nbad={r['nbad']} range_err={r['range_err']:.3g} worst_col={wc:.6f}", flush=True)
    assert r["nbad"] == 0 and r["nonfinite"] == 0 and r["range_err"] <= 1e-2 and wc >= 0.999, label


def _attn_ok(label, ref, got):
    r = compare(ref, got)
    print(f"  {label}: max_abs={r['max_abs']:.3g} range_err={r['range_err']:.3g}", flush=True)
    assert r["nonfinite"] == 0 and r["max_abs"] <= 2e-2 and r["range_err"] <= 1e-2, label


@pytest.fixture
def be(torch_cuda):
    b = mx.Backend()
    yield b
    b.free()


def test_attention_then_o_reads_the_device_copy(be):
    """{FLASH_ATTN_EXT, O}: O takes the attention's device copy (one mirror hit), and both dst
    are delivered."""
    g = mx.Graph()
    q, k, v, m = _attn_inputs(0x7100)
    fa, fa2d = _fa(g, q, k, v, m, np.zeros(D * T * 4, np.uint8))
    Wo, Wo16 = _w(g, D, D, 0x7110, "blk.0.attn_output.weight")
    o = g.mul_mat(Wo, fa2d)
    h0 = be.host_stats()
    assert be.compute([fa, fa2d, o]) == mx.STATUS_SUCCESS
    hs = be.host_stats()
    assert hs["fa_mirror_hits"] - h0["fa_mirror_hits"] == 1 and be.cpu_fallbacks() == 0
    attn = g.get(fa, np.float32, (T, D))
    _attn_ok("attention", _attn_ref(q, k, v, m), attn)
    _gemm_ok("O", O.mul_mat(O.F16, Wo16, attn, D, D), g.get(o, np.float32, (T, D)))


def test_node_over_the_attention_dst_disables_the_device_copy(be):
    """A node of the call that writes over the attention's host bytes: O must read those bytes
    as the host holds them after that node (its result), not the attention's device copy."""
    g = mx.Graph()
    q, k, v, m = _attn_inputs(0x7200)
    buf = np.zeros(D * T * 4, np.uint8)
    fa, fa2d = _fa(g, q, k, v, m, buf)
    W2, W2_16 = _w(g, D, D, 0x7210, "blk.0.other.weight")
    Y = g.new_tensor(mx.F32, [D, T])
    y = O.fill_uniform((T, D), 0x7211, amp_for(D, 1.0))
    g.set(Y, y)
    over = g._new(mx.F32, [D, T], op=mx.OP_MUL_MAT, srcs=(W2, Y), data=buf)   # same host bytes as fa
    Wo, Wo16 = _w(g, D, D, 0x7212, "blk.0.attn_output.weight")
    o = g.mul_mat(Wo, fa2d)
    h0 = be.host_stats()
    assert be.compute([fa, fa2d, over, o]) == mx.STATUS_SUCCESS
    assert be.host_stats()["fa_mirror_hits"] == h0["fa_mirror_hits"] and be.cpu_fallbacks() == 0
    final = g.get(over, np.float32, (T, D))
    _gemm_ok("node over the attention", O.mul_mat(O.F16, W2_16, y, D, D), final)
    _gemm_ok("O over the final host bytes", O.mul_mat(O.F16, Wo16, final, D, D), g.get(o, np.float32, (T, D)))


def test_second_attention_clears_the_device_copy(be):
    """Two attentions, then O reading the first: the device copy held is the second's, so O
    uploads the first's host bytes, which must be delivered before that upload."""
    g = mx.Graph()
    q1, k1, v1, m1 = _attn_inputs(0x7300)
    q2, k2, v2, m2 = _attn_inputs(0x7310)
    fa1, fa1_2d = _fa(g, q1, k1, v1, m1, np.zeros(D * T * 4, np.uint8))
    fa2, _ = _fa(g, q2, k2, v2, m2, np.zeros(D * T * 4, np.uint8))
    Wo, Wo16 = _w(g, D, D, 0x7320, "blk.0.attn_output.weight")
    o = g.mul_mat(Wo, fa1_2d)
    h0 = be.host_stats()
    assert be.compute([fa1, fa2, fa1_2d, o]) == mx.STATUS_SUCCESS
    assert be.host_stats()["fa_mirror_hits"] == h0["fa_mirror_hits"] and be.cpu_fallbacks() == 0
    a1 = g.get(fa1, np.float32, (T, D))
    _attn_ok("first attention", _attn_ref(q1, k1, v1, m1), a1)
    _attn_ok("second attention", _attn_ref(q2, k2, v2, m2), g.get(fa2, np.float32, (T, D)))
    _gemm_ok("O over the first", O.mul_mat(O.F16, Wo16, a1, D, D), g.get(o, np.float32, (T, D)))


def test_chained_mul_mat_reads_a_queued_result(be):
    """Z = W2 . (W1 . X) in one call: Z's upload of Y's host bytes waits for Y's queued
    download."""
    g = mx.Graph()
    K, N1, N2, M = 512, 768, 384, 320
    W1, W1_16 = _w(g, N1, K, 0x7400, "blk.0.a.weight")
    W2, W2_16 = _w(g, N2, N1, 0x7401, "blk.0.b.weight")
    X = g.new_tensor(mx.F32, [K, M])
    x = O.fill_uniform((M, K), 0x7402, amp_for(K, 1.0))
    g.set(X, x)
    y = g.mul_mat(W1, X)
    z = g.mul_mat(W2, y)
    assert be.compute([y, z]) == mx.STATUS_SUCCESS and be.cpu_fallbacks() == 0
    yh = g.get(y, np.float32, (M, N1))
    _gemm_ok("Y", O.mul_mat(O.F16, W1_16, x, N1, K), yh)
    _gemm_ok("Z over the delivered Y", O.mul_mat(O.F16, W2_16, yh, N2, N1), g.get(z, np.float32, (M, N2)))


def test_failed_copyback_recomputes_on_the_cpu(be):
    """The attention's first result piece reports a failed copy-back: the attention and the O
    queued after it (which read its device copy) are recomputed on the CPU, counted as
    fallbacks, with correct results; the next call runs on the device again."""
    g = mx.Graph()
    q, k, v, m = _attn_inputs(0x7500)
    fa, fa2d = _fa(g, q, k, v, m, np.zeros(D * T * 4, np.uint8))
    Wo, Wo16 = _w(g, D, D, 0x7510, "blk.0.attn_output.weight")
    o = g.mul_mat(Wo, fa2d)
    fb0, h0 = be.cpu_fallbacks(), be.host_stats()
    be.inject_faults("copyback", 1)
    assert be.compute([fa, fa2d, o]) == mx.STATUS_SUCCESS
    assert be.cpu_fallbacks() - fb0 == 2 and be.host_stats()["copyback_redone"] - h0["copyback_redone"] == 2
    attn = g.get(fa, np.float32, (T, D))
    assert compare(_attn_ref(q, k, v, m, q_mode=1), attn)["max_abs"] <= 1e-5   # the CPU's double attention
    assert compare(O.mul_mat(O.F16, Wo16, attn, D, D), g.get(o, np.float32, (T, D)))["range_err"] <= 1e-5
    fb1 = be.cpu_fallbacks()
    g.set(o, np.zeros((T, D), np.float32))
    assert be.compute([fa, fa2d, o]) == mx.STATUS_SUCCESS and be.cpu_fallbacks() == fb1
    _gemm_ok("O on the device again", O.mul_mat(O.F16, Wo16, attn, D, D), g.get(o, np.float32, (T, D)))


def test_buffer_growth_does_not_wait_for_other_streams(torch_cuda):
    """A backend whose buffers grow frees the old ones in its own stream's order: with ~0.5 s of
    GEMMs queued on another stream, a call that regrows the activation, pack and output buffers
    returns while that work is still running (a device-wide synchronization would have waited
    for all of it)."""
    torch = torch_cuda
    be = mx.Backend()
    K, N = 512, 256
    W16 = O.f32_to_f16_bits(O.fill_uniform((N, K), 0x7600, 1.0))

    def call(M):
        g = mx.Graph()
        W = g.new_tensor(mx.F16, [K, N], "blk.0.grow.weight")
        g.set(W, W16)
        X = g.new_tensor(mx.F32, [K, M])
        x = O.fill_uniform((M, K), 0x7601 + M, amp_for(K, 1.0))
        g.set(X, x)
        d = g.mul_mat(W, X)
        assert be.compute([d]) == mx.STATUS_SUCCESS
        return x, g.get(d, np.float32, (M, N))

    call(64)                                   # staging, streams, first buffers
    a = torch.randn(8192, 8192, device="cuda", dtype=torch.float16)
    b = torch.randn(8192, 8192, device="cuda", dtype=torch.float16)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        for _ in range(3):                   # the library's first calls pick and load kernels
            torch.mm(a, b)
        side.synchronize()
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record()
        for _ in range(8):
            torch.mm(a, b)
        s1.record()
    s1.synchronize()
    per = s0.elapsed_time(s1) / 8            # ms per GEMM
    n = min(4000, max(8, int(500.0 / per)))
    with torch.cuda.stream(side):
        for _ in range(n):
            torch.mm(a, b)
        busy_until = torch.cuda.Event()
        busy_until.record()
    x, got = call(4096)                        # act, a16, scales and out regrow
    still_busy = not busy_until.query()
    side.synchronize()
    print(f"  {n} side GEMMs of {per:.2f} ms queued; side stream still busy after the call: {still_busy}", flush=True)
    assert still_busy
    assert be.cpu_fallbacks() == 0
    _gemm_ok("regrown call", O.mul_mat(O.F16, W16, x, N, K), got)
    be.free()


def test_free_returns_the_decode_first_scratch(torch_cuda):
    """init, a MUL_MAT that takes the decode-first form (its tiled fp16 weight in per-call
    scratch), free: three times over, device free memory comes back to where it started."""
    torch = torch_cuda
    K, N, M = 3072, 3072, 512
    L = mx.lib()
    assert L.mi355x_mul_mat_decode_first(O.Q6_K, M, N, K) == 1
    Wq = O.quantize(O.Q6_K, O.fill_normal((N, K), 0x7700, 0.0, 0.02))
    x = O.fill_normal((M, K), 0x7701)
    ref = None
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for i in range(3):
        be = mx.Backend()
        be.set_quant_resident(0)
        g = mx.Graph()
        W = g.new_tensor(O.Q6_K, [K, N], "blk.0.ffn_up.weight")
        g.set(W, Wq)
        X = g.new_tensor(mx.F32, [K, M])
        g.set(X, x)
        d = g.mul_mat(W, X)
        assert be.compute([d]) == mx.STATUS_SUCCESS
        assert be.route_ops("mt") == 1 and be.cpu_fallbacks() == 0
        if ref is None:
            ref = O.mul_mat(O.Q6_K, Wq, x[:64], N, K)
            _gemm_ok("decode-first Q6_K", ref, g.get(d, np.float32, (M, N))[:64])
        be.free()
        torch.cuda.synchronize()
        free = torch.cuda.mem_get_info()[0]
        print(f"  round {i}: free HBM {free / 2**20:.0f} MiB (start {free0 / 2**20:.0f} MiB)", flush=True)
        assert free >= free0 - (16 << 20), (i, free0, free)


@pytest.mark.parametrize("K,Ns,M,chunk", [(512, (768, 384), 520, 128), (14336, (4096,), 512, 128),
                                          (4096, (6144,), 512, 256)])
def test_row_chunked_mul_mat(torch_cuda, monkeypatch, K, Ns, M, chunk):
    """MI355X_ROW_CHUNK: a MUL_MAT (or fused group) whose activations are uploaded runs in chunks
    of rows, each chunk's upload, pack, GEMM and download overlapping its neighbours'; every dst
    row lands where the unchunked call puts it (ragged last chunk included), within the MUL_MAT
    bars of the fp64 oracle on sampled rows; the K-split accumulate form (deep K) included."""
    monkeypatch.setenv("MI355X_ROW_CHUNK", str(chunk))
    be = mx.Backend()
    g = mx.Graph()
    Ws = [_w(g, N, K, 0x7800 + i, f"blk.0.chunked{i}.weight") for i, N in enumerate(Ns)]
    X = g.new_tensor(mx.F32, [K, M])
    x = O.fill_uniform((M, K), 0x7810, amp_for(K, 1.0))
    g.set(X, x)
    ds = [g.mul_mat(W, X) for W, _ in Ws]
    assert be.compute(ds) == mx.STATUS_SUCCESS and be.cpu_fallbacks() == 0
    rows = np.unique(np.r_[0, chunk - 1, chunk, M - 1, np.random.default_rng(5).choice(M, 24, replace=False)])
    for (W, W16), d, N in zip(Ws, ds, Ns):
        got = g.get(d, np.float32, (M, N))
        _gemm_ok(f"chunked {chunk} rows N {N} K {K}", O.mul_mat(O.F16, W16, x[rows], N, K), got[rows])
    be.free()
