"""mi355x_mul_mat_noalloc (no counterpart in the reference: an entry for callers that cannot
allocate) against mi355x_mul_mat, the entry it wraps, through the C ABI: two calls in a row on
the shared static scratch, the second with a smaller input, each checked against mi355x_mul_mat
on the same inputs (bit-identical: both sum their K splits in a fixed order and the scratch holds
the partials of the split mi355x_mul_mat_workspace_for sizes) and against the oracle's fp64 GEMM with the MUL_MAT bars. A
workspace past the static scratch is refused with MI355X_E_NOMEM before anything launches."""
import numpy as np
import pytest

import ggml_mi355x as mx
from oracle import oracle as O
from bars import compare, worst_col_cos

pytestmark = pytest.mark.gpu


def _case(torch, wt, N, K, M, seed):
    W = O.fill_normal((N, K), seed, 0.0, 0.02)
    P = O.quantize(wt, W) if wt != O.F16 else O.f32_to_f16_bits(W)
    X = O.fill_normal((M, K), seed + 1)
    w = mx.upload_weight(wt, P, N, K)
    x = torch.from_numpy(X).cuda()
    return P, X, w, x


def test_noalloc_matches_mul_mat(torch_cuda):
    torch = torch_cuda
    L = mx.lib()
    assert hasattr(L, "mi355x_mul_mat_noalloc")
    # (wtype, N, K, M): the first call the larger; the second smaller, on the same scratch
    for wt, N, K, M in ((O.Q4_K, 4096, 4096, 512), (O.Q8_0, 1024, 2048, 96), (O.F16, 2048, 1024, 300)):
        P, X, w, x = _case(torch, wt, N, K, M, 9100 + M)
        got = torch.full((M, N), float("nan"), device="cuda")
        st = mx.mul_mat_noalloc(wt, w, N, K, x, got)
        assert st == mx.OK, mx.status_str(st)
        want = mx.mul_mat(wt, w, N, K, x)
        torch.cuda.synchronize()
        g, e = got.cpu().numpy(), want.cpu().numpy()
        assert np.isfinite(g).all()
        d = float(np.abs(g - e).max())
        print(f"type {wt} N={N} K={K} M={M}: max |noalloc - mul_mat| = {d:.3g}", flush=True)
        assert d == 0.0
        ref = O.mul_mat(wt, P, X, N, K)
        r = compare(ref, g)
        assert r["nbad"] == 0 and r["range_err"] <= 1e-2 and worst_col_cos(ref, g) >= 0.999


def test_noalloc_when_the_decoded_weight_does_not_fit(torch_cuda):
    """Q6_K 8192 x 4096 at M 512: mi355x_mul_mat with mi355x_mul_mat_workspace_for bytes decodes
    the weight into tiled fp16 first (4 MiB of pack + 64 MiB of fp16 weight), which the 64 MiB
    static scratch cannot hold, so the no-allocation entry decodes inside the GEMM instead. Both
    forms against the oracle's fp64 GEMM on sampled rows, with the MUL_MAT bars (not bit equality:
    the two forms round in a different order)."""
    torch = torch_cuda
    L = mx.lib()
    wt, N, K, M = O.Q6_K, 8192, 4096, 512
    assert L.mi355x_mul_mat_decode_first(wt, M, N, K) == 1
    assert int(L.mi355x_mul_mat_workspace_for(wt, N, K, M)) > (64 << 20) >= int(L.mi355x_mul_mat_workspace(M, K))
    P, X, w, x = _case(torch, wt, N, K, M, 9300)
    got = torch.full((M, N), float("nan"), device="cuda")
    st = mx.mul_mat_noalloc(wt, w, N, K, x, got)
    assert st == mx.OK, mx.status_str(st)
    first = mx.mul_mat(wt, w, N, K, x)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(93).choice(M, 40, replace=False))
    ref = O.mul_mat(wt, P, X[rows], N, K)
    for label, out in (("noalloc (in-GEMM decode)", got), ("mul_mat (decode first)", first)):
        g = out.cpu().numpy()[rows]
        r = compare(ref, g)
        print(f"{label}: nbad={r['nbad']} range_err={r['range_err']:.3g}", flush=True)
        assert np.isfinite(g).all() and r["nbad"] == 0 and r["range_err"] <= 1e-2 and worst_col_cos(ref, g) >= 0.999


def test_noalloc_refuses_past_scratch(torch_cuda):
    torch = torch_cuda
    K, N = 14336, 256
    M = 4096                                   # 4096 x 14336 fp16 = 112 MiB > 64 MiB
    assert mx.lib().mi355x_mul_mat_workspace(M, K) > (64 << 20)
    w = torch.zeros(N * K, dtype=torch.float16, device="cuda")
    x = torch.zeros(M, K, device="cuda")
    out = torch.full((M, N), 7.0, device="cuda")
    assert mx.mul_mat_noalloc(O.F16, w, N, K, x, out) == mx.E_NOMEM
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())            # nothing launched
