"""MUL_MAT_ID on the GPU against the oracle, through the C ABI.

Cases follow test-rocket-moe.cpp (F16 and quantized expert stacks, both b forms ne11 = 1 and
ne11 = n_used, pad rows, 16 experts / 4 used, skewed routing with the last expert empty,
outlier activation channels, one weight upload serving several token counts) plus the MoE prefill
shape: 128 experts, top-8 routing from a softmax over seeded N(0,1) router logits, 512 tokens,
d_model 2048, expert FFN 768, gate/up/down Q4_K, and the reference's MXFP4 (gpt-oss) stacks,
decoded exactly to fp16 here (the reference merges block exponents onto int8 codes instead, so
its bars hold with room).
Bars: the element bar, aggregate cosine, worst row / column cosine at 1 - 10 (1 - floor)
(test-rocket-moe.cpp:200-219, 279-289), and max|d|/max|ref| <= 1e-2.
"""
import numpy as np
import pytest

from oracle import oracle as O
from bars import compare, worst_col_cos, worst_row_cos

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mx(torch_cuda):
    import ggml_mi355x
    ggml_mi355x.lib()
    return ggml_mi355x


def make_ids(T, U, E):
    t = np.arange(T)[:, None]
    s = np.arange(U)[None, :]
    return ((t * 3 + s * 7 + t // 5) % (E - 1)).astype(np.int32)   # last expert stays empty


def make_input(T, ne11, K):
    X = O.fill_uniform((T, ne11, K), 2000 + K, 0.25)
    X[..., (np.arange(K) % 97) == 13] *= 20.0                    # ~1% outlier channels
    return X


def expert_payload(wtype, E, N, K, seed0=1000, wide=False):
    W = np.stack([O.fill_uniform((N, K), seed0 + e, 0.3) for e in range(E)])
    if wide:   # a 9-octave spread of block magnitudes (test-rocket-moe.cpp's WIDE weights)
        oct_ = (np.arange(E * N * K // 32).reshape(E, N, K // 32) * 7919) % 9
        W = (W.reshape(E, N, K // 32, 32) * np.exp2(-oct_.astype(np.float32))[..., None]).reshape(E, N, K)
        W = W.astype(np.float32)
    if wtype == O.F16:
        return O.f32_to_f16_bits(W)
    return O.quantize(wtype, W)


def topk_ids(T, E, k, seed):
    logits = O.fill_normal((T, E), seed)
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    # top-k, ties to the lowest index: stable sort on -p
    return np.argsort(-p, axis=1, kind="stable")[:, :k].astype(np.int32)


def run(mx, wtype, payload, E, N, K, X, ids, w_dev=None):
    import torch
    if w_dev is None:
        w_dev = mx.upload_weight(wtype, payload, E * N, K)
    out = mx.mul_mat_id(wtype, w_dev, E, N, K, torch.from_numpy(X).cuda(), torch.from_numpy(ids).cuda())
    torch.cuda.synchronize()
    return out.cpu().numpy(), w_dev


def check_bars(ref, got, N, floor, label):
    r = compare(ref, got)
    part = 1.0 - 10.0 * (1.0 - floor)
    R = ref.size // N
    rc = worst_row_cos(ref.reshape(R, N), got.reshape(R, N))
    cc = worst_col_cos(ref.reshape(R, N), got.reshape(R, N))
    print(f"{label}: cos={r['cos']:.7f} nbad={r['nbad']} range_err={r['range_err']:.3g} "
          f"worst row {rc:.6f} worst col {cc:.6f}")
    assert r["nonfinite"] == 0 and r["nbad"] == 0, label
    assert r["cos"] >= floor and rc >= part and cc >= part, label
    assert r["range_err"] <= 1e-2, label


# (K, N, E, ne11, U, T, wtype, floor, wide) -- test-rocket-moe.cpp:200-219
CASES = [
    (256, 128, 8, 1, 2, 64, O.F16, 0.9999, False),
    (256, 128, 8, 2, 2, 64, O.F16, 0.9999, False),
    (256, 128, 8, 1, 2, 66, O.F16, 0.9999, False),
    (256, 128, 16, 1, 4, 96, O.F16, 0.9999, False),
    (256, 128, 8, 1, 2, 64, O.MXFP4, 0.9990, False),
    (256, 128, 8, 2, 2, 64, O.MXFP4, 0.9990, False),
    (1152, 128, 8, 1, 2, 64, O.MXFP4, 0.9990, False),
    (2048, 128, 8, 1, 2, 66, O.MXFP4, 0.9990, False),
    (1152, 128, 8, 1, 2, 64, O.MXFP4, 0.9985, True),
    (1024, 128, 8, 1, 2, 64, O.Q4_K, 0.9990, False),
    (1152, 128, 8, 2, 2, 64, O.Q8_0, 0.9990, False),
    (512, 256, 8, 2, 4, 80, O.Q6_K, 0.9990, False),
    (1152, 128, 8, 2, 2, 64, O.Q4_0, 0.9985, False),
    (1024, 128, 8, 1, 2, 66, O.Q5_K, 0.9990, False),
]


@pytest.mark.parametrize("K,N,E,ne11,U,T,wtype,floor,wide", CASES)
def test_moe_reference_cases(mx, K, N, E, ne11, U, T, wtype, floor, wide):
    P = expert_payload(wtype, E, N, K, wide=wide)
    X = make_input(T, ne11, K)
    ids = make_ids(T, U, E)
    got, _ = run(mx, wtype, P, E, N, K, X, ids)
    ref = O.mul_mat_id(wtype, P, K, N, E, X, ne11, ids)
    check_bars(ref, got, N, floor, f"moe {O.TYPE_NAMES[wtype]} K={K} T={T}")


def test_moe_one_upload_serves_every_token_count(mx):
    """test-rocket-moe.cpp:299-361: one weight, micro-batches of 64/130/96/258 tokens."""
    K, N, E, U = 1024, 128, 8, 2
    P = expert_payload(O.Q4_K, E, N, K, seed0=3000)
    w = None
    for T in (64, 130, 96, 258):
        X = make_input(T, 1, K)
        ids = make_ids(T, U, E)
        got, w = run(mx, O.Q4_K, P, E, N, K, X, ids, w_dev=w)
        ref = O.mul_mat_id(O.Q4_K, P, K, N, E, X, 1, ids)
        check_bars(ref, got, N, 0.999, f"cross-M T={T}")


def test_moe_bad_id_flags_error(mx):
    import torch
    K, N, E, U, T = 256, 64, 4, 2, 16
    P = expert_payload(O.F16, E, N, K)
    X = make_input(T, 1, K)
    ids = make_ids(T, U, E)
    ids[3, 1] = E                   # out of range
    w = mx.upload_weight(O.F16, P, E * N, K)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    out = torch.full((T, U, N), 7.0, dtype=torch.float32, device="cuda")
    mx.mul_mat_id(O.F16, w, E, N, K, torch.from_numpy(X).cuda(), torch.from_numpy(ids).cuda(), out=out, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 1
    o = out.cpu().numpy()
    assert np.all(o[3, 1] == 7.0)                  # the bad row is left unwritten
    good = ids.copy()
    good[3, 1] = 0
    ref = O.mul_mat_id(O.F16, P, K, N, E, X, 1, good)
    mask = np.ones((T, U), bool)
    mask[3, 1] = False
    assert compare(ref[mask], o[mask])["range_err"] <= 1e-2


X32_LAYOUTS = [("Q4_K", "Q4_K_X"), ("Q8_0", "Q8_0_X"), ("Q6_K", "Q6_K_X"), ("MXFP4", "MXFP4_X")]


@pytest.mark.parametrize("base_name,x_name", X32_LAYOUTS)
@pytest.mark.parametrize("K,N,E,ne11,U,T", [(1024, 128, 8, 1, 2, 64), (2048, 96, 8, 2, 2, 66), (768, 2048, 4, 8, 2, 40)])
def test_moe_x32_layout(mx, K, N, E, ne11, U, T, base_name, x_name):
    """Expert stacks regrouped by 32 rows (Q4_K_X, Q8_0_X, Q6_K_X, MXFP4_X) give the same bits as the
    layout of their base type (same decode, same MFMA order; only where the bytes sit differs),
    and meet the oracle's bars; N = 96 leaves a partial 128-column block."""
    wt = getattr(O, base_name)
    P = expert_payload(wt, E, N, K)
    X = make_input(T, ne11, K)
    ids = make_ids(T, U, E)
    base, _ = run(mx, wt, P, E, N, K, X, ids)
    got, _ = run(mx, getattr(mx, x_name), P, E, N, K, X, ids)
    assert np.array_equal(base.view(np.uint32), got.view(np.uint32))
    ref = O.mul_mat_id(wt, P, K, N, E, X, ne11, ids)
    check_bars(ref, got, N, 0.9990, f"moe {x_name} K={K} N={N} T={T}")


@pytest.mark.parametrize("base_name,x_name", [("F16", None), ("Q4_0", None), ("Q8_0", "Q8_0_X"), ("MXFP4", "MXFP4_X")])
def test_moe_k_ending_mid_slab(mx, base_name, x_name):
    """K = 1056 ends half-way through the expert GEMM's last 64-deep slab (32-value blocks): the
    chunks past K read zeros and the weights there decode to zero, in the row-strided layouts and
    the regrouped ones alike (the same bits), within the oracle's bars."""
    K, N, E, ne11, U, T = 1056, 64, 8, 2, 2, 40
    wt = getattr(O, base_name)
    P = expert_payload(wt, E, N, K)
    X = make_input(T, ne11, K)
    ids = make_ids(T, U, E)
    base, _ = run(mx, wt, P, E, N, K, X, ids)
    ref = O.mul_mat_id(wt, P, K, N, E, X, ne11, ids)
    check_bars(ref, base, N, 0.9985, f"moe {base_name} K={K}")
    if x_name:
        got, _ = run(mx, getattr(mx, x_name), P, E, N, K, X, ids)
        assert np.array_equal(base.view(np.uint32), got.view(np.uint32))


@pytest.mark.parametrize("layout", ["q4_k", "q4_k_x"])
@pytest.mark.parametrize("proj", ["gate", "up", "down"])
def test_moe_baseline_shape(mx, proj, layout):
    """128 experts, top-8 of a softmax over N(0,1) router logits, 512 tokens, d_model 2048,
    expert FFN 768; expert weights Q4_K from N(0,0.02), activations N(0,1)."""
    E, T, U, D, F = 128, 512, 8, 2048, 768
    ids = topk_ids(T, E, U, 0x5EED0000 + 64)
    if proj == "down":
        N, K, ne11 = D, F, U
    else:
        N, K, ne11 = F, D, 1
    seed = 0x5EED0000 + 65 + ("gate", "up", "down").index(proj)
    W = O.fill_normal((E, N, K), seed, 0.0, 0.02)
    P = O.quantize(O.Q4_K, W)
    X = O.fill_normal((T, ne11, K), seed + 8)
    got, _ = run(mx, O.Q4_K if layout == "q4_k" else mx.Q4_K_X, P, E, N, K, X, ids)
    # the oracle on a sample of 64 tokens (every slot of each)
    toks = np.unique(np.linspace(0, T - 1, 64).astype(int))
    ref = O.mul_mat_id(O.Q4_K, P, K, N, E, np.ascontiguousarray(X[toks]), ne11, np.ascontiguousarray(ids[toks]))
    check_bars(ref, got[toks], N, 0.9999, f"baseline {proj}")
