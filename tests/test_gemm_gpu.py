"""MUL_MAT on the GPU against the CPU oracle, through the C ABI.

Cases follow test-rocket-matmul.cpp: its F16 shapes (incl. M not a multiple of 4), the
outlier-row case, the fused shared-src1 groups, its quantized shapes, plus the single-op shapes:
the F16 [8192 x 2048] x [512 x 2048] case and the Q8_0 / Q4_K / Q6_K sweep, and the Q4_0 / Q5_K
decoders on the same shapes. Bars (tests/bars.py):
the element bar, worst-column cosine >= 0.999, and max|d|/max|ref| <= 1e-2.
"""
import numpy as np
import pytest

from oracle import oracle as O
from bars import compare, worst_col_cos, amp_for

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mx(torch_cuda):
    import ggml_mi355x
    ggml_mi355x.lib()
    return ggml_mi355x


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _run_mul_mat(mx, wtype, payload, N, K, X):
    import torch
    w = mx.upload_weight(wtype, payload, N, K)
    out = mx.mul_mat(wtype, w, N, K, _dev(X))
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _assert_bars(ref, got, M, N, label, cos_floor=0.999, range_tol=1e-2):
    r = compare(ref, got)
    wc = worst_col_cos(ref.reshape(M, N), got.reshape(M, N))
    print(f"{label}: nbad={r['nbad']} max_abs={r['max_abs']:.4g} range_err={r['range_err']:.3g} "
          f"worst_col_cos={wc:.6f}")
    assert r["nonfinite"] == 0, label
    assert r["nbad"] == 0, label
    assert wc >= cos_floor, label
    assert r["range_err"] <= range_tol, label


def test_pack_act_bitexact(mx):
    X = O.fill_normal((67, 512), 7)
    X[3] *= 3000.0                 # outlier row
    X[5] = 0.0                     # zero row -> scale 1
    X[9, 17] = 1e6                 # a value past fp16 range before scaling
    a16, sc = mx.pack_act(_dev(X))
    want_a, want_s = O.pack_act(X)
    got_a = a16.cpu().numpy().view(np.uint16)
    assert np.array_equal(sc.cpu().numpy(), want_s)
    assert np.array_equal(got_a, want_a)


@pytest.mark.parametrize("K", [4, 764, 2048, 4096, 4100, 14336])
@pytest.mark.parametrize("form", ["wave", "block"])
@pytest.mark.parametrize("tiled", [False, True])
def test_pack_act_forms_bitexact(mx, monkeypatch, K, form, tiled):
    """Both forms of the activation pack (one wave a row up to 4096 values, one block a row past
    that or with MI355X_PACK_WAVE_K=0) against the oracle's pack, row-major and tiled, with an
    outlier row, a zero row and a value past fp16 range; the clearing variant leaves exactly the
    columns it is asked to clear at zero."""
    import torch
    if tiled and K % 32:
        pytest.skip("the tiled layout needs K % 32 == 0")
    monkeypatch.setenv("MI355X_PACK_WAVE_K", "4096" if form == "wave" else "0")
    M = 37
    X = O.fill_normal((M, K), 8 + K)
    X[3] *= 3000.0
    X[5] = 0.0
    X[9, K // 2] = 1e6
    a16, sc = mx.pack_act(_dev(X), tiled=tiled)
    want_a, want_s = O.pack_act(X)
    got = a16.cpu().numpy().view(np.uint16)
    if tiled:   # tile (r / 16, k / 32) of 16 x 32 values, row-major inside
        rows = got.shape[0]
        got = got.reshape(rows // 16, K // 32, 16, 32).transpose(0, 2, 1, 3).reshape(rows, K)[:M]
    assert np.array_equal(sc.cpu().numpy(), want_s)
    assert np.array_equal(got, want_a)
    if not tiled:
        L = mx.lib()
        a2 = torch.empty((M, K), dtype=torch.float16, device="cuda")
        s2 = torch.empty((M,), dtype=torch.float32, device="cuda")
        z = torch.full((M, 40), 7.0, device="cuda")
        x = _dev(X)
        st = L.mi355x_pack_act_clear(0, mx._ptr(x), K, M, K, mx._ptr(a2), mx._ptr(s2), mx._ptr(z), 40, 33,
                                     mx.stream_handle())
        assert st == mx.OK
        torch.cuda.synchronize()
        zz = z.cpu().numpy()
        assert np.all(zz[:, :33] == 0.0) and np.all(zz[:, 33:] == 7.0)
        assert np.array_equal(a2.cpu().numpy().view(np.uint16), want_a)


@pytest.mark.parametrize("wtype", [O.F16, O.Q8_0, O.Q4_0, O.Q4_K, O.Q5_K, O.Q6_K, O.MXFP4])
def test_dequant_f16_bitexact(mx, wtype):
    N, K = 96, 1024
    W = O.fill_normal((N, K), 11 + wtype, 0.0, 0.02)
    W[0, :256] *= 50.0             # a wide block
    W[1, :] = 0.0                  # an all-zero row
    W[2, 5] = -3.0                 # one extreme value
    if wtype == O.F16:
        payload = O.f32_to_f16_bits(W)
        want = payload
    else:
        payload = O.quantize(wtype, W)
        want = O.dequantize_f16(wtype, payload, K)
    w = mx.upload_weight(wtype, payload, N, K)
    got = mx.dequant_f16(wtype, w, N, K).cpu().numpy().view(np.uint16)
    assert np.array_equal(got, want.reshape(N, K))


F16_SHAPES = [(64, 32, 8), (384, 256, 256), (3840, 4096, 512), (64, 64, 7), (384, 256, 130),
              (3840, 4096, 250)]


@pytest.mark.parametrize("K,N,M", F16_SHAPES)
def test_mul_mat_f16_shapes(mx, K, N, M):
    Wf = O.fill_uniform((N, K), 101 + K, 1.0)
    Xf = O.fill_uniform((M, K), 202 + M, amp_for(K, 1.0))
    W16 = O.f32_to_f16_bits(Wf)
    ref = O.mul_mat(O.F16, W16, Xf, N, K)
    got = _run_mul_mat(mx, O.F16, W16, N, K, Xf)
    _assert_bars(ref, got, M, N, f"F16 K={K} N={N} M={M}")


def test_outlier_row(mx):
    """test-rocket-matmul.cpp:181-221: an outlier row must not crush the other rows."""
    K, N, M = 256, 64, 8
    i = np.arange(K * N)
    Wf = ((((i * 7) % 13) - 6) * 0.05).astype(np.float32).reshape(N, K)
    j = np.arange(K * M)
    Xf = ((((j * 5) % 11) - 5) * 0.02).astype(np.float32).reshape(M, K)
    Xf[3] = ((np.arange(K) % 7) - 3) * 300.0
    W16 = O.f32_to_f16_bits(Wf)
    ref = O.mul_mat(O.F16, W16, Xf, N, K)
    got = _run_mul_mat(mx, O.F16, W16, N, K, Xf)
    assert np.isfinite(got).all()
    small = np.delete(np.arange(M), 3)
    rd = np.abs(got[small] - ref[small]) / (np.abs(ref[small]) + 1e-6)
    assert rd.max() < 0.05


def test_cfg_f16_8192x2048_m512(mx):
    """F16 weight [N=8192, K=2048] ~N(0,0.02), F32 activations [512, 2048] ~N(0,1)."""
    K, N, M = 2048, 8192, 512
    W16 = O.f32_to_f16_bits(O.fill_normal((N, K), 0x5EED0000 + 16, 0.0, 0.02))
    Xf = O.fill_normal((M, K), 0x5EED0000 + 16 + 8)
    ref = O.mul_mat(O.F16, W16, Xf, N, K)
    got = _run_mul_mat(mx, O.F16, W16, N, K, Xf)
    _assert_bars(ref, got, M, N, "F16 cfg 8192x2048 M=512")


QSHAPES = [(256, 128, 64, O.Q8_0), (3840, 256, 128, O.Q8_0), (256, 128, 64, O.Q4_K),
           (3840, 256, 128, O.Q4_K), (512, 256, 128, O.Q6_K), (2880, 256, 128, O.MXFP4),
           (256, 128, 64, O.Q4_0), (2880, 256, 128, O.Q4_0), (256, 128, 64, O.Q5_K), (3840, 256, 128, O.Q5_K)]


@pytest.mark.parametrize("K,N,M,wtype", QSHAPES)
def test_mul_mat_quant_reference_shapes(mx, K, N, M, wtype):
    """test-rocket-matmul.cpp:316-366: golden = fp64 dot of the dequantized weight."""
    i = np.arange(N * K, dtype=np.float32)
    Wf = (np.sin(i * np.float32(0.013)) * np.float32(0.5)).astype(np.float32).reshape(N, K)
    Xf = O.fill_uniform((M, K), 505 + K, amp_for(K, 0.61))
    Q = O.quantize(wtype, Wf)
    ref = O.mul_mat(wtype, Q, Xf, N, K)
    got = _run_mul_mat(mx, wtype, Q, N, K, Xf)
    r = compare(ref, got)
    assert r["nbad"] == 0 and r["nonfinite"] == 0
    assert r["range_err"] <= 1e-2


# The quantized sweep at its full sizes. The oracle runs on a sample of 48 activation rows (an
# exact subset of the output), so the check stays seconds long at M = 2048.
SWEEP = [(K, N, M, t) for t in (O.Q8_0, O.Q4_K, O.Q6_K)
         for (K, N) in ((3072, 3072), (3072, 8192), (8192, 3072)) for M in (32, 128, 512, 2048)]


@pytest.mark.parametrize("K,N,M,wtype", SWEEP)
def test_mul_mat_quant_sweep(mx, K, N, M, wtype):
    W = O.fill_normal((N, K), 0x5EED0000 + 32 + wtype, 0.0, 0.02)
    Xf = O.fill_normal((M, K), 0x5EED0000 + 40 + M)
    Q = O.quantize(wtype, W)
    got = _run_mul_mat(mx, wtype, Q, N, K, Xf)
    rows = np.unique(np.linspace(0, M - 1, min(M, 48)).astype(int))
    ref = O.mul_mat(wtype, Q, Xf[rows], N, K)
    _assert_bars(ref, got[rows], len(rows), N, f"{O.TYPE_NAMES[wtype]} K={K} N={N} M={M}")


@pytest.mark.parametrize("wtype,M,N,K", [(O.Q6_K, 512, 768, 1024), (O.Q8_0, 1024, 512, 2048),
                                         (O.Q8_0, 512, 8192, 3072), (O.Q5_K, 512, 384, 768),
                                         (O.MXFP4, 512, 256, 512), (O.Q4_0, 512, 512, 256),
                                         (O.Q4_K, 512, 512, 256),
                                         # ragged: M off the 16-row groups of the tiled pack, N off the
                                         # 32 / 128-row tiles (N % 16 == 0, as every MUL_MAT here takes)
                                         (O.Q6_K, 520, 112, 256), (O.Q8_0, 530, 208, 192)])
def test_mul_mat_decode_first(mx, wtype, M, N, K):
    """Q6_K / Q5_K / MXFP4 / Q8_0 / Q4_0 / Q4_K at M >= 512: with mi355x_mul_mat_workspace_for bytes the weight is decoded once
    into tiled fp16 in the workspace and multiplied by the fp16 GEMM; with only the pack's bytes it
    is decoded inside the GEMM. Both forms meet the oracle's bars and agree with each other to
    fp32 summation order (same fp16 weights and activations)."""
    import ctypes
    import torch
    W = O.fill_normal((N, K), 0x5EED0100 + wtype, 0.0, 0.02)
    Xf = O.fill_normal((M, K), 0x5EED0200 + M)
    Q = O.quantize(wtype, W)
    w = mx.upload_weight(wtype, Q, N, K)
    L = mx.lib()
    x = _dev(Xf)
    outs = []
    for nbytes in (int(L.mi355x_mul_mat_workspace_for(wtype, N, K, M)), int(L.mi355x_mul_mat_workspace(M, K))):
        ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        out = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        mx.check(L.mi355x_mul_mat(wtype, ctypes.c_void_p(w.data_ptr()), N, K, ctypes.c_void_p(x.data_ptr()), K, M,
                                  ctypes.c_void_p(out.data_ptr()), N, ctypes.c_void_p(ws.data_ptr()), nbytes,
                                  mx.stream_handle()), "mul_mat")
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    first, in_gemm = outs
    assert int(L.mi355x_mul_mat_workspace_for(wtype, N, K, M)) >= int(L.mi355x_mul_mat_workspace(M, K)) + 2 * N * K
    rows = np.unique(np.linspace(0, M - 1, 48).astype(int))
    ref = O.mul_mat(wtype, Q, Xf[rows], N, K)
    _assert_bars(ref, first[rows], len(rows), N, f"{O.TYPE_NAMES[wtype]} decode-first M={M}")
    _assert_bars(ref, in_gemm[rows], len(rows), N, f"{O.TYPE_NAMES[wtype]} in-GEMM decode M={M}")
    assert np.abs(first - in_gemm).max() <= 1e-5 * np.abs(in_gemm).max()


@pytest.mark.parametrize("Ns", [(4096, 4096), (4096, 2048, 2048)])
def test_fused_group(mx, Ns):
    """test-rocket-matmul.cpp:259-314: members sharing src1 in one launch over concatenated N."""
    import torch
    K, M = 3840, 128
    Xf = O.fill_uniform((M, K), 303, amp_for(K, 1.0))
    a16, sc = mx.pack_act(_dev(Xf))
    outs, refs = [], []
    for g, N in enumerate(Ns):
        W16 = O.f32_to_f16_bits(O.fill_uniform((N, K), 404 + g, 1.0))
        refs.append(O.mul_mat(O.F16, W16, Xf, N, K))
        w = mx.upload_weight(O.F16, W16, N, K)
        c = torch.empty((M, N), dtype=torch.float32, device="cuda")
        outs.append((w, N, 0, N, c))
    mx.gemm(O.F16, a16, sc, K, outs)
    torch.cuda.synchronize()
    for (w, _, _, N, c), ref in zip(outs, refs):
        _assert_bars(ref, c.cpu().numpy(), M, N, f"fused N={N}")


def test_gemm_rows_of_a_panel(mx):
    """row0/rows_total: a weight addressed inside a larger split-layout panel (the expert stacks)."""
    import torch
    K, N, E, M = 512, 128, 3, 40
    W = O.fill_normal((E * N, K), 77, 0.0, 0.02)
    for wtype in (O.Q8_0, O.Q6_K, O.Q4_K, O.Q4_0, O.Q5_K):
        Q = O.quantize(wtype, W)
        w = mx.upload_weight(wtype, Q, E * N, K)
        Xf = O.fill_normal((M, K), 78)
        a16, sc = mx.pack_act(_dev(Xf))
        c = torch.empty((M, N), dtype=torch.float32, device="cuda")
        mx.gemm(wtype, a16, sc, K, [(w, E * N, 2 * N, N, c)])
        torch.cuda.synchronize()
        ref = O.mul_mat(wtype, Q[2 * N:3 * N], Xf, N, K)
        _assert_bars(ref, c.cpu().numpy(), M, N, f"panel {O.TYPE_NAMES[wtype]}")


def _untile(buf, rows, K):
    """The tiled fp16 layout (16 x 32 tiles of 1 KB, tile (r/16, k/32) at ((r/16)*(K/32) + k/32)
    * 512 values, row-major inside, rows padded to 16) back to [rows][K]."""
    rp = (rows + 15) // 16 * 16
    t = np.asarray(buf).view(np.uint16).reshape(-1)[:rp * K].reshape(rp // 16, K // 32, 16, 32)
    return t.transpose(0, 2, 1, 3).reshape(rp, K)[:rows]


@pytest.mark.parametrize("wtype", [O.F16, O.Q8_0, O.Q4_0, O.Q4_K, O.Q5_K, O.Q6_K, O.MXFP4])
def test_f16_tiled_bitexact(mx, wtype):
    """The tiled resident form holds exactly the fp16 values of the row-major one (rows not a
    multiple of 16: padded, the padding never read)."""
    N, K = 300, 1024                # rows padded to 304
    W = O.fill_normal((N, K), 21 + wtype, 0.0, 0.02)
    W[0, :256] *= 50.0
    W[1, :] = 0.0
    payload = O.f32_to_f16_bits(W) if wtype == O.F16 else O.quantize(wtype, W)
    want = payload if wtype == O.F16 else O.dequantize_f16(wtype, payload, K)
    w = mx.upload_weight(wtype, payload, N, K)
    t = mx.tile_f16(wtype, w, N, K)
    assert t.numel() == mx.weight_bytes(mx.F16_T, N, K) == 304 * K * 2
    assert np.array_equal(_untile(t.cpu().numpy(), N, K), want.reshape(N, K))


def test_pack_act_tiled_bitexact(mx):
    X = O.fill_normal((67, 512), 8)
    X[3] *= 3000.0
    X[5] = 0.0
    X[9, 17] = 1e6
    a16, sc = mx.pack_act(_dev(X), tiled=True)
    want_a, want_s = O.pack_act(X)
    got = _untile(a16.cpu().numpy(), 67, 512)
    assert np.array_equal(sc.cpu().numpy(), want_s)
    bad = np.argwhere(got != want_a)
    assert len(bad) == 0, f"{len(bad)} differ, first {[(int(r), int(c), int(got[r, c]), int(want_a[r, c])) for r, c in bad[:8]]}"


# Every tile configuration of mi355x_gemm, forced through MI355X_GEMM_CFG, on a ragged fused
# launch (M and both N not multiples of any tile). Configurations 0-3 are the register-staged
# kernel (every weight layout but the tiled fp16 one); 4-15 and 21-24 the LDS-DMA kernels,
# which take fp16 weights only, row-major (F16) or tiled (F16_T); 16-19 the kernel with every
# operand by DMA (K % 256 == 0; Q4_K, and Q8_0 on the 128 x 256 tiles 17 and 19). 20 is the skinny kernel (M <= 128), covered
# by its own tests.
REG_CFGS = list(range(0, 4))
DMA_CFGS = list(range(4, 16)) + [21, 22, 23, 24]
QDMA_CFGS = list(range(16, 20))
F16_T = 0x101
QUANT = (O.Q4_K, O.MXFP4, O.Q8_0, O.Q6_K, O.Q4_0, O.Q5_K)


@pytest.mark.parametrize("cfg", REG_CFGS + DMA_CFGS + QDMA_CFGS)
@pytest.mark.parametrize("wtype", [O.F16, O.Q4_K, F16_T, O.MXFP4, O.Q8_0, O.Q6_K, O.Q4_0, O.Q5_K])
def test_gemm_every_tile_config(mx, monkeypatch, cfg, wtype):
    import torch
    if cfg in DMA_CFGS and wtype in QUANT:
        pytest.skip("the LDS-DMA configurations take fp16 weights only")
    if cfg in REG_CFGS and wtype == F16_T:
        pytest.skip("the register-staged configurations do not read the tiled layout")
    if cfg in QDMA_CFGS and wtype != O.Q4_K and not (wtype == O.Q8_0 and cfg in (17, 19)):
        pytest.skip("the all-DMA configurations take Q4_K weights, and Q8_0 on the 128-row tiles")
    monkeypatch.setenv("MI355X_GEMM_CFG", str(cfg))
    K, M, Ns = 1280, 300, (528, 144)
    Xf = O.fill_normal((M, K), 900 + cfg)
    a16, sc = mx.pack_act(_dev(Xf), tiled=wtype == F16_T)
    outs, refs = [], []
    for g, N in enumerate(Ns):
        W = O.fill_normal((N, K), 910 + g, 0.0, 0.02)
        payload = O.quantize(wtype, W) if wtype in QUANT else O.f32_to_f16_bits(W)
        refs.append(O.mul_mat(wtype if wtype in QUANT else O.F16, payload, Xf, N, K))
        if wtype == F16_T:
            w = mx.tile_f16(O.F16, mx.upload_weight(O.F16, payload, N, K), N, K)
        else:
            w = mx.upload_weight(wtype, payload, N, K)
        c = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        outs.append((w, N, 0, N, c))
    mx.gemm(wtype, a16, sc, K, outs)
    torch.cuda.synchronize()
    first = [c.cpu().numpy() for (_, _, _, _, c) in outs]
    for (w, _, _, N, c), ref in zip(outs, refs):
        _assert_bars(ref, c.cpu().numpy(), M, N, f"cfg {cfg} {O.TYPE_NAMES.get(wtype, 'F16_T')} N={N}")
    # reproducible: a second launch on NaN-filled outputs gives the same bits
    for (_, _, _, _, c) in outs:
        c.fill_(float("nan"))
    mx.gemm(wtype, a16, sc, K, outs)
    torch.cuda.synchronize()
    for (_, _, _, N, c), f in zip(outs, first):
        assert np.array_equal(c.cpu().numpy(), f), f"cfg {cfg} N={N}: second launch differs"


@pytest.mark.parametrize("K", [1312, 96])
def test_f16_k_not_multiple_of_64(mx, K):
    """K % 64 != 0: only the 32-deep DMA configuration (or the register-staged kernel) takes it."""
    N, M = 272, 130
    W16 = O.f32_to_f16_bits(O.fill_normal((N, K), 930, 0.0, 0.02))
    Xf = O.fill_normal((M, K), 931)
    ref = O.mul_mat(O.F16, W16, Xf, N, K)
    got = _run_mul_mat(mx, O.F16, W16, N, K, Xf)
    _assert_bars(ref, got, M, N, f"F16 K={K}")


@pytest.mark.parametrize("K,N,M", [(1024, 512, 7), (4096, 1024, 130), (2048, 8192, 512)])
def test_mul_mat_f16_tiled(mx, K, N, M):
    """mi355x_mul_mat on a tiled resident weight (the tiled activation pack inside), M ragged."""
    import torch
    W16 = O.f32_to_f16_bits(O.fill_normal((N, K), 940 + M, 0.0, 0.02))
    Xf = O.fill_normal((M, K), 941 + M)
    w = mx.tile_f16(O.F16, mx.upload_weight(O.F16, W16, N, K), N, K)
    out = mx.mul_mat(F16_T, w, N, K, _dev(Xf))
    torch.cuda.synchronize()
    rows = np.unique(np.linspace(0, M - 1, min(M, 48)).astype(int))
    ref = O.mul_mat(O.F16, W16, Xf[rows], N, K)
    _assert_bars(ref, out.cpu().numpy()[rows], len(rows), N, f"F16_T K={K} N={N} M={M}")


def test_gemm_tiled_rows_of_a_panel(mx):
    """row0 inside a tiled panel (not a multiple of 16): the slabs are rows_total rows long."""
    import torch
    K, N, M = 512, 96, 33
    W16 = O.f32_to_f16_bits(O.fill_normal((3 * N, K), 950, 0.0, 0.02))
    w = mx.tile_f16(O.F16, mx.upload_weight(O.F16, W16, 3 * N, K), 3 * N, K)
    Xf = O.fill_normal((M, K), 951)
    a16, sc = mx.pack_act(_dev(Xf), tiled=True)
    c = torch.empty((M, N), dtype=torch.float32, device="cuda")
    for row0 in (2 * N, 40):
        mx.gemm(F16_T, a16, sc, K, [(w, 3 * N, row0, N, c)])
        torch.cuda.synchronize()
        ref = O.mul_mat(O.F16, W16.reshape(3 * N, K)[row0:row0 + N], Xf, N, K)
        _assert_bars(ref, c.cpu().numpy(), M, N, f"tiled panel row0={row0}")


# The skinny kernel (M <= 128, every format but the tiled fp16 one): each M-tile count, a ragged
# N (not a multiple of the 128-row block), a K with a 32-value tail where the format allows one,
# K splits added atomically into an output cleared by the pack (mi355x_mul_mat) or by the GEMM
# launch itself (mi355x_gemm on NaN-filled outputs, two fused weights).
SKINNY_TYPES = [O.F16, O.Q8_0, O.Q4_K, O.Q6_K, O.MXFP4, O.Q4_0, O.Q5_K]
SUPER_BLOCK = (O.Q4_K, O.Q5_K, O.Q6_K)   # 256-value blocks: no 32-value K tail


@pytest.mark.parametrize("M", [1, 33, 96, 128])
@pytest.mark.parametrize("wtype", SKINNY_TYPES)
def test_skinny_mul_mat(mx, wtype, M):
    K = 2560 if wtype in SUPER_BLOCK else 1312
    N = 400
    W = O.fill_normal((N, K), 960 + wtype, 0.0, 0.02)
    Xf = O.fill_normal((M, K), 961 + M)
    payload = O.f32_to_f16_bits(W) if wtype == O.F16 else O.quantize(wtype, W)
    import torch
    ref = O.mul_mat(wtype, payload, Xf, N, K)
    w = mx.upload_weight(wtype, payload, N, K)
    # a row stride wider than N: the pack clears only the N columns the GEMM adds into
    wide = torch.full((M, N + 24), float("nan"), dtype=torch.float32, device="cuda")
    mx.mul_mat(wtype, w, N, K, _dev(Xf), wide[:, :N])
    torch.cuda.synchronize()
    got = wide.cpu().numpy()
    assert np.isnan(got[:, N:]).all(), "wrote past N"
    _assert_bars(ref, got[:, :N], M, N, f"skinny {O.TYPE_NAMES[wtype]} M={M}")


def test_mxfp4_fast_decode_is_exact(mx, monkeypatch):
    """The skinny kernel's packed MXFP4 decoder gives the exact decode's fp16 values for block
    scales 2^(e-127), e in 80..140 (below 89 every value rounds to zero, to 104 the products are
    fp16 subnormals, past 128 the scale takes two steps; 140 keeps 12 x 2^(e-128) finite, since an
    infinite weight would turn the zero products of the row into NaN): with one-hot activation
    rows (pack scale 1, every other product zero, so the K split's partial sums are exact),
    out[m][n] is the decoded weight W[n][k_m], compared with the oracle's dequantization to fp16
    (as values: a zero weight of either sign sums to +0). The one-hot positions take both
    nibbles of a byte (weights j and j + 16 of a block) and every block."""
    import torch
    N, K = 256, 512
    nblk = K // 32
    rng = np.random.default_rng(1234)
    blocks = rng.integers(0, 256, size=(N, nblk, 17), dtype=np.uint8)
    blocks[:, :, 0] = (80 + (np.arange(N * nblk).reshape(N, nblk) * 7) % 61).astype(np.uint8)
    payload = blocks.reshape(-1)
    want = O.f16_bits_to_f32(O.dequantize_f16(O.MXFP4, payload, K))
    ks = np.array([32 * (m % nblk) + (m * 5) % 32 for m in range(64)])
    X = np.zeros((64, K), np.float32)
    X[np.arange(64), ks] = 1.0
    monkeypatch.setenv("MI355X_GEMM_CFG", "20")
    w = mx.upload_weight(O.MXFP4, payload, N, K)
    out = mx.mul_mat(O.MXFP4, w, N, K, _dev(X))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ref = want[:, ks].T
    assert np.isfinite(ref).all()
    bad = np.argwhere(got != ref)
    assert len(bad) == 0, [(int(m), int(n), float(got[m, n]), float(ref[m, n])) for m, n in bad[:8]]


@pytest.mark.parametrize("M", [1, 32, 64, 100, 128])
@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_K, O.Q6_K])
def test_skinny_dma_matches_register_kernel(mx, monkeypatch, wtype, M):
    """The skinny kernel with the weight staged by LDS DMA (Q8_0, Q4_K, Q6_K) against the
    register-staged one (MI355X_SKINNY_DMA=0) on the same packed activations: both walk the same
    64-deep chunks in the same order with the same decoders, so where their K splits coincide
    (one split: K within one block's groups) the bits are equal; the DMA form also meets the
    oracle bars. N 400 (ragged against the 128-row block), K with a 32-value tail for Q8_0."""
    import torch
    K = 1024 if wtype in SUPER_BLOCK else 1056
    N = 400
    W = O.fill_normal((N, K), 990 + wtype, 0.0, 0.02)
    Xf = O.fill_normal((M, K), 991 + M)
    P = O.quantize(wtype, W)
    w = mx.upload_weight(wtype, P, N, K)
    a16, sc = mx.pack_act(_dev(Xf))
    got = {}
    for dma in ("1", "0"):
        monkeypatch.setenv("MI355X_SKINNY_DMA", dma)
        monkeypatch.setenv("MI355X_SKINNY_BLOCKS", "4")   # one K split: the whole K in each block
        c = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        mx.gemm(wtype, a16, sc, K, [(w, N, 0, N, c)])
        torch.cuda.synchronize()
        got[dma] = c.cpu().numpy()
    assert np.isfinite(got["1"]).all()
    assert np.array_equal(got["1"], got["0"]), float(np.abs(got["1"] - got["0"]).max())
    _assert_bars(O.mul_mat(wtype, P, Xf, N, K), got["1"], M, N, f"skinny dma {O.TYPE_NAMES[wtype]} M={M}",
                 cos_floor=0.999 if M >= 8 else -1.0)


@pytest.mark.parametrize("wtype", SKINNY_TYPES)
def test_skinny_gemm_fused_nan_outputs(mx, wtype):
    import torch
    K = 1536 if wtype in SUPER_BLOCK else 1248
    M, Ns = 70, (144, 272)
    Xf = O.fill_normal((M, K), 970)
    a16, sc = mx.pack_act(_dev(Xf))
    outs, refs = [], []
    for g, N in enumerate(Ns):
        W = O.fill_normal((N, K), 971 + g, 0.0, 0.02)
        payload = O.f32_to_f16_bits(W) if wtype == O.F16 else O.quantize(wtype, W)
        refs.append(O.mul_mat(wtype, payload, Xf, N, K))
        w = mx.upload_weight(wtype, payload, N, K)
        c = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        outs.append((w, N, 0, N, c))
    mx.gemm(wtype, a16, sc, K, outs)
    torch.cuda.synchronize()
    for (w, _, _, N, c), ref in zip(outs, refs):
        _assert_bars(ref, c.cpu().numpy(), M, N, f"skinny fused {O.TYPE_NAMES[wtype]} N={N}")


# K splits are summed in a fixed order. Each split form, launched three times on NaN-filled
# outputs, must give the same bits every time and meet the oracle bars: the skinny kernel's wide
# split and the register-staged split (partials in the workspace, summed by a second launch),
# the Q4_K DMA split (configuration 19, K 14336), and mi355x_gemm without a workspace (at most
# two ways, added into the zeroed output).
SPLIT_CASES = [  # (wtype, M, N, K, cfg or None, split_workspace)
    (O.Q4_K, 1, 4096, 4096, None, True),
    (O.Q8_0, 33, 1024, 4096, None, True),
    (O.Q4_K, 128, 2048, 14336, None, True),
    (O.Q6_K, 200, 256, 8192, "1", True),
    (O.Q4_K, 512, 1024, 14336, "19", True),
    (O.Q4_K, 8, 4096, 4096, None, False),
    (O.Q4_K, 512, 1024, 14336, "19", False),
]


@pytest.mark.parametrize("wtype,M,N,K,cfg,use_ws", SPLIT_CASES)
def test_split_k_reproducible(mx, monkeypatch, wtype, M, N, K, cfg, use_ws):
    import torch
    if cfg is not None:
        monkeypatch.setenv("MI355X_GEMM_CFG", cfg)
    W = O.fill_normal((N, K), 1300 + M, 0.0, 0.02)
    P = O.quantize(wtype, W)
    Xf = O.fill_normal((M, K), 1301 + M)
    w = mx.upload_weight(wtype, P, N, K)
    a16, sc = mx.pack_act(_dev(Xf))
    arr = (mx.GemmOut * 1)()
    arr[0] = mx.GemmOut(None, N, 0, N, None, N)
    part = int(mx.lib().mi355x_gemm_workspace(wtype, M, K, arr, 1))
    print(f"{O.TYPE_NAMES[wtype]} M={M} N={N} K={K} cfg={cfg}: split workspace {part} bytes, used={use_ws}")
    got = []
    for _ in range(3):
        c = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        mx.gemm(wtype, a16, sc, K, [(w, N, 0, N, c)], split_workspace=use_ws)
        torch.cuda.synchronize()
        got.append(c.cpu().numpy())
    for g in got[1:]:
        assert np.array_equal(g, got[0]), "launches differ"
    rows = np.unique(np.linspace(0, M - 1, min(M, 40)).astype(int))
    ref = O.mul_mat(wtype, P, Xf[rows], N, K)
    # a column cosine over fewer than 8 rows says nothing (one near-zero value can flip its sign)
    _assert_bars(ref, got[0][rows], len(rows), N, f"split {O.TYPE_NAMES[wtype]} M={M} cfg={cfg}",
                 cos_floor=0.999 if len(rows) >= 8 else -1.0)


def test_pack_clear_then_accumulating_gemm(mx):
    """mi355x_pack_act_clear + MI355X_GEMM_OUT_ZEROED (the pack clears the output of a GEMM that
    adds a two-way K split into it) gives the bits of the launch that clears its output itself."""
    import torch
    M, N, K = 512, 4096, 14336
    W16 = O.f32_to_f16_bits(O.fill_normal((N, K), 1400, 0.0, 0.02))
    Xf = O.fill_normal((M, K), 1401)
    w = mx.tile_f16(O.F16, mx.upload_weight(O.F16, W16, N, K), N, K)
    arr = (mx.GemmOut * 1)()
    arr[0] = mx.GemmOut(None, N, 0, N, None, N)
    part = int(mx.lib().mi355x_gemm_workspace(F16_T, M, K, arr, 1))
    acc = int(mx.lib().mi355x_gemm_accumulates(F16_T, M, K, arr, 1, part))
    print(f"split workspace {part} bytes, accumulates {acc}")
    assert acc in (0, 1)
    x = _dev(Xf)
    a16, sc = mx.pack_act(x, tiled=True)
    ws = torch.empty(max(part, 256), dtype=torch.uint8, device="cuda")
    outs = []
    for zeroed in (False, True):
        c = torch.full((M, N + 8), float("nan"), dtype=torch.float32, device="cuda")
        arr[0] = mx.GemmOut(w.data_ptr(), N, 0, N, c.data_ptr(), c.stride(0))
        if zeroed:
            mx.check(mx.lib().mi355x_pack_act_clear(1, mx._ptr(x), x.stride(0), M, K, mx._ptr(a16), mx._ptr(sc),
                                                    mx._ptr(c), c.stride(0), N, mx.stream_handle()), "pack_clear")
        mx.check(mx.lib().mi355x_gemm_ws(F16_T, mx._ptr(a16), mx._ptr(sc), M, K, arr, 1, mx._ptr(ws), part,
                                         1 if (zeroed and acc) else 0, mx.stream_handle()), "gemm_ws")
        torch.cuda.synchronize()
        got = c.cpu().numpy()
        assert np.isnan(got[:, N:]).all(), "wrote past N"
        outs.append(got[:, :N])
    assert np.array_equal(outs[0], outs[1])
    rows = np.arange(0, M, 16)
    _assert_bars(O.mul_mat(O.F16, W16, Xf[rows], N, K), outs[1][rows], len(rows), N, "pack-clear + zeroed GEMM")
