"""Pins the CPU oracle before anything is checked against it (CPU only).

The reference's tests hold no stored vectors for this path (they compare against ggml's CPU
backend at run time, test-common.h:48-100), and ggml is absent here. So each oracle function is
pinned by known answers written by hand from ggml's published block formats, by closed forms and
independent implementations (numpy's float16 conversion and float64 matmul), by invariants, and
by brute force on tiny inputs -- chosen so that a plausible mistake (a swapped nibble order, a
wrong scale index, a transposed operand, a dropped mask) fails one of them.
"""
import numpy as np
import pytest

from oracle import oracle as O
from fa_cases import fill_case, OVERFLOW, causal_mask


# ---- fp16 -------------------------------------------------------------------------------------

def test_f16_roundtrip_all_halves():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = O.f16_bits_to_f32(h)
    # numpy's independent conversion
    assert np.array_equal(np.isnan(f), np.isnan(h.view(np.float16).astype(np.float32)))
    fin = ~np.isnan(f)
    assert np.array_equal(f[fin], h.view(np.float16).astype(np.float32)[fin])
    back = O.f32_to_f16_bits(f)
    assert np.array_equal(back[fin], h[fin])


def test_f32_to_f16_matches_numpy_rne():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(1000),
        rng.standard_normal(200000).astype(np.float32) * np.float32(1e-5),   # subnormal halves
        np.array([65504, 65519.99, 65520, 65536, -65520, 1e9, 6.1e-5, 5.96e-8, 2.98e-8,
                  2.99e-8, 0.0, -0.0, 1.0 + 2**-11, 1.0 + 3 * 2**-11, np.inf, -np.inf],
                 dtype=np.float32)])
    assert np.array_equal(O.f32_to_f16_bits(x), x.astype(np.float16).view(np.uint16))


# ---- fills ------------------------------------------------------------------------------------

def test_fill_uniform_known_values():
    # rk_hash(seed=1, i=0) by hand from test-common.h:181-187
    z = (1 * 0x9E3779B97F4A7C15 + 0 + 0x9E3779B97F4A7C15) & (2**64 - 1)
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & (2**64 - 1)
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & (2**64 - 1)
    z = z ^ (z >> 31)
    want = np.float32(2.0 * float(np.float32((z >> 11) * (2.0 / 9007199254740992.0) - 1.0)) / 2.0)
    got = O.fill_uniform((4,), 1, 1.0)
    assert got[0] == want
    u = O.fill_uniform((100000,), 7, 3.0)
    assert u.min() >= -3.0 and u.max() < 3.0 and abs(u.mean()) < 0.05


def test_fill_normal_moments():
    x = O.fill_normal((1 << 20,), 123, 0.0, 0.02)
    assert abs(x.mean()) < 1e-4 and abs(x.std() - 0.02) < 1e-4
    assert np.array_equal(x, O.fill_normal((1 << 20,), 123, 0.0, 0.02))


# ---- block formats: hand-built known answers ---------------------------------------------------

def _h(x):
    return int(np.float32(x).astype(np.float16).view(np.uint16))


def test_q8_0_known_block():
    blk = np.zeros(34, dtype=np.uint8)
    blk[0:2] = np.frombuffer(np.uint16(_h(0.5)).tobytes(), np.uint8)
    q = np.array([-128, -1, 0, 1, 127] + list(range(-13, 14)), dtype=np.int8)[:32]
    blk[2:] = q.view(np.uint8)
    y = O.dequantize(O.Q8_0, blk, 32)
    assert np.array_equal(y, 0.5 * q.astype(np.float32))


def _q4k_block(d, dmin, scale_bytes, qs):
    b = np.zeros(144, dtype=np.uint8)
    b[0:2] = np.frombuffer(np.uint16(_h(d)).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.uint16(_h(dmin)).tobytes(), np.uint8)
    b[4:16] = scale_bytes
    b[16:] = qs
    return b


def test_q4_k_scale_unpacking_known_answer():
    # 12 scale bytes chosen by hand. ggml's get_scale_min_k4: for j < 4, sc = q[j] & 63 and
    # m = q[j+4] & 63; for j >= 4, sc = (q[j+4] & 15) | (q[j-4] >> 6) << 4 and
    # m = (q[j+4] >> 4) | (q[j] >> 6) << 4. Expected pairs worked out by hand:
    sb = np.array([0xC1, 0x02, 0x43, 0x84, 0x05, 0xC6, 0x07, 0x48, 0x21, 0x43, 0x65, 0x87], np.uint8)
    sc = [1, 2, 3, 4, 49, 3, 5 | (1 << 4), 7 | (2 << 4)]
    mn = [5, 6, 7, 8, 2, 4 | (3 << 4), 6, 8 | (1 << 4)]
    # all nibbles 0: y = -dmin * m of the weight's sub-block (p // 32)
    y0 = O.dequantize(O.Q4_K, _q4k_block(1.0, 0.5, sb, np.zeros(128, np.uint8)), 256)
    assert np.array_equal(y0, np.repeat(-0.5 * np.array(mn, np.float32), 32))
    # all nibbles 1: y = d*sc - dmin*m
    y1 = O.dequantize(O.Q4_K, _q4k_block(2.0, 0.5, sb, np.full(128, 0x11, np.uint8)), 256)
    assert np.array_equal(y1, np.repeat(np.float32(2.0) * np.array(sc, np.float32)
                                        - np.float32(0.5) * np.array(mn, np.float32), 32))


def test_q4_k_nibble_order_known_answer():
    # qs byte 32j + l holds weight 64j + l in its low nibble and 64j + 32 + l in its high one.
    sb = np.array([1] * 4 + [0] * 4 + [0x01] * 4, np.uint8)   # every sc = 1, every m = 0
    qs = np.zeros(128, np.uint8)
    qs[32 * 2 + 5] = 0x9C                                    # low 12 -> w 133, high 9 -> w 165
    y = O.dequantize(O.Q4_K, _q4k_block(1.0, 0.0, sb, qs), 256)
    want = np.zeros(256, np.float32)
    want[133], want[165] = 12.0, 9.0
    assert np.array_equal(y, want)


def test_q6_k_known_answer():
    b = np.zeros(210, np.uint8)
    sc = np.arange(1, 17, dtype=np.int8)
    sc[3] = -7
    b[192:208] = sc.view(np.uint8)
    b[208:210] = np.frombuffer(np.uint16(_h(0.25)).tobytes(), np.uint8)
    # all codes zero -> q = -32: y[p] = d * sc[p // 16] * -32
    y = O.dequantize(O.Q6_K, b, 256)
    assert np.array_equal(y, np.repeat(np.float32(0.25) * sc.astype(np.float32), 16) * np.float32(-32.0))
    # one weight per bit plane: weight 128 + 32*k + 3 (second half, quarter k) gets code 6-bit v_k
    b2 = b.copy()
    codes = {0: 0x3F, 1: 0x21, 2: 0x10, 3: 0x05}
    for k, v in codes.items():
        l = 3
        ql_idx = 64 + l + (32 if k in (1, 3) else 0)
        shift = 4 if k in (2, 3) else 0
        b2[ql_idx] |= (v & 15) << shift
        b2[128 + 32 + l] |= (v >> 4) << (2 * k)
    y2 = O.dequantize(O.Q6_K, b2, 256)
    for k, v in codes.items():
        p = 128 + 32 * k + 3
        assert y2[p] == np.float32(0.25) * np.float32(sc[p // 16]) * np.float32(v - 32), (k, p)
    other = np.setdiff1d(np.arange(256), [128 + 32 * k + 3 for k in codes])
    assert np.array_equal(y2[other], y[other])


def test_q4_0_known_block():
    # ggml's block_q4_0: qs[j] low nibble = weight j, high nibble = weight j + 16; y = d * (q - 8)
    blk = np.zeros(18, dtype=np.uint8)
    blk[0:2] = np.frombuffer(np.uint16(_h(0.25)).tobytes(), np.uint8)
    lo = np.arange(16, dtype=np.uint8)              # weights 0..15: codes 0..15
    hi = (15 - np.arange(16)).astype(np.uint8)      # weights 16..31: codes 15..0
    blk[2:] = lo | (hi << 4)
    y = O.dequantize(O.Q4_0, blk, 32)
    want = np.float32(0.25) * np.concatenate([lo, hi]).astype(np.float32) - np.float32(2.0)
    assert np.array_equal(y, want)
    assert y[8] == 0.0 and y[0] == -2.0 and y[16] == 1.75


def _q5k_block(d, dmin, scale_bytes, qh, qs):
    b = np.zeros(176, dtype=np.uint8)
    b[0:2] = np.frombuffer(np.uint16(_h(d)).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.uint16(_h(dmin)).tobytes(), np.uint8)
    b[4:16] = scale_bytes
    b[16:48] = qh
    b[48:] = qs
    return b


def test_q5_k_known_answer():
    # the scales and mins of Q4_K (same 12-byte packing, pinned above); the fifth bit of weight
    # 32 i + l (sub-block i) is bit i of qh[l] and adds 16 to its code before the scale
    sb = np.array([0xC1, 0x02, 0x43, 0x84, 0x05, 0xC6, 0x07, 0x48, 0x21, 0x43, 0x65, 0x87], np.uint8)
    sc = np.array([1, 2, 3, 4, 49, 3, 5 | (1 << 4), 7 | (2 << 4)], np.float32)
    mn = np.array([5, 6, 7, 8, 2, 4 | (3 << 4), 6, 8 | (1 << 4)], np.float32)
    # all codes 0: y = -dmin * m
    y0 = O.dequantize(O.Q5_K, _q5k_block(1.0, 0.5, sb, np.zeros(32, np.uint8), np.zeros(128, np.uint8)), 256)
    assert np.array_equal(y0, np.repeat(np.float32(-0.5) * mn, 32))
    # every fifth bit set, nibbles 0: code 16 in every weight
    y1 = O.dequantize(O.Q5_K, _q5k_block(2.0, 0.5, sb, np.full(32, 0xFF, np.uint8), np.zeros(128, np.uint8)), 256)
    assert np.array_equal(y1, np.repeat(np.float32(2.0) * sc * np.float32(16.0) - np.float32(0.5) * mn, 32))
    # one weight per sub-block: weight 32 i + 7 gets code 16 * (i % 2 == 0) + i via qh bit i / nibble
    qh = np.zeros(32, np.uint8)
    qs = np.zeros(128, np.uint8)
    for i in range(8):
        if i % 2 == 0:
            qh[7] |= 1 << i
        qs[32 * (i // 2) + 7] |= i << (4 * (i % 2))
    y2 = O.dequantize(O.Q5_K, _q5k_block(1.0, 0.0, np.array([1] * 4 + [0] * 4 + [0x01] * 4, np.uint8), qh, qs), 256)
    want = np.zeros(256, np.float32)
    for i in range(8):
        want[32 * i + 7] = (16 if i % 2 == 0 else 0) + i
    assert np.array_equal(y2, want)


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_K, O.Q6_K, O.Q4_0, O.Q5_K])
def test_quant_roundtrip(wtype):
    """Within about half a quantization step of each sub-block: symmetric amax/127 (Q8_0),
    amax/31 (Q6_K) and amax/7 (Q4_0) steps, the asymmetric (max-min)/15 step of Q4_K and
    (max-min)/31 of Q5_K; slack for the fp16 / 6-bit / 8-bit rounding of the scales."""
    W = O.fill_normal((64, 1024), 5, 0.0, 0.02)
    d = O.dequantize(wtype, O.quantize(wtype, W), 1024)
    blk = {O.Q8_0: 32, O.Q4_K: 32, O.Q6_K: 16, O.Q4_0: 32, O.Q5_K: 32}[wtype]
    Wb = W.reshape(64, -1, blk)
    amax = np.abs(Wb).max(-1)
    step = {O.Q8_0: amax / 127, O.Q6_K: amax / 31, O.Q4_K: (Wb.max(-1) - Wb.min(-1)) / 15,
            O.Q4_0: amax / 7, O.Q5_K: (Wb.max(-1) - Wb.min(-1)) / 31}[wtype]
    err = np.abs(d - W).reshape(64, -1, blk).max(-1)
    assert np.all(err <= 0.75 * step + 1e-6)


def test_row_size():
    assert O.row_size(O.Q8_0, 64) == 68 and O.row_size(O.Q4_K, 512) == 288
    assert O.row_size(O.Q6_K, 256) == 210 and O.row_size(O.Q4_K, 100) == -1
    assert O.row_size(O.MXFP4, 64) == 34 and O.row_size(O.MXFP4, 48) == -1
    assert O.row_size(O.Q4_0, 64) == 36 and O.row_size(O.Q5_K, 512) == 352 and O.row_size(O.Q5_K, 128) == -1


# The OCP microscaling FP4 definition the MXFP4 decoder restates: an E2M1 code is
# sign * {0, 0.5, 1, 1.5, 2, 3, 4, 6}[low 3 bits] (bit 3 = sign), the E8M0 byte e scales the
# block by 2^(e-127), and ggml puts weight j in the low nibble of qs[j], weight j+16 in the high.
E2M1 = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6, -0.0, -0.5, -1, -1.5, -2, -3, -4, -6], dtype=np.float64)


def _mxfp4_block(e, codes):
    codes = np.asarray(codes, dtype=np.uint8)
    return np.concatenate([[np.uint8(e)], (codes[:16] | (codes[16:] << 4)).astype(np.uint8)]).astype(np.uint8)


def test_mxfp4_known_answer():
    """Every code at unit scale (e = 127), the nibble order, the bias, doubling per exponent
    step, and the two subnormal scales (e = 0, 1 -> 2^-127, 2^-126 times the E2M1 value)."""
    codes = np.array(list(range(16)) + list(range(15, -1, -1)), dtype=np.uint8)
    for e in (0, 1, 2, 100, 126, 127, 128, 140):
        y = O.dequantize(O.MXFP4, _mxfp4_block(e, codes), 32)
        want = E2M1[codes] * np.ldexp(1.0, e - 127)
        assert np.array_equal(y.astype(np.float64), want), e
    # low nibble -> weight j, high nibble -> weight j + 16
    one = np.zeros(32, dtype=np.uint8)
    one[3], one[16 + 9] = 7, 12         # 6.0 at weight 3, -2.0 at weight 25
    y = O.dequantize(O.MXFP4, _mxfp4_block(127, one), 32)
    assert y[3] == 6.0 and y[25] == -2.0 and np.count_nonzero(y) == 2


def test_mxfp4_quant_roundtrip():
    """Values that are E2M1 codes times the block scale come back exactly; others within half
    the widest code gap (2 units of the scale, between 4 and 6) of each block."""
    rng = np.random.default_rng(11)
    codes = rng.integers(0, 16, (8, 64)).astype(np.uint8)
    exps = rng.integers(110, 140, (8, 2))
    W = (E2M1[codes].reshape(8, 2, 32) * np.ldexp(1.0, exps - 127)[..., None]).reshape(8, 64)
    W[:, 0] = 6.0 * np.ldexp(1.0, exps[:, 0] - 127)      # each block's largest code is present
    W[:, 32] = -6.0 * np.ldexp(1.0, exps[:, 1] - 127)
    W = W.astype(np.float32)
    assert np.array_equal(O.dequantize(O.MXFP4, O.quantize(O.MXFP4, W), 64), W)
    X = O.fill_normal((16, 256), 12, 0.0, 0.02)
    d = O.dequantize(O.MXFP4, O.quantize(O.MXFP4, X), 256)
    scale = np.abs(X.reshape(16, -1, 32)).max(-1, keepdims=True) / 6.0
    assert np.all(np.abs(d - X).reshape(16, -1, 32) <= 2.0 * scale + 1e-12)


# ---- ops --------------------------------------------------------------------------------------

def test_mul_mat_vs_numpy():
    W = O.fill_normal((96, 512), 1)
    X = O.fill_normal((17, 512), 2)
    for wt in (O.F32, O.F16, O.Q8_0, O.Q4_K, O.Q6_K):
        P = W if wt == O.F32 else (O.f32_to_f16_bits(W) if wt == O.F16 else O.quantize(wt, W))
        Wd = W if wt == O.F32 else (O.f16_bits_to_f32(P) if wt == O.F16 else O.dequantize(wt, P, 512))
        want = X.astype(np.float64) @ Wd.astype(np.float64).T
        got = O.mul_mat(wt, P, X, 96, 512)
        assert np.allclose(got, want, rtol=1e-6, atol=1e-6)


def test_pack_act_invariants():
    X = O.fill_normal((9, 256), 3)
    X[2] = 0.0
    X[4] *= 1e5
    a16, sc = O.pack_act(X)
    assert sc[2] == 1.0 and np.all(a16[2] == 0)
    amax = np.abs(X).max(1)
    assert np.array_equal(sc[[0, 1, 3, 4]], amax[[0, 1, 3, 4]])
    # independent: numpy's float16 of x * (1/s)
    inv = (np.float32(1.0) / sc).astype(np.float32)
    assert np.array_equal(a16, (X * inv[:, None]).astype(np.float16).view(np.uint16))
    assert np.all(np.abs(a16.view(np.float16)).max(1)[[0, 1, 3, 4]] == 1.0)


def test_mul_mat_id_brute_force():
    K, N, E, T, U = 64, 32, 5, 7, 3
    As = O.fill_normal((E, N, K), 4)
    rng = np.random.default_rng(1)
    ids = rng.integers(0, E - 1, size=(T, U)).astype(np.int32)   # last expert empty
    for ne11 in (1, U):
        B = O.fill_normal((T, ne11, K), 5)
        got = O.mul_mat_id(O.F32, As, K, N, E, B, ne11, ids)
        for t in range(T):
            for s in range(U):
                want = As[ids[t, s]].astype(np.float64) @ B[t, s % ne11].astype(np.float64)
                assert np.allclose(got[t, s], want, rtol=1e-6, atol=1e-6)
    bad = ids.copy()
    bad[2, 1] = E
    with pytest.raises(ValueError):
        O.mul_mat_id(O.F32, As, K, N, E, O.fill_normal((T, 1, K), 5), 1, bad)


def _np_attn(Q, K, V, M, scale, softcap=0.0, q16=True):
    H, T, D = Q.shape
    HK = K.shape[0]
    out = np.zeros((T, H, V.shape[2]))
    Qd = Q.astype(np.float16).astype(np.float64) if q16 else Q.astype(np.float64)
    for h in range(H):
        hk = h // (H // HK)
        s = Qd[h] @ K[hk].astype(np.float64).T * scale
        if softcap:
            s = softcap * np.tanh(s / softcap)
        if M is not None:
            s = s + M[:T, :K.shape[1]].astype(np.float64)
        mx = s.max(1, keepdims=True)
        p = np.where(np.isinf(s), 0.0, np.exp(s - np.where(np.isinf(mx), 0, mx)))
        den = p.sum(1, keepdims=True)
        out[:, h, :] = np.where(den > 0, (p @ V[hk].astype(np.float64)) / np.where(den > 0, den, 1), 0)
    return out


def test_flash_attn_vs_numpy_and_masked_rows():
    D, T, H, KV, HK = 32, 9, 4, 40, 2
    Q = O.fill_normal((H, T, D), 6)
    K16 = O.f32_to_f16_bits(O.fill_normal((HK, KV, D), 7))
    V16 = O.f32_to_f16_bits(O.fill_normal((HK, KV, D), 8))
    M = causal_mask(T, KV)
    M[3] = -np.inf
    M16 = O.f32_to_f16_bits(M)
    Kf, Vf, Mf = O.f16_bits_to_f32(K16), O.f16_bits_to_f32(V16), O.f16_bits_to_f32(M16)
    for softcap in (0.0, 2.5):
        got = O.flash_attn(Q, K16, V16, M16, 0.2, softcap=softcap)
        want = _np_attn(Q, Kf, Vf, Mf, 0.2, softcap)
        assert np.allclose(got, want, rtol=1e-5, atol=1e-6)
        assert np.all(got[3] == 0.0)
    gotf = O.flash_attn(Q, K16, V16, None, 0.2, q_mode=1)
    assert np.allclose(gotf, _np_attn(Q, Kf, Vf, None, 0.2, q16=False), rtol=1e-5, atol=1e-6)


def test_flash_attn_one_hot_known_answer():
    """The overflow construction: each query's softmax is one-hot on its largest key, so the
    output is that key's V row (test-rocket-fa.cpp:13-32)."""
    D, T, H, KV, HK = 64, 32, 4, 1024, 2
    Q, K, V, M = fill_case(D, T, H, KV, HK, OVERFLOW)
    K16, V16 = O.f32_to_f16_bits(K), O.f32_to_f16_bits(V)
    got = O.flash_attn(Q, K16, V16, O.f32_to_f16_bits(M), 1.0 / 8.0)
    Vf = O.f16_bits_to_f32(V16)
    for h in range(H):
        hk = h // (H // HK)
        for t in range(T):
            d = (t + h) % D
            j = max(j for j in range(KV) if j % D == d)   # largest k along direction d
            assert np.array_equal(got[t, h], Vf[hk, j]), (h, t)


def test_flash_attn_uniform_is_mean():
    """Q = 0 makes every score equal: the output is the mean of the visible V rows."""
    D, T, H, KV, HK = 16, 5, 2, 12, 1
    Q = np.zeros((H, T, D), np.float32)
    K16 = O.f32_to_f16_bits(O.fill_normal((HK, KV, D), 9))
    V16 = O.f32_to_f16_bits(O.fill_normal((HK, KV, D), 10))
    M = causal_mask(T, KV)
    got = O.flash_attn(Q, K16, V16, O.f32_to_f16_bits(M), 0.5)
    Vf = O.f16_bits_to_f32(V16)
    for t in range(T):
        vis = KV - T + t + 1
        assert np.allclose(got[t, 0], Vf[0, :vis].astype(np.float64).mean(0), rtol=1e-6, atol=1e-7)


def test_flash_attn_value_width_differs_from_key_width():
    """K rows of 48 and V rows of 24 (the MLA shape family: keys wider than values); a wrong
    stride on either operand breaks the match with the float64 softmax."""
    D, DV, T, H, KV, HK = 48, 24, 7, 4, 33, 2
    Q = O.fill_normal((H, T, D), 11)
    K16 = O.f32_to_f16_bits(O.fill_normal((HK, KV, D), 12))
    V16 = O.f32_to_f16_bits(O.fill_normal((HK, KV, DV), 13))
    M16 = O.f32_to_f16_bits(causal_mask(T, KV))
    Kf, Vf, Mf = O.f16_bits_to_f32(K16), O.f16_bits_to_f32(V16), O.f16_bits_to_f32(M16)
    got = O.flash_attn(Q, K16, V16, M16, 0.15)
    assert got.shape == (T, H, DV)
    assert np.allclose(got, _np_attn(Q, Kf, Vf, Mf, 0.15), rtol=1e-5, atol=1e-6)
