"""FLASH_ATTN_EXT fixtures of test-rocket-fa.cpp (fill_case, 137-171), restated for numpy.

Layouts: Q [H][T][D] f32, K/V [HK][KV][D] f32 (converted to fp16 by the caller, as the
reference's run_fa does), mask [T][KV] f32 (0 or -inf).
"""
import numpy as np

TYPICAL, OVERFLOW, SCALED, QRANGE = "typical", "overflow", "scaled", "qrange"

# (name, D, T, H, KV, HK, kind, tol) -- test-rocket-fa.cpp:184-192
REFERENCE_CASES = [
    ("overflow d64", 64, 32, 4, 1024, 2, OVERFLOW, 1e-3),
    ("overflow d128", 128, 32, 4, 1024, 2, OVERFLOW, 1e-3),
    ("typical d64", 64, 64, 8, 1024, 2, TYPICAL, 2e-2),
    ("typical d128", 128, 64, 4, 1536, 4, TYPICAL, 2e-2),
    ("scaled d64", 64, 32, 4, 1024, 2, SCALED, 1e-3),
    ("scaled d128", 128, 32, 4, 1024, 2, SCALED, 1e-3),
    ("q range d64", 64, 32, 4, 1024, 2, QRANGE, 1e-3),
]

_M64 = (1 << 64) - 1


def _xorshift_uniform(seed: int, n: int) -> np.ndarray:
    """The case fill's xorshift64 stream: s ^= s<<13; s ^= s>>7; s ^= s<<17; then
    (float)((s >> 11) / 2^52) - 1, uniform in [-1, 1)."""
    s = seed & _M64
    out = np.empty(n, dtype=np.float32)
    inv = 1.0 / float(1 << 52)
    for i in range(n):
        s ^= (s << 13) & _M64
        s ^= s >> 7
        s ^= (s << 17) & _M64
        out[i] = np.float32(np.float32((s >> 11) * inv) - np.float32(1.0))
    return out


def fill_case(D, T, H, KV, HK, kind):
    Q = np.zeros((H, T, D), dtype=np.float32)
    K = np.zeros((HK, KV, D), dtype=np.float32)
    M = np.zeros((T, KV), dtype=np.float32)
    seed = 0x9E3779B97F4A7C15 ^ (D * 131 + KV)
    nv = D * KV * HK
    if kind == TYPICAL:
        r = _xorshift_uniform(seed, nv + Q.size + K.size)
        V = r[:nv].reshape(HK, KV, D)
        Q = r[nv:nv + Q.size].reshape(H, T, D).copy()
        K = r[nv + Q.size:].reshape(HK, KV, D).copy()
        for t in range(T):
            M[t, KV - T + t + 1:] = -np.inf
    else:
        V = _xorshift_uniform(seed, nv).reshape(HK, KV, D)
        qa = 500.0 * np.sqrt(np.float32(D)) if kind == SCALED else (1.0e6 if kind == QRANGE else 1000.0)
        k0 = 140.0 if kind == SCALED else 60.0
        kd = 1000.0 if kind == QRANGE else 1.0
        for h in range(H):
            for t in range(T):
                Q[h, t, (t + h) % D] = np.float32(qa)
        for hk in range(HK):
            for j in range(KV):
                K[hk, j, j % D] = np.float32((np.float32(k0) + np.float32(5.0) * np.float32(j // D)) / np.float32(kd))
    return Q, K, V.copy(), M


def causal_mask(T: int, KV: int) -> np.ndarray:
    """M[t, j] = -inf iff j > KV - T + t (the last T of KV positions are the queries)."""
    j = np.arange(KV)[None, :]
    t = np.arange(T)[:, None]
    return np.where(j > KV - T + t, -np.inf, 0.0).astype(np.float32)
