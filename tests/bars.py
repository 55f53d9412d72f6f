"""The reference's comparison bars, restated for numpy.

  element bar   an element is bad only if |d| >= 0.5 AND |d|/(|ref|+1e-6) >= 0.05; a non-finite
                element is bad outright (test-common.h:110-129, test-rocket-matmul.cpp:158-178)
  cosine        aggregate cosine over the flattened tile (test-common.h:121-129)
  worst column  / worst row cosine over a [rows, N] result (test-common.h:203-242)
  range error   max|d| / max|ref| (test-rocket-matmul.cpp:244-253), the "max rel err <= 1e-2"
                bar stated for fp16 GEMM and attention.
"""
import numpy as np


def compare(ref, got):
    ref = np.asarray(ref, dtype=np.float64).ravel()
    got = np.asarray(got, dtype=np.float64).ravel()
    fin = np.isfinite(got)
    d = np.abs(got - ref)
    rd = d / (np.abs(ref) + 1e-6)
    nbad = int((~fin).sum()) + int(((d >= 0.5) & (rd >= 0.05) & fin).sum())
    g = np.where(fin, got, 0.0)
    na, nb = np.sqrt((ref * ref).sum()), np.sqrt((g * g).sum())
    cos = float((ref * g).sum() / (na * nb)) if na > 0 and nb > 0 else 0.0
    dmax = float(np.max(d[fin])) if fin.any() else float("inf")
    rng = float(np.max(np.abs(ref))) if ref.size else 0.0
    return {"nbad": nbad, "cos": cos, "max_abs": dmax,
            "max_rel": float(np.max(rd[fin])) if fin.any() else float("inf"),
            "range_err": dmax / rng if rng > 0 else (0.0 if dmax == 0 else float("inf")),
            "nonfinite": int((~fin).sum())}


def _worst_cos(ref, got, axis):
    ref = np.asarray(ref, dtype=np.float64)
    got = np.asarray(got, dtype=np.float64)
    if not (np.isfinite(ref).all() and np.isfinite(got).all()):
        return -2.0
    dot = (ref * got).sum(axis=axis)
    na = np.sqrt((ref * ref).sum(axis=axis))
    nb = np.sqrt((got * got).sum(axis=axis))
    keep = na > 0
    if not keep.any():
        return 1.0
    c = np.where(nb[keep] > 0, dot[keep] / (na[keep] * np.where(nb[keep] > 0, nb[keep], 1.0)), 0.0)
    return float(c.min())


def worst_col_cos(ref, got):
    """ref/got [rows, N]: the worst per-column cosine."""
    return _worst_cos(ref, got, axis=0)


def worst_row_cos(ref, got):
    """ref/got [rows, N]: the worst per-row cosine."""
    return _worst_cos(ref, got, axis=1)


def amp_for(K: int, other_amp: float, target: float = 10.0) -> float:
    """Amplitude that puts a K-deep dot of two uniform fills near `target` rms
    (test-common.h:195-200)."""
    return 3.0 * target / (np.sqrt(float(K)) * other_amp)
