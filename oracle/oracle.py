"""ctypes binding of the CPU oracle (liboracle.so, built from oracle.c).

Test infrastructure only: tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
it to check or time the HIP path. Nothing in the product library imports it.

Each function names the reference code it restates (see oracle.c for the C side).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(_HERE, "liboracle.so")

F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, BF16, MXFP4 = 0, 1, 2, 8, 12, 13, 14, 30, 39
TYPE_NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K",
              BF16: "BF16", MXFP4: "MXFP4"}

_lib = None


def build(force: bool = False) -> str:
    """Compile liboracle.so with the Makefile beside this file."""
    if force or not os.path.exists(_LIB):
        subprocess.run(["make", "-C", _HERE, "-B" if force else "liboracle.so"], check=True,
                       stdout=subprocess.DEVNULL)
    return _LIB


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            build()
        L = ctypes.CDLL(_LIB)
        i64, i32, f32, vp = ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_void_p
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [f32]
        L.orc_f16_to_f32.restype = f32
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f32_to_f16_row.argtypes = [vp, vp, i64]
        L.orc_f16_to_f32_row.argtypes = [vp, vp, i64]
        L.orc_fill_uniform.argtypes = [vp, i64, ctypes.c_uint64, f32]
        L.orc_fill_normal.argtypes = [vp, i64, ctypes.c_uint64, f32, f32]
        L.orc_block_size.restype = i64
        L.orc_block_size.argtypes = [i32]
        L.orc_type_size.restype = i64
        L.orc_type_size.argtypes = [i32]
        L.orc_row_size.restype = i64
        L.orc_row_size.argtypes = [i32, i64]
        L.orc_dequant_row.argtypes = [i32, vp, vp, i64]
        L.orc_dequant_rows_f16.argtypes = [i32, vp, vp, i64, i64]
        L.orc_dequant_rows_f32.argtypes = [i32, vp, vp, i64, i64]
        L.orc_quantize_rows.argtypes = [i32, vp, vp, i64, i64]
        L.orc_mul_mat.argtypes = [i32, vp, vp, vp, i64, i64, i64, i32]
        L.orc_mul_mat_id.argtypes = [i32, vp, i64, i64, i64, vp, i64, vp, i64, i64, vp, i32]
        L.orc_flash_attn.argtypes = [vp, vp, vp, vp, i64, vp, i32, i32, i32, i32, i32, i32,
                                     f32, f32, i32, i32]
        L.orc_pack_act.argtypes = [vp, i64, i64, vp, vp]
        L.orc_max_threads.restype = i32
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


# ---- fp16 ---------------------------------------------------------------------------------

def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_f16_row(_p(x), _p(out), x.size)
    return out


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_f16_to_f32_row(_p(h), _p(out), h.size)
    return out


# ---- fills (test-common.h:181-193) --------------------------------------------------------

def fill_uniform(shape, seed: int, amp: float) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    lib().orc_fill_uniform(_p(out), out.size, seed & 0xFFFFFFFFFFFFFFFF, amp)
    return out


def fill_normal(shape, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    lib().orc_fill_normal(_p(out), out.size, seed & 0xFFFFFFFFFFFFFFFF, mean, std)
    return out


# ---- quant formats ------------------------------------------------------------------------

def row_size(wtype: int, K: int) -> int:
    return int(lib().orc_row_size(wtype, K))


def quantize(wtype: int, W: np.ndarray) -> np.ndarray:
    """W f32 [..., K] -> the ggml block payload, uint8 [..., row_size]."""
    W = np.ascontiguousarray(W, dtype=np.float32)
    K = W.shape[-1]
    rb = row_size(wtype, K)
    if rb < 0:
        raise ValueError(f"K={K} is not a whole number of {TYPE_NAMES.get(wtype)} blocks")
    nrows = W.size // K
    out = np.empty(W.shape[:-1] + (rb,), dtype=np.uint8)
    if lib().orc_quantize_rows(wtype, _p(W), _p(out), nrows, K) != 0:
        raise ValueError("quantize failed")
    return out


def dequantize(wtype: int, Q: np.ndarray, K: int) -> np.ndarray:
    """The ggml payload [..., row_size] -> f32 [..., K] (the to_float contract)."""
    Q = np.ascontiguousarray(Q)
    rb = row_size(wtype, K)
    nrows = Q.nbytes // rb
    shape = Q.shape[:-1] + (K,) if (Q.dtype == np.uint8 and Q.shape[-1] == rb) else (nrows, K)
    out = np.empty(shape, dtype=np.float32)
    if lib().orc_dequant_rows_f32(wtype, _p(Q), _p(out), nrows, K) != 0:
        raise ValueError("dequantize failed")
    return out


def dequantize_f16(wtype: int, Q: np.ndarray, K: int) -> np.ndarray:
    """Dequantized then rounded to fp16, as uint16 bits (rocket_weight_to_fp16)."""
    Q = np.ascontiguousarray(Q)
    rb = row_size(wtype, K)
    nrows = Q.nbytes // rb
    out = np.empty((nrows, K), dtype=np.uint16)
    if lib().orc_dequant_rows_f16(wtype, _p(Q), _p(out), nrows, K) != 0:
        raise ValueError("dequantize failed")
    return out


def pack_act(X: np.ndarray):
    """Per-row max-abs scaled fp16 activations (rk_pack_act_row, ggml-rocket.cpp:1451-1475).
    Returns (a16 uint16 [M, K], scales f32 [M])."""
    X = np.ascontiguousarray(X, dtype=np.float32)
    M, K = X.shape
    a16 = np.empty((M, K), dtype=np.uint16)
    sc = np.empty((M,), dtype=np.float32)
    lib().orc_pack_act(_p(X), M, K, _p(a16), _p(sc))
    return a16, sc


# ---- ops ----------------------------------------------------------------------------------

def mul_mat(wtype: int, W: np.ndarray, X: np.ndarray, N: int, K: int, nthreads: int = 0) -> np.ndarray:
    """fp64 dst[M, N] = X[M, K] . W[N, K]^T, W in its stored format (rocket_cpu_matmul_slice)."""
    X = np.ascontiguousarray(X, dtype=np.float32)
    M = X.size // K
    W = np.ascontiguousarray(W)
    out = np.empty((M, N), dtype=np.float32)
    rc = lib().orc_mul_mat(wtype, _p(W), _p(X), _p(out), M, N, K, nthreads)
    if rc != 0:
        raise ValueError(f"orc_mul_mat rc={rc}")
    return out


def mul_mat_id(wtype: int, As: np.ndarray, K: int, N: int, n_expert: int, B: np.ndarray,
               ne11: int, ids: np.ndarray, nthreads: int = 0) -> np.ndarray:
    """dst[T, n_used, N] = as[ids[t, e]] . b[t, e % ne11] (ggml-rocket.cpp:6654-6662)."""
    As = np.ascontiguousarray(As)
    B = np.ascontiguousarray(B, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    n_tokens, n_used = ids.shape
    out = np.empty((n_tokens, n_used, N), dtype=np.float32)
    rc = lib().orc_mul_mat_id(wtype, _p(As), K, N, n_expert, _p(B), ne11, _p(ids), n_used,
                              n_tokens, _p(out), nthreads)
    if rc != 0:
        raise ValueError(f"orc_mul_mat_id rc={rc}")
    return out


def flash_attn(q: np.ndarray, k16: np.ndarray, v16: np.ndarray, mask16, scale: float,
               softcap: float = 0.0, q_mode: int = 0, nthreads: int = 0) -> np.ndarray:
    """q [H, T, D] f32; k16 [HK, KV, D], v16 [HK, KV, DV] fp16 bits; mask16 [T_pad, KV_pad] fp16
    bits or None. Returns dst [T, H, DV] f32. q_mode 0 rounds Q to fp16 (test-rocket-fa.cpp:
    101-135); q_mode 1 keeps it F32 (rocket_fa_ref_f32, ggml-rocket.cpp:5392-5442)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k16 = np.ascontiguousarray(k16, dtype=np.uint16)
    v16 = np.ascontiguousarray(v16, dtype=np.uint16)
    H, T, D = q.shape
    HK, KV, _ = k16.shape
    DV = v16.shape[2]
    out = np.empty((T, H, DV), dtype=np.float32)
    if mask16 is not None:
        mask16 = np.ascontiguousarray(mask16, dtype=np.uint16)
        mp, ms = _p(mask16), mask16.shape[1]
    else:
        mp, ms = None, 0
    rc = lib().orc_flash_attn(_p(q), _p(k16), _p(v16), mp, ms, _p(out), D, DV, T, H, KV, HK,
                              scale, softcap, q_mode, nthreads)
    if rc != 0:
        raise ValueError(f"orc_flash_attn rc={rc}")
    return out


def max_threads() -> int:
    return int(lib().orc_max_threads())
