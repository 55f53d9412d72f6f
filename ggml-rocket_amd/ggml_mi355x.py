"""Python binding of libggml-mi355x.so (the gfx950 prefill backend).

Two layers, both plain ctypes over the C ABI in include/:
  * the kernel entry points of mi355x_kernels.h (device pointers, sizes, a HIP stream), with
    torch-tensor helpers: torch only allocates device memory and names the stream;
  * the backend's host layer of ggml-mi355x.h (claim rules, graph compute, counters), which
    mirrors ggml-rocket.h.

There is no fallback: if the shared library is missing, `lib()` raises.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libggml-mi355x.so")

F32, F16, Q8_0, Q4_K, Q6_K, I32, BF16 = 0, 1, 8, 12, 14, 26, 30
BLOCK = {F16: 1, F32: 1, BF16: 1, Q8_0: 32, Q4_K: 256, Q6_K: 256}
TYPE_SIZE = {F16: 2, F32: 4, BF16: 2, Q8_0: 34, Q4_K: 144, Q6_K: 210}

_lib = None


class MI355XError(RuntimeError):
    pass


class GemmOut(ctypes.Structure):
    _fields_ = [("w_dev", ctypes.c_void_p), ("rows_total", ctypes.c_int64),
                ("row0", ctypes.c_int64), ("N", ctypes.c_int64),
                ("c_dev", ctypes.c_void_p), ("ldc", ctypes.c_int64)]


class DeviceInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 64), ("compute_units", ctypes.c_int),
                ("lds_bytes_per_block", ctypes.c_int), ("clock_khz", ctypes.c_int),
                ("hbm_total", ctypes.c_size_t), ("hbm_free", ctypes.c_size_t)]


class FaArgs(ctypes.Structure):
    _fields_ = [("q_dev", ctypes.c_void_p), ("q_nb1", ctypes.c_int64), ("q_nb2", ctypes.c_int64),
                ("k_dev", ctypes.c_void_p), ("k_nb1", ctypes.c_int64), ("k_nb2", ctypes.c_int64),
                ("v_dev", ctypes.c_void_p), ("v_nb1", ctypes.c_int64), ("v_nb2", ctypes.c_int64),
                ("mask_dev", ctypes.c_void_p), ("mask_nb1", ctypes.c_int64),
                ("dst_dev", ctypes.c_void_p), ("dst_nb1", ctypes.c_int64), ("dst_nb2", ctypes.c_int64),
                ("D", ctypes.c_int), ("DV", ctypes.c_int), ("T", ctypes.c_int), ("H", ctypes.c_int),
                ("KV", ctypes.c_int), ("HK", ctypes.c_int),
                ("scale", ctypes.c_float), ("max_bias", ctypes.c_float), ("softcap", ctypes.c_float)]


class MoeArgs(ctypes.Structure):
    _fields_ = [("wtype", ctypes.c_int),
                ("as_dev", ctypes.c_void_p), ("n_expert", ctypes.c_int64), ("N", ctypes.c_int64),
                ("K", ctypes.c_int64),
                ("b_dev", ctypes.c_void_p), ("ne11", ctypes.c_int64), ("b_nb1", ctypes.c_int64),
                ("b_nb2", ctypes.c_int64),
                ("ids_dev", ctypes.c_void_p), ("n_used", ctypes.c_int64), ("ids_nb0", ctypes.c_int64),
                ("ids_nb1", ctypes.c_int64),
                ("n_tokens", ctypes.c_int64),
                ("dst_dev", ctypes.c_void_p), ("dst_nb1", ctypes.c_int64), ("dst_nb2", ctypes.c_int64)]


def lib():
    """Load the built backend library. Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise MI355XError(f"{LIB_PATH} is missing: build it first (python -c "
                          f"'import __graft_entry__ as g; g.build()')")
    L = ctypes.CDLL(LIB_PATH)
    i64, i32, vp, sz = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t
    f32 = ctypes.c_float
    L.mi355x_status_str.restype = ctypes.c_char_p
    L.mi355x_status_str.argtypes = [i32]
    L.mi355x_get_device_info.argtypes = [ctypes.POINTER(DeviceInfo)]
    L.mi355x_weight_bytes.restype = i64
    L.mi355x_weight_bytes.argtypes = [i32, i64, i64]
    L.mi355x_weight_pack.argtypes = [i32, vp, i64, i64, vp, vp]
    L.mi355x_weight_dequant_f16.argtypes = [i32, vp, i64, i64, vp, vp]
    L.mi355x_pack_act.argtypes = [vp, i64, i64, i64, vp, vp, vp]
    L.mi355x_gemm.argtypes = [i32, vp, vp, i64, i64, ctypes.POINTER(GemmOut), i32, vp]
    L.mi355x_mul_mat_workspace.restype = sz
    L.mi355x_mul_mat_workspace.argtypes = [i64, i64]
    L.mi355x_mul_mat.argtypes = [i32, vp, i64, i64, vp, i64, i64, vp, i64, vp, sz, vp]
    _bind_optional(L)
    _lib = L
    return L


def _bind_optional(L):
    """Entry points of later kernel families; bound when the library exports them."""
    i64, i32, vp, sz, f32 = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_float
    if hasattr(L, "mi355x_flash_attn"):
        pa = ctypes.POINTER(FaArgs)
        L.mi355x_flash_attn_auto_split.restype = i32
        L.mi355x_flash_attn_auto_split.argtypes = [pa]
        L.mi355x_flash_attn_workspace.restype = sz
        L.mi355x_flash_attn_workspace.argtypes = [pa, i32]
        L.mi355x_flash_attn.argtypes = [pa, i32, vp, sz, vp]
    if hasattr(L, "mi355x_mul_mat_id"):
        pm = ctypes.POINTER(MoeArgs)
        L.mi355x_mul_mat_id_workspace.restype = sz
        L.mi355x_mul_mat_id_workspace.argtypes = [pm]
        L.mi355x_mul_mat_id.argtypes = [pm, vp, sz, vp, vp]


def check(status: int, what: str = "call"):
    if status != 0:
        msg = lib().mi355x_status_str(status).decode()
        raise MI355XError(f"{what}: status {status} ({msg})")


def status_str(status: int) -> str:
    return lib().mi355x_status_str(status).decode()


def device_info() -> dict:
    d = DeviceInfo()
    check(lib().mi355x_get_device_info(ctypes.byref(d)), "get_device_info")
    return {"name": d.name.decode(), "compute_units": d.compute_units,
            "lds_bytes_per_block": d.lds_bytes_per_block, "clock_khz": d.clock_khz,
            "hbm_total": d.hbm_total, "hbm_free": d.hbm_free}


# ---- torch helpers ------------------------------------------------------------------------

def _torch():
    import torch
    return torch


def stream_handle(stream=None):
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def weight_bytes(wtype: int, rows: int, K: int) -> int:
    return int(lib().mi355x_weight_bytes(wtype, rows, K))


def upload_weight(wtype: int, payload, rows: int, K: int, device="cuda"):
    """A ggml payload (numpy uint8 / uint16 / torch) -> its HBM layout, as a uint8 device tensor."""
    torch = _torch()
    import numpy as np
    if isinstance(payload, np.ndarray):
        raw = torch.from_numpy(np.ascontiguousarray(payload).view(np.uint8).reshape(-1)).to(device)
    else:
        raw = payload.contiguous().view(torch.uint8).reshape(-1).to(device)
    nbytes = weight_bytes(wtype, rows, K)
    if nbytes < 0 or raw.numel() != nbytes:
        raise MI355XError(f"payload of {raw.numel()} bytes is not {rows} rows of K={K} of type {wtype}")
    if wtype in (F16, Q4_K):
        return raw
    out = torch.empty(nbytes, dtype=torch.uint8, device=device)
    check(lib().mi355x_weight_pack(wtype, _ptr(raw), rows, K, _ptr(out), stream_handle()), "weight_pack")
    return out


def dequant_f16(wtype: int, w_dev, rows: int, K: int):
    torch = _torch()
    out = torch.empty((rows, K), dtype=torch.float16, device=w_dev.device)
    check(lib().mi355x_weight_dequant_f16(wtype, _ptr(w_dev), rows, K, _ptr(out), stream_handle()),
          "weight_dequant_f16")
    return out


def pack_act(x):
    torch = _torch()
    M, K = x.shape
    a16 = torch.empty((M, K), dtype=torch.float16, device=x.device)
    sc = torch.empty((M,), dtype=torch.float32, device=x.device)
    check(lib().mi355x_pack_act(_ptr(x), x.stride(0), M, K, _ptr(a16), _ptr(sc), stream_handle()), "pack_act")
    return a16, sc


def gemm(wtype: int, a16, scales, K: int, outs):
    """outs: list of (w_dev, rows_total, row0, N, c_tensor)."""
    arr = (GemmOut * len(outs))()
    for i, (w, rows_total, row0, N, c) in enumerate(outs):
        arr[i] = GemmOut(w.data_ptr(), rows_total, row0, N, c.data_ptr(), c.stride(0))
    M = a16.shape[0]
    check(lib().mi355x_gemm(wtype, _ptr(a16), _ptr(scales), M, K, arr, len(outs), stream_handle()), "gemm")


def mul_mat(wtype: int, w_dev, N: int, K: int, x, out=None, workspace=None):
    """dst[M, N] = x[M, K] . W[N, K]^T with W already in HBM layout."""
    torch = _torch()
    M = x.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32, device=x.device)
    need = int(lib().mi355x_mul_mat_workspace(M, K))
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
    check(lib().mi355x_mul_mat(wtype, _ptr(w_dev), N, K, _ptr(x), x.stride(0), M, _ptr(out), out.stride(0),
                               _ptr(workspace), workspace.numel(), stream_handle()), "mul_mat")
    return out


def flash_attn(q, k, v, mask, scale: float, softcap: float = 0.0, nsplit: int = 0, out=None,
               workspace=None, max_bias: float = 0.0):
    """q [H, T, D] f32 (any strides with unit last-dim stride), k/v [HK, KV, D] fp16, mask
    [T', KV'] fp16 or None. Returns dst [T, H, D] f32."""
    torch = _torch()
    H, T, D = q.shape
    HK, KV, DV = v.shape
    if out is None:
        out = torch.empty((T, H, DV), dtype=torch.float32, device=q.device)
    a = FaArgs(q.data_ptr(), q.stride(1), q.stride(0),
               k.data_ptr(), k.stride(1), k.stride(0),
               v.data_ptr(), v.stride(1), v.stride(0),
               mask.data_ptr() if mask is not None else None, mask.stride(0) if mask is not None else 0,
               out.data_ptr(), out.stride(1), out.stride(0),
               D, DV, T, H, KV, HK, scale, max_bias, softcap)
    need = int(lib().mi355x_flash_attn_workspace(ctypes.byref(a), nsplit))
    if need and (workspace is None or workspace.numel() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    wp = workspace.data_ptr() if need else None
    check(lib().mi355x_flash_attn(ctypes.byref(a), nsplit, wp, need, stream_handle()), "flash_attn")
    return out


def mul_mat_id(wtype: int, as_dev, n_expert: int, N: int, K: int, b, ids, out=None, workspace=None,
               err=None):
    """as_dev: expert panel in HBM layout (n_expert*N rows); b [T, ne11, K] f32; ids [T, n_used]
    int32. Returns dst [T, n_used, N] f32."""
    torch = _torch()
    T, ne11, _ = b.shape
    n_used = ids.shape[1]
    if out is None:
        out = torch.empty((T, n_used, N), dtype=torch.float32, device=b.device)
    a = MoeArgs(wtype, as_dev.data_ptr(), n_expert, N, K, b.data_ptr(), ne11, b.stride(1), b.stride(0),
                ids.data_ptr(), n_used, ids.stride(1), ids.stride(0), T,
                out.data_ptr(), out.stride(1), out.stride(0))
    need = int(lib().mi355x_mul_mat_id_workspace(ctypes.byref(a)))
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=b.device)
    check(lib().mi355x_mul_mat_id(ctypes.byref(a), _ptr(workspace), workspace.numel(),
                                  _ptr(err) if err is not None else None, stream_handle()), "mul_mat_id")
    return out
