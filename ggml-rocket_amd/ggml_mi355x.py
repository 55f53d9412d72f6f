"""Python binding of libmi355x.so (the gfx950 prefill backend).

Two layers, both plain ctypes over the C ABI in include/:
  * the kernel entry points of mi355x_kernels.h (device pointers, sizes, a HIP stream), with
    torch-tensor helpers: torch only allocates device memory and names the stream;
  * the backend's host layer of mi355x_backend.h (claim rules, graph compute, counters), which
    mirrors ggml-rocket.h.

There is no fallback: if the shared library is missing, `lib()` raises.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libmi355x.so")

F32, F16, Q8_0, Q4_K, Q6_K, I32, BF16, MXFP4 = 0, 1, 8, 12, 14, 26, 30, 39
Q4_0, Q4_1, Q5_0, Q2_K, Q5_K = 2, 3, 6, 10, 13
F16_T = 0x101   # the library's tiled fp16 layout (16 x 32 tiles of 1 KB); not a ggml type
Q4_K_X = 0x10C  # Q4_K blocks regrouped by 32 rows, for expert stacks (MUL_MAT_ID); not a ggml type
Q8_0_X = 0x108  # Q8_0 blocks regrouped by 32 rows (quant plane, then scale plane); expert stacks only
MXFP4_X = 0x127  # MXFP4 blocks regrouped by 32 rows, as Q8_0_X; expert stacks only
Q6_K_X = 0x10E  # Q6_K blocks regrouped by 32 rows (four planes); expert stacks only
OK, E_ARG, E_DEVICE, E_UNSUPPORTED, E_NOMEM, E_IDS = 0, -1, -2, -3, -4, -5   # mi355x_status
BLOCK = {F16: 1, F32: 1, BF16: 1, Q8_0: 32, Q4_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256, MXFP4: 32}
TYPE_SIZE = {F16: 2, F32: 4, BF16: 2, Q8_0: 34, Q4_0: 18, Q4_K: 144, Q5_K: 176, Q6_K: 210, MXFP4: 17}

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
    L.mi355x_weight_f16_tiled.argtypes = [i32, vp, i64, i64, vp, vp]
    L.mi355x_pack_act.argtypes = [vp, i64, i64, i64, vp, vp, vp]
    L.mi355x_pack_act_tiled.argtypes = [vp, i64, i64, i64, vp, vp, vp]
    L.mi355x_gemm.argtypes = [i32, vp, vp, i64, i64, ctypes.POINTER(GemmOut), i32, vp]
    L.mi355x_gemm_workspace.restype = sz
    L.mi355x_gemm_workspace.argtypes = [i32, i64, i64, ctypes.POINTER(GemmOut), i32]
    L.mi355x_gemm_ws.argtypes = [i32, vp, vp, i64, i64, ctypes.POINTER(GemmOut), i32, vp, sz, i32, vp]
    L.mi355x_gemm_accumulates.argtypes = [i32, i64, i64, ctypes.POINTER(GemmOut), i32, sz]
    L.mi355x_pack_act_clear.argtypes = [i32, vp, i64, i64, i64, vp, vp, vp, i64, i64, vp]
    L.mi355x_mul_mat_workspace.restype = sz
    L.mi355x_mul_mat_workspace.argtypes = [i64, i64]
    L.mi355x_mul_mat_workspace_for.restype = sz
    L.mi355x_mul_mat_workspace_for.argtypes = [i32, i64, i64, i64]
    L.mi355x_mul_mat_decode_first.restype = i32
    L.mi355x_mul_mat_decode_first.argtypes = [i32, i64, i64, i64]
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
        L.mi355x_flash_attn_ex.argtypes = [pa, i32, i32, vp, sz, vp]
    if hasattr(L, "mi355x_mul_mat_noalloc"):
        L.mi355x_mul_mat_noalloc.argtypes = [i32, vp, i64, i64, vp, i64, i64, vp, i64, vp]
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
    """A ggml payload (numpy uint8 / uint16 / torch) -> its HBM layout, as a uint8 device tensor.
    Q4_K_X, Q8_0_X, Q6_K_X and MXFP4_X take the ggml blocks of their base type (rows % 32 == 0)
    and regroup them."""
    torch = _torch()
    import numpy as np
    if isinstance(payload, np.ndarray):
        raw = torch.from_numpy(np.ascontiguousarray(payload).view(np.uint8).reshape(-1)).to(device)
    else:
        raw = payload.contiguous().view(torch.uint8).reshape(-1).to(device)
    nbytes = weight_bytes(wtype, rows, K)
    if nbytes < 0 or raw.numel() != nbytes:
        raise MI355XError(f"payload of {raw.numel()} bytes is not {rows} rows of K={K} of type {wtype}")
    if wtype in (F16, Q4_K, Q5_K):
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


def tile_f16(wtype: int, w_dev, rows: int, K: int):
    """A weight in HBM layout -> the tiled fp16 layout (F16_T), as a uint8 device tensor."""
    torch = _torch()
    out = torch.empty(weight_bytes(F16_T, rows, K), dtype=torch.uint8, device=w_dev.device)
    check(lib().mi355x_weight_f16_tiled(wtype, _ptr(w_dev), rows, K, _ptr(out), stream_handle()),
          "weight_f16_tiled")
    return out


def pack_act(x, tiled: bool = False):
    """F32 [M, K] -> (fp16 activations, row scales [M]). tiled: the F16_T layout over M rows,
    returned as [ceil(M/16)*16, K] (the padding rows are never read)."""
    torch = _torch()
    M, K = x.shape
    rows = (M + 15) // 16 * 16 if tiled else M
    a16 = torch.empty((rows, K), dtype=torch.float16, device=x.device)
    sc = torch.empty((M,), dtype=torch.float32, device=x.device)
    fn = lib().mi355x_pack_act_tiled if tiled else lib().mi355x_pack_act
    check(fn(_ptr(x), x.stride(0), M, K, _ptr(a16), _ptr(sc), stream_handle()), "pack_act")
    return a16, sc


def gemm(wtype: int, a16, scales, K: int, outs, split_workspace: bool = True):
    """outs: list of (w_dev, rows_total, row0, N, c_tensor). M = len(scales). With
    split_workspace, mi355x_gemm_ws with the workspace its fastest K split asks for; without,
    mi355x_gemm (K split at most two ways)."""
    arr = (GemmOut * len(outs))()
    for i, (w, rows_total, row0, N, c) in enumerate(outs):
        arr[i] = GemmOut(w.data_ptr(), rows_total, row0, N, c.data_ptr(), c.stride(0))
    M = scales.shape[0]
    if not split_workspace:
        check(lib().mi355x_gemm(wtype, _ptr(a16), _ptr(scales), M, K, arr, len(outs), stream_handle()), "gemm")
        return
    need = int(lib().mi355x_gemm_workspace(wtype, M, K, arr, len(outs)))
    ws = _torch().empty(max(need, 1), dtype=_torch().uint8, device=a16.device)
    check(lib().mi355x_gemm_ws(wtype, _ptr(a16), _ptr(scales), M, K, arr, len(outs), _ptr(ws), need, 0,
                               stream_handle()), "gemm_ws")


def mul_mat(wtype: int, w_dev, N: int, K: int, x, out=None, workspace=None):
    """dst[M, N] = x[M, K] . W[N, K]^T with W already in HBM layout."""
    torch = _torch()
    M = x.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32, device=x.device)
    need = int(lib().mi355x_mul_mat_workspace_for(wtype, N, K, M))
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
    check(lib().mi355x_mul_mat(wtype, _ptr(w_dev), N, K, _ptr(x), x.stride(0), M, _ptr(out), out.stride(0),
                               _ptr(workspace), workspace.numel(), stream_handle()), "mul_mat")
    return out


def mul_mat_noalloc(wtype: int, w_dev, N: int, K: int, x, out):
    """mul_mat through mi355x_mul_mat_noalloc: the workspace is the library's static device
    scratch; `out` [M, >= N] is the caller's. Returns the status (no exception), so callers can
    check the size limit."""
    return lib().mi355x_mul_mat_noalloc(wtype, _ptr(w_dev), N, K, _ptr(x), x.stride(0), x.shape[0], _ptr(out),
                                        out.stride(0), stream_handle())


def _fa_args(q, k, v, mask, out, scale, softcap=0.0, max_bias=0.0):
    H, T, D = q.shape
    HK, KV, DV = v.shape
    return FaArgs(q.data_ptr(), q.stride(1), q.stride(0),
                  k.data_ptr(), k.stride(1), k.stride(0),
                  v.data_ptr(), v.stride(1), v.stride(0),
                  mask.data_ptr() if mask is not None else None, mask.stride(0) if mask is not None else 0,
                  out.data_ptr(), out.stride(1), out.stride(0),
                  D, DV, T, H, KV, HK, scale, max_bias, softcap)


def flash_attn_workspace(q, k, v, mask, out, scale: float = 1.0, softcap: float = 0.0, nsplit: int = 0) -> int:
    """Workspace bytes mi355x_flash_attn needs for these operands (0 for an unsupported op)."""
    return int(lib().mi355x_flash_attn_workspace(ctypes.byref(_fa_args(q, k, v, mask, out, scale, softcap)), nsplit))


FA_CLASSES_READY = 1


def flash_attn(q, k, v, mask, scale: float, softcap: float = 0.0, nsplit: int = 0, out=None,
               workspace=None, max_bias: float = 0.0, classes_ready: bool = False):
    """q [H, T, D] f32 (any strides with unit last-dim stride), k/v [HK, KV, D] fp16, mask
    [T', KV'] fp16 or None. Returns dst [T, H, D] f32. classes_ready: `workspace` holds the mask
    classes of an earlier call with the same mask, shapes and split (mi355x_flash_attn_ex)."""
    torch = _torch()
    H, T, D = q.shape
    HK, KV, DV = v.shape
    if out is None:
        out = torch.empty((T, H, DV), dtype=torch.float32, device=q.device)
    a = _fa_args(q, k, v, mask, out, scale, softcap, max_bias)
    need = int(lib().mi355x_flash_attn_workspace(ctypes.byref(a), nsplit))
    if need and (workspace is None or workspace.numel() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    wp = workspace.data_ptr() if need else None
    if classes_ready and workspace is None:
        raise MI355XError("flash_attn: classes_ready needs the workspace of the call that classified the mask")
    flags = FA_CLASSES_READY if classes_ready else 0
    check(lib().mi355x_flash_attn_ex(ctypes.byref(a), nsplit, flags, wp, need, stream_handle()), "flash_attn")
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


# ==== the backend host layer (include/mi355x_backend.h) =========================================
# A numpy-backed stand-in for the few ggml graph constructors the reference's tests use
# (ggml_new_tensor_*, ggml_mul_mat, ggml_mul_mat_id, ggml_flash_attn_ext, permute / view), with
# ggml's ne / nb conventions, so the host-layer tests read like the reference's.

OP_NONE, OP_MUL_MAT, OP_MUL_MAT_ID, OP_FLASH_ATTN_EXT, OP_RESHAPE, OP_VIEW, OP_PERMUTE, \
    OP_TRANSPOSE, OP_ADD, OP_SCALE, OP_OTHER = range(11)
BUF_NONE, BUF_HOST, BUF_REPACK, BUF_OTHER = range(4)
STATUS_SUCCESS, STATUS_FAILED = 0, -1
# ggml's published (block values, block bytes) of the types the descriptors here may carry
_TYPE_SIZE_ALL = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
                  10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 26: (1, 4),
                  30: (1, 2), 39: (32, 17)}


class Tensor(ctypes.Structure):
    pass


Tensor._fields_ = [("type", ctypes.c_int32), ("op", ctypes.c_int32),
                   ("ne", ctypes.c_int64 * 4), ("nb", ctypes.c_size_t * 4),
                   ("op_params", ctypes.c_int32 * 16), ("src", ctypes.POINTER(Tensor) * 10),
                   ("data", ctypes.c_void_p), ("name", ctypes.c_char * 64),
                   ("buffer_kind", ctypes.c_int32), ("buffer_id", ctypes.c_void_p),
                   ("buffer_size", ctypes.c_size_t)]


# ggml_to_float_t: (const void * src, float * dst, int64_t n)
TO_FLOAT_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.POINTER(ctypes.c_float), ctypes.c_int64)
_decoders = {}


def set_to_float(ttype, block, type_size, fn):
    """Registers a row decoder for a quantized type the kernels do not decode (the plugin passes
    ggml's to_float). `fn(src_addr, dst_float_ptr, n)`; kept alive for the process. Returns the
    status (0 or -1)."""
    cb = TO_FLOAT_FN(fn)
    st = host().mi355x_backend_set_to_float(ttype, block, type_size, cb)
    if st == 0:
        _decoders[ttype] = cb
    return st


def _bind_host(L):
    if getattr(L, "_host_bound", False):
        return L
    vp, i32, lng, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_long, ctypes.c_size_t
    pt = ctypes.POINTER(Tensor)
    L.mi355x_backend_name.restype = ctypes.c_char_p
    L.mi355x_backend_description.restype = ctypes.c_char_p
    L.mi355x_backend_get_memory.argtypes = [ctypes.POINTER(sz), ctypes.POINTER(sz)]
    L.mi355x_backend_get_host_memory.argtypes = [ctypes.POINTER(sz), ctypes.POINTER(sz)]
    L.mi355x_backend_supports_op.restype = ctypes.c_bool
    L.mi355x_backend_supports_op.argtypes = [pt]
    L.mi355x_backend_offload_op.restype = ctypes.c_bool
    L.mi355x_backend_offload_op.argtypes = [pt]
    L.mi355x_backend_supports_buft.restype = ctypes.c_bool
    L.mi355x_backend_supports_buft.argtypes = [i32]
    L.mi355x_backend_init.restype = vp
    L.mi355x_backend_free.argtypes = [vp]
    L.mi355x_backend_is.restype = ctypes.c_bool
    L.mi355x_backend_is.argtypes = [vp]
    L.mi355x_backend_set_n_threads.argtypes = [vp, i32]
    L.mi355x_backend_get_n_threads.argtypes = [vp]
    L.mi355x_backend_set_quant_resident.argtypes = [vp, i32]
    L.mi355x_backend_graph_compute.argtypes = [vp, ctypes.POINTER(pt), i32]
    L.mi355x_backend_route_ops.restype = lng
    L.mi355x_backend_route_ops.argtypes = [vp, ctypes.c_char_p]
    L.mi355x_backend_cpu_fallbacks.restype = lng
    L.mi355x_backend_cpu_fallbacks.argtypes = [vp]
    L.mi355x_backend_moe_stats.argtypes = [vp, ctypes.POINTER(lng), ctypes.POINTER(lng)]
    L.mi355x_backend_route_stats.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(lng), ctypes.POINTER(lng),
                                                  ctypes.POINTER(lng)]
    L.mi355x_backend_inject_faults.argtypes = [vp, ctypes.c_char_p, i32]
    L.mi355x_backend_host_stats.argtypes = [vp, ctypes.POINTER(HostStats)]
    L.mi355x_backend_weight_key.argtypes = [pt, ctypes.c_char_p, i32]
    L.mi355x_backend_register_weight_source.argtypes = [pt, vp, sz]
    L.mi355x_backend_parse_mb.restype = ctypes.c_bool
    L.mi355x_backend_parse_mb.argtypes = [ctypes.c_char_p, ctypes.POINTER(sz)]
    L.mi355x_backend_set_to_float.restype = i32
    L.mi355x_backend_set_to_float.argtypes = [i32, ctypes.c_int64, ctypes.c_int64, TO_FLOAT_FN]
    L._host_bound = True
    return L


class HostStats(ctypes.Structure):
    """mi355x_host_stats: where graph_compute's time goes on the host."""
    _fields_ = [("calls", ctypes.c_long), ("fa_mirror_hits", ctypes.c_long), ("copyback_redone", ctypes.c_long),
                ("bytes_up", ctypes.c_double), ("bytes_down", ctypes.c_double), ("wall_s", ctypes.c_double),
                ("up_copy_s", ctypes.c_double), ("up_wait_s", ctypes.c_double), ("down_copy_s", ctypes.c_double),
                ("down_wait_s", ctypes.c_double), ("copy_api_s", ctypes.c_double), ("weight_s", ctypes.c_double),
                ("pieces_up", ctypes.c_long), ("pieces_down", ctypes.c_long)]


def host():
    return _bind_host(lib())


class Graph:
    """Owns the descriptors and numpy buffers of one graph (a ggml_context stand-in). With
    alloc=False (a no_alloc context) tensors have no data, as in a supports_op probe."""

    def __init__(self, alloc=True):
        self.alloc = alloc
        self.tensors = []
        self.keep = []

    def _new(self, ttype, ne, name=None, op=OP_NONE, srcs=(), data=None):
        import numpy as np
        t = Tensor()
        t.type = ttype
        t.op = op
        ne = list(ne) + [1] * (4 - len(ne))
        blk, bsz = _TYPE_SIZE_ALL[ttype]
        for i in range(4):
            t.ne[i] = ne[i]
        t.nb[0] = bsz
        t.nb[1] = bsz * (ne[0] // blk)
        t.nb[2] = t.nb[1] * ne[1]
        t.nb[3] = t.nb[2] * ne[2]
        for i, s in enumerate(srcs):
            if s is not None:
                t.src[i] = ctypes.pointer(s)
        if name:
            t.name = name.encode()[:63]
        nbytes = t.nb[3] * ne[3]
        if self.alloc and op in (OP_NONE, OP_MUL_MAT, OP_MUL_MAT_ID, OP_FLASH_ATTN_EXT, OP_OTHER, OP_ADD, OP_SCALE):
            buf = np.zeros(max(nbytes, 1), dtype=np.uint8) if data is None else data
            self.keep.append(buf)
            t.data = buf.ctypes.data
            t.buffer_kind = BUF_HOST
            t.buffer_size = buf.nbytes
            t.buffer_id = buf.ctypes.data
        self.tensors.append(t)
        return t

    def new_tensor(self, ttype, ne, name=None):
        return self._new(ttype, ne, name)

    def set(self, t, arr):
        import numpy as np
        a = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
        n = min(a.nbytes, t.buffer_size)
        ctypes.memmove(t.data, a.ctypes.data, n)

    def get(self, t, dtype, shape):
        import numpy as np
        n = int(np.prod(shape)) * np.dtype(dtype).itemsize
        out = np.empty(shape, dtype=dtype)
        ctypes.memmove(out.ctypes.data, t.data, n)
        return out

    def mul_mat(self, a, b):
        return self._new(F32, [a.ne[1], b.ne[1], b.ne[2], b.ne[3]], op=OP_MUL_MAT, srcs=(a, b))

    def mul_mat_id(self, a, b, ids):
        return self._new(F32, [a.ne[1], ids.ne[0], b.ne[2], 1], op=OP_MUL_MAT_ID, srcs=(a, b, ids))

    def flash_attn_ext(self, q, k, v, mask, scale, max_bias=0.0, softcap=0.0, acc_prec=0):
        t = self._new(F32, [v.ne[0], q.ne[2], q.ne[1], q.ne[3]], op=OP_FLASH_ATTN_EXT, srcs=(q, k, v, mask))
        fp = (ctypes.c_float * 3)(scale, max_bias, softcap)
        ctypes.memmove(ctypes.addressof(t.op_params), fp, 12)
        if acc_prec:
            t.op_params[3] = acc_prec
        return t

    def op(self, ttype, ne, op, srcs=()):
        """A node of any other op (e.g. an ADD or a SCALE) for placement probes."""
        return self._new(ttype, ne, op=op, srcs=srcs)

    def permute_view(self, src, ne, nb, offset=0):
        """A strided view of `src` (ggml_view_* / ggml_permute): same bytes, new ne / nb."""
        t = Tensor()
        t.type = src.type
        t.op = OP_VIEW
        for i in range(4):
            t.ne[i] = ne[i]
            t.nb[i] = nb[i]
        t.src[0] = ctypes.pointer(src)
        if src.data:
            t.data = src.data + offset
            t.buffer_kind = src.buffer_kind
            t.buffer_size = src.buffer_size
            t.buffer_id = src.buffer_id
        self.tensors.append(t)
        return t


class Backend:
    """One backend instance (mi355x_backend_init .. free)."""

    def __init__(self):
        self.L = host()
        self.h = self.L.mi355x_backend_init()
        if not self.h:
            raise MI355XError("init failed")

    def free(self):
        if self.h:
            self.L.mi355x_backend_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def compute(self, nodes):
        arr = (ctypes.POINTER(Tensor) * len(nodes))(*[ctypes.pointer(n) for n in nodes])
        return self.L.mi355x_backend_graph_compute(self.h, arr, len(nodes))

    def route_ops(self, route=None):
        return self.L.mi355x_backend_route_ops(self.h, route.encode() if route else None)

    def cpu_fallbacks(self):
        return self.L.mi355x_backend_cpu_fallbacks(self.h)

    def moe_stats(self):
        a, b = ctypes.c_long(), ctypes.c_long()
        self.L.mi355x_backend_moe_stats(self.h, ctypes.byref(a), ctypes.byref(b))
        return a.value, b.value

    def route_stats(self, group):
        a, b, c = ctypes.c_long(), ctypes.c_long(), ctypes.c_long()
        self.L.mi355x_backend_route_stats(self.h, group.encode(), ctypes.byref(a), ctypes.byref(b), ctypes.byref(c))
        return a.value, b.value, c.value

    def set_quant_resident(self, mode):
        self.L.mi355x_backend_set_quant_resident(self.h, mode)

    def inject_faults(self, group, n):
        self.L.mi355x_backend_inject_faults(self.h, group.encode(), n)

    def host_stats(self):
        st = HostStats()
        self.L.mi355x_backend_host_stats(self.h, ctypes.byref(st))
        return {name: getattr(st, name) for name, _ in HostStats._fields_}


_registered = {}


def register_weight_source(t, src):
    """The original bytes of a weight whose tensor sits in CPU_REPACK (numpy array, or None to
    unregister); the array is kept alive while registered."""
    import numpy as np
    key = ctypes.addressof(t)
    if src is None:
        host().mi355x_backend_register_weight_source(ctypes.byref(t), None, 0)
        _registered.pop(key, None)
        return
    a = np.ascontiguousarray(src).view(np.uint8).reshape(-1)
    _registered[key] = a
    host().mi355x_backend_register_weight_source(ctypes.byref(t), ctypes.c_void_p(a.ctypes.data), a.nbytes)


def supports_op(t):
    return bool(host().mi355x_backend_supports_op(ctypes.byref(t)))


def offload_op(t):
    return bool(host().mi355x_backend_offload_op(ctypes.byref(t)))


def weight_key(t):
    buf = ctypes.create_string_buffer(256)
    host().mi355x_backend_weight_key(ctypes.byref(t), buf, 256)
    return buf.value.decode()


def parse_mb(text):
    v = ctypes.c_size_t(12345)
    ok = host().mi355x_backend_parse_mb(text.encode(), ctypes.byref(v))
    return ok, v.value
