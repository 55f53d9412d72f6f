// SPDX-License-Identifier: MIT
// The C ABI of the kernel library (include/mi355x_kernels.h): argument checks, HIP error
// mapping and launches. Nothing here allocates device memory.

#include "../../include/mi355x_kernels.h"

#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>

#include "mx_fa_dims.h"
#include "mx_kernels_impl.h"
#include "mx_weights.h"

namespace {

inline hipStream_t S(void * s) { return (hipStream_t)s; }

inline int hip_status(hipError_t e) {
    if (e == hipSuccess) return MI355X_OK;
    fprintf(stderr, "[mi355x] HIP error: %s\n", hipGetErrorString(e));
    return MI355X_E_DEVICE;
}

inline bool known_wtype(int wt) {
    return wt == mx::T_F16 || wt == mx::T_Q8_0 || wt == mx::T_Q4_0 || wt == mx::T_Q4_K || wt == mx::T_Q5_K ||
           wt == mx::T_Q6_K || wt == mx::T_MXFP4;
}

// the layouts regrouped by 32 rows, built from ggml blocks for expert stacks
inline bool x32_wtype(int wt) { return wt == mx::T_Q4_KX || wt == mx::T_Q8_0X || wt == mx::T_Q6_KX || wt == mx::T_MXFP4X; }

// the expert-stack layouts: every weight type, and the regrouped ones
inline bool known_moe_wtype(int wt) { return known_wtype(wt) || x32_wtype(wt); }

inline int64_t blck(int wt) {
    if (wt == mx::T_Q4_K || wt == mx::T_Q4_KX || wt == mx::T_Q5_K || wt == mx::T_Q6_K || wt == mx::T_Q6_KX) return 256;
    return (wt == mx::T_Q8_0 || wt == mx::T_Q8_0X || wt == mx::T_Q4_0 || wt == mx::T_MXFP4 || wt == mx::T_MXFP4X) ? 32 : 1;
}

inline bool aligned(const void * p, size_t a) { return ((uintptr_t)p % a) == 0; }

}  // namespace

extern "C" {

MI355X_API const char * mi355x_status_str(int st) {
    switch (st) {
        case MI355X_OK: return "ok";
        case MI355X_E_ARG: return "invalid argument";
        case MI355X_E_DEVICE: return "device error";
        case MI355X_E_UNSUPPORTED: return "unsupported";
        case MI355X_E_NOMEM: return "workspace too small";
        case MI355X_E_IDS: return "expert id out of range";
        default: return "unknown status";
    }
}

MI355X_API int mi355x_get_device_info(mi355x_device_info * out) {
    if (!out) return MI355X_E_ARG;
    memset(out, 0, sizeof(*out));
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e);
    hipDeviceProp_t p;
    e = hipGetDeviceProperties(&p, dev);
    if (e != hipSuccess) return hip_status(e);
    snprintf(out->name, sizeof(out->name), "%s", p.gcnArchName);
    out->compute_units = p.multiProcessorCount;
    out->lds_bytes_per_block = (int)p.sharedMemPerBlock;
    out->clock_khz = p.clockRate;
    size_t fr = 0, tot = 0;
    if (hipMemGetInfo(&fr, &tot) == hipSuccess) {
        out->hbm_free = fr;
        out->hbm_total = tot;
    }
    return MI355X_OK;
}

MI355X_API int64_t mi355x_weight_bytes(int wtype, int64_t rows, int64_t K) {
    if (wtype == mx::T_F16T) return (rows < 0 || K <= 0 || K % 32) ? -1 : mx::packed_weight_bytes(wtype, rows, K);
    if (x32_wtype(wtype)) return (rows < 0 || K <= 0 || K % blck(wtype)) ? -1 : mx::packed_weight_bytes(wtype, rows, K);
    if (!known_wtype(wtype) || rows < 0 || K <= 0 || K % blck(wtype)) return -1;
    return mx::packed_weight_bytes(wtype, rows, K);
}

MI355X_API int mi355x_weight_pack(int wtype, const void * src_dev, int64_t rows, int64_t K,
                                  void * dst_dev, void * stream) {
    if (x32_wtype(wtype)) {   // from ggml blocks; a regrouping, so never in place
        if (rows < 0 || rows % 32 || K <= 0 || K % blck(wtype)) return MI355X_E_ARG;
        if (rows == 0) return MI355X_OK;
        if (!src_dev || !dst_dev || src_dev == dst_dev || !aligned(dst_dev, 16)) return MI355X_E_ARG;
        if (wtype == mx::T_Q4_KX) {
            if (!aligned(src_dev, 16)) return MI355X_E_ARG;
            return hip_status(mx::launch_pack_q4kx(src_dev, rows, K, dst_dev, S(stream)));
        }
        return hip_status(mx::launch_pack_x32(wtype, src_dev, rows, K, dst_dev, S(stream)));
    }
    if (!known_wtype(wtype) || rows < 0 || K <= 0 || K % blck(wtype) || K % 32) return MI355X_E_ARG;
    if (rows == 0) return MI355X_OK;
    if (!src_dev || !dst_dev) return MI355X_E_ARG;
    if ((wtype == mx::T_Q8_0 || wtype == mx::T_Q4_0 || wtype == mx::T_Q6_K || wtype == mx::T_MXFP4) && src_dev == dst_dev)
        return MI355X_E_ARG;
    return hip_status(mx::launch_pack_weight(wtype, src_dev, rows, K, dst_dev, S(stream)));
}

MI355X_API int mi355x_weight_dequant_f16(int wtype, const void * w_dev, int64_t rows, int64_t K,
                                         uint16_t * out_dev, void * stream) {
    if (!known_wtype(wtype) || rows < 0 || K <= 0 || K % blck(wtype) || K % 64) return MI355X_E_ARG;
    if (rows == 0) return MI355X_OK;
    if (!w_dev || !out_dev || !aligned(w_dev, 16) || !aligned(out_dev, 16)) return MI355X_E_ARG;
    return hip_status(mx::launch_dequant_f16(wtype, w_dev, rows, K, out_dev, S(stream)));
}

MI355X_API int mi355x_weight_f16_tiled(int wtype, const void * w_dev, int64_t rows, int64_t K,
                                       uint16_t * out_dev, void * stream) {
    if (!known_wtype(wtype) || rows < 0 || K <= 0 || K % blck(wtype) || K % 64) return MI355X_E_ARG;
    if (rows == 0) return MI355X_OK;
    if (!w_dev || !out_dev || !aligned(w_dev, 16) || !aligned(out_dev, 16) || w_dev == (const void *)out_dev)
        return MI355X_E_ARG;
    return hip_status(mx::launch_f16_tiled(wtype, w_dev, rows, K, out_dev, S(stream)));
}

MI355X_API int mi355x_convert_f16(int type, const void * src_dev, int64_t n, uint16_t * dst_dev, void * stream) {
    if ((type != mx::T_F32 && type != mx::T_BF16) || n < 0) return MI355X_E_ARG;
    if (n == 0) return MI355X_OK;
    if (!src_dev || !dst_dev || !aligned(src_dev, type == mx::T_F32 ? 4 : 2) || !aligned(dst_dev, 2)) return MI355X_E_ARG;
    return hip_status(mx::launch_convert_f16(type, src_dev, n, dst_dev, S(stream)));
}

// zc (optional): an output [M][ldzc] whose first zn columns the pack kernel also clears
static int pack_impl(bool tiled, const float * x_dev, int64_t ldx, int64_t M, int64_t K, uint16_t * a16_dev,
                     float * scales_dev, void * stream, float * zc, int64_t ldzc, int64_t zn) {
    if (M < 0 || K <= 0 || K % (tiled ? 32 : 4) || ldx < K || ldx % 4 || M > INT32_MAX - 15 || K > INT32_MAX)
        return MI355X_E_ARG;
    if (M == 0) return MI355X_OK;
    if (!x_dev || !a16_dev || !scales_dev || !aligned(x_dev, 16) || !aligned(a16_dev, 8)) return MI355X_E_ARG;
    if (zc && (ldzc < zn || zn > INT32_MAX)) return MI355X_E_ARG;
    return tiled ? hip_status(mx::launch_pack_act_tiled(x_dev, ldx, (int)M, (int)K, a16_dev, scales_dev, S(stream),
                                                        zc, ldzc, (int)zn))
                 : hip_status(mx::launch_pack_act(x_dev, ldx, (int)M, (int)K, a16_dev, K, scales_dev, S(stream), zc,
                                                  ldzc, (int)zn));
}

MI355X_API int mi355x_pack_act(const float * x_dev, int64_t ldx, int64_t M, int64_t K,
                               uint16_t * a16_dev, float * scales_dev, void * stream) {
    return pack_impl(false, x_dev, ldx, M, K, a16_dev, scales_dev, stream, nullptr, 0, 0);
}

MI355X_API int mi355x_pack_act_tiled(const float * x_dev, int64_t ldx, int64_t M, int64_t K,
                                     uint16_t * a16_dev, float * scales_dev, void * stream) {
    return pack_impl(true, x_dev, ldx, M, K, a16_dev, scales_dev, stream, nullptr, 0, 0);
}

MI355X_API int mi355x_pack_act_clear(int tiled, const float * x_dev, int64_t ldx, int64_t M, int64_t K,
                                     uint16_t * a16_dev, float * scales_dev, float * clear_dev, int64_t ld_clear,
                                     int64_t n_clear, void * stream) {
    if (!clear_dev || n_clear <= 0 || !aligned(clear_dev, 4)) return MI355X_E_ARG;
    return pack_impl(tiled != 0, x_dev, ldx, M, K, a16_dev, scales_dev, stream, clear_dev, ld_clear, n_clear);
}

// The launch arguments of a GEMM, checked; `with_ptrs` also checks the operand pointers.
static int gemm_lower(int wtype, const uint16_t * a16_dev, const float * scales_dev, int64_t M, int64_t K,
                      const mi355x_gemm_out * outs, int n_out, bool with_ptrs, mx::GemmArgs & a) {
    const bool tiled = wtype == mx::T_F16T;
    if ((!known_wtype(wtype) && !tiled) || M < 0 || K <= 0 || K % 32 || K % blck(wtype) || M > INT32_MAX ||
        K > INT32_MAX)
        return MI355X_E_ARG;
    if (n_out < 1 || n_out > mx::GEMM_MAX_GROUPS || !outs) return MI355X_E_ARG;
    if (with_ptrs && M > 0 && (!a16_dev || !scales_dev || !aligned(a16_dev, 16))) return MI355X_E_ARG;
    memset(&a, 0, sizeof(a));
    a.A = a16_dev;
    a.scales = scales_dev;
    a.lda = K;
    a.M = (int)M;
    a.K = (int)K;
    a.m_tiles = (int)((M + 127) / 128);
    a.ng = n_out;
    int nt = 0;
    for (int i = 0; i < n_out; i++) {
        const mi355x_gemm_out & o = outs[i];
        if (o.N <= 0 || o.N % 16 || o.N > INT32_MAX || o.ldc < o.N || o.row0 < 0 || o.rows_total < o.row0 + o.N)
            return MI355X_E_ARG;
        if (with_ptrs && (!o.w_dev || !o.c_dev || !aligned(o.w_dev, 16))) return MI355X_E_ARG;
        a.g[i].W = o.w_dev;
        a.g[i].rows_total = o.rows_total;
        a.g[i].row0 = o.row0;
        a.g[i].N = (int)o.N;
        a.g[i].C = o.c_dev;
        a.g[i].ldc = o.ldc;
        a.g[i].ntile_begin = nt;
        nt += (int)((o.N + 127) / 128);
    }
    return MI355X_OK;
}

// c_zeroed: the outputs were cleared by the activation pack (mi355x_mul_mat); part / part_bytes:
// workspace for the partial sums of a K split past two ways
static int gemm_impl(int wtype, const uint16_t * a16_dev, const float * scales_dev, int64_t M, int64_t K,
                     const mi355x_gemm_out * outs, int n_out, void * stream, bool c_zeroed, void * part,
                     size_t part_bytes) {
    mx::GemmArgs a;
    const int st = gemm_lower(wtype, a16_dev, scales_dev, M, K, outs, n_out, true, a);
    if (st != MI355X_OK || M == 0) return st;
    if (part && !aligned(part, 16)) return MI355X_E_ARG;
    return hip_status(mx::launch_gemm(wtype, a, 0, S(stream), c_zeroed, (float *)part, part ? part_bytes : 0));
}

MI355X_API int mi355x_gemm(int wtype, const uint16_t * a16_dev, const float * scales_dev,
                           int64_t M, int64_t K, const mi355x_gemm_out * outs, int n_out,
                           void * stream) {
    return gemm_impl(wtype, a16_dev, scales_dev, M, K, outs, n_out, stream, false, nullptr, 0);
}

MI355X_API size_t mi355x_gemm_workspace(int wtype, int64_t M, int64_t K, const mi355x_gemm_out * outs, int n_out) {
    mx::GemmArgs a;
    if (M <= 0 || gemm_lower(wtype, nullptr, nullptr, M, K, outs, n_out, false, a) != MI355X_OK) return 0;
    return mx::gemm_split_bytes(wtype, a);
}

MI355X_API int mi355x_gemm_accumulates(int wtype, int64_t M, int64_t K, const mi355x_gemm_out * outs, int n_out,
                                       size_t workspace_bytes) {
    mx::GemmArgs a;
    const int st = gemm_lower(wtype, nullptr, nullptr, M, K, outs, n_out, false, a);
    if (st != MI355X_OK) return st;
    return M > 0 && mx::gemm_accumulates(wtype, a, workspace_bytes) ? 1 : 0;
}

MI355X_API int mi355x_gemm_ws(int wtype, const uint16_t * a16_dev, const float * scales_dev,
                              int64_t M, int64_t K, const mi355x_gemm_out * outs, int n_out,
                              void * workspace_dev, size_t workspace_bytes, int flags, void * stream) {
    return gemm_impl(wtype, a16_dev, scales_dev, M, K, outs, n_out, stream, (flags & MI355X_GEMM_OUT_ZEROED) != 0,
                     workspace_dev, workspace_bytes);
}

// M rows rounded up to 16: the tiled layout's padding (the row-major pack uses M rows of it).
static size_t mul_mat_a16_bytes(int64_t M, int64_t K) {
    return ((size_t)((M + 15) / 16 * 16) * (size_t)K * 2 + 255) & ~(size_t)255;
}

MI355X_API size_t mi355x_mul_mat_workspace(int64_t M, int64_t K) {
    if (M <= 0 || K <= 0) return 0;
    return mul_mat_a16_bytes(M, K) + (size_t)M * 4;
}

// The K-split partials of mi355x_mul_mat start at this offset of its workspace.
static size_t mul_mat_part_offset(int64_t M, int64_t K) {
    return (mi355x_mul_mat_workspace(M, K) + 255) & ~(size_t)255;
}

// Weights of the register-staged decode kernel run faster at M >= 512 decoded once per call into
// tiled fp16 (one pass over the weight) and multiplied by the fp16 GEMM than decoded inside the
// GEMM, where the decode sits on every tile's load path. Measured per call on MI355X with cold
// weights over N, K in {3072, 4096, 8192, 14336}: Q6_K, Q5_K and MXFP4 1.06-1.48x at M 512 and
// 1.24-1.91x at M 2048; Q8_0 and Q4_0 1.08-1.15x at M 512 with N >= K, 0.92-0.99x with N < K (the
// fp16 GEMM's few output tiles there), 1.19-1.52x at M 2048. Not M 128 and below (the decode pass
// costs more than the GEMM saves). Q4_K's all-DMA decode kernel is 0.83-1.38x of the two-pass
// form depending on the shape: the two-pass form wins where N >= K and the fp16 weight is at most
// 64 MB (1.02-1.38x, e.g. 1.20x for N 6144, K 4096 at M 512), and loses on larger panels, whose
// fp16 form no longer stays in the 256 MB last-level cache (0.83x for N 28672, K 4096 at M 512).
// Q8_0 with whole 256-value blocks has an all-DMA kernel of its own, which wins at M < 1024 but
// on one kind of shape (mx::q8_0_decode_first). Same fp16 weights and activations either way.
static bool mul_mat_decode_first(int wtype, int64_t M, int64_t N, int64_t K) {
    if (K % 64 || M < 512) return false;
    if (wtype == mx::T_Q6_K || wtype == mx::T_Q5_K || wtype == mx::T_MXFP4) return true;
    if (wtype == mx::T_Q4_K) return N >= K && N * K <= ((int64_t)1 << 25);
    if (wtype == mx::T_Q8_0) return mx::q8_0_decode_first(M, N, K);
    return wtype == mx::T_Q4_0 && (N >= K || M >= 1024);
}

MI355X_API int mi355x_mul_mat_decode_first(int wtype, int64_t M, int64_t N, int64_t K) {
    return known_wtype(wtype) && N > 0 && K > 0 && mul_mat_decode_first(wtype, M, N, K) ? 1 : 0;
}

// The tiled fp16 weight of the decode-first form sits right after the pack; the K-split
// partials after it.
static size_t mul_mat_w16_bytes(int64_t N, int64_t K) {
    return ((size_t)mi355x_weight_bytes(mx::T_F16T, N, K) + 255) & ~(size_t)255;
}

MI355X_API size_t mi355x_mul_mat_workspace_for(int wtype, int64_t N, int64_t K, int64_t M) {
    const size_t need = mi355x_mul_mat_workspace(M, K);
    if (need == 0) return 0;
    const mi355x_gemm_out o = {nullptr, N, 0, N, nullptr, N};
    if (known_wtype(wtype) && N > 0 && mul_mat_decode_first(wtype, M, N, K))
        return mul_mat_part_offset(M, K) + mul_mat_w16_bytes(N, K) + mi355x_gemm_workspace(mx::T_F16T, M, K, &o, 1);
    const size_t part = mi355x_gemm_workspace(wtype, M, K, &o, 1);
    return part ? mul_mat_part_offset(M, K) + part : need;
}

MI355X_API int mi355x_mul_mat(int wtype, const void * w_dev, int64_t N, int64_t K,
                              const float * x_dev, int64_t ldx, int64_t M,
                              float * dst_dev, int64_t ldd,
                              void * workspace_dev, size_t workspace_bytes, void * stream) {
    if (M == 0) return MI355X_OK;
    const size_t need = mi355x_mul_mat_workspace(M, K);
    if (need == 0) return MI355X_E_ARG;
    if (!workspace_dev || workspace_bytes < need) return MI355X_E_NOMEM;
    uint16_t * a16 = (uint16_t *)workspace_dev;
    float * scales = (float *)((char *)workspace_dev + mul_mat_a16_bytes(M, K));
    // the room past the pack holds the decode-first form's fp16 weight, if it runs, then K-split
    // partials
    size_t poff = mul_mat_part_offset(M, K);
    uint16_t * w16 = nullptr;
    if (known_wtype(wtype) && N > 0 && N <= INT32_MAX && mul_mat_decode_first(wtype, M, N, K) &&
        workspace_bytes >= poff + mul_mat_w16_bytes(N, K)) {
        w16 = (uint16_t *)((char *)workspace_dev + poff);
        poff += mul_mat_w16_bytes(N, K);
    }
    void * part = workspace_bytes > poff ? (char *)workspace_dev + poff : nullptr;
    const size_t part_bytes = part ? workspace_bytes - poff : 0;
    if (w16) {   // checks the weight's type, K and alignment like any other call of it
        const int st = mi355x_weight_f16_tiled(wtype, w_dev, N, K, w16, stream);
        if (st != MI355X_OK) return st;
        wtype = mx::T_F16T;
        w_dev = w16;
    }
    // a GEMM that adds a two-way K split into dst has it cleared by the pack, in the same launch
    bool zero = false;
    if ((known_wtype(wtype) || wtype == mx::T_F16T) && K > 0 && K <= INT32_MAX && M <= INT32_MAX && N > 0 &&
        N <= INT32_MAX && dst_dev && ldd >= N) {
        mx::GemmArgs probe;
        memset(&probe, 0, sizeof(probe));
        probe.M = (int)M;
        probe.K = (int)K;
        probe.ng = 1;
        probe.g[0].N = (int)N;
        zero = mx::gemm_accumulates(wtype, probe, part_bytes);
    }
    int st = pack_impl(wtype == mx::T_F16T, x_dev, ldx, M, K, a16, scales, stream, zero ? dst_dev : nullptr, ldd, N);
    if (st != MI355X_OK) return st;
    mi355x_gemm_out o = {w_dev, N, 0, N, dst_dev, ldd};
    return gemm_impl(wtype, a16, scales, M, K, &o, 1, stream, zero, part, part_bytes);
}

// ---- FLASH_ATTN_EXT ---------------------------------------------------------------------------

// Head dims past the fused kernel's builds (dk or dv > 256): two GEMMs around a softmax pass
// (mx_fa_wide.hip).
static bool fa_is_wide(const mi355x_fa_args * a) {
    return !mx::fa_dims_supported(a->D, a->DV) && mx::fa_wide_dims(a->D, a->DV);
}
static constexpr int64_t FA_WIDE_MAX_KV = 1 << 20;

static int fa_check(const mi355x_fa_args * a) {
    if (!a || !a->q_dev || !a->k_dev || !a->v_dev || !a->dst_dev) return MI355X_E_ARG;
    const bool wide = fa_is_wide(a);
    // dk, dv <= 256, multiples of 8 (fused kernel); else dk % 32 == 0, dv % 8 == 0 up to 1024
    if (!wide && !mx::fa_dims_supported(a->D, a->DV)) return MI355X_E_UNSUPPORTED;
    if (a->max_bias != 0.0f) return MI355X_E_UNSUPPORTED;
    if (a->T < 0 || a->H <= 0 || a->HK <= 0 || a->KV < 0 || a->H % a->HK) return MI355X_E_ARG;
    if (a->q_nb1 % 4 || a->q_nb2 % 4 || !aligned(a->q_dev, 16)) return MI355X_E_ARG;
    if (a->k_nb1 % 8 || a->k_nb2 % 8 || a->v_nb1 % 8 || a->v_nb2 % 8) return MI355X_E_ARG;
    if (!aligned(a->k_dev, 16) || !aligned(a->v_dev, 16)) return MI355X_E_ARG;
    if (a->dst_nb1 % 4 || a->dst_nb2 % 4 || !aligned(a->dst_dev, 16)) return MI355X_E_ARG;
    if (a->mask_dev && (a->mask_nb1 % 4 || a->mask_nb1 < a->KV || !aligned(a->mask_dev, 8))) return MI355X_E_ARG;
    if (wide ? (int64_t)a->KV > FA_WIDE_MAX_KV : (size_t)a->KV > mx::fa_max_kv(a->D, a->DV)) return MI355X_E_UNSUPPORTED;
    return MI355X_OK;
}

// Workspace of the wide path: fp16 queries and their row scales, one KV head's keys and
// transposed values, and one chunk of query rows' scores, fp16 P, 1 / row sums and output rows.
struct FaWideLayout {
    size_t q16, qsc, kc, vt, s, p16, psc, o, total;
    int kvp, rows_chunk;
};
static size_t up256_fa(size_t n) { return (n + 255) & ~(size_t)255; }
static FaWideLayout fa_wide_layout(const mi355x_fa_args * a) {
    FaWideLayout L;
    L.kvp = (int)((a->KV + 63) / 64 * 64);
    if (L.kvp == 0) L.kvp = 64;
    L.rows_chunk = mx::fa_wide_rows_chunk(a->T, a->H, a->HK, L.kvp);
    const size_t rows = (size_t)a->H * a->T, rc = (size_t)L.rows_chunk, kvp = (size_t)L.kvp;
    size_t o = 0;
    L.q16 = o;  o += up256_fa(rows * a->D * 2);
    L.qsc = o;  o += up256_fa(rows * 4);
    L.kc = o;   o += up256_fa(kvp * a->D * 2);
    L.vt = o;   o += up256_fa((size_t)a->DV * kvp * 2);
    L.s = o;    o += up256_fa(rc * kvp * 4);
    L.p16 = o;  o += up256_fa(rc * kvp * 2);
    L.psc = o;  o += up256_fa(rc * 4);
    L.o = o;    o += up256_fa(rc * a->DV * 4);
    L.total = o;
    return L;
}

static mx::FaArgs fa_lower(const mi355x_fa_args * a, int nsplit) {
    mx::FaArgs f;
    memset(&f, 0, sizeof(f));
    f.q = a->q_dev; f.k = a->k_dev; f.v = a->v_dev; f.mask = a->mask_dev; f.dst = a->dst_dev;
    f.q_nb1 = a->q_nb1; f.q_nb2 = a->q_nb2; f.k_nb1 = a->k_nb1; f.k_nb2 = a->k_nb2;
    f.v_nb1 = a->v_nb1; f.v_nb2 = a->v_nb2; f.mask_nb1 = a->mask_nb1;
    f.dst_nb1 = a->dst_nb1; f.dst_nb2 = a->dst_nb2;
    f.dk = a->D; f.dv = a->DV;
    mx::fa_pad_dims(a->D, a->DV, f.D, f.DV);   // the kernel's dims (checked by fa_check)
    f.T = a->T; f.H = a->H; f.HK = a->HK; f.KV = a->KV; f.nsplit = nsplit;
    f.tasks = 4;
    f.kvp = (int)((a->KV + 63) / 64 * 64);
    f.cls_stride = (f.kvp / 64 + 15) / 16 * 16;
    f.scale = a->scale; f.softcap = a->softcap;
    return f;
}

static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// Workspace: mask classes [T/32][cls_stride] | 256 bytes, the first 16 zeroed by the prep kernel |
// partial O [nsplit][T][H][DV] f32 and (max, sum) [nsplit][T][H][2] f32 when nsplit > 1 (DV as
// the kernel is built).
struct FaLayout {
    size_t cls, zero, po, pml, total;
};
static FaLayout fa_layout(const mx::FaArgs & f) {
    FaLayout L;
    const size_t nqt = (size_t)(f.T + 31) / 32;
    const size_t rows = (size_t)f.T * f.H * f.nsplit;
    L.cls = 0;
    L.zero = L.cls + align256(nqt * (size_t)f.cls_stride);
    L.po = L.zero + 256;
    L.pml = L.po + (f.nsplit > 1 ? align256(rows * f.DV * 4) : 0);
    L.total = L.pml + (f.nsplit > 1 ? align256(rows * 8) : 0);
    return L;
}

static int device_cus() {
    static int cus = 0;   // read once: this may run while a stream is being captured
    if (cus == 0) {
        int dev = 0;
        hipDeviceProp_t p;
        cus = (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&p, dev) == hipSuccess &&
               p.multiProcessorCount > 0) ? p.multiProcessorCount : 256;
    }
    return cus;
}

// The launch of an op: wave tasks per block and KV split (nsplit_req > 0: that split). One block
// per CU (their LDS rings take 128 KB). A step is two 64-key tiles for every task of a block:
// measured at head dims 128 / 128 on MI355X, 2.4 us with four tasks a block and 1.55 us with
// two (half the MFMA work, but the same barrier, DMA and latency chain per step), scaled here by
// the MFMA work of other head dims. A split writes its unnormalised partials and reads them back
// in the combine launch (about 3 us plus the partial bytes at 6 TB/s: 8.6 us at 512 queries x 32
// heads split two ways), and keeps at least 12 key tiles. MI355X_FA_TASKS (2 or 4) pins the
// task count, for tests.
struct FaPlan {
    int tasks, nsplit;
};
static FaPlan fa_plan(const mi355x_fa_args * a, int nsplit_req) {
    mx::FaArgs f = fa_lower(a, 1);
    const int ntiles = (int)((a->KV + 63) / 64);
    const int cus = device_cus();
    int pin = 0;
    if (const char * e = getenv("MI355X_FA_TASKS"))
        if (*e) pin = atoi(e);
    const int max_by_len = ntiles / 12 > 0 ? ntiles / 12 : 1;
    FaPlan best{4, nsplit_req > 0 ? nsplit_req : 1};
    double best_us = 0.0;
    bool have = false;
    for (int tasks = 2; tasks <= 4; tasks += 2) {
        if (!mx::fa_tasks_ok(f.DV, tasks) || (pin && pin != tasks)) continue;
        f.tasks = tasks;
        const int nb = mx::fa_blocks_per_split(f);
        const double step_us = (tasks == 2 ? 1.55 : 2.4) * (f.D + f.DV) / 256.0;
        const int lo = nsplit_req > 0 ? nsplit_req : 1, hi = nsplit_req > 0 ? nsplit_req : std::min(max_by_len, 16);
        for (int ns = lo; ns <= hi; ns++) {
            const double rounds = (double)((int64_t)nb * ns + cus - 1) / cus;
            const int steps = ((ntiles + ns - 1) / ns + 1) / 2;
            const double part_mb = (double)ns * a->T * a->H * f.DV * 8.0 / 1e6;
            const double us = (int64_t)rounds * steps * step_us + (ns > 1 ? 3.0 + part_mb / 6.0 : 0.0);
            if (!have || us < best_us - 1e-9) {
                best = {tasks, ns};
                best_us = us;
                have = true;
            }
        }
    }
    return best;
}

MI355X_API int mi355x_flash_attn_auto_split(const mi355x_fa_args * a) {
    if (fa_check(a) != MI355X_OK || fa_is_wide(a)) return 1;
    return fa_plan(a, 0).nsplit;
}

MI355X_API size_t mi355x_flash_attn_workspace(const mi355x_fa_args * a, int nsplit) {
    if (fa_check(a) != MI355X_OK) return 0;
    if (fa_is_wide(a)) return fa_wide_layout(a).total;   // no KV split on this path
    if (nsplit <= 0) nsplit = fa_plan(a, 0).nsplit;
    if (nsplit > 64) return 0;
    return fa_layout(fa_lower(a, nsplit)).total;
}

MI355X_API int mi355x_flash_attn(const mi355x_fa_args * a, int nsplit,
                                 void * workspace_dev, size_t workspace_bytes, void * stream) {
    return mi355x_flash_attn_ex(a, nsplit, 0, workspace_dev, workspace_bytes, stream);
}

MI355X_API int mi355x_flash_attn_ex(const mi355x_fa_args * a, int nsplit, int flags,
                                    void * workspace_dev, size_t workspace_bytes, void * stream) {
    if (flags & ~MI355X_FA_CLASSES_READY) return MI355X_E_ARG;
    const int st = fa_check(a);
    if (st != MI355X_OK) return st;
    if (a->T == 0) return MI355X_OK;
    if (fa_is_wide(a)) {
        const FaWideLayout L = fa_wide_layout(a);
        if (!workspace_dev || workspace_bytes < L.total || !aligned(workspace_dev, 256)) return MI355X_E_NOMEM;
        char * ws = (char *)workspace_dev;
        mx::FaWideArgs w;
        memset(&w, 0, sizeof(w));
        w.q = a->q_dev; w.k = a->k_dev; w.v = a->v_dev; w.mask = a->mask_dev; w.dst = a->dst_dev;
        w.q_nb1 = a->q_nb1; w.q_nb2 = a->q_nb2; w.k_nb1 = a->k_nb1; w.k_nb2 = a->k_nb2;
        w.v_nb1 = a->v_nb1; w.v_nb2 = a->v_nb2; w.mask_nb1 = a->mask_nb1;
        w.dst_nb1 = a->dst_nb1; w.dst_nb2 = a->dst_nb2;
        w.dk = a->D; w.dv = a->DV; w.T = a->T; w.H = a->H; w.HK = a->HK; w.KV = a->KV;
        w.kvp = L.kvp; w.rows_chunk = L.rows_chunk;
        w.scale = a->scale; w.softcap = a->softcap;
        w.q16 = (uint16_t *)(ws + L.q16); w.qsc = (float *)(ws + L.qsc);
        w.kc = (uint16_t *)(ws + L.kc); w.vt = (uint16_t *)(ws + L.vt);
        w.s = (float *)(ws + L.s); w.p16 = (uint16_t *)(ws + L.p16);
        w.psc = (float *)(ws + L.psc); w.o = (float *)(ws + L.o);
        return hip_status(mx::launch_fa_wide(w, S(stream)));
    }
    if (nsplit > 64) return MI355X_E_ARG;
    const FaPlan plan = fa_plan(a, nsplit);
    mx::FaArgs f = fa_lower(a, plan.nsplit);
    f.tasks = plan.tasks;
    nsplit = plan.nsplit;
    const FaLayout L = fa_layout(f);
    if (!workspace_dev || workspace_bytes < L.total || !aligned(workspace_dev, 256)) return MI355X_E_NOMEM;
    char * ws = (char *)workspace_dev;
    f.cls = (uint8_t *)(ws + L.cls);
    f.kzero = (uint16_t *)(ws + L.zero);
    if (nsplit > 1) {
        f.part_o = (float *)(ws + L.po);
        f.part_ml = (float *)(ws + L.pml);
    }
    return hip_status(mx::launch_fa(f, !(flags & MI355X_FA_CLASSES_READY), S(stream)));
}

// ---- MUL_MAT_ID -------------------------------------------------------------------------------

namespace {

struct MoeLayout {
    size_t a16, scales, off, rows, tiles, n_tiles, err, zero, total;
};

inline size_t up256(size_t x) { return (x + 255) & ~(size_t)255; }

bool moe_layout(const mi355x_moe_args * a, MoeLayout & L) {
    if (!a || a->n_tokens < 0 || a->n_used <= 0 || a->ne11 <= 0 || a->n_expert <= 0 || a->K <= 0 || a->N <= 0)
        return false;
    const size_t rows_b = (size_t)a->n_tokens * a->ne11;
    const size_t R = (size_t)a->n_tokens * a->n_used;
    const size_t tiles = (size_t)mx::moe_max_tiles((int)a->n_tokens, (int)a->n_used, (int)a->n_expert);
    size_t o = 0;
    L.a16 = o;     o += up256(rows_b * a->K * 2);
    L.scales = o;  o += up256(rows_b * 4);
    L.off = o;     o += up256(((size_t)a->n_expert + 1) * 4);
    L.rows = o;    o += up256((R > 0 ? R : 1) * 4);
    L.tiles = o;   o += up256(tiles * 8);
    L.n_tiles = o; o += 256;
    L.err = o;     o += 256;
    L.zero = o;    o += 256;
    L.total = o;
    return true;
}

}  // namespace

MI355X_API size_t mi355x_mul_mat_id_workspace(const mi355x_moe_args * a) {
    MoeLayout L;
    return moe_layout(a, L) ? L.total : 0;
}

MI355X_API int mi355x_mul_mat_id(const mi355x_moe_args * a, void * workspace_dev, size_t workspace_bytes,
                                 int32_t * err_dev, void * stream) {
    MoeLayout L;
    if (!moe_layout(a, L)) return MI355X_E_ARG;
    if (!known_moe_wtype(a->wtype) || a->K % 32 || a->K % blck(a->wtype) || a->N % 16) return MI355X_E_ARG;
    // experts are whole 32-row groups, each plane's share of one expert under 2^31 bytes
    if (x32_wtype(a->wtype) && (a->N % 32 || a->N * a->K > ((int64_t)1 << 31))) return MI355X_E_ARG;
    if (!a->as_dev || !a->b_dev || !a->ids_dev || !a->dst_dev || !aligned(a->as_dev, 16) || !aligned(a->b_dev, 16))
        return MI355X_E_ARG;
    if (a->b_nb1 < a->K || a->b_nb1 % 4 || a->b_nb2 != a->ne11 * a->b_nb1) return MI355X_E_ARG;
    if (a->n_expert * a->N > INT32_MAX || a->n_tokens * a->n_used > INT32_MAX || a->n_expert > 8192 ||
        a->n_tokens * a->ne11 > INT32_MAX || a->K > INT32_MAX)
        return MI355X_E_ARG;
    if (a->n_tokens == 0) return MI355X_OK;
    if (!workspace_dev || workspace_bytes < L.total) return MI355X_E_NOMEM;
    char * ws = (char *)workspace_dev;
    mx::MoeArgs m;
    memset(&m, 0, sizeof(m));
    m.w = a->as_dev; m.E = (int)a->n_expert; m.N = (int)a->N; m.K = (int)a->K;
    m.b = a->b_dev; m.b_nb1 = a->b_nb1; m.ne11 = (int)a->ne11; m.T = (int)a->n_tokens; m.U = (int)a->n_used;
    m.ids = a->ids_dev; m.ids_nb0 = a->ids_nb0; m.ids_nb1 = a->ids_nb1;
    m.dst = a->dst_dev; m.dst_nb1 = a->dst_nb1; m.dst_nb2 = a->dst_nb2;
    m.a16 = (uint16_t *)(ws + L.a16);
    m.scales = (float *)(ws + L.scales);
    m.off = (int32_t *)(ws + L.off);
    m.rows = (int32_t *)(ws + L.rows);
    m.tiles = (int32_t *)(ws + L.tiles);
    m.n_tiles = (int32_t *)(ws + L.n_tiles);
    m.err = err_dev ? err_dev : (int32_t *)(ws + L.err);
    m.zero = (uint16_t *)(ws + L.zero);
    return hip_status(mx::launch_moe(a->wtype, m, S(stream)));
}

}  // extern "C"
