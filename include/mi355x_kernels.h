/* SPDX-License-Identifier: MIT
 *
 * mi355x_kernels.h -- the C ABI of the gfx950 prefill kernels (libmi355x.so).
 *
 * This is the device library of the backend: what librocketnpu is to the reference (its call
 * sites in ggml-rocket.cpp are cited per entry). Plain pointers, sizes and an opaque stream;
 * no ggml or torch types cross it. Every pointer named *_dev is device memory (HBM) that the
 * caller owns; the library allocates nothing inside these calls unless a comment says so.
 * `stream` is a hipStream_t (NULL = the legacy default stream). Every call is asynchronous on
 * that stream and returns a status (MI355X_OK = 0, or a negative code below).
 *
 * Layouts follow ggml's contiguous tensors:
 *   MUL_MAT      W [N][K] (src0 ne=[K,N]), X [M][K] F32 (src1 ne=[K,M]), dst [M][N] F32.
 *   FLASH_ATTN   q [H][T][D] F32, k [HK][KV][D] fp16, v [HK][KV][DV] fp16,
 *                mask [T'][KV'] fp16 (T' >= T, KV' >= KV), dst [T][H][DV] F32.
 *   MUL_MAT_ID   as [E][N][K], b [T][ne11][K] F32, ids [T][n_used] I32, dst [T][n_used][N] F32.
 *
 * Weight types are ggml type ids: F16 = 1, Q4_0 = 2, Q8_0 = 8, Q4_K = 12, Q5_K = 13, Q6_K = 14,
 * MXFP4 = 39. A weight reaches a GEMM in its HBM layout: F16, Q4_K and Q5_K are the ggml payload
 * unchanged; Q4_0, Q8_0, Q6_K and MXFP4 are re-laid out once by mi355x_weight_pack (same bytes,
 * split into 16-byte-aligned planes).
 */
#ifndef MI355X_KERNELS_H
#define MI355X_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MI355X_API __attribute__((visibility("default")))

enum mi355x_status {
    MI355X_OK = 0,
    MI355X_E_ARG = -1,          /* a shape, stride, alignment or type the entry does not take */
    MI355X_E_DEVICE = -2,       /* a HIP error: launch, copy or allocation failure */
    MI355X_E_UNSUPPORTED = -3,  /* a structural decline (like ROCKET_E_UNSUPPORTED) */
    MI355X_E_NOMEM = -4,        /* workspace too small */
    MI355X_E_IDS = -5,          /* MUL_MAT_ID: an expert id outside [0, n_expert) */
};

enum mi355x_wtype { MI355X_F16 = 1, MI355X_Q4_0 = 2, MI355X_Q8_0 = 8, MI355X_Q4_K = 12, MI355X_Q5_K = 13,
                    MI355X_Q6_K = 14, MI355X_MXFP4 = 39,
                    /* not a ggml type: fp16 [rows][K] in 16 x 32 tiles of 1 KB, row-major inside,
                     * tile (r/16, k/32) at element ((r/16)*(K/32) + k/32)*512; rows padded to a
                     * multiple of 16 (padding never read). The resident fp16 form the GEMM streams
                     * fastest: each 64-lane load instruction reads one whole tile. */
                    MI355X_F16_T = 0x101,
                    /* not a ggml type: Q4_K blocks of [rows][K] (rows % 32 == 0) regrouped by 32
                     * rows, for expert stacks (mi355x_mul_mat_id only): for each group of 32 rows
                     * and 256-value block, the 32 rows' 16-byte headers (d, dmin, scales), then
                     * for each 64-value quarter the 32 rows' 32 bytes of nibbles. Same bytes as
                     * Q4_K; a wave's loads of a quarter are one contiguous KiB. Built from ggml
                     * Q4_K blocks by mi355x_weight_pack. */
                    MI355X_Q4_K_X = 0x10C,
                    /* not ggml types: Q8_0 / MXFP4 blocks of [rows][K] (rows % 32 == 0) regrouped
                     * by 32 rows, for expert stacks (mi355x_mul_mat_id only). Two planes, each in
                     * (32-row group, 32-value block, row) order: the quants (Q8_0: 32 int8 a
                     * block, MXFP4: 16 bytes of FP4 codes), then the block scales (Q8_0: fp16 d,
                     * MXFP4: the E8M0 byte). Same bytes as the ggml blocks; a wave's quant load
                     * of a block is 1 KiB (Q8_0) or 512 B (MXFP4) of consecutive bytes. Built from
                     * ggml blocks by mi355x_weight_pack. */
                    MI355X_Q8_0_X = 0x108, MI355X_MXFP4_X = 0x127,
                    /* not a ggml type: Q6_K blocks of [rows][K] (rows % 32 == 0) regrouped by 32
                     * rows, for expert stacks (mi355x_mul_mat_id only): the four planes ql, qh,
                     * scales, d, each in (32-row group, 256-value block) order, ql and qh as
                     * [16-byte chunk][row], scales as [row][16 bytes], d as [row]. Same bytes as
                     * the ggml blocks. Built from ggml Q6_K blocks by mi355x_weight_pack. */
                    MI355X_Q6_K_X = 0x10E };

typedef struct mi355x_device_info {
    char name[64];              /* e.g. "gfx950" */
    int  compute_units;
    int  lds_bytes_per_block;
    int  clock_khz;
    size_t hbm_total;
    size_t hbm_free;
} mi355x_device_info;

/* The current device's properties. Replaces rocket_hw_current() (ggml-rocket.cpp:4402, 7262)
 * and rocket_driver_name() (7273), which describe the NPU part and its driver. */
MI355X_API int mi355x_get_device_info(mi355x_device_info * out);

/* Human-readable text for a status code. */
MI355X_API const char * mi355x_status_str(int status);

/* ---- weights ------------------------------------------------------------------------------ */

/* Bytes of `rows` rows of K values of `wtype` in HBM layout (equal to the ggml payload size),
 * or -1 if K is not a whole number of the type's blocks. */
MI355X_API int64_t mi355x_weight_bytes(int wtype, int64_t rows, int64_t K);

/* ggml payload (device) -> HBM layout (device). For F16, Q4_K and Q5_K this is a copy (or
 * nothing, when src_dev == dst_dev); the split layouts need dst_dev != src_dev. Replaces the resident pack rocket_weights_pack (ggml-rocket.cpp:
 * 4362) and its segment form rocket_weights_pack_seg (5121). */
MI355X_API int mi355x_weight_pack(int wtype, const void * src_dev, int64_t rows, int64_t K,
                                  void * dst_dev, void * stream);

/* A weight in HBM layout -> fp16 [rows][K]: each value decoded exactly as ggml's dequantizer
 * does, then rounded once to fp16. The on-device form of rocket_weight_to_fp16 (ggml-rocket.cpp:
 * 3843-3931), used for the resident-fp16 ("prepacked-q") cache. */
MI355X_API int mi355x_weight_dequant_f16(int wtype, const void * w_dev, int64_t rows, int64_t K,
                                         uint16_t * out_dev, void * stream);

/* A weight in HBM layout (any weight type above) -> MI355X_F16_T, decoded exactly as
 * mi355x_weight_dequant_f16 decodes it (the same fp16 values, tiled). K % 64 == 0; out_dev holds
 * mi355x_weight_bytes(MI355X_F16_T, rows, K) bytes and does not alias w_dev. The tiled resident
 * form of rocket_weight_to_fp16 + the resident pack (ggml-rocket.cpp:3843-3931, 4362). */
MI355X_API int mi355x_weight_f16_tiled(int wtype, const void * w_dev, int64_t rows, int64_t K,
                                       uint16_t * out_dev, void * stream);

/* F32 (type 0) or BF16 (type 30) values -> fp16, round to nearest even: the resident form of an
 * F32 / BF16 weight (the F32 and BF16 branches of rocket_weight_to_fp16, ggml-rocket.cpp:
 * 3855-3890). n values; src 4- or 2-byte aligned, dst 2-byte aligned. */
MI355X_API int mi355x_convert_f16(int type, const void * src_dev, int64_t n, uint16_t * dst_dev, void * stream);

/* ---- MUL_MAT ----------------------------------------------------------------------------- */

/* F32 activations [M][ldx] -> fp16 [M][K] divided by each row's max |x| (1 for a zero row),
 * and the row scales [M]. The device form of rocket_pack_activations (ggml-rocket.cpp:
 * 1451-1502). K % 4 == 0, ldx % 4 == 0, x 16-byte aligned. */
MI355X_API int mi355x_pack_act(const float * x_dev, int64_t ldx, int64_t M, int64_t K,
                               uint16_t * a16_dev, float * scales_dev, void * stream);

/* mi355x_pack_act (tiled != 0: mi355x_pack_act_tiled) that also clears columns [0, n_clear) of
 * the M rows of an F32 matrix clear_dev (row stride ld_clear elements): the output of a GEMM that
 * adds a two-way K split into it (mi355x_gemm_accumulates), cleared in the same launch instead
 * of by a fill of the GEMM's own (pass MI355X_GEMM_OUT_ZEROED to mi355x_gemm_ws). No counterpart
 * in the reference, whose NPU GEMM writes its output. */
MI355X_API int mi355x_pack_act_clear(int tiled, const float * x_dev, int64_t ldx, int64_t M, int64_t K,
                                     uint16_t * a16_dev, float * scales_dev, float * clear_dev, int64_t ld_clear,
                                     int64_t n_clear, void * stream);

/* mi355x_pack_act with the fp16 output in the MI355X_F16_T layout (ceil(M/16)*16 rows; the
 * padding rows are never read), for a GEMM on MI355X_F16_T weights. K % 32 == 0. Same values and
 * scales as mi355x_pack_act (rocket_pack_activations, ggml-rocket.cpp:1451-1502). */
MI355X_API int mi355x_pack_act_tiled(const float * x_dev, int64_t ldx, int64_t M, int64_t K,
                                     uint16_t * a16_dev, float * scales_dev, void * stream);

/* One output of a (fused) GEMM launch. */
typedef struct mi355x_gemm_out {
    const void * w_dev;     /* weight panel in HBM layout */
    int64_t rows_total;     /* rows of the whole panel (the split layouts index planes by it) */
    int64_t row0;           /* first row of this weight in the panel */
    int64_t N;              /* rows of this weight = output columns; N % 16 == 0 */
    float * c_dev;          /* output [M][ldc] F32 */
    int64_t ldc;
} mi355x_gemm_out;

/* c[m][n] = scales[m] * sum_k a16[m][k] * w[row0 + n][k], for each of `n_out` (1..4) weights of
 * one type that share the activation, in ONE launch over their concatenated N. fp16 MFMA, fp32
 * accumulation, F32 output. K % 32 == 0 (and a whole number of the type's blocks). For
 * MI355X_F16_T weights a16 is tiled too (mi355x_pack_act_tiled).
 * Replaces rocket_matmul_fp16_prepacked (ggml-rocket.cpp:4449, 5144),
 * rocket_matmul_fp16_stream (4834), rocket_matmul_fp16_mt (4844) and the fused
 * rocket_matmul_fp16_stream_fused (5004).
 * Results are reproducible: equal inputs give equal bits on every call. A launch may split K
 * over blocks; this entry has no workspace, so it splits at most two ways, adding both parts
 * into the zeroed output (two addends on zero sum the same in either order). Wider splits, the
 * fast form for M <= 128 and for deep K, need mi355x_gemm_ws. */
MI355X_API int mi355x_gemm(int wtype, const uint16_t * a16_dev, const float * scales_dev,
                           int64_t M, int64_t K, const mi355x_gemm_out * outs, int n_out,
                           void * stream);

/* Bytes of device workspace with which mi355x_gemm_ws runs this launch's fastest K split: one
 * F32 slab [M][sum of the outputs' N] per split when it splits more than two ways, else 0 (0 also
 * for invalid arguments; the pointers in `outs` are not read). */
MI355X_API size_t mi355x_gemm_workspace(int wtype, int64_t M, int64_t K, const mi355x_gemm_out * outs, int n_out);

/* mi355x_gemm with a workspace (16-byte aligned) for the partial sums of a K split past two ways.
 * Each split writes its slab; a second launch sums the slabs in split order into the outputs,
 * so the result does not depend on the order in which blocks finish (reproducible, as the CPU
 * backend's MUL_MAT is). With fewer bytes than mi355x_gemm_workspace asks, the split narrows to
 * what fits (down to two ways). The same bytes give the same bits on every call; a different
 * workspace size may pick a different split and round differently. */
MI355X_API int mi355x_gemm_ws(int wtype, const uint16_t * a16_dev, const float * scales_dev,
                              int64_t M, int64_t K, const mi355x_gemm_out * outs, int n_out,
                              void * workspace_dev, size_t workspace_bytes, int flags, void * stream);

/* flags of mi355x_gemm_ws: the outputs are already zero (cleared by mi355x_pack_act_clear), so a
 * launch that adds a two-way split into them launches no fill of its own. */
#define MI355X_GEMM_OUT_ZEROED 1

/* 1 if mi355x_gemm_ws with `workspace_bytes` of workspace adds a two-way K split into zeroed
 * outputs for this launch (the outputs must then be zero: cleared by the caller, with
 * MI355X_GEMM_OUT_ZEROED, or by the launch itself), 0 if it writes them, or a negative status
 * for arguments mi355x_gemm_ws would refuse (the pointers in `outs` are not read). */
MI355X_API int mi355x_gemm_accumulates(int wtype, int64_t M, int64_t K, const mi355x_gemm_out * outs, int n_out,
                                       size_t workspace_bytes);

/* 1 if a MUL_MAT of M rows with this weight layout and N x K weight runs faster in the
 * decode-first form (the weight decoded once into tiled fp16, mi355x_weight_f16_tiled, then
 * multiplied as MI355X_F16_T) than decoded inside the GEMM, else 0: Q6_K, Q5_K and MXFP4
 * weights at M >= 512, Q8_0 and Q4_0 at M >= 1024 or at M >= 512 with N >= K, Q4_K at M >= 512
 * with N >= K and N * K <= 2^25, K % 64 == 0 (measured on MI355X).
 * No counterpart in the reference, whose per-call fp16 route always decodes first. */
MI355X_API int mi355x_mul_mat_decode_first(int wtype, int64_t M, int64_t N, int64_t K);

/* Workspace bytes mi355x_mul_mat needs for M rows of K: the activation pack. */
MI355X_API size_t mi355x_mul_mat_workspace(int64_t M, int64_t K);

/* Workspace bytes with which mi355x_mul_mat runs its fastest form for this shape: the pack,
 * then (from the next 256-byte boundary) the decode-first form's tiled fp16 weight where that
 * form runs (mi355x_mul_mat_decode_first), then the split
 * partials mi355x_gemm_workspace names. */
MI355X_API size_t mi355x_mul_mat_workspace_for(int wtype, int64_t N, int64_t K, int64_t M);

/* dst[M][ldd] = x[M][ldx] . w[N][K]^T: mi355x_pack_act (mi355x_pack_act_tiled for MI355X_F16_T)
 * then mi355x_gemm_ws, the activation pack at the start of `workspace_dev` and the K-split
 * partials in the bytes past it (mi355x_mul_mat_workspace_for sizes both; with only
 * mi355x_mul_mat_workspace bytes the split is at most two ways). Reproducible as mi355x_gemm_ws.
 * Decode-first form: where mi355x_mul_mat_decode_first says so, the weight is decoded once per
 * call into tiled fp16 in the workspace
 * (mi355x_weight_f16_tiled) and multiplied as MI355X_F16_T, when the workspace holds that
 * weight; the same fp16 weights and activations as the in-GEMM decode, faster at those shapes.
 * The whole MUL_MAT of ggml-rocket.cpp:4548-4871 on device. */
MI355X_API int mi355x_mul_mat(int wtype, const void * w_dev, int64_t N, int64_t K,
                              const float * x_dev, int64_t ldx, int64_t M,
                              float * dst_dev, int64_t ldd,
                              void * workspace_dev, size_t workspace_bytes, void * stream);

/* Bytes of the static device scratch of mi355x_mul_mat_noalloc (64 MiB per GPU). */
#define MI355X_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

/* mi355x_mul_mat without a workspace argument: no counterpart in the reference. For callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). The workspace lives in a file-scope device array of
 * MI355X_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends; the call allocates nothing
 * and frees nothing. Limit: mi355x_mul_mat_workspace(M, K) <= MI355X_NOALLOC_SCRATCH_BYTES
 * (e.g. M 2048 at K 14336), else MI355X_E_NOMEM with a message. Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (two streams, two threads) race and must be
 * serialized by the caller. The first call on a device resolves the array's address there
 * (make it outside a stream capture); later calls may be captured. It computes exactly what
 * mi355x_mul_mat computes given MI355X_NOALLOC_SCRATCH_BYTES of workspace: the scratch holds
 * the activation pack, then, where the decode-first form runs (mi355x_mul_mat_decode_first) and
 * the pack plus the tiled fp16 weight fit, that weight, and the K-split partials in what is left.
 * So the form depends on the fit: a quantized weight whose fp16 image does not fit beside the
 * pack (e.g. Q6_K 8192 x 4096 at M 512: 4 MiB + 64 MiB) is decoded inside the GEMM here while
 * mi355x_mul_mat with mi355x_mul_mat_workspace_for bytes decodes it first; both forms meet the
 * same MUL_MAT bars, but their bits can differ in the last place. */
MI355X_API int mi355x_mul_mat_noalloc(int wtype, const void * w_dev, int64_t N, int64_t K,
                                      const float * x_dev, int64_t ldx, int64_t M,
                                      float * dst_dev, int64_t ldd, void * stream);

/* ---- FLASH_ATTN_EXT ---------------------------------------------------------------------- */

/* One attention op. Strides are in ELEMENTS, so strided ggml views (a KV-cache slice, a
 * permuted Q) are read in place. */
typedef struct mi355x_fa_args {
    const float * q_dev;      int64_t q_nb1, q_nb2;      /* token, head strides */
    const uint16_t * k_dev;   int64_t k_nb1, k_nb2;      /* key, kv-head strides (fp16) */
    const uint16_t * v_dev;   int64_t v_nb1, v_nb2;      /* key, kv-head strides (fp16) */
    const uint16_t * mask_dev; int64_t mask_nb1;         /* token stride; NULL = unmasked */
    float * dst_dev;          int64_t dst_nb1, dst_nb2;  /* head, token strides */
    int D, DV, T, H, KV, HK;
    float scale, max_bias, softcap;
} mi355x_fa_args;

/* The KV-split count mi355x_flash_attn uses when called with nsplit = 0. The launch is planned per
 * call: the block layout (two or four 32-query tasks per block) and the split that together
 * minimise an estimate from measured per-step costs; MI355X_FA_TASKS=2|4 in the environment pins
 * the layout (for tests). The result does not depend on the layout beyond fp32 summation order. */
MI355X_API int mi355x_flash_attn_auto_split(const mi355x_fa_args * a);

/* Workspace bytes for `nsplit` KV splits (0 = auto): the per-tile mask classes, 16 zero bytes
 * (the source of zero-padded head dims) and, for nsplit > 1, the partial outputs and their
 * (max, sum); for head dims past 256, the fp16 queries, one KV head's keys and transposed
 * values, and a chunk of query rows' scores and fp16 P (at most 64 MiB of F32 scores). Always
 * non-zero for a valid op; the workspace must be 256-byte aligned. */
MI355X_API size_t mi355x_flash_attn_workspace(const mi355x_fa_args * a, int nsplit);

/* dst = softmax(cap(scale * q.k) + mask) . v for every (token, head); head h reads KV head
 * h / (H / HK). On `stream`: a prep pass over the mask, the attention, and for a KV split a
 * launch that merges the splits.
 * Concurrent calls must not share a workspace. D and DV up to 256, multiples of 8, run fused (the
 * kernels are built for (64, 64), (128, 128), the MLA (192, 128) and (256, 256); other dims run
 * zero-padded on the smallest that holds them); past 256 (the absorbed MLA's 576 / 512: D % 32
 * == 0, DV % 8 == 0, both up to 1024) as two GEMMs around a softmax pass over a bounded chunk
 * of query rows at a time, with no KV split; H % HK == 0; max_bias
 * must be 0 (no ALiBi); the mask
 * covers [T][KV] with mask_nb1 % 4 == 0; q rows and dst rows 16-byte aligned; k/v rows 16-byte
 * aligned. Rows whose every key is masked are written as zeros. Replaces
 * rocket_flash_attn_fp16_ctx / _mt (ggml-rocket.cpp:5589-5606) and, because no fp16 score
 * surface exists here, the range fallback rocket_fa_ref_f32 (5617-5626) as well. */
MI355X_API int mi355x_flash_attn(const mi355x_fa_args * a, int nsplit,
                                 void * workspace_dev, size_t workspace_bytes, void * stream);

/* mi355x_flash_attn with flags. MI355X_FA_CLASSES_READY: skip the prep pass, because this
 * workspace already holds its results for this mask -- written by an earlier call on the same
 * stream with the same mask bytes, T, KV, head dims and split (nsplit as resolved), and not
 * overwritten since. A graph's layers share one KQ mask per micro-batch, so the first attention
 * of the micro-batch classifies the mask tiles and the others reuse them. The flag is ignored for
 * head dims past 256. No counterpart in the reference (its NPU path has no prep pass). */
#define MI355X_FA_CLASSES_READY 1
MI355X_API int mi355x_flash_attn_ex(const mi355x_fa_args * a, int nsplit, int flags,
                                    void * workspace_dev, size_t workspace_bytes, void * stream);

/* ---- MUL_MAT_ID --------------------------------------------------------------------------- */

/* One expert-GEMM op. Strides in ELEMENTS. */
typedef struct mi355x_moe_args {
    int wtype;
    const void * as_dev;      int64_t n_expert, N, K;     /* experts [E][N][K], HBM layout over E*N rows */
    const float * b_dev;      int64_t ne11, b_nb1, b_nb2; /* activations [T][ne11][K]; rows contiguous */
    const int32_t * ids_dev;  int64_t n_used, ids_nb0, ids_nb1;  /* ids[t][s] */
    int64_t n_tokens;
    float * dst_dev;          int64_t dst_nb1, dst_nb2;   /* dst[t][s][:] */
} mi355x_moe_args;

/* Workspace bytes of mi355x_mul_mat_id for this op. */
MI355X_API size_t mi355x_mul_mat_id_workspace(const mi355x_moe_args * a);

/* dst[t][s][:] = as[ids[t][s]] . b[t][s % ne11][:] for every token t and slot s, in one device
 * pipeline with no host synchronisation: the distinct activation rows are packed once, the rows
 * are bucketed by expert on the device, and one grouped launch runs every (expert tile, N block)
 * with the expert's weight dequantized in LDS. An id outside [0, n_expert) leaves its row
 * unwritten and sets *err_dev (a device int32, may be NULL) to 1; the host-buffer path checks ids
 * before calling. K % 32 == 0 and a whole number of blocks, N % 16 == 0; for the layouts
 * regrouped by 32 rows (MI355X_*_X) N % 32 == 0 and N * K <= 2^31 (one expert's weights).
 * Replaces the per-expert loop of ggml-rocket.cpp:6783-6941 and its device calls
 * rocket_matmul_int8_prepacked_gw (6833) / rocket_matmul_fp16_mt (6922). */
MI355X_API int mi355x_mul_mat_id(const mi355x_moe_args * a, void * workspace_dev, size_t workspace_bytes,
                                 int32_t * err_dev, void * stream);

#ifdef __cplusplus
}
#endif

#endif /* MI355X_KERNELS_H */
