// SPDX-License-Identifier: MIT
// Launch interfaces between the C ABI (mx_api.cpp) and the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mx {

constexpr int GEMM_MAX_GROUPS = 4;

// One weight of a (possibly fused) GEMM launch: its panel, its output, and where its N tiles
// start in the launch's concatenated N.
struct GemmGroup {
    const void * W;        // HBM weight, layout per mx_weights.h
    int64_t rows_total;    // rows of the whole panel W (the split layouts index planes by it)
    int64_t row0;          // first row of this weight inside the panel
    int N;                 // rows used (output columns)
    float * C;             // output [M][ldc]
    int64_t ldc;
    int ntile_begin;       // first global N tile of this group
    int64_t pcol;          // first column of this group in a row of the K-split partials
};

struct GemmArgs {
    const uint16_t * A;    // fp16 activations [M][lda], row-scaled (tiled for T_F16T weights)
    const float * scales;  // [M]
    int64_t lda;
    int M, K;
    int m_tiles;
    int ng;
    int ksplit;            // K split of a register-staged split configuration (set by the launcher)
    float * part;          // K splits past two: [ksplit][M][ldp] partial sums, one slab per split,
                           // summed in split order by a second launch (null: no such split)
    int64_t ldp;           // row length of the partials: the groups' N, concatenated
    GemmGroup g[GEMM_MAX_GROUPS];
};

// FLASH_ATTN_EXT launch: strides in elements.
struct FaArgs {
    const float * q;           // [H][T][D] via q_nb2 (head), q_nb1 (token)
    const uint16_t * k;        // [HK][KV][D] via k_nb2, k_nb1
    const uint16_t * v;        // [HK][KV][D] via v_nb2, v_nb1
    const uint16_t * mask;     // [T'][KV'] via mask_nb1, or null
    float * dst;               // [T][H][D] via dst_nb2 (token), dst_nb1 (head)
    float * part_o;            // [nsplit][T][H][D] when nsplit > 1
    float * part_ml;           // [nsplit][T][H][2]
    uint8_t * cls;             // workspace: mask class per (32-query tile, 64-key tile), rows of cls_stride
    int64_t q_nb1, q_nb2, k_nb1, k_nb2, v_nb1, v_nb2, mask_nb1, dst_nb1, dst_nb2;
    uint16_t * kzero;          // workspace: 16 zero bytes (written by the prep kernel), the K and
                               // V source of the padded columns
    int D, DV, T, H, HK, KV, kvp, cls_stride, nsplit;   // D: Q / K head dim, DV: V / output, as
                                                        // the kernel is built (fa_pad_dims)
    int tasks;                 // wave tasks per block: 4, or 2 (DV <= 128; four waves a task)
    int dk, dv;                // the op's head dims (<= D, DV): columns past them are padding
    float scale, softcap;
};

// FLASH_ATTN_EXT with head dims past 256 (two GEMMs around a softmax pass): strides in
// elements as in FaArgs; scratch pointers carved from the caller's workspace.
struct FaWideArgs {
    const float * q;
    const uint16_t * k;
    const uint16_t * v;
    const uint16_t * mask;
    float * dst;
    int64_t q_nb1, q_nb2, k_nb1, k_nb2, v_nb1, v_nb2, mask_nb1, dst_nb1, dst_nb2;
    int dk, dv, T, H, HK, KV, kvp, rows_chunk;   // kvp: KV rounded up to 64
    float scale, softcap;
    uint16_t * q16;            // [HK][H/HK * T][dk] fp16 queries, rows (local head, token)
    float * qsc;               // their row scales
    uint16_t * kc;             // [kvp][dk] one KV head's keys, rows past KV zero
    uint16_t * vt;             // [dv][kvp] its values transposed, columns past KV zero
    float * s;                 // [rows_chunk][kvp] scores of a chunk of query rows
    uint16_t * p16;            // [rows_chunk][kvp] fp16 P
    float * psc;               // [rows_chunk] 1 / row sum of P
    float * o;                 // [rows_chunk][dv] normalised output rows
};

int fa_wide_rows_chunk(int T, int H, int HK, int kvp);    // query rows per chunk
hipError_t launch_fa_wide(const FaWideArgs & a, hipStream_t st);

// MUL_MAT_ID launch: strides in elements; scratch pointers carved from the caller's workspace.
struct MoeArgs {
    const void * w;            // expert panel, E*N rows of K, HBM layout
    int E, N, K;
    const float * b;           // [T][ne11][K], row stride b_nb1 (rows contiguous)
    int64_t b_nb1;
    int ne11, T, U;
    const int32_t * ids;       // ids[t][s] at t*ids_nb1 + s*ids_nb0
    int64_t ids_nb0, ids_nb1;
    float * dst;               // dst[t][s][:] at t*dst_nb2 + s*dst_nb1
    int64_t dst_nb1, dst_nb2;
    uint16_t * a16;            // [T*ne11][K] packed activations
    float * scales;            // [T*ne11]
    int32_t * off;             // [E+1] bucket offsets
    int32_t * rows;            // [T*U] bucketed row ids (t*U + s)
    int32_t * tiles;           // [2*max_tiles] (expert, first row)
    int32_t * n_tiles;         // [1]
    int32_t * err;             // [1] set when an id is out of range
    uint16_t * zero;           // [64] zeros (written by the bucketing pass), read for k past K
};

int moe_max_tiles(int T, int U, int E);
hipError_t launch_pack_q4kx(const void * src, int64_t rows, int64_t K, void * dst, hipStream_t st);   // rows % 32 == 0
hipError_t launch_pack_x32(int wt, const void * src, int64_t rows, int64_t K, void * dst, hipStream_t st);   // T_Q8_0X, T_Q6_KX, T_MXFP4X
hipError_t launch_moe(int wt, const MoeArgs & a, hipStream_t st);

// FaArgs::tasks: 4 for every build, 2 for DV <= 128
__host__ __device__ constexpr bool fa_tasks_ok(int DV, int tasks) { return tasks == 4 || (tasks == 2 && DV <= 128); }
int fa_blocks_per_split(const FaArgs & a);   // for a.tasks
int fa_prep_blocks(const FaArgs & a);
bool fa_dims_supported(int dk, int dv);   // fa_pad_dims: dk, dv <= 256, multiples of 8
size_t fa_max_kv(int dk, int dv);          // the longest KV range one launch takes
hipError_t launch_fa(const FaArgs & a, bool prep, hipStream_t st);

// zc (optional): an F32 output [M][ldzc] whose first zn columns the pack also clears
hipError_t launch_pack_act(const float * X, int64_t ldx, int M, int K, uint16_t * A16, int64_t lda,
                           float * scales, hipStream_t st, float * zc = nullptr, int64_t ldzc = 0, int zn = 0);
hipError_t launch_pack_act_tiled(const float * X, int64_t ldx, int M, int K, uint16_t * A16, float * scales,
                                 hipStream_t st, float * zc = nullptr, int64_t ldzc = 0, int zn = 0);
// c_zeroed: the outputs are already zero (the pack cleared them), so a launch that adds its K
// splits into them needs no fill of its own. part / part_bytes: workspace for the partial sums
// of a K split past two ways; a split that does not fit is narrowed, down to two ways (added
// into the zeroed output: with two addends on zero the order cannot change the sum). Every
// split is therefore reduced in a fixed order, and equal inputs give equal bits.
hipError_t launch_gemm(int wt, const GemmArgs & a, int n_tiles_total, hipStream_t st, bool c_zeroed = false,
                       float * part = nullptr, size_t part_bytes = 0);
// whether launch_gemm, with part_bytes of partial workspace, would add into its outputs (a
// two-way K split) rather than write them
bool gemm_accumulates(int wt, const GemmArgs & a, size_t part_bytes);
// partial workspace bytes of the launch's fastest K split (0 if it splits two ways or less)
size_t gemm_split_bytes(int wt, const GemmArgs & a);
bool q8_0_decode_first(int64_t M, int64_t N, int64_t K);   // mi355x_mul_mat's form for Q8_0
hipError_t launch_dequant_f16(int wt, const void * W, int64_t rows, int64_t K, uint16_t * out, hipStream_t st);
hipError_t launch_f16_tiled(int wt, const void * W, int64_t rows, int64_t K, uint16_t * out, hipStream_t st);
hipError_t launch_pack_weight(int wt, const void * src, int64_t rows, int64_t K, void * dst, hipStream_t st);
hipError_t launch_convert_f16(int type, const void * src, int64_t n, uint16_t * dst, hipStream_t st);

}  // namespace mx
