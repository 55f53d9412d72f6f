// SPDX-License-Identifier: MIT
// FLASH_ATTN_EXT for head dims past the fused kernel's 256: the absorbed MLA of DeepSeek-style
// models (dk 576, dv 512) and any dk % 32 == 0, dv % 8 == 0 up to 1024, the claim range of
// ggml-rocket.cpp:7740-7760. Same semantics as the fused kernel (ggml-rocket.cpp:5444-5691):
//   O[t,h,:] = softmax_j( cap(scale * q[h,t].k[hk,j]) + mask[t,j] ) . v[hk,j,:],  hk = h / (H/HK)
// computed as two GEMMs around a softmax pass, per KV head and chunk of query rows:
//   Q16 = fp16(scale * q), row-scaled like the activation pack; its rows are ordered (local
//         head, token) within each KV head, so a KV head's query rows are one block of rows
//   S   = Q16 . K^T in F32                           (gemm_f16 kernels; K copied to [KVp][dk])
//   P16 = fp16(exp(cap(S) + mask - rowmax)), 1 / sum (one block per row; the sum is over the
//         rounded P, as the P.V product sees it)
//   O   = (P16 . V) / sum                            (gemm_f16 kernels; V^T copied to [dv][KVp])
//   dst[t][h][:] = O row                             (scatter)
// The scores stay in fp32, P is rounded to fp16 for the P.V product and both products accumulate
// in fp32, as in the fused kernel; a row whose every key is masked has sum 0 and is written as
// zeros. The query rows are taken a chunk at a time, so the F32 scores take a bounded slab of
// the workspace whatever T and n_kv are.

#include <algorithm>

#include "mx_common.h"
#include "mx_fa_dims.h"
#include "mx_kernels_impl.h"

namespace mx {

constexpr int FW_THREADS = 256;

__device__ __forceinline__ float fw_block_max(float v, float * red) {
    v = wave_max(v);
    const int wave = threadIdx.x / WAVE;
    __syncthreads();   // red is reused by consecutive reductions
    if (threadIdx.x % WAVE == 0) red[wave] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}
__device__ __forceinline__ float fw_block_sum(float v, float * red) {
    v = wave_sum(v);
    const int wave = threadIdx.x / WAVE;
    __syncthreads();
    if (threadIdx.x % WAVE == 0) red[wave] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// Q rows -> fp16, one block per row: block (r, hk) is row r = hl * T + t of KV head hk (query head
// hk * g + hl, token t). 4 values per thread (dk <= 1024, dk % 32 == 0).
__global__ void __launch_bounds__(FW_THREADS) fa_wide_pack_q(FaWideArgs w) {
    __shared__ float red[FW_THREADS / WAVE];
    const int r = blockIdx.x, hk = blockIdx.y;
    const int g = w.H / w.HK;
    const int hl = r / w.T, t = r % w.T, h = hk * g + hl;
    const float * q = w.q + (int64_t)h * w.q_nb2 + (int64_t)t * w.q_nb1;
    const int64_t row = (int64_t)hk * g * w.T + r;
    const int c = 4 * threadIdx.x;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float amax = 0.0f;
    if (c < w.dk) {
        const float4v x = *(const float4v *)(q + c);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            v[e] = mul_rn(x[e], w.scale);
            amax = fmaxf(amax, fabsf(v[e]));
        }
    }
    amax = fw_block_max(amax, red);
    const float s = amax > 0.0f ? amax : 1.0f;
    const float inv = 1.0f / s;
    if (c < w.dk) {
        u32x2 o;
        o[0] = pack2h(mul_rn(v[0], inv), mul_rn(v[1], inv));
        o[1] = pack2h(mul_rn(v[2], inv), mul_rn(v[3], inv));
        *(u32x2 *)(w.q16 + row * w.dk + c) = o;
    }
    if (threadIdx.x == 0) w.qsc[row] = s;
}

// KV head hk's keys as a [KVp][dk] fp16 matrix (rows past KV zero): one block per key row.
__global__ void __launch_bounds__(FW_THREADS) fa_wide_keys(FaWideArgs w, int hk) {
    const int j = blockIdx.x, c = 4 * threadIdx.x;
    if (c >= w.dk) return;
    u32x2 x = {0u, 0u};
    if (j < w.KV) x = *(const u32x2 *)(w.k + (int64_t)hk * w.k_nb2 + (int64_t)j * w.k_nb1 + c);
    *(u32x2 *)(w.kc + (int64_t)j * w.dk + c) = x;
}

// KV head hk's values transposed, [dv][KVp] fp16 (columns past KV zero), through 64 x 64 LDS
// tiles: block (key tile, dim tile); thread t loads 16 dims of key 64 bx + t / 4 and stores 16
// keys of dim 64 by + t / 4.
__global__ void __launch_bounds__(FW_THREADS) fa_wide_values(FaWideArgs w, int hk) {
    __shared__ uint16_t tile[64][64 + 2];
    const int j0 = 64 * blockIdx.x, d0 = 64 * blockIdx.y;
    const int rr = threadIdx.x / 4, cc = 16 * (threadIdx.x % 4);
    {
        const int j = j0 + rr;
        const uint16_t * src = w.v + (int64_t)hk * w.v_nb2 + (int64_t)j * w.v_nb1 + d0 + cc;
#pragma unroll
        for (int e = 0; e < 16; e++) tile[rr][cc + e] = (j < w.KV && d0 + cc + e < w.dv) ? src[e] : (uint16_t)0;
    }
    __syncthreads();
    const int d = d0 + rr;
    if (d >= w.dv) return;
    uint32_t o[8];
#pragma unroll
    for (int e = 0; e < 8; e++) o[e] = (uint32_t)tile[cc + 2 * e][rr] | ((uint32_t)tile[cc + 2 * e + 1][rr] << 16);
    uint16_t * dst = w.vt + (int64_t)d * w.kvp + j0 + cc;
    *(u32x4 *)dst = u32x4{o[0], o[1], o[2], o[3]};
    *(u32x4 *)(dst + 8) = u32x4{o[4], o[5], o[6], o[7]};
}

// One block per query row r of the chunk (row r0 + r of KV head hk): the capped, masked scores'
// max, then P = exp(x - max) rounded to fp16 and the row's 1 / sum of the rounded P (0 for a row
// with every key masked). The capped, masked scores are written back in place between the two
// passes so tanh runs once per score.
__global__ void __launch_bounds__(FW_THREADS) fa_wide_softmax(FaWideArgs w, int r0) {
    __shared__ float red[FW_THREADS / WAVE];
    const int r = blockIdx.x;
    const int t = (r0 + r) % w.T;
    float * srow = w.s + (int64_t)r * w.kvp;
    const uint16_t * mrow = w.mask ? w.mask + (int64_t)t * w.mask_nb1 : nullptr;
    const float inv_cap = w.softcap != 0.0f ? 1.0f / w.softcap : 0.0f;
    float m = -INFINITY;
    for (int j = threadIdx.x; j < w.kvp; j += FW_THREADS) {
        float x = -INFINITY;
        if (j < w.KV) {
            x = srow[j];
            if (w.softcap != 0.0f) x = w.softcap * tanhf(x * inv_cap);
            if (mrow) x += h2f_bits(mrow[j]);
        }
        srow[j] = x;
        m = fmaxf(m, x);
    }
    m = fw_block_max(m, red);
    const float LOG2E = 1.4426950408889634f;
    const float mb = m == -INFINITY ? 0.0f : m * LOG2E;
    uint16_t * prow = w.p16 + (int64_t)r * w.kvp;
    float sum = 0.0f;
    for (int j = threadIdx.x; j < w.kvp; j += FW_THREADS) {
        // v_exp_f32: exp2(-inf) = 0
        const uint16_t ph = f2h_bits(__builtin_amdgcn_exp2f(fmaf(srow[j], LOG2E, -mb)));
        prow[j] = ph;
        sum += h2f_bits(ph);
    }
    sum = fw_block_sum(sum, red);
    if (threadIdx.x == 0) w.psc[r] = sum > 0.0f ? 1.0f / sum : 0.0f;
}

// Output row r of the chunk -> dst[t][h][0 .. dv): one block per row, a float4 per thread.
__global__ void __launch_bounds__(FW_THREADS) fa_wide_scatter(FaWideArgs w, int hk, int r0) {
    const int r = blockIdx.x, c = 4 * threadIdx.x;
    if (c >= w.dv) return;
    const int g = w.H / w.HK;
    const int hl = (r0 + r) / w.T, t = (r0 + r) % w.T, h = hk * g + hl;
    *(float4v *)(w.dst + (int64_t)t * w.dst_nb2 + (int64_t)h * w.dst_nb1 + c) = *(const float4v *)(w.o + (int64_t)r * w.dv + c);
}

int fa_wide_rows_chunk(int T, int H, int HK, int kvp) {
    const int rows = (H / HK) * T;
    // the F32 scores of a chunk take at most 64 MiB
    int rc = (int)std::min<int64_t>((int64_t)rows, (64LL << 20) / ((int64_t)kvp * 4));
    rc = std::max(64, rc / 64 * 64);
    return std::min(rc, std::max(rows, 1));
}

hipError_t launch_fa_wide(const FaWideArgs & w, hipStream_t st) {
    const int g = w.H / w.HK;
    const int rows = g * w.T;
    if (rows == 0) return hipSuccess;
    hipLaunchKernelGGL(fa_wide_pack_q, dim3(rows, w.HK), dim3(FW_THREADS), 0, st, w);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    for (int hk = 0; hk < w.HK; hk++) {
        hipLaunchKernelGGL(fa_wide_keys, dim3(w.kvp), dim3(FW_THREADS), 0, st, w, hk);
        hipLaunchKernelGGL(fa_wide_values, dim3(w.kvp / 64, (w.dv + 63) / 64), dim3(FW_THREADS), 0, st, w, hk);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        for (int r0 = 0; r0 < rows; r0 += w.rows_chunk) {
            const int R = std::min(w.rows_chunk, rows - r0);
            const int64_t qrow = (int64_t)hk * rows + r0;
            GemmArgs s{};
            s.A = w.q16 + qrow * w.dk;
            s.scales = w.qsc + qrow;
            s.lda = w.dk;
            s.M = R;
            s.K = w.dk;
            s.ng = 1;
            s.g[0].W = w.kc;
            s.g[0].rows_total = w.kvp;
            s.g[0].row0 = 0;
            s.g[0].N = w.KV;
            s.g[0].C = w.s;
            s.g[0].ldc = w.kvp;
            if ((e = launch_gemm(T_F16, s, 0, st)) != hipSuccess) return e;
            hipLaunchKernelGGL(fa_wide_softmax, dim3(R), dim3(FW_THREADS), 0, st, w, r0);
            if ((e = hipGetLastError()) != hipSuccess) return e;
            GemmArgs o{};
            o.A = w.p16;
            o.scales = w.psc;
            o.lda = w.kvp;
            o.M = R;
            o.K = w.kvp;
            o.ng = 1;
            o.g[0].W = w.vt;
            o.g[0].rows_total = w.dv;
            o.g[0].row0 = 0;
            o.g[0].N = w.dv;
            o.g[0].C = w.o;
            o.g[0].ldc = w.dv;
            if ((e = launch_gemm(T_F16, o, 0, st)) != hipSuccess) return e;
            hipLaunchKernelGGL(fa_wide_scatter, dim3(R), dim3(FW_THREADS), 0, st, w, hk, r0);
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

}  // namespace mx
