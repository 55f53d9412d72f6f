// SPDX-License-Identifier: MIT
// The prefill GEMM family for gfx950.
//
//   pack_act      F32 activations [M][K] -> fp16 [M][K] divided by a per-row scale (the row's
//                 max |x|), plus the scales. This is the activation contract of the reference
//                 (rk_pack_act_row, ggml-rocket.cpp:1451-1475): C = s * ((A/s) . W).
//   gemm          C[M][N] (F32) = scale[m] * sum_k A16[m][k] * W[n][k], W in any of the HBM
//                 weight formats of mx_weights.h, decoded to fp16 while it is staged into LDS.
//                 fp16 MFMA (v_mfma_f32_32x32x16_f16) with fp32 accumulation, F32 written
//                 straight from the accumulators: no fp16 output surface.
//                 Up to four weights that share A run in one launch over their concatenated N
//                 (the fused QKV / gate-up groups of ggml-rocket.cpp:4956-5160).
//   dequant_f16   a weight panel -> fp16 [rows][K] (the resident-fp16 form, "prepacked-q").
//   pack_weight   a ggml Q8_0 / Q6_K payload -> its split HBM layout (mx_weights.h).
//
// Tiling: 256 threads (4 waves) per block, a 128x128 output tile, K staged 64 at a time through
// a double-buffered, XOR-swizzled LDS tile; each wave owns a 64x64 quadrant (2x2 MFMA blocks).

#include "mx_weights.h"
#include "mx_kernels_impl.h"

namespace mx {

// ---------------------------------------------------------------------------------------------
// activation pack: one wave per row
// ---------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) pack_act_kernel(const float * __restrict__ X, int64_t ldx,
                                                       int M, int K, uint16_t * __restrict__ A16,
                                                       int64_t lda, float * __restrict__ scales) {
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int m = blockIdx.x * 4 + wave;
    if (m >= M) return;
    const float * x = X + (int64_t)m * ldx;
    float amax = 0.0f;
    for (int k = lane * 4; k < K; k += WAVE * 4) {
        const float4v v = *(const float4v *)(x + k);
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
    }
    amax = wave_max(amax);
    const float s = amax > 0.0f ? amax : 1.0f;
    const float inv = 1.0f / s;
    uint16_t * a = A16 + (int64_t)m * lda;
    for (int k = lane * 4; k < K; k += WAVE * 4) {
        const float4v v = *(const float4v *)(x + k);
        u32x2 o;
        o[0] = pack2h(v[0] * inv, v[1] * inv);
        o[1] = pack2h(v[2] * inv, v[3] * inv);
        *(u32x2 *)(a + k) = o;
    }
    if (lane == 0) scales[m] = s;
}

// ---------------------------------------------------------------------------------------------
// GEMM
// ---------------------------------------------------------------------------------------------
constexpr int BM = 128, BN = 128, BK = 64;
constexpr int GEMM_THREADS = 256;
constexpr int TILE_BYTES = BM * BK * 2;   // 16 KiB, A and B tiles alike (BM == BN)

// A-tile load stage: thread t takes row t/2, values 32*(t%2) .. +31 of the 64-wide K slab.
struct ALoad {
    u32x4 v[4];
    __device__ __forceinline__ void load(const uint16_t * A, int64_t lda, int M, int K, int m0,
                                         int64_t k0, int t) {
        const int r = m0 + t / 2;
        const int64_t k = k0 + 32 * (t % 2);
        const bool ok = r < M && k < K;
        const u32x4 * p = (const u32x4 *)(A + (int64_t)r * lda + k);
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = ok ? p[i] : u32x4{0, 0, 0, 0};
    }
    __device__ __forceinline__ void store(uint8_t * lds, int t) const {
        const int r = t / 2, c0 = 4 * (t % 2);
#pragma unroll
        for (int i = 0; i < 4; i++) *(u32x4 *)(lds + swz<8>(r, c0 + i)) = v[i];
    }
};

template <int WT>
__device__ __forceinline__ void store_w(uint8_t * lds, int t, const WLoad<WT> & w) {
    u32x4 out[4];
    int run0, run1;
    w.decode(t % 2, out, run0, run1);
    const int r = t / 2;
    *(u32x4 *)(lds + swz<8>(r, run0 / 8)) = out[0];
    *(u32x4 *)(lds + swz<8>(r, run0 / 8 + 1)) = out[1];
    *(u32x4 *)(lds + swz<8>(r, run1 / 8)) = out[2];
    *(u32x4 *)(lds + swz<8>(r, run1 / 8 + 1)) = out[3];
}

// One K slab (64) of MFMA work for a wave's 64x64 quadrant.
__device__ __forceinline__ void mma_slab(const uint8_t * As, const uint8_t * Bs, int wm, int wn,
                                         int lane, float16v acc[2][2]) {
    const int lr = lane % 32, lg = lane / 32;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ks++) {
        const int c = 2 * ks + lg;
        half8 a[2], b[2];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            a[i] = *(const half8 *)(As + swz<8>(wm * 64 + i * 32 + lr, c));
            b[i] = *(const half8 *)(Bs + swz<8>(wn * 64 + i * 32 + lr, c));
        }
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) acc[i][j] = mfma32(a[i], b[j], acc[i][j]);
    }
}

template <int WT>
__global__ void __launch_bounds__(GEMM_THREADS) gemm_kernel(GemmArgs args) {
    extern __shared__ __align__(16) uint8_t smem[];
    // stage s: A tile at smem + s*TILE_BYTES, B tile at smem + (2+s)*TILE_BYTES

    const int t = threadIdx.x, lane = t % WAVE, wave = t / WAVE;
    const int wm = wave / 2, wn = wave % 2;

    // tile id -> (global n tile, m tile); m is the fast index so the blocks that share a
    // weight panel are neighbours (and, after xcd_tile, on one XCD).
    const int nblocks = gridDim.x;
    const int tile = xcd_tile(blockIdx.x, nblocks);
    const int mt = tile % args.m_tiles, nt = tile / args.m_tiles;
    int g = 0;
#pragma unroll
    for (int i = 1; i < GEMM_MAX_GROUPS; i++)
        if (i < args.ng && nt >= args.g[i].ntile_begin) g = i;
    const GemmGroup & G = args.g[g];
    const int n0 = (nt - G.ntile_begin) * BN;
    const int m0 = mt * BM;
    const int M = args.M, K = args.K;

    const uint8_t * W = (const uint8_t *)G.W;
    const int64_t wrow = G.row0 + n0 + t / 2;
    const bool wok = (n0 + t / 2) < G.N;

    float16v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

    const int nk = (K + BK - 1) / BK;
    ALoad al;
    WLoad<WT> wl;
    al.load(args.A, args.lda, M, K, m0, 0, t);
    wl.load(W, G.rows_total, K, wrow, 0, t % 2, wok);
    al.store(smem, t);
    store_w<WT>(smem + 2 * TILE_BYTES, t, wl);
    __syncthreads();

    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) {
            const int64_t k0 = (int64_t)(kt + 1) * BK;
            al.load(args.A, args.lda, M, K, m0, k0, t);
            wl.load(W, G.rows_total, K, wrow, k0, t % 2, wok);
        }
        mma_slab(smem + cur * TILE_BYTES, smem + (2 + cur) * TILE_BYTES, wm, wn, lane, acc);
        if (more) {
            al.store(smem + (cur ^ 1) * TILE_BYTES, t);
            store_w<WT>(smem + (2 + (cur ^ 1)) * TILE_BYTES, t, wl);
        }
        __syncthreads();
    }

    // epilogue: C = scale[m] * acc
    const int lr = lane % 32, lg = lane / 32;
#pragma unroll
    for (int i = 0; i < 2; i++) {
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int r = m0 + wm * 64 + i * 32 + 8 * (e / 4) + 4 * lg + (e % 4);
            if (r >= M) continue;
            const float s = args.scales[r];
            float * crow = G.C + (int64_t)r * G.ldc;
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int n = n0 + wn * 64 + j * 32 + lr;
                if (n < G.N) crow[n] = acc[i][j][e] * s;
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------
// dequant to fp16 and the weight re-layout
// ---------------------------------------------------------------------------------------------

// One thread per (row, 32-value half of a 64-wide slab): the same decoders the GEMM uses.
template <int WT>
__global__ void __launch_bounds__(256) dequant_f16_kernel(const uint8_t * __restrict__ W, int64_t rows,
                                                          int64_t K, uint16_t * __restrict__ out) {
    const int64_t per_row = K / 32;   // thread items per row
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * per_row) return;
    const int64_t row = i / per_row, item = i % per_row;
    const int64_t k0 = (item / 2) * 64;
    const int u = (int)(item % 2);
    WLoad<WT> wl;
    wl.load(W, rows, K, row, k0, u, true);
    u32x4 o[4];
    int run0, run1;
    wl.decode(u, o, run0, run1);
    uint16_t * d = out + row * K + k0;
    *(u32x4 *)(d + run0) = o[0];
    *(u32x4 *)(d + run0 + 8) = o[1];
    *(u32x4 *)(d + run1) = o[2];
    *(u32x4 *)(d + run1 + 8) = o[3];
}

// ggml Q8_0 -> split planes. One thread per block.
__global__ void pack_q8_0_kernel(const uint8_t * __restrict__ src, int64_t rows, int64_t K,
                                 uint8_t * __restrict__ dst) {
    const int64_t nb = K / 32;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * nb) return;
    const int64_t row = i / nb, b = i % nb;
    const uint8_t * s = src + i * 34;
    uint8_t * qs = dst + row * K + b * 32;
    for (int l = 0; l < 32; l++) qs[l] = s[2 + l];
    uint8_t * d = dst + rows * K + (row * nb + b) * 2;
    d[0] = s[0];
    d[1] = s[1];
}

// ggml Q6_K -> split planes. One thread per block.
__global__ void pack_q6_k_kernel(const uint8_t * __restrict__ src, int64_t rows, int64_t K,
                                 uint8_t * __restrict__ dst) {
    const int64_t nb = K / 256;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * nb) return;
    const int64_t row = i / nb, b = i % nb;
    const uint8_t * s = src + i * 210;
    uint8_t * ql = dst + row * (K / 2) + b * 128;
    uint8_t * qh = dst + rows * (K / 2) + row * (K / 4) + b * 64;
    uint8_t * sc = dst + rows * (K / 2) + rows * (K / 4) + row * (K / 16) + b * 16;
    uint8_t * d = dst + rows * (K / 2) + rows * (K / 4) + rows * (K / 16) + (row * nb + b) * 2;
    for (int l = 0; l < 128; l++) ql[l] = s[l];
    for (int l = 0; l < 64; l++) qh[l] = s[128 + l];
    for (int l = 0; l < 16; l++) sc[l] = s[192 + l];
    d[0] = s[208];
    d[1] = s[209];
}

// ---------------------------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------------------------

hipError_t launch_pack_act(const float * X, int64_t ldx, int M, int K, uint16_t * A16, int64_t lda,
                           float * scales, hipStream_t st) {
    if (M <= 0) return hipSuccess;
    hipLaunchKernelGGL(pack_act_kernel, dim3((M + 3) / 4), dim3(256), 0, st, X, ldx, M, K, A16, lda, scales);
    return hipGetLastError();
}

hipError_t launch_gemm(int wt, const GemmArgs & a, int n_tiles_total, hipStream_t st) {
    const int nblocks = n_tiles_total * a.m_tiles;
    if (nblocks <= 0) return hipSuccess;
    const size_t lds = 4 * TILE_BYTES;
    switch (wt) {
        case T_F16: hipLaunchKernelGGL(gemm_kernel<T_F16>, dim3(nblocks), dim3(GEMM_THREADS), lds, st, a); break;
        case T_Q8_0: hipLaunchKernelGGL(gemm_kernel<T_Q8_0>, dim3(nblocks), dim3(GEMM_THREADS), lds, st, a); break;
        case T_Q4_K: hipLaunchKernelGGL(gemm_kernel<T_Q4_K>, dim3(nblocks), dim3(GEMM_THREADS), lds, st, a); break;
        case T_Q6_K: hipLaunchKernelGGL(gemm_kernel<T_Q6_K>, dim3(nblocks), dim3(GEMM_THREADS), lds, st, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_dequant_f16(int wt, const void * W, int64_t rows, int64_t K, uint16_t * out, hipStream_t st) {
    const int64_t items = rows * (K / 32);
    if (items <= 0) return hipSuccess;
    const dim3 grid((unsigned)((items + 255) / 256));
    const uint8_t * w = (const uint8_t *)W;
    switch (wt) {
        case T_F16: hipLaunchKernelGGL(dequant_f16_kernel<T_F16>, grid, dim3(256), 0, st, w, rows, K, out); break;
        case T_Q8_0: hipLaunchKernelGGL(dequant_f16_kernel<T_Q8_0>, grid, dim3(256), 0, st, w, rows, K, out); break;
        case T_Q4_K: hipLaunchKernelGGL(dequant_f16_kernel<T_Q4_K>, grid, dim3(256), 0, st, w, rows, K, out); break;
        case T_Q6_K: hipLaunchKernelGGL(dequant_f16_kernel<T_Q6_K>, grid, dim3(256), 0, st, w, rows, K, out); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_pack_weight(int wt, const void * src, int64_t rows, int64_t K, void * dst, hipStream_t st) {
    const uint8_t * s = (const uint8_t *)src;
    uint8_t * d = (uint8_t *)dst;
    switch (wt) {
        case T_F16:
        case T_Q4_K: {
            const int64_t bytes = packed_weight_bytes(wt, rows, K);
            if (s != d) return hipMemcpyAsync(d, s, (size_t)bytes, hipMemcpyDeviceToDevice, st);
            return hipSuccess;
        }
        case T_Q8_0: {
            const int64_t n = rows * (K / 32);
            if (n <= 0) return hipSuccess;
            hipLaunchKernelGGL(pack_q8_0_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, s, rows, K, d);
            return hipGetLastError();
        }
        case T_Q6_K: {
            const int64_t n = rows * (K / 256);
            if (n <= 0) return hipSuccess;
            hipLaunchKernelGGL(pack_q6_k_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, s, rows, K, d);
            return hipGetLastError();
        }
        default: return hipErrorInvalidValue;
    }
}

}  // namespace mx
