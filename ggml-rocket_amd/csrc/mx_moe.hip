// SPDX-License-Identifier: MIT
// MUL_MAT_ID (mixture-of-experts expert GEMM) for gfx950: token-grouped, one launch per op.
//
// Semantics (ggml-rocket.cpp:6654-6662): for every token t and slot s,
//   dst[t][s][:] = as[ids[t][s]] . b[t][s % ne11][:]
// The reference buckets the (slot, token) rows by expert with a counting sort (6706-6732) and
// runs one GEMM per expert with rows (6783-6941). Here the whole op stays on the device:
//   1. pack_act converts each distinct activation row b[t][i] (T * ne11 of them) to fp16 with
//      its per-row scale, once, however many experts read it;
//   2. moe_sort buckets the rows by expert (counting sort in LDS) and writes a work list of
//      (expert, first row) tiles of MOE_BM rows;
//   3. moe_gemm runs every (tile, N block) pair in ONE launch: it gathers the tile's activation
//      rows by index, streams that expert's weight panel through the same fused-dequant LDS
//      staging as the dense GEMM, and scatters each output row to dst[t][s]. Blocks past the
//      work list's length exit at once, so the grid is sized from an upper bound and nothing
//      waits on the host.
// A row's result does not depend on which tile or position it lands in (every row's K
// accumulation order is the same), so the bucket order inside an expert is free.

#include "mx_weights.h"
#include "mx_kernels_impl.h"

namespace mx {

constexpr int MOE_BM = 32;            // rows per tile (an expert receives ~32 rows at 512 tokens, top-8 of 128)
constexpr int MOE_BN = 256;           // output columns per block: 4 waves x 64
constexpr int MOE_BK = 64;
constexpr int MOE_THREADS = 256;
constexpr int MOE_A_BYTES = MOE_BM * MOE_BK * 2;   // 4 KiB
constexpr int MOE_B_BYTES = MOE_BN * MOE_BK * 2;   // 32 KiB
constexpr int MOE_STAGE = MOE_A_BYTES + MOE_B_BYTES;
constexpr int MOE_SORT_THREADS = 1024;

// ---------------------------------------------------------------------------------------------
// bucketing
// ---------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(MOE_SORT_THREADS) moe_sort_kernel(MoeArgs a) {
    extern __shared__ __align__(16) int32_t sh[];
    int32_t * cnt = sh;              // [E]
    int32_t * cur = sh + a.E;        // [E]
    __shared__ int32_t bad;
    const int t = threadIdx.x;
    const int R = a.T * a.U;
    for (int e = t; e < a.E; e += MOE_SORT_THREADS) cnt[e] = 0;
    if (t == 0) bad = 0;
    __syncthreads();
    for (int r = t; r < R; r += MOE_SORT_THREADS) {
        const int tok = r / a.U, s = r % a.U;
        const int e = a.ids[(int64_t)tok * a.ids_nb1 + (int64_t)s * a.ids_nb0];
        if (e < 0 || e >= a.E) atomicOr(&bad, 1);
        else atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    if (t == 0) {
        int32_t o = 0, tl = 0;
        for (int e = 0; e < a.E; e++) {
            const int c = cnt[e];
            a.off[e] = o;
            cur[e] = o;
            for (int m0 = 0; m0 < c; m0 += MOE_BM) {
                a.tiles[2 * tl] = e;
                a.tiles[2 * tl + 1] = m0;
                tl++;
            }
            o += c;
        }
        a.off[a.E] = o;
        a.n_tiles[0] = tl;
        a.err[0] = bad;
    }
    __syncthreads();
    for (int r = t; r < R; r += MOE_SORT_THREADS) {
        const int tok = r / a.U, s = r % a.U;
        const int e = a.ids[(int64_t)tok * a.ids_nb1 + (int64_t)s * a.ids_nb0];
        if (e < 0 || e >= a.E) continue;
        const int p = atomicAdd(&cur[e], 1);
        a.rows[p] = r;
    }
}

// ---------------------------------------------------------------------------------------------
// grouped expert GEMM
// ---------------------------------------------------------------------------------------------
template <int WT>
__global__ void __launch_bounds__(MOE_THREADS) moe_gemm_kernel(MoeArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int32_t arow[MOE_BM];   // A16 row of each tile row (-1 = pad)
    __shared__ int32_t orow[MOE_BM];   // flattened (t * U + s) of each tile row

    const int n_nt = (a.N + MOE_BN - 1) / MOE_BN;
    const int tile = blockIdx.x / n_nt, nt = blockIdx.x % n_nt;
    if (tile >= a.n_tiles[0]) return;   // uniform for the block
    const int e = a.tiles[2 * tile], m0 = a.tiles[2 * tile + 1];
    const int base = a.off[e];
    const int cnt = a.off[e + 1] - base;
    const int rows_here = min(MOE_BM, cnt - m0);

    const int t = threadIdx.x, lane = t % WAVE, wave = t / WAVE;
    if (t < MOE_BM) {
        if (t < rows_here) {
            const int r = a.rows[base + m0 + t];
            const int tok = r / a.U, s = r % a.U;
            arow[t] = tok * a.ne11 + (s % a.ne11);
            orow[t] = r;
        } else {
            arow[t] = -1;
            orow[t] = -1;
        }
    }
    __syncthreads();

    const int K = a.K;
    const int n0 = nt * MOE_BN;
    const uint8_t * W = (const uint8_t *)a.w;
    const int64_t rows_total = (int64_t)a.E * a.N;
    // weight rows: thread t stages row n0 + t (both 32-value halves of each slab)
    const int64_t wrow = (int64_t)e * a.N + min(n0 + t, a.N - 1);   // clamped: loads are unconditional
    const bool wok = n0 + t < a.N;
    // A: thread t stages row t / 8, chunk t % 8
    const int ar = t / 8, ac = t % 8;
    const int arow_t = arow[ar];

    float16v acc[2];
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int i = 0; i < 16; i++) acc[j][i] = 0.0f;

    auto load_a = [&](int64_t k0) -> u32x4 {
        const int64_t k = k0 + 8 * ac;
        if (arow_t < 0 || k >= K) return u32x4{0, 0, 0, 0};
        return *(const u32x4 *)(a.a16 + (int64_t)arow_t * K + k);
    };
    auto store_stage = [&](uint8_t * st, const u32x4 & av, const WLoad<WT> & w0, const WLoad<WT> & w1) {
        *(u32x4 *)(st + swz<8>(ar, ac)) = av;
        uint8_t * bs = st + MOE_A_BYTES;
        u32x4 o[4];
        int r0, r1;
        w0.decode(0, o, r0, r1);
        *(u32x4 *)(bs + swz<8>(t, r0 / 8)) = o[0];
        *(u32x4 *)(bs + swz<8>(t, r0 / 8 + 1)) = o[1];
        *(u32x4 *)(bs + swz<8>(t, r1 / 8)) = o[2];
        *(u32x4 *)(bs + swz<8>(t, r1 / 8 + 1)) = o[3];
        w1.decode(1, o, r0, r1);
        *(u32x4 *)(bs + swz<8>(t, r0 / 8)) = o[0];
        *(u32x4 *)(bs + swz<8>(t, r0 / 8 + 1)) = o[1];
        *(u32x4 *)(bs + swz<8>(t, r1 / 8)) = o[2];
        *(u32x4 *)(bs + swz<8>(t, r1 / 8 + 1)) = o[3];
    };

    const int nk = (K + MOE_BK - 1) / MOE_BK;
    WLoad<WT> w0, w1;
    u32x4 av = load_a(0);
    w0.load(W, rows_total, K, wrow, 0, 0, wok);
    w1.load(W, rows_total, K, wrow, 0, 1, wok);
    store_stage(smem, av, w0, w1);
    __syncthreads();

    const int lr = lane % 32, lg = lane / 32;
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) {
            const int64_t k0 = (int64_t)(kt + 1) * MOE_BK;
            av = load_a(k0);
            w0.load(W, rows_total, K, wrow, k0, 0, wok);
            w1.load(W, rows_total, K, wrow, k0, 1, wok);
        }
        const uint8_t * As = smem + cur * MOE_STAGE;
        const uint8_t * Bs = As + MOE_A_BYTES;
#pragma unroll
        for (int ks = 0; ks < MOE_BK / 16; ks++) {
            const int c = 2 * ks + lg;
            const half8 af = *(const half8 *)(As + swz<8>(lr, c));
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const half8 bf = *(const half8 *)(Bs + swz<8>(wave * 64 + j * 32 + lr, c));
                acc[j] = mfma32(af, bf, acc[j]);
            }
        }
        if (more) store_stage(smem + (cur ^ 1) * MOE_STAGE, av, w0, w1);
        __syncthreads();
    }

    // scatter: tile row i -> dst[t][s][:], scaled back by the row's activation scale. Every
    // scale is loaded and applied before the first store: a load issued, or first used, after a
    // store waits for that store too (one in-order counter).
    float rs[16];
#pragma unroll
    for (int i = 0; i < 16; i++) rs[i] = a.scales[max(arow[8 * (i / 4) + 4 * lg + (i % 4)], 0)];
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int i = 0; i < 16; i++) acc[j][i] *= rs[i];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int rl = 8 * (i / 4) + 4 * lg + (i % 4);
        const int r = orow[rl];
        if (r < 0) continue;
        float * d = a.dst + (int64_t)(r / a.U) * a.dst_nb2 + (int64_t)(r % a.U) * a.dst_nb1;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int n = n0 + wave * 64 + j * 32 + lr;
            if (n < a.N) d[n] = acc[j][i];
        }
    }
}

int moe_max_tiles(int T, int U, int E) { return (T * U + MOE_BM - 1) / MOE_BM + E; }

hipError_t launch_moe(int wt, const MoeArgs & a, hipStream_t st) {
    const int R = a.T * a.U;
    // 1. pack the distinct activation rows
    hipError_t e = launch_pack_act(a.b, a.b_nb1, a.T * a.ne11, a.K, a.a16, a.K, a.scales, st);
    if (e != hipSuccess) return e;
    // 2. bucket
    hipLaunchKernelGGL(moe_sort_kernel, dim3(1), dim3(MOE_SORT_THREADS), (size_t)2 * a.E * sizeof(int32_t), st, a);
    e = hipGetLastError();
    if (e != hipSuccess || R == 0) return e;
    // 3. grouped GEMM over an upper bound of tiles
    const int n_nt = (a.N + MOE_BN - 1) / MOE_BN;
    const int64_t nb = (int64_t)moe_max_tiles(a.T, a.U, a.E) * n_nt;
    const size_t lds = 2 * MOE_STAGE;
    switch (wt) {
        case T_F16: hipLaunchKernelGGL(moe_gemm_kernel<T_F16>, dim3((unsigned)nb), dim3(MOE_THREADS), lds, st, a); break;
        case T_Q8_0: hipLaunchKernelGGL(moe_gemm_kernel<T_Q8_0>, dim3((unsigned)nb), dim3(MOE_THREADS), lds, st, a); break;
        case T_Q4_K: hipLaunchKernelGGL(moe_gemm_kernel<T_Q4_K>, dim3((unsigned)nb), dim3(MOE_THREADS), lds, st, a); break;
        case T_Q6_K: hipLaunchKernelGGL(moe_gemm_kernel<T_Q6_K>, dim3((unsigned)nb), dim3(MOE_THREADS), lds, st, a); break;
        case T_MXFP4: hipLaunchKernelGGL(moe_gemm_kernel<T_MXFP4>, dim3((unsigned)nb), dim3(MOE_THREADS), lds, st, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace mx
