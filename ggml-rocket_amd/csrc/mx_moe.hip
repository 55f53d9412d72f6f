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
//      (expert, first row) tiles of MOE_BM rows; steps 1 and 2 share one launch (moe_prep) when
//      the rows fit a one-wave pack;
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

constexpr int MOE_BM = 64;            // rows per tile: an expert receives ~32 rows (20-45) at 512 tokens, top-8
                                      // of 128, so one tile each and every weight is decoded once
constexpr int MOE_BN = 128;           // output columns per block: 4 waves x 32
constexpr int MOE_BK = 64;
constexpr int MOE_THREADS = 256;
constexpr int MOE_A_BYTES = MOE_BM * MOE_BK * 2;   // 8 KiB
constexpr int MOE_STAGE = MOE_A_BYTES;   // the activation slab only: the weights go to registers
constexpr int MOE_SORT_THREADS = 1024;

// ---------------------------------------------------------------------------------------------
// bucketing
// ---------------------------------------------------------------------------------------------
// Exclusive prefix sums of (x, y) over the block's threads, in thread order; returns the totals.
__device__ __forceinline__ int2 block_scan2(int & x, int & y, int2 * wsum) {
    const int t = threadIdx.x, lane = t % WAVE, wave = t / WAVE;
    constexpr int NWAVES = MOE_SORT_THREADS / WAVE;
    int ix = x, iy = y;   // inclusive within the wave
#pragma unroll
    for (int o = 1; o < WAVE; o <<= 1) {
        const int px = __shfl_up(ix, o, WAVE), py = __shfl_up(iy, o, WAVE);
        if (lane >= o) { ix += px; iy += py; }
    }
    if (lane == WAVE - 1) wsum[wave] = make_int2(ix, iy);
    __syncthreads();
    int bx = 0, by = 0, tx = 0, ty = 0;
    for (int w = 0; w < NWAVES; w++) {
        const int2 v = wsum[w];
        if (w < wave) { bx += v.x; by += v.y; }
        tx += v.x;
        ty += v.y;
    }
    x = bx + ix - x;
    y = by + iy - y;
    return make_int2(tx, ty);
}

// One block: counts the (token, slot) rows of every expert, lays the experts' rows out
// contiguously (bucket offsets off[e]) and lists the tiles of MOE_BM rows as (expert, first row).
// Both prefix sums run across the block; rows are placed with LDS cursors. A thread keeps the
// first SORT_KEEP ids it reads in registers for the placement pass, so up to
// SORT_KEEP * MOE_SORT_THREADS rows are read from memory once.
constexpr int SORT_KEEP = 8;
__device__ __forceinline__ void moe_sort_block(const MoeArgs & a) {
    extern __shared__ __align__(16) int32_t sh[];
    int32_t * cnt = sh;              // [E] rows per expert, then the placement cursor
    __shared__ int32_t bad;
    __shared__ int2 wsum[MOE_SORT_THREADS / WAVE];
    const int t = threadIdx.x;
    const int R = a.T * a.U;
    if (t < 8) ((u32x4 *)a.zero)[t] = u32x4{0, 0, 0, 0};
    for (int e = t; e < a.E; e += MOE_SORT_THREADS) cnt[e] = 0;
    if (t == 0) bad = 0;
    __syncthreads();
    auto id_of = [&](int r) {
        const int tok = r / a.U, s = r % a.U;
        return a.ids[(int64_t)tok * a.ids_nb1 + (int64_t)s * a.ids_nb0];
    };
    int keep[SORT_KEEP];
#pragma unroll
    for (int i = 0; i < SORT_KEEP; i++) {
        const int r = t + i * MOE_SORT_THREADS;
        keep[i] = r < R ? id_of(r) : -1;
    }
    auto count = [&](int e) {
        if (e < 0 || e >= a.E) atomicOr(&bad, 1);
        else atomicAdd(&cnt[e], 1);
    };
#pragma unroll
    for (int i = 0; i < SORT_KEEP; i++)
        if (t + i * MOE_SORT_THREADS < R) count(keep[i]);
    for (int r = t + SORT_KEEP * MOE_SORT_THREADS; r < R; r += MOE_SORT_THREADS) count(id_of(r));
    __syncthreads();
    // thread t owns experts [t * per, (t + 1) * per)
    const int per = (a.E + MOE_SORT_THREADS - 1) / MOE_SORT_THREADS;
    const int e0 = min(t * per, a.E), e1 = min(e0 + per, a.E);
    int rows = 0, tiles = 0;
    for (int e = e0; e < e1; e++) {
        rows += cnt[e];
        tiles += (cnt[e] + MOE_BM - 1) / MOE_BM;
    }
    const int2 tot = block_scan2(rows, tiles, wsum);   // rows, tiles: this thread's first offsets
    for (int e = e0; e < e1; e++) {
        const int c = cnt[e];
        a.off[e] = rows;
        for (int m0 = 0; m0 < c; m0 += MOE_BM, tiles++) {
            a.tiles[2 * tiles] = e;
            a.tiles[2 * tiles + 1] = m0;
        }
        cnt[e] = rows;   // placement cursor
        rows += c;
    }
    if (t == 0) {
        a.off[a.E] = tot.x;
        a.n_tiles[0] = tot.y;
        a.err[0] = bad;
    }
    __syncthreads();
    auto place = [&](int r, int e) {
        if (e < 0 || e >= a.E) return;
        const int p = atomicAdd(&cnt[e], 1);
        a.rows[p] = r;
    };
#pragma unroll
    for (int i = 0; i < SORT_KEEP; i++) {
        const int r = t + i * MOE_SORT_THREADS;
        if (r < R) place(r, keep[i]);
    }
    for (int r = t + SORT_KEEP * MOE_SORT_THREADS; r < R; r += MOE_SORT_THREADS) place(r, id_of(r));
}

__global__ void __launch_bounds__(MOE_SORT_THREADS) moe_sort_kernel(MoeArgs a) { moe_sort_block(a); }

// The op's two passes before the GEMM in one launch, since neither needs the other: block 0
// buckets the rows, every other block packs MOE_SORT_THREADS / WAVE distinct activation rows,
// one wave a row (rows of at most PACK_WAVE_K values).
__global__ void __launch_bounds__(MOE_SORT_THREADS) moe_prep_kernel(MoeArgs a) {
    if (blockIdx.x == 0) {
        moe_sort_block(a);
        return;
    }
    const int m = (blockIdx.x - 1) * (MOE_SORT_THREADS / WAVE) + threadIdx.x / WAVE;
    if (m >= a.T * a.ne11) return;   // the whole wave
    pack_row_wave<false>(a.b + (int64_t)m * a.b_nb1, m, a.K, a.a16, a.K, a.scales, threadIdx.x % WAVE);
}

// ---------------------------------------------------------------------------------------------
// grouped expert GEMM
// ---------------------------------------------------------------------------------------------
// Block = (tile of MOE_BM rows of one expert, MOE_BN output columns); wave w owns columns
// w*32 .. w*32+31 of the block for all MOE_BM rows (2 MFMA tiles of 32x32, one where the tile has
// 32 rows or fewer). Lane l of wave w loads and decodes one 32-value half (l / 32) of weight row
// n0 + 32 w + l % 32 per 64-deep K slab straight into its MFMA B operand: the decoder yields the
// half as four runs of 8 consecutive k, and MFMA step i takes run i, so lane l's B slots of step
// i hold those 8 k and its A slots read the same 8 k of its activation row from LDS (the order in
// which K enters the MFMAs is free as long as both operands follow it; the two halves together
// are the slab's 64 k). The weights never pass through LDS; the tile's gathered activation rows
// do (every thread stages two 16-byte chunks), double-buffered, one barrier per slab. Loads run R
// K slabs ahead of the MFMAs, so an HBM round trip has R - 1 slabs of work to hide behind before
// its data is decoded. 128-column blocks: 768 of them (128 experts x 6 column blocks of a
// 768-wide gate/up) are one round of three blocks per CU over 256 CUs.
// Waves per SIMD and register stages of slab lookahead: Q4_K, Q8_0 and MXFP4 (each in both
// layouts) run four waves a SIMD with two stages (128 registers), measured 1-12% faster than
// three waves with four stages, most on the down projection's 2048 blocks (MXFP4 since its packed
// decoder fits); the other formats keep three waves with four stages, or three where the stage
// is wider (F16, Q5_K, Q6_K; Q6_K would spill at four waves, and three stages at four waves
// spill for every format).
template <int WT> constexpr int moe_waves() {
    return (WT == T_Q4_K || WT == T_Q4_KX || WT == T_Q8_0 || WT == T_Q8_0X || WT == T_MXFP4 || WT == T_MXFP4X) ? 4 : 3;
}
template <int WT> constexpr int moe_stages() {
    return moe_waves<WT>() == 4 ? 2 : (WT == T_F16 || WT == T_Q6_K || WT == T_Q6_KX || WT == T_Q5_K) ? 3 : 4;
}

template <int WT> constexpr bool moe_x32() { return WT == T_Q4_KX || WT == T_Q8_0X || WT == T_Q6_KX || WT == T_MXFP4X; }
// formats whose K may end half-way through a 64-deep slab (32-value blocks)
template <int WT> constexpr bool moe_k_tail() {
    return !(WT == T_Q4_K || WT == T_Q4_KX || WT == T_Q5_K || WT == T_Q6_K || WT == T_Q6_KX);
}

// A lane's weight loads: the row-strided formats keep the lane's panel row and half; the
// regrouped layouts keep WLoad's Lane (a block-uniform base and fixed lane offsets).
template <int WT, bool X = moe_x32<WT>()> struct MoeLane {
    int64_t row;
    int u;
    __device__ __forceinline__ void init(const MoeArgs & a, int e, int nloc, int u_) {
        row = (int64_t)e * a.N + nloc;
        u = u_;
    }
    __device__ __forceinline__ void load(WLoad<WT> & w, const MoeArgs & a, int64_t k0, bool ok) const {
        w.load((const uint8_t *)a.w, (int64_t)a.E * a.N, a.K, row, k0, u, ok);
    }
};
template <int WT> struct MoeLane<WT, true> {
    typename WLoad<WT>::Lane l;
    __device__ __forceinline__ void init(const MoeArgs & a, int e, int nloc, int u) {
        l = WLoad<WT>::lane((const uint8_t *)a.w, (int64_t)a.E * a.N, a.K, (int64_t)e * a.N, nloc, u);
    }
    __device__ __forceinline__ void load(WLoad<WT> & w, const MoeArgs & a, int64_t k0, bool ok) const {
        w.load(l, a.K, k0, ok);
    }
};

template <int WT>
__global__ void __launch_bounds__(MOE_THREADS) __attribute__((amdgpu_waves_per_eu(moe_waves<WT>(), moe_waves<WT>())))
moe_gemm_kernel(MoeArgs a) {
    constexpr int R = moe_stages<WT>();
    extern __shared__ __align__(16) uint8_t smem[];

    const int n_nt = (a.N + MOE_BN - 1) / MOE_BN;
    const int tile = blockIdx.x / n_nt, nt = blockIdx.x % n_nt;
    if (tile >= a.n_tiles[0]) return;   // uniform for the block
    const int e = a.tiles[2 * tile], m0 = a.tiles[2 * tile + 1];
    const int base = a.off[e];
    const int rows_here = min(MOE_BM, a.off[e + 1] - base - m0);
    const int32_t * trows = a.rows + base + m0;   // the tile's bucketed rows (t * U + s)

    const int t = threadIdx.x, lane = t % WAVE, wave = t / WAVE;
    // the packed activation row of tile row r (-1: pad row)
    auto act_row = [&](int r) -> int {
        if (r >= rows_here) return -1;
        const int rr = trows[r];
        const int tok = rr / a.U, s = rr % a.U;
        return tok * a.ne11 + (s % a.ne11);
    };
    // each tile row's output row offset in dst (-1: pad row) and activation scale, worked out
    // once per block (the epilogue would otherwise divide by U for each of a lane's 32 rows)
    __shared__ int64_t row_dst[MOE_BM];
    __shared__ float row_sc[MOE_BM];
    if (t < MOE_BM) {
        int64_t off = -1;
        float sc = 0.0f;
        if (t < rows_here) {
            const int rr = trows[t];
            const int tok = rr / a.U, s = rr % a.U;
            off = (int64_t)tok * a.dst_nb2 + (int64_t)s * a.dst_nb1;
            sc = a.scales[tok * a.ne11 + (s % a.ne11)];
        }
        row_dst[t] = off;
        row_sc[t] = sc;
    }

    const int K = a.K;
    const int n0 = nt * MOE_BN;
    const int lr = lane % 32, lg = lane / 32;
    const int wr = wave * 32 + lr, wu = lg;   // this lane's weight row (output column) in the block, and its half
    const bool wok = n0 + wr < a.N;
    MoeLane<WT> wl;
    wl.init(a, e, min(n0 + wr, a.N - 1), wu);   // clamped: loads are unconditional
    // A: thread t stages rows t / 8 and 32 + t / 8, chunk t % 8. A pad row reads packed row 0:
    // MFMA output row i depends on A row i alone, and pad rows' outputs are never stored.
    const int ar = t / 8, ac = t % 8;
    const uint16_t * ap0 = a.a16 + (int64_t)max(act_row(ar), 0) * K + 8 * ac;
    const uint16_t * ap1 = a.a16 + (int64_t)max(act_row(ar + 32), 0) * K + 8 * ac;

    float16v acc[2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int q = 0; q < 16; q++) acc[i][q] = 0.0f;

    struct Stage {
        u32x4 a0, a1;
        WLoad<WT> w;
    };
    // Past K (the last slab of a K that ends half-way through it) a chunk reads the zero block;
    // the weights there decode to zero as well. A branch around a load, or a select on its
    // value, would make the compiler wait for the newest loads at the join and cut the register
    // stages' lookahead to one, so the address is what is chosen.
    auto load_a = [&](const uint16_t * ap, int64_t k0) -> u32x4 {
        const uint16_t * p = ap + k0;
        if constexpr (moe_k_tail<WT>()) p = k0 + 8 * ac < K ? p : a.zero + 8 * ac;
        return *(const u32x4 *)p;
    };
    const int nk = (K + MOE_BK - 1) / MOE_BK;
    auto load = [&](Stage & g, int kt) {
        const int64_t k0 = (int64_t)min(kt, nk - 1) * MOE_BK;   // past the end: a repeat nobody uses
        g.a0 = load_a(ap0, k0);
        g.a1 = load_a(ap1, k0);
        wl.load(g.w, a, k0, wok);
    };
    // the lane's B operand of the next slab to multiply (four runs of 8 fp16 weights) and the
    // slab's 8-k chunk each run holds
    u32x4 bq[4];
    int kc[4];
    auto store = [&](uint8_t * st, const Stage & g) {
        *(u32x4 *)(st + swz<8>(ar, ac)) = g.a0;
        *(u32x4 *)(st + swz<8>(ar + 32, ac)) = g.a1;
        int r0, r1;
        g.w.decode_fast(wu, bq, r0, r1);
        kc[0] = r0 / 8;
        kc[1] = r0 / 8 + 1;
        kc[2] = r1 / 8;
        kc[3] = r1 / 8 + 1;
    };

    const bool two = rows_here > 32;   // block-uniform: the second 32-row MFMA tile has real rows
    auto mma = [&](const uint8_t * st) {
#pragma unroll
        for (int ks = 0; ks < MOE_BK / 16; ks++) {
            const half8 bf = __builtin_bit_cast(half8, bq[ks]);
            acc[0] = mfma32(*(const half8 *)(st + swz<8>(lr, kc[ks])), bf, acc[0]);
            if (two) acc[1] = mfma32(*(const half8 *)(st + swz<8>(32 + lr, kc[ks])), bf, acc[1]);
        }
    };

    // R register stages: step kk requests slab kk+R into the stage slab kk came from (already in
    // LDS), multiplies slab kk, then writes slab kk+1 into the other LDS buffer. The same loads
    // and stores every step, no branch around them; the ring index of every step is a constant
    // (loop unrolled by R, the remainder by a switch), so the stages stay in registers.
    Stage g[R];
#pragma unroll
    for (int q = 0; q < R; q++) load(g[q], q);
    store(smem, g[0]);
    __syncthreads();
    auto step = [&](int kk, Stage & mine, Stage & next) {
        load(mine, kk + R);
        mma(smem + (kk & 1) * MOE_STAGE);
        store(smem + ((kk + 1) & 1) * MOE_STAGE, next);
        __syncthreads();
    };
    int kk = 0;
    for (; kk + R <= nk; kk += R) {
#pragma unroll
        for (int q = 0; q < R; q++) step(kk + q, g[q], g[(q + 1) % R]);
    }
    switch (nk - kk) {   // 0 .. R-1 steps left, ring positions 0 .. R-2
        case 3:
            if constexpr (R > 3) {
                step(kk, g[0], g[1]);
                step(kk + 1, g[1], g[2]);
                step(kk + 2, g[2], g[3 % R]);
            }
            break;
        case 2:
            if constexpr (R > 2) {
                step(kk, g[0], g[1]);
                step(kk + 1, g[1], g[2 % R]);
            }
            break;
        case 1: step(kk, g[0], g[1]); break;
        default: break;
    }

    // scatter: tile row -> dst[t][s][:], scaled back by the row's activation scale (both from
    // the block's row table in LDS, written before the loop's first barrier)
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int q = 0; q < 16; q++) acc[i][q] *= row_sc[i * 32 + 8 * (q / 4) + 4 * lg + (q % 4)];
#pragma unroll
    for (int i = 0; i < 2; i++) asm volatile("" : "+v"(acc[i]));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int q = 0; q < 16; q++) {
            const int64_t off = row_dst[i * 32 + 8 * (q / 4) + 4 * lg + (q % 4)];
            if (off < 0) continue;
            float * d = a.dst + off;
            const int n = n0 + wave * 32 + lr;
            if (n < a.N) d[n] = acc[i][q];
        }
}

// ggml Q4_K blocks -> T_Q4_KX: one thread per 16-byte chunk of a source block (the header, then
// eight chunks of nibbles: quarter (c - 1) / 2, half (c - 1) % 2).
__global__ void __launch_bounds__(256) pack_q4kx_kernel(const uint8_t * __restrict__ src, int64_t rows, int64_t nblk,
                                                        uint8_t * __restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * nblk * 9) return;
    const int c = (int)(i % 9);
    const int64_t rb = i / 9, row = rb / nblk, blk = rb % nblk;
    const u32x4 v = *(const u32x4 *)(src + rb * 144 + 16 * c);
    uint8_t * b = dst + q4kx_block(row, blk, nblk);
    const int r = (int)(row % Q4KX_GROUP);
    uint8_t * d = c == 0 ? b + 16 * r : b + 16 * Q4KX_GROUP + 32 * Q4KX_GROUP * ((c - 1) / 2) + 32 * r + 16 * ((c - 1) % 2);
    *(u32x4 *)d = v;
}

hipError_t launch_pack_q4kx(const void * src, int64_t rows, int64_t K, void * dst, hipStream_t st) {
    const int64_t n = rows * (K / 256) * 9;
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(pack_q4kx_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, (const uint8_t *)src, rows,
                       K / 256, (uint8_t *)dst);
    return hipGetLastError();
}

// ggml Q8_0 (34-byte) or MXFP4 (17-byte) blocks -> T_Q8_0X / T_MXFP4X: one thread per source
// block; the blocks are only 2- or 1-byte aligned, so the quants move as bytes gathered into
// words (a one-time layout build of an expert stack, bound by HBM either way).
template <bool Q8>
__global__ void __launch_bounds__(256) pack_x32_kernel(const uint8_t * __restrict__ src, int64_t rows, int64_t nblk,
                                                       uint8_t * __restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * nblk) return;
    constexpr int BB = Q8 ? 34 : 17, QB = Q8 ? 32 : 16, Q0 = Q8 ? 2 : 1;
    const uint8_t * b = src + i * BB;
    const int64_t x = x32_index(i / nblk, i % nblk, nblk);
    uint32_t * q = (uint32_t *)(dst + x * QB);
#pragma unroll
    for (int w = 0; w < QB / 4; w++)
        q[w] = (uint32_t)b[Q0 + 4 * w] | ((uint32_t)b[Q0 + 4 * w + 1] << 8) | ((uint32_t)b[Q0 + 4 * w + 2] << 16) |
               ((uint32_t)b[Q0 + 4 * w + 3] << 24);
    uint8_t * scales = dst + rows * nblk * QB;
    if (Q8) {
        scales[2 * x] = b[0];
        scales[2 * x + 1] = b[1];
    } else {
        scales[x] = b[0];
    }
}

// ggml Q6_K blocks (210 bytes: ql[128] qh[64] scales[16] d) -> T_Q6_KX: one thread per source
// block, bytes gathered into words as above.
__global__ void __launch_bounds__(256) pack_q6kx_kernel(const uint8_t * __restrict__ src, int64_t rows, int64_t K,
                                                        uint8_t * __restrict__ dst) {
    const int64_t nblk = K / 256;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * nblk) return;
    const uint8_t * b = src + i * 210;
    const Q6kxPlanes p = q6kx_planes(rows, K, i / nblk, i % nblk);
    auto word = [&](int o) {
        return (uint32_t)b[o] | ((uint32_t)b[o + 1] << 8) | ((uint32_t)b[o + 2] << 16) | ((uint32_t)b[o + 3] << 24);
    };
    auto chunk = [&](int o, uint8_t * d) {
#pragma unroll
        for (int w = 0; w < 4; w++) ((uint32_t *)d)[w] = word(o + 4 * w);
    };
#pragma unroll
    for (int c = 0; c < 8; c++) chunk(16 * c, dst + p.ql + (c * 32 + p.r) * 16);
#pragma unroll
    for (int c = 0; c < 4; c++) chunk(128 + 16 * c, dst + p.qh + (c * 32 + p.r) * 16);
    chunk(192, dst + p.sc + p.r * 16);
    dst[p.d + 2 * p.r] = b[208];
    dst[p.d + 2 * p.r + 1] = b[209];
}

hipError_t launch_pack_x32(int wt, const void * src, int64_t rows, int64_t K, void * dst, hipStream_t st) {
    if (wt == T_Q6_KX) {
        const int64_t n = rows * (K / 256);
        if (n <= 0) return hipSuccess;
        hipLaunchKernelGGL(pack_q6kx_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, (const uint8_t *)src, rows, K,
                           (uint8_t *)dst);
        return hipGetLastError();
    }
    const int64_t n = rows * (K / 32);
    if (n <= 0) return hipSuccess;
    const dim3 grid((unsigned)((n + 255) / 256));
    if (wt == T_Q8_0X) hipLaunchKernelGGL(pack_x32_kernel<true>, grid, dim3(256), 0, st, (const uint8_t *)src, rows, K / 32, (uint8_t *)dst);
    else if (wt == T_MXFP4X) hipLaunchKernelGGL(pack_x32_kernel<false>, grid, dim3(256), 0, st, (const uint8_t *)src, rows, K / 32, (uint8_t *)dst);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

int moe_max_tiles(int T, int U, int E) { return (T * U + MOE_BM - 1) / MOE_BM + E; }

hipError_t launch_moe(int wt, const MoeArgs & a, hipStream_t st) {
    const int R = a.T * a.U;
    // 1. pack the distinct activation rows and 2. bucket the rows by expert: one launch when the
    // rows fit the one-wave pack, else the block-per-row pack, then the bucketing
    hipError_t e = hipSuccess;
    const int prows = a.T * a.ne11;
    constexpr int RPB = MOE_SORT_THREADS / WAVE;
    if (a.K <= PACK_WAVE_K) {
        hipLaunchKernelGGL(moe_prep_kernel, dim3(1 + (prows + RPB - 1) / RPB), dim3(MOE_SORT_THREADS),
                           (size_t)a.E * sizeof(int32_t), st, a);
    } else {
        e = launch_pack_act(a.b, a.b_nb1, prows, a.K, a.a16, a.K, a.scales, st);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(moe_sort_kernel, dim3(1), dim3(MOE_SORT_THREADS), (size_t)a.E * sizeof(int32_t), st, a);
    }
    e = hipGetLastError();
    if (e != hipSuccess || R == 0) return e;
    // 3. grouped GEMM over an upper bound of tiles
    const int n_nt = (a.N + MOE_BN - 1) / MOE_BN;
    const int64_t nb = (int64_t)moe_max_tiles(a.T, a.U, a.E) * n_nt;
    const size_t lds = 2 * MOE_STAGE;
    switch (wt) {
        case T_F16: hipLaunchKernelGGL(moe_gemm_kernel<T_F16>, dim3((unsigned)nb), dim3(MOE_THREADS), lds, st, a); break;
        case T_Q8_0: hipLaunchKernelGGL(moe_gemm_kernel<T_Q8_0>, dim3((unsigned)nb), dim3(MOE_THREADS), lds, st, a); break;
        case T_Q4_0: hipLaunchKernelGGL(moe_gemm_kernel<T_Q4_0>, dim3((unsigned)nb), dim3(MOE_THREADS), lds, st, a); break;
        case T_Q5_K: hipLaunchKernelGGL(moe_gemm_kernel<T_Q5_K>, dim3((unsigned)nb), dim3(MOE_THREADS), lds, st, a); break;
        case T_Q4_K: hipLaunchKernelGGL(moe_gemm_kernel<T_Q4_K>, dim3((unsigned)nb), dim3(MOE_THREADS), lds, st, a); break;
        case T_Q4_KX: hipLaunchKernelGGL(moe_gemm_kernel<T_Q4_KX>, dim3((unsigned)nb), dim3(MOE_THREADS), lds, st, a); break;
        case T_Q6_K: hipLaunchKernelGGL(moe_gemm_kernel<T_Q6_K>, dim3((unsigned)nb), dim3(MOE_THREADS), lds, st, a); break;
        case T_MXFP4: hipLaunchKernelGGL(moe_gemm_kernel<T_MXFP4>, dim3((unsigned)nb), dim3(MOE_THREADS), lds, st, a); break;
        case T_Q8_0X: hipLaunchKernelGGL(moe_gemm_kernel<T_Q8_0X>, dim3((unsigned)nb), dim3(MOE_THREADS), lds, st, a); break;
        case T_MXFP4X: hipLaunchKernelGGL(moe_gemm_kernel<T_MXFP4X>, dim3((unsigned)nb), dim3(MOE_THREADS), lds, st, a); break;
        case T_Q6_KX: hipLaunchKernelGGL(moe_gemm_kernel<T_Q6_KX>, dim3((unsigned)nb), dim3(MOE_THREADS), lds, st, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace mx
