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
//   pack_weight   a ggml Q8_0 / Q6_K / MXFP4 payload -> its split HBM layout (mx_weights.h).
//
// Three GEMM kernels: a register-staged one that decodes any weight format into LDS
// (gemm_kernel), for fp16 weights one that moves both operands into LDS by DMA (gemm_f16_kernel,
// and its two-width variant gemm_f16_cols_kernel), and for M <= 128 one that decodes the weight
// straight into MFMA operands (gemm_skinny_kernel). The launcher picks a kernel and tile
// configuration per call from the output shape.

#include <algorithm>
#include <cmath>

#include "mx_weights.h"
#include "mx_kernels_impl.h"

namespace mx {

// ---------------------------------------------------------------------------------------------
// activation pack: one 256-thread block per row. A row of up to PACK_REG_MAX floats is read
// once into registers (all loads in flight together), reduced, scaled and written; longer rows
// take a second pass over memory.
// ---------------------------------------------------------------------------------------------
constexpr int PACK_THREADS = 256;
constexpr int PACK_VEC = 16;                                 // float4 per thread held in registers
constexpr int PACK_REG_MAX = PACK_THREADS * PACK_VEC * 4;    // 16384 floats

// TL: write A16 in the tiled layout (tiled_index over M rows) instead of rows of lda.
// ZC (optional): an F32 output whose row m (ZN values) the block also clears, for a GEMM that
// adds its K splits into it; one launch fewer than a separate fill.
template <bool TL>
__global__ void __launch_bounds__(PACK_THREADS) pack_act_kernel(const float * __restrict__ X, int64_t ldx,
                                                                int M, int K, uint16_t * __restrict__ A16,
                                                                int64_t lda, float * __restrict__ scales,
                                                                float * __restrict__ ZC, int64_t ldzc, int ZN) {
    __shared__ float red[PACK_THREADS / WAVE];
    const int t = threadIdx.x, lane = t % WAVE, wave = t / WAVE;
    const int m = blockIdx.x;
    if (ZC) {
        float * zrow = ZC + (int64_t)m * ldzc;
        int c0 = 0;
        if ((reinterpret_cast<uintptr_t>(zrow) & 15) == 0) {
            for (int c = 4 * t; c + 3 < ZN; c += 4 * PACK_THREADS) *(float4v *)(zrow + c) = float4v{0, 0, 0, 0};
            c0 = ZN & ~3;
        }
        for (int c = c0 + t; c < ZN; c += PACK_THREADS) zrow[c] = 0.0f;
    }
    const int n4 = K / 4;
    // the destination of the 4 values starting at column 4c
    auto dst = [&](int c) -> uint16_t * {
        return TL ? A16 + tiled_index(m, 4 * c, K) : A16 + (int64_t)m * lda + 4 * c;
    };
    const float * x = X + (int64_t)m * ldx;
    float4v v[PACK_VEC];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < PACK_VEC; i++) {
        const int c = t + i * PACK_THREADS;
        v[i] = c < n4 ? *(const float4v *)(x + 4 * c) : float4v{0, 0, 0, 0};
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[i][0]), fabsf(v[i][1])), fmaxf(fabsf(v[i][2]), fabsf(v[i][3]))));
    }
    for (int c = t + PACK_VEC * PACK_THREADS; c < n4; c += PACK_THREADS) {
        const float4v w = *(const float4v *)(x + 4 * c);
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(w[0]), fabsf(w[1])), fmaxf(fabsf(w[2]), fabsf(w[3]))));
    }
    amax = wave_max(amax);
    if (lane == 0) red[wave] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float s = amax > 0.0f ? amax : 1.0f;
    const float inv = 1.0f / s;
    // x * inv is rounded to f32 and then to fp16, as the CPU pack does: mul_rn keeps the compiler
    // from folding the product into the conversion (v_fma_mix rounds once)
#pragma unroll
    for (int i = 0; i < PACK_VEC; i++) {
        const int c = t + i * PACK_THREADS;
        if (c < n4) {
            u32x2 o;
            o[0] = pack2h(mul_rn(v[i][0], inv), mul_rn(v[i][1], inv));
            o[1] = pack2h(mul_rn(v[i][2], inv), mul_rn(v[i][3], inv));
            *(u32x2 *)dst(c) = o;
        }
    }
    for (int c = t + PACK_VEC * PACK_THREADS; c < n4; c += PACK_THREADS) {
        const float4v w = *(const float4v *)(x + 4 * c);
        u32x2 o;
        o[0] = pack2h(mul_rn(w[0], inv), mul_rn(w[1], inv));
        o[1] = pack2h(mul_rn(w[2], inv), mul_rn(w[3], inv));
        *(u32x2 *)dst(c) = o;
    }
    if (t == 0) scales[m] = s;
}

// Rows of up to PACK_WAVE_K values: one wave a row (pack_row_wave), four rows a block; for
// short rows (an expert's 768- or 2048-wide activations, thousands of them) the block form's
// barrier and its idle threads dominate.
template <bool TL>
__global__ void __launch_bounds__(PACK_THREADS) pack_act_wave_kernel(const float * __restrict__ X, int64_t ldx,
                                                                     int M, int K, uint16_t * __restrict__ A16,
                                                                     int64_t lda, float * __restrict__ scales,
                                                                     float * __restrict__ ZC, int64_t ldzc, int ZN) {
    const int lane = threadIdx.x % WAVE;
    const int m = blockIdx.x * (PACK_THREADS / WAVE) + threadIdx.x / WAVE;
    if (m >= M) return;   // the whole wave
    if (ZC) {
        float * zrow = ZC + (int64_t)m * ldzc;
        int c0 = 0;
        if ((reinterpret_cast<uintptr_t>(zrow) & 15) == 0) {
            for (int c = 4 * lane; c + 3 < ZN; c += 4 * WAVE) *(float4v *)(zrow + c) = float4v{0, 0, 0, 0};
            c0 = ZN & ~3;
        }
        for (int c = c0 + lane; c < ZN; c += WAVE) zrow[c] = 0.0f;
    }
    pack_row_wave<TL>(X + (int64_t)m * ldx, m, K, A16, lda, scales, lane);
}

// The widest row the wave form packs: 2048 values (measured: 8.5% faster for the 4096 rows of 768
// of an expert down projection, within 3% either way for 512 rows of 4096; MI355X_PACK_WAVE_K
// overrides, for tests and tuning, up to 4096; 0 keeps every row on the block form).
static int pack_wave_k() {
    const char * e = getenv("MI355X_PACK_WAVE_K");
    return (e && *e) ? std::min(atoi(e), PACK_WAVE_K) : 2048;
}

// ---------------------------------------------------------------------------------------------
// GEMM
//
// Block = 256 threads (4 waves in a WM x WN grid), output tile BM x BN, K staged BK = 64 at a
// time through a double-buffered, XOR-swizzled LDS tile. Global loads run R slabs ahead in a ring
// of register sets (the loop is unrolled by R so the sets are static registers): slab k+R is
// requested while slab k is multiplied, and slab k+1 is written to LDS only after that, which
// hides HBM latency behind R-1 slabs of MFMA work.
// KSPLIT > 1 splits K between that many blocks that add their parts atomically into a zeroed
// output; KSPLIT = 0 takes the split count from the launcher (args.ksplit), which sizes it to fill
// the chip when the output has few tiles (a skinny M: 32 rows of a 3072-wide output are 24
// tiles). Two addends sum the same in either order; with more, the rounding of the sum depends
// on the order the blocks finish in.
// ---------------------------------------------------------------------------------------------
constexpr int BK = 64;
constexpr int GEMM_THREADS = 256;

template <int BM, int BN, int WM, int WN, int R>
struct GemmCfg {
    static constexpr int TM = BM / WM, TN = BN / WN;        // wave tile
    static constexpr int MI = TM / 32, NJ = TN / 32;        // MFMA blocks per wave
    static constexpr int A_CHUNKS = BM * (BK / 8) / GEMM_THREADS;   // 16-byte chunks per thread
    static constexpr int B_ITEMS = BN * 2 / GEMM_THREADS;           // (row, half) items per thread
    static constexpr int A_BYTES = BM * BK * 2, B_BYTES = BN * BK * 2;
    static constexpr int STAGE = A_BYTES + B_BYTES;
    static constexpr int LDS = 2 * STAGE;
    static_assert(WM * WN == 4, "4 waves");
    static_assert(A_CHUNKS >= 1 && B_ITEMS >= 1, "tile too small");
};

// One pipeline stage in registers: raw loads plus whether each item is real; the masking is
// applied when the stage is written to LDS, so the loads stay in flight until then.
template <int WT, int NA, int NB>
struct Slab {
    u32x4 a[NA];
    bool a_ok[NA];
    WLoad<WT> b[NB];
};

template <int WT, class C>
__device__ __forceinline__ void slab_load(Slab<WT, C::A_CHUNKS, C::B_ITEMS> & s, const GemmArgs & args,
                                          const GemmGroup & G, int m0, int n0, int64_t k0, int t) {
    const int M = args.M, K = args.K;
#pragma unroll
    for (int i = 0; i < C::A_CHUNKS; i++) {
        const int c = t + i * GEMM_THREADS;
        const int r = m0 + c / 8;
        const int64_t k = k0 + 8 * (c % 8);
        s.a_ok[i] = r < M && k < K;
        s.a[i] = *(const u32x4 *)(args.A + (int64_t)(r < M ? r : M - 1) * args.lda + (k < K ? k : 0));
    }
    const uint8_t * W = (const uint8_t *)G.W;
#pragma unroll
    for (int i = 0; i < C::B_ITEMS; i++) {
        const int it = t + i * GEMM_THREADS;
        const int n = n0 + it / 2;
        const bool ok = n < G.N;
        s.b[i].load(W, G.rows_total, K, G.row0 + (ok ? n : G.N - 1), k0, it % 2, ok);
    }
}

template <int WT, class C>
__device__ __forceinline__ void slab_store(const Slab<WT, C::A_CHUNKS, C::B_ITEMS> & s, uint8_t * st, int t) {
#pragma unroll
    for (int i = 0; i < C::A_CHUNKS; i++) {
        const int c = t + i * GEMM_THREADS;
        *(u32x4 *)(st + swz<8>(c / 8, c % 8)) = s.a_ok[i] ? s.a[i] : u32x4{0, 0, 0, 0};
    }
    uint8_t * bs = st + C::A_BYTES;
#pragma unroll
    for (int i = 0; i < C::B_ITEMS; i++) {
        const int it = t + i * GEMM_THREADS;
        const int r = it / 2;
        u32x4 out[4];
        int run0, run1;
        s.b[i].decode(it % 2, out, run0, run1);
        *(u32x4 *)(bs + swz<8>(r, run0 / 8)) = out[0];
        *(u32x4 *)(bs + swz<8>(r, run0 / 8 + 1)) = out[1];
        *(u32x4 *)(bs + swz<8>(r, run1 / 8)) = out[2];
        *(u32x4 *)(bs + swz<8>(r, run1 / 8 + 1)) = out[3];
    }
}

template <class C>
__device__ __forceinline__ void mma_slab(const uint8_t * st, int wm, int wn, int lane,
                                         float16v (&acc)[C::MI][C::NJ]) {
    const uint8_t * As = st;
    const uint8_t * Bs = st + C::A_BYTES;
    const int lr = lane % 32, lg = lane / 32;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ks++) {
        const int c = 2 * ks + lg;
        half8 a[C::MI], b[C::NJ];
#pragma unroll
        for (int i = 0; i < C::MI; i++) a[i] = *(const half8 *)(As + swz<8>(wm * C::TM + i * 32 + lr, c));
#pragma unroll
        for (int j = 0; j < C::NJ; j++) b[j] = *(const half8 *)(Bs + swz<8>(wn * C::TN + j * 32 + lr, c));
#pragma unroll
        for (int i = 0; i < C::MI; i++)
#pragma unroll
            for (int j = 0; j < C::NJ; j++) acc[i][j] = mfma32(a[i], b[j], acc[i][j]);
    }
}

// Where a K-split block writes: with partials (a split past two ways) its split's slab of them,
// row stride ldp, group g's columns from pcol; otherwise the group's own output, which it adds
// into when the split is two ways.
__device__ __forceinline__ void split_target(const GemmArgs & a, int g, int split, float *& Cp, int64_t & ldc) {
    if (!a.part) return;
    int64_t pcol = a.g[0].pcol;
#pragma unroll
    for (int i = 1; i < GEMM_MAX_GROUPS; i++)
        if (i == g) pcol = a.g[i].pcol;
    Cp = a.part + (int64_t)split * a.M * a.ldp + pcol;
    ldc = a.ldp;
}

template <int WT, int BM, int BN, int WM, int WN, int R, int KSPLIT>
__global__ void __launch_bounds__(GEMM_THREADS)
__attribute__((amdgpu_waves_per_eu((BM == 128 && BN == 128) ? 2 : 1, (BM == 128 && BN == 128) ? 2 : 1)))
gemm_kernel(GemmArgs args) {
    // waves_per_eu pins the register budget to the occupancy the LDS allows anyway (2 blocks of
    // a 128x128 tile per CU, 1 of the larger tiles), so the scheduler does not sink the prefetch
    // loads next to their use to save registers.
    using C = GemmCfg<BM, BN, WM, WN, R>;
    extern __shared__ __align__(16) uint8_t smem[];

    const int t = threadIdx.x, lane = t % WAVE, wave = t / WAVE;
    const int wm = wave / WN, wn = wave % WN;

    // block -> (k split, global n tile, m tile); m is the fast index so the blocks that share a
    // weight panel are neighbours (and, after xcd_tile, on one XCD)
    const int nblocks = gridDim.x;
    const int ks = KSPLIT > 0 ? KSPLIT : args.ksplit;   // 0: the launcher's split count
    int tile = xcd_tile(blockIdx.x, nblocks);
    const int split = tile % ks;
    tile /= ks;
    const int mt = tile % args.m_tiles, nt = tile / args.m_tiles;
    int g = 0;
#pragma unroll
    for (int i = 1; i < GEMM_MAX_GROUPS; i++)
        if (i < args.ng && nt >= args.g[i].ntile_begin) g = i;
    GemmGroup G;
    G.W = args.g[0].W; G.rows_total = args.g[0].rows_total; G.row0 = args.g[0].row0; G.N = args.g[0].N;
    G.C = args.g[0].C; G.ldc = args.g[0].ldc; G.ntile_begin = args.g[0].ntile_begin;
#pragma unroll
    for (int i = 1; i < GEMM_MAX_GROUPS; i++)
        if (i == g) {
            G.W = args.g[i].W; G.rows_total = args.g[i].rows_total; G.row0 = args.g[i].row0; G.N = args.g[i].N;
            G.C = args.g[i].C; G.ldc = args.g[i].ldc; G.ntile_begin = args.g[i].ntile_begin;
        }
    split_target(args, g, split, G.C, G.ldc);
    const int n0 = (nt - G.ntile_begin) * BN;
    const int m0 = mt * BM;

    const int nk_all = (args.K + BK - 1) / BK;
    const int per = (nk_all + ks - 1) / ks;
    const int kb = split * per;
    const int nk = max(0, min(nk_all, kb + per) - kb);

    float16v acc[C::MI][C::NJ];
#pragma unroll
    for (int i = 0; i < C::MI; i++)
#pragma unroll
        for (int j = 0; j < C::NJ; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

    // Two register stages. Step kk: request slab kk+2 into ring[kk&1] (its previous contents,
    // slab kk, are already in LDS), multiply slab kk from LDS, then write slab kk+1 (requested a
    // step earlier) into the other LDS buffer. Slab indices past the end are clamped to the last
    // slab, so every step issues the same loads and stores with no branch around them (a load
    // behind a branch makes the compiler wait for every outstanding load); the extra slab written
    // on the last step lands in the buffer nobody reads again.
    static_assert(R == 2, "two register stages");
    Slab<WT, C::A_CHUNKS, C::B_ITEMS> ring[2];
    const int last = kb + (nk > 0 ? nk - 1 : 0);
    auto slab_k0 = [&](int kk) -> int64_t { return (int64_t)min(kb + kk, last) * BK; };
    auto step = [&](int kk, Slab<WT, C::A_CHUNKS, C::B_ITEMS> & mine, Slab<WT, C::A_CHUNKS, C::B_ITEMS> & next) {
        slab_load<WT, C>(mine, args, G, m0, n0, slab_k0(kk + 2), t);
        mma_slab<C>(smem + (kk & 1) * C::STAGE, wm, wn, lane, acc);
        slab_store<WT, C>(next, smem + ((kk + 1) & 1) * C::STAGE, t);
        __syncthreads();
    };
    if (nk > 0) {
        slab_load<WT, C>(ring[0], args, G, m0, n0, slab_k0(0), t);
        slab_load<WT, C>(ring[1], args, G, m0, n0, slab_k0(1), t);
        slab_store<WT, C>(ring[0], smem, t);
        __syncthreads();
        int kk = 0;
        for (; kk + 2 <= nk; kk += 2) {
            step(kk, ring[0], ring[1]);
            step(kk + 1, ring[1], ring[0]);
        }
        if (kk < nk) step(kk, ring[0], ring[1]);
    }

    // epilogue: C = scale[m] * acc
    const int lr = lane % 32, lg = lane / 32;
    scale_rows(acc, args.scales, m0 + wm * C::TM, lg, args.M);
#pragma unroll
    for (int i = 0; i < C::MI; i++) {
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int r = m0 + wm * C::TM + i * 32 + 8 * (e / 4) + 4 * lg + (e % 4);
            if (r >= args.M) continue;
            float * crow = G.C + (int64_t)r * G.ldc;
#pragma unroll
            for (int j = 0; j < C::NJ; j++) {
                const int n = n0 + wn * C::TN + j * 32 + lr;
                if (n < G.N) {
                    if (ks == 1 || args.part) crow[n] = acc[i][j][e];
                    else unsafeAtomicAdd(crow + n, acc[i][j][e]);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Skinny GEMM (M <= 128): a launch this narrow is bound by how many weight bytes it keeps in
// flight, not by MFMA rate, so the weight goes from HBM straight into registers and is decoded
// there into MFMA operands (no LDS round trip for the weight). A block is SK_NW waves over
// SK_NW*32 weight rows and a run of K groups of CH 64-deep chunks; lane (r, g) of a wave loads
// decoder item g of each chunk for weight row r, and the 32 values it decodes (two runs of 16
// consecutive k) are its B operands for the chunk's four 16-deep MFMA steps, so lane (r, g) of
// the A operand reads the same k from activation row r. Per group the activation slice
// [32 MT][64 CH] fp16 sits in LDS (16-byte chunks XOR-swizzled by row), double-buffered, and the
// weight of the next group is in flight in a second register set while this one is multiplied.
// Issue order matters: one vmcnt counter covers every load in issue order, so each step issues
// the next group's activation loads before its weight loads (their LDS store then waits for them
// alone, not for the weight), and nothing consumes a loaded value before the step's compute: the
// activation's row / K mask is applied at its LDS store, since a select right after a load would
// make the compiler wait for that load before issuing the next. Past the block's last group the
// loads re-fetch it and are never multiplied, so the loop body has no branch between a load and
// its use. The weights are decoded by the packed-fp16 decoders (decode_fast: a quarter to a half
// of the VALU instructions of the exact decode, which bounded this kernel). Blocks split K: past
// two ways each writes its slab of the partials, summed in split order by reduce_splits_kernel;
// two ways add into a zeroed output.
// ---------------------------------------------------------------------------------------------
constexpr int SK_MAX_M = 128;
constexpr int SK_NW = 4;

// Two waves per SIMD (two blocks per CU) where the two register sets fit in half the register
// file without spilling, one otherwise.
template <int WT, int MT>
constexpr int skinny_occupancy() {
    return (WT == T_Q4_K || WT == T_MXFP4 || WT == T_Q4_0 || MT == 1) ? 2 : 1;
}

template <int WT, int MT, int CH>
__global__ void __launch_bounds__(SK_NW * WAVE)
__attribute__((amdgpu_waves_per_eu(skinny_occupancy<WT, MT>(), skinny_occupancy<WT, MT>())))
gemm_skinny_kernel(GemmArgs args, int groups_per_block) {
    constexpr int NW = SK_NW;
    constexpr int CPR = 8 * CH;               // 16-byte chunks per activation row of the slice
    constexpr int ACH = 32 * MT * CPR;        // 16-byte chunks of the slice
    constexpr int APT = ACH / (NW * WAVE);    // per thread
    constexpr int SLICE = ACH * 16;
    static_assert(ACH % (NW * WAVE) == 0, "slice split");
    __shared__ __align__(16) uint8_t sa[2 * SLICE];

    const int t = threadIdx.x, lane = t % WAVE, wave = t / WAVE;
    const int lr = lane % 32, lg = lane / 32;
    const int ks = args.ksplit;
    const int split = blockIdx.x % ks;
    const int nt = blockIdx.x / ks;
    int g = 0;
#pragma unroll
    for (int i = 1; i < GEMM_MAX_GROUPS; i++)
        if (i < args.ng && nt >= args.g[i].ntile_begin) g = i;
    GemmGroup G;
    G.W = args.g[0].W; G.rows_total = args.g[0].rows_total; G.row0 = args.g[0].row0; G.N = args.g[0].N;
    G.C = args.g[0].C; G.ldc = args.g[0].ldc; G.ntile_begin = args.g[0].ntile_begin;
#pragma unroll
    for (int i = 1; i < GEMM_MAX_GROUPS; i++)
        if (i == g) {
            G.W = args.g[i].W; G.rows_total = args.g[i].rows_total; G.row0 = args.g[i].row0; G.N = args.g[i].N;
            G.C = args.g[i].C; G.ldc = args.g[i].ldc; G.ntile_begin = args.g[i].ntile_begin;
        }
    split_target(args, g, split, G.C, G.ldc);
    const int n = (nt - G.ntile_begin) * (32 * NW) + 32 * wave + lr;   // this lane's weight row
    const bool okn = n < G.N;
    const int64_t row = G.row0 + (okn ? n : G.N - 1);
    const int nchunks = (args.K + 63) / 64;
    const int ngroups = (nchunks + CH - 1) / CH;
    const int gb = split * groups_per_block;                             // first group of the block
    const int gn = max(0, min(ngroups, gb + groups_per_block) - gb);    // groups of the block
    const int glast = gb + max(gn, 1) - 1;

    // rows past M and k past K read as zero: the load takes a valid address and the mask is
    // applied when the value is stored to LDS (where the load is waited for anyway), so no
    // wait sits between one load and the next
    auto load_a = [&](u32x4 (&av)[APT], uint32_t & amask, int grp) {
        const int64_t kb = (int64_t)min(grp, glast) * CH * 64;
        amask = 0;
#pragma unroll
        for (int i = 0; i < APT; i++) {
            const int q = t + i * NW * WAVE, r = q / CPR, c = q % CPR;
            const int64_t k = kb + 8 * c;
            const bool ok = r < args.M && k < args.K;
            av[i] = *(const u32x4 *)(args.A + (ok ? (int64_t)r * args.lda + k : 0));
            amask |= ok ? (1u << i) : 0u;
        }
    };
    auto store_a = [&](const u32x4 (&av)[APT], uint32_t amask, int buf) {
#pragma unroll
        for (int i = 0; i < APT; i++) {
            const int q = t + i * NW * WAVE, r = q / CPR, c = q % CPR;
            const bool ok = (amask >> i) & 1u;
            const u32x4 v = {ok ? av[i][0] : 0u, ok ? av[i][1] : 0u, ok ? av[i][2] : 0u, ok ? av[i][3] : 0u};
            *(u32x4 *)(sa + buf * SLICE + (r * CPR + (c ^ (r & 7))) * 16) = v;
        }
    };
    auto load_w = [&](WLoad<WT> (&w)[CH], int grp) {
        const bool live = okn && grp <= glast && gn > 0;
        const int c0 = min(grp, glast) * CH;
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const int cc = c0 + c;
            w[c].load((const uint8_t *)G.W, G.rows_total, args.K, row, (int64_t)min(cc, nchunks - 1) * 64, lg,
                      live && cc < nchunks);
        }
    };
    float16v acc[MT][1];
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[i][0][e] = 0.0f;
    auto compute = [&](const WLoad<WT> (&w)[CH], int buf) {
#pragma unroll
        for (int c = 0; c < CH; c++) {
            u32x4 b[4];
            int run0, run1;
            w[c].decode_fast(lg, b, run0, run1);
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const int ch = 8 * c + (s < 2 ? run0 + 8 * s : run1 + 8 * (s - 2)) / 8;   // slice chunk
                const half8 bf = __builtin_bit_cast(half8, b[s]);
#pragma unroll
                for (int i = 0; i < MT; i++) {
                    const int r = 32 * i + lr;
                    const half8 af = *(const half8 *)(sa + buf * SLICE + (r * CPR + (ch ^ (r & 7))) * 16);
                    acc[i][0] = mfma32(af, bf, acc[i][0]);
                }
            }
        }
    };

    WLoad<WT> w0[CH], w1[CH];
    u32x4 av[APT];
    uint32_t amask;
    load_a(av, amask, gb);
    load_w(w0, gb);
    store_a(av, amask, 0);
    __syncthreads();
    int q = 0;
    for (; q + 2 <= gn; q += 2) {
        load_a(av, amask, gb + q + 1);
        load_w(w1, gb + q + 1);
        compute(w0, 0);
        store_a(av, amask, 1);
        __syncthreads();
        load_a(av, amask, gb + q + 2);
        load_w(w0, gb + q + 2);
        compute(w1, 1);
        store_a(av, amask, 0);
        __syncthreads();
    }
    if (q < gn) compute(w0, 0);

    scale_rows(acc, args.scales, 0, lg, args.M);
    if (!okn || gn == 0) return;
#pragma unroll
    for (int i = 0; i < MT; i++) {
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int r = i * 32 + 8 * (e / 4) + 4 * lg + (e % 4);
            if (r >= args.M) continue;
            float * p = G.C + (int64_t)r * G.ldc + n;
            if (ks == 1 || args.part) *p = acc[i][0][e];
            else unsafeAtomicAdd(p, acc[i][0][e]);
        }
    }
}

// ---------------------------------------------------------------------------------------------
// fp16-weight GEMM with LDS DMA
//
// For fp16 weights nothing has to be decoded between HBM and LDS, so both operands go straight
// into LDS with global_load_lds_dwordx4 (gfx950): no staging registers, no ds_write. K is staged
// DK (32, 64 or 128) values at a time through a ring of NS LDS stages; while one stage is
// multiplied the next NS-1 are landing. A block is WGM x WGN waves, each owning a
// (BM/WGM) x (BN/WGN) tile of 32x32x16 MFMAs with its accumulators in AGPRs. With 8 waves two
// share each SIMD, so one wave's MFMAs cover the other's LDS reads and barrier waits.
//
// A DMA instruction writes 64 lanes x 16 bytes to 1 KB of consecutive LDS; lane l lands at
// base + 16 l. Each lane therefore fetches the global chunk that belongs at its LDS slot under
// the swizzle: a row of DK values holds CH = DK/8 chunks, and slot (row, p) holds logical chunk
// p ^ ((row / (16/CH)) & (CH-1)), so the 16 rows of an MFMA fragment read hit 16 distinct bank
// groups. With DK >= 64 every DMA instruction covers whole 128-byte lines of A and W, which
// halves the cache-line lookups per byte against DK = 32 (the limit of this path when all its
// data hits in L2). Rows past M or N are clamped to the last real row (their results are never
// stored); K must be a multiple of DK, so there is no K tail.
//
// The waits are explicit, and the compiler is kept from adding its own around the DMA:
//   * before every barrier, s_waitcnt on this wave's DMA count (the stage about to be read has
//     landed, the NS-2 behind it may still be in flight) and on lgkmcnt (this wave's LDS reads of
//     the stage about to be overwritten are done);
//   * every iteration issues exactly one stage of DMA (past the last stage it re-fetches the last
//     one into a buffer nobody reads again), so those counts are the same every time and the loop
//     body has no branch;
//   * the compiler waits for all outstanding LDS reads before an MFMA whose fragment is still in
//     flight (it cannot order them against the DMA), so each fragment read is issued after the
//     first MFMA that would otherwise wait for it, and scheduling barriers keep that order.
// KSPLIT = 2 splits K between two blocks that add their halves atomically into a zeroed output
// (two addends: the sum is the same in either order).
// ---------------------------------------------------------------------------------------------
template <int BM, int BN, int WGM, int WGN, int DK, int NS>
struct F16Cfg {
    static constexpr int NW = WGM * WGN, THREADS = WAVE * NW;
    static constexpr int TM = BM / WGM, TN = BN / WGN, MI = TM / 32, NJ = TN / 32;
    static constexpr int CH = DK / 8, RPW = 16 / CH, RB = DK * 2;
    static constexpr int A_BYTES = BM * RB, B_BYTES = BN * RB, STAGE = A_BYTES + B_BYTES;
    static constexpr int LDS = NS * STAGE;
    static constexpr int PA = A_BYTES / (THREADS * 16), PB = B_BYTES / (THREADS * 16);   // DMA per wave
    static constexpr int PER = PA + PB;
    static_assert(MI >= 1 && NJ >= 1 && TM % 32 == 0 && TN % 32 == 0, "wave tile");
    static_assert(PA >= 1 && PB >= 1 && PA * THREADS * 16 == A_BYTES && PB * THREADS * 16 == B_BYTES, "DMA split");
    static_assert(NS >= 2 && (NS - 1) * PER <= 63, "vmcnt range");
    static_assert(LDS <= 160 * 1024, "LDS");
};

typedef const void __attribute__((address_space(1))) * gptr_t;
typedef void __attribute__((address_space(3))) * lptr_t;

__device__ __forceinline__ void dma16(const void * g, void * l) {
    __builtin_amdgcn_global_load_lds((gptr_t)g, (lptr_t)l, 16, 0, 0);
}

// s_waitcnt with vmcnt(N), expcnt(7) (no wait), lgkmcnt(0): gfx9 encoding.
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
    static_assert(N >= 0 && N <= 63, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | ((N >> 4) << 14));
}

template <int BM, int BN, int WGM, int WGN, int DK, int NS, int KSPLIT, bool TL>
__global__ void __launch_bounds__(WAVE * WGM * WGN)
__attribute__((amdgpu_waves_per_eu(WGM * WGN / 4, WGM * WGN / 4)))
gemm_f16_kernel(GemmArgs args) {
    using C = F16Cfg<BM, BN, WGM, WGN, DK, NS>;
    extern __shared__ __align__(16) uint8_t smem[];
    const int t = threadIdx.x, lane = t % WAVE, wave = t / WAVE;
    const int wm = wave / WGN, wn = wave % WGN;

    int tile = xcd_tile(blockIdx.x, gridDim.x);
    const int split = tile % KSPLIT;
    tile /= KSPLIT;
    const int mt = tile % args.m_tiles, nt = tile / args.m_tiles;
    int g = 0;
#pragma unroll
    for (int i = 1; i < GEMM_MAX_GROUPS; i++)
        if (i < args.ng && nt >= args.g[i].ntile_begin) g = i;
    const uint16_t * W = (const uint16_t *)args.g[0].W;
    int64_t row0 = args.g[0].row0;
    int N = args.g[0].N, ntb = args.g[0].ntile_begin;
    float * Cp = args.g[0].C;
    int64_t ldc = args.g[0].ldc;
#pragma unroll
    for (int i = 1; i < GEMM_MAX_GROUPS; i++)
        if (i == g) {
            W = (const uint16_t *)args.g[i].W; row0 = args.g[i].row0; N = args.g[i].N;
            ntb = args.g[i].ntile_begin; Cp = args.g[i].C; ldc = args.g[i].ldc;
        }
    const int n0 = (nt - ntb) * BN, m0 = mt * BM;
    const int M = args.M, K = args.K;
    const int nk_all = K / DK;
    const int per = (nk_all + KSPLIT - 1) / KSPLIT;
    const int kb = split * per;
    const int nk = max(0, min(nk_all, kb + per) - kb);

    // this lane's global sources, one row chunk per DMA instruction, advanced by one stage's K
    // per stage: DK values in rows, DK/32 tiles of 512 values in the tiled layout (TL), where the
    // 16 rows x DK of one instruction are whole 64-byte tile rows
    const uint16_t * asrc[C::PA];
    const uint16_t * bsrc[C::PB];
#pragma unroll
    for (int q = 0; q < C::PA; q++) {
        const int slot = (q * C::NW + wave) * WAVE + lane;
        const int r = slot / C::CH, c = (slot % C::CH) ^ ((r / C::RPW) & (C::CH - 1));
        const int64_t row = min(m0 + r, M - 1), k = (int64_t)kb * DK + 8 * c;
        asrc[q] = args.A + (TL ? tiled_index(row, k, K) : row * args.lda + k);
    }
#pragma unroll
    for (int q = 0; q < C::PB; q++) {
        const int slot = (q * C::NW + wave) * WAVE + lane;
        const int r = slot / C::CH, c = (slot % C::CH) ^ ((r / C::RPW) & (C::CH - 1));
        const int64_t row = row0 + min(n0 + r, N - 1), k = (int64_t)kb * DK + 8 * c;
        bsrc[q] = W + (TL ? tiled_index(row, k, K) : row * K + k);
    }
    // the LDS destination of a DMA instruction must be wave-uniform (it goes to M0): take the
    // wave index from an SGPR so the address arithmetic stays scalar
    const int wave_s = __builtin_amdgcn_readfirstlane(wave);
    // stage s into ring buffer s % NS; past the last stage the last one is fetched again into
    // the buffer just freed (nobody reads it again)
    auto issue = [&](int s) {
        uint8_t * st = smem + (s % NS) * C::STAGE;
        s = min(s, nk - 1);
        const int64_t off = (int64_t)s * (TL ? DK * 16 : DK);
#pragma unroll
        for (int q = 0; q < C::PA; q++) dma16(asrc[q] + off, st + (q * C::NW + wave_s) * 1024);
#pragma unroll
        for (int q = 0; q < C::PB; q++) dma16(bsrc[q] + off, st + C::A_BYTES + (q * C::NW + wave_s) * 1024);
    };

    float16v acc[C::MI][C::NJ];
#pragma unroll
    for (int i = 0; i < C::MI; i++)
#pragma unroll
        for (int j = 0; j < C::NJ; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

    // fragment rows (w*T + i*32 + lr), logical chunk (2 ks + lg); the row part of the swizzle
    // depends on lr only, because w*T + i*32 is a multiple of 16
    const int lr = lane % 32, lg = lane / 32, x = (lr / C::RPW) & (C::CH - 1);
    const int a_off = (wm * C::TM + lr) * C::RB, b_off = C::A_BYTES + (wn * C::TN + lr) * C::RB;
    struct Frags {
        half8 a[C::MI], b[C::NJ];
    };
    auto read_frags = [&](int s, int ks, Frags & f) {
        const uint8_t * st = smem + (s % NS) * C::STAGE;
        const int co = ((2 * ks + lg) ^ x) * 16;
#pragma unroll
        for (int i = 0; i < C::MI; i++) f.a[i] = *(const half8 *)(st + a_off + i * 32 * C::RB + co);
#pragma unroll
        for (int j = 0; j < C::NJ; j++) f.b[j] = *(const half8 *)(st + b_off + j * 32 * C::RB + co);
    };
    // the MFMAs of one 16-deep K step; `part` 0 = only the first, 1 = all but the first
    auto mma = [&](const Frags & f, int part) {
#pragma unroll
        for (int i = 0; i < C::MI; i++)
#pragma unroll
            for (int j = 0; j < C::NJ; j++)
                if ((part == 0) == (i == 0 && j == 0)) acc[i][j] = mfma32(f.a[i], f.b[j], acc[i][j]);
    };

    // Software pipeline over the 16-deep K steps of each stage, fragments alternating between f0
    // and f1: the next step's fragments are read while this step's MFMAs run. At the last step of
    // a stage: one barrier (the next stage has landed for every wave, and every wave is done
    // reading this one), the next stage's first fragments, and the DMA of the stage NS ahead
    // into the buffer just freed.
    if (nk > 0) {
        Frags f0, f1;
#pragma unroll
        for (int p = 0; p < NS; p++) issue(p);
        wait_vm_lgkm0<(NS - 1) * C::PER>();
        __builtin_amdgcn_s_barrier();
        read_frags(0, 0, f0);
        constexpr int KS = DK / 16;
        for (int s = 0; s < nk; s++) {
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                Frags & F = (ks % 2 == 0) ? f0 : f1;
                Frags & G = (ks % 2 == 0) ? f1 : f0;
                mma(F, 0);
                __builtin_amdgcn_sched_barrier(0);
                if (ks + 1 < KS) {
                    read_frags(s, ks + 1, G);
                    __builtin_amdgcn_sched_barrier(0);
                } else {
                    wait_vm_lgkm0<(NS - 2) * C::PER>();
                    __builtin_amdgcn_s_barrier();
                    read_frags(s + 1, 0, G);
                    __builtin_amdgcn_sched_barrier(0);
                    issue(s + NS);
                    __builtin_amdgcn_sched_barrier(0);
                }
                mma(F, 1);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        wait_vm_lgkm0<0>();   // no DMA may still be writing this block's LDS when it exits
    }

    // epilogue: C = scale[m] * acc
    scale_rows(acc, args.scales, m0 + wm * C::TM, lg, M);
#pragma unroll
    for (int i = 0; i < C::MI; i++) {
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int r = m0 + wm * C::TM + i * 32 + 8 * (e / 4) + 4 * lg + (e % 4);
            if (r >= M) continue;
            float * crow = Cp + (int64_t)r * ldc;
#pragma unroll
            for (int j = 0; j < C::NJ; j++) {
                const int n = n0 + wn * C::TN + j * 32 + lr;
                if (n < N) {
                    if (KSPLIT == 1) crow[n] = acc[i][j][e];
                    else unsafeAtomicAdd(crow + n, acc[i][j][e]);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------
// The same LDS-DMA pipeline with a block tile whose two wave columns differ in width: BN0 + BN1
// columns (e.g. 128 + 96 = 224), 8 waves in a 4 x 2 grid. A 256 x 224 tile cuts an N of 28672
// (the fused gate/up of an 8B model) into 128 x 2 = 256 blocks, one per CU, where 256 x 256
// leaves 32 CUs idle. Wave w takes column w / 4, so each SIMD (w % 4) holds one wave of each
// width. Each column's four waves fetch that column's B rows, so the DMA count per stage, and
// with it the vmcnt of every wait, is a per-column constant; the body below is instantiated once
// per column width, and both instances meet at the same barriers (one before the loop, one per
// stage).
// Where a column's B rows of one stage are not a whole number of DMA instructions per wave of
// that column (96 rows x 32 K: 6 KB for four waves), all eight waves share the B tile instead:
// instruction i (1 KB, 1024 / RB rows) goes to wave i % 8, and the waves whose last slot has no
// real instruction fetch the last real chunk again into a 1 KB LDS slot nobody reads, so every
// wave issues the same number of DMA instructions a stage and the wait counts stay constants.
// ---------------------------------------------------------------------------------------------
template <int BM_, int BN0, int BN1, int DK, int NS>
struct ColsCfg {
    static constexpr int NW = 8, THREADS = WAVE * NW, WGM = 4;
    static constexpr int BM = BM_, BN = BN0 + BN1, TM = BM / WGM, MI = TM / 32;
    static constexpr int CH = DK / 8, RPW = 16 / CH, RB = DK * 2, NSTAGES = NS;
    static constexpr int A_BYTES = BM * RB, B_BYTES = BN * RB, STAGE = A_BYTES + B_BYTES;
    static constexpr bool PERCOL = (BN0 * RB) % (4 * 1024) == 0 && (BN1 * RB) % (4 * 1024) == 0;
    static constexpr int NBI = B_BYTES / 1024;                       // B DMA instructions a stage
    static constexpr int PBW = (NBI + NW - 1) / NW;                  // per wave when shared
    static constexpr int RING = NS * STAGE;
    static constexpr int LDS = RING + (PERCOL ? 0 : (NW * PBW - NBI) * 1024);
    static constexpr int PA = A_BYTES / (THREADS * 16);
    static constexpr int PER_MAX = PA + (PERCOL ? BN0 * RB / 4096 : PBW);
    static_assert(MI >= 1 && TM % 32 == 0 && BN0 % 32 == 0 && BN1 % 32 == 0 && BN0 % 16 == 0, "wave tile");
    static_assert(PA * THREADS * 16 == A_BYTES, "A DMA split");
    static_assert(B_BYTES % 1024 == 0, "B DMA split");
    static_assert(NS >= 2 && (NS - 1) * PER_MAX <= 63, "vmcnt range");
    static_assert(LDS <= 160 * 1024, "LDS");
};

// The weight group a block's N tile falls in, resolved once per block from the kernel
// arguments (a select chain: indexing args.g with a runtime value would copy the array to
// scratch).
struct ColsTile {
    const uint16_t * W;
    int64_t row0;
    float * C;
    int64_t ldc;
    int N, n0, m0;
};

template <class C, int TNW, int COL0, bool TL>
__device__ __forceinline__ void cols_body(const uint16_t * __restrict__ Ap, const float * __restrict__ scales,
                                          int64_t lda, int M, int K, ColsTile tb, uint8_t * smem, int wm) {
    constexpr int DK = C::RB / 2, NS = C::NSTAGES, NJ = TNW / 32;
    constexpr int PB = C::PERCOL ? TNW * C::RB / 4096 : C::PBW;   // this wave's B DMA a stage
    constexpr int PER = C::PA + PB;
    const int t = threadIdx.x, lane = t % WAVE, wave = t / WAVE;
    const uint16_t * W = tb.W;
    const int64_t row0 = tb.row0;
    const int N = tb.N;
    float * Cp = tb.C;
    const int64_t ldc = tb.ldc;
    const int n0 = tb.n0, m0 = tb.m0;
    const int nk = K / DK;

    const uint16_t * asrc[C::PA];
    const uint16_t * bsrc[PB];
#pragma unroll
    for (int q = 0; q < C::PA; q++) {
        const int slot = (q * C::NW + wave) * WAVE + lane;
        const int r = slot / C::CH, c = (slot % C::CH) ^ ((r / C::RPW) & (C::CH - 1));
        const int64_t row = min(m0 + r, M - 1), k = 8 * c;
        asrc[q] = Ap + (TL ? tiled_index(row, k, K) : row * lda + k);
    }
#pragma unroll
    for (int q = 0; q < PB; q++) {
        if constexpr (C::PERCOL) {
            // rows COL0 .. COL0 + TNW of the B tile, fetched by this column's four waves; COL0 is a
            // multiple of 16, so the swizzle of a row depends on its offset inside the column only
            const int slot = (q * 4 + wm) * WAVE + lane;
            const int r = slot / C::CH, c = (slot % C::CH) ^ ((r / C::RPW) & (C::CH - 1));
            const int64_t row = row0 + min(n0 + COL0 + r, N - 1), k = 8 * c;
            bsrc[q] = W + (TL ? tiled_index(row, k, K) : row * K + k);
        } else {
            // instruction q * 8 + wave of the whole B tile (rows of both columns in order; the
            // swizzle is the same, since BN0 is a multiple of 16)
            const int slot = min(q * C::NW + wave, C::NBI - 1) * WAVE + lane;
            const int r = slot / C::CH, c = (slot % C::CH) ^ ((r / C::RPW) & (C::CH - 1));
            const int64_t row = row0 + min(n0 + r, N - 1), k = 8 * c;
            bsrc[q] = W + (TL ? tiled_index(row, k, K) : row * K + k);
        }
    }
    const int wave_s = __builtin_amdgcn_readfirstlane(wave), wm_s = __builtin_amdgcn_readfirstlane(wm);
    auto issue = [&](int s) {
        uint8_t * st = smem + (s % NS) * C::STAGE;
        s = min(s, nk - 1);
        const int64_t off = (int64_t)s * (TL ? DK * 16 : DK);
#pragma unroll
        for (int q = 0; q < C::PA; q++) dma16(asrc[q] + off, st + (q * C::NW + wave_s) * 1024);
#pragma unroll
        for (int q = 0; q < PB; q++) {
            if constexpr (C::PERCOL) {
                dma16(bsrc[q] + off, st + C::A_BYTES + COL0 * C::RB + (q * 4 + wm_s) * 1024);
            } else {
                const int gi = q * C::NW + wave_s;
                dma16(bsrc[q] + off, gi < C::NBI ? st + C::A_BYTES + gi * 1024 : smem + C::RING + (gi - C::NBI) * 1024);
            }
        }
    };

    float16v acc[C::MI][NJ];
#pragma unroll
    for (int i = 0; i < C::MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

    const int lr = lane % 32, lg = lane / 32, x = (lr / C::RPW) & (C::CH - 1);
    const int a_off = (wm * C::TM + lr) * C::RB, b_off = C::A_BYTES + (COL0 + lr) * C::RB;
    struct Frags {
        half8 a[C::MI], b[NJ];
    };
    auto read_frags = [&](int s, int ks, Frags & f) {
        const uint8_t * st = smem + (s % NS) * C::STAGE;
        const int co = ((2 * ks + lg) ^ x) * 16;
#pragma unroll
        for (int i = 0; i < C::MI; i++) f.a[i] = *(const half8 *)(st + a_off + i * 32 * C::RB + co);
#pragma unroll
        for (int j = 0; j < NJ; j++) f.b[j] = *(const half8 *)(st + b_off + j * 32 * C::RB + co);
    };
    auto mma = [&](const Frags & f, int part) {
#pragma unroll
        for (int i = 0; i < C::MI; i++)
#pragma unroll
            for (int j = 0; j < NJ; j++)
                if ((part == 0) == (i == 0 && j == 0)) acc[i][j] = mfma32(f.a[i], f.b[j], acc[i][j]);
    };

    // the pipeline of gemm_f16_kernel, stage for stage (same barriers, same DMA order)
    if (nk > 0) {
        Frags f0, f1;
#pragma unroll
        for (int p = 0; p < NS; p++) issue(p);
        wait_vm_lgkm0<(NS - 1) * PER>();
        __builtin_amdgcn_s_barrier();
        read_frags(0, 0, f0);
        constexpr int KS = DK / 16;
        for (int s = 0; s < nk; s++) {
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                Frags & F = (ks % 2 == 0) ? f0 : f1;
                Frags & G = (ks % 2 == 0) ? f1 : f0;
                mma(F, 0);
                __builtin_amdgcn_sched_barrier(0);
                if (ks + 1 < KS) {
                    read_frags(s, ks + 1, G);
                    __builtin_amdgcn_sched_barrier(0);
                } else {
                    wait_vm_lgkm0<(NS - 2) * PER>();
                    __builtin_amdgcn_s_barrier();
                    read_frags(s + 1, 0, G);
                    __builtin_amdgcn_sched_barrier(0);
                    issue(s + NS);
                    __builtin_amdgcn_sched_barrier(0);
                }
                mma(F, 1);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        wait_vm_lgkm0<0>();
    }

    scale_rows(acc, scales, m0 + wm * C::TM, lg, M);
#pragma unroll
    for (int i = 0; i < C::MI; i++) {
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int r = m0 + wm * C::TM + i * 32 + 8 * (e / 4) + 4 * lg + (e % 4);
            if (r >= M) continue;
            float * crow = Cp + (int64_t)r * ldc;
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const int n = n0 + COL0 + j * 32 + lr;
                if (n < N) crow[n] = acc[i][j][e];
            }
        }
    }
}

template <int BM, int BN0, int BN1, int DK, int NS, bool TL>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
gemm_f16_cols_kernel(GemmArgs args) {
    using C = ColsCfg<BM, BN0, BN1, DK, NS>;
    extern __shared__ __align__(16) uint8_t smem[];
    const int wave = threadIdx.x / WAVE;
    const int tile = xcd_tile(blockIdx.x, gridDim.x);
    const int mt = tile % args.m_tiles, nt = tile / args.m_tiles;
    ColsTile tb;
    tb.W = (const uint16_t *)args.g[0].W; tb.row0 = args.g[0].row0; tb.N = args.g[0].N;
    tb.C = args.g[0].C; tb.ldc = args.g[0].ldc;
    int ntb = args.g[0].ntile_begin;
#pragma unroll
    for (int i = 1; i < GEMM_MAX_GROUPS; i++)
        if (i < args.ng && nt >= args.g[i].ntile_begin) {
            tb.W = (const uint16_t *)args.g[i].W; tb.row0 = args.g[i].row0; tb.N = args.g[i].N;
            tb.C = args.g[i].C; tb.ldc = args.g[i].ldc; ntb = args.g[i].ntile_begin;
        }
    tb.n0 = (nt - ntb) * C::BN;
    tb.m0 = mt * C::BM;
    if (wave / 4 == 0) cols_body<C, BN0, 0, TL>(args.A, args.scales, args.lda, args.M, args.K, tb, smem, wave % 4);
    else cols_body<C, BN1, BN0, TL>(args.A, args.scales, args.lda, args.M, args.K, tb, smem, wave % 4);
}

// Zero the outputs of a split-K launch (a fill kernel rather than a memset, so the launch
// sequence stays capturable).
// Zeroes the outputs a split-K launch adds into: one block per (row, weight group), 16-byte
// stores where the row start allows them.
// ---------------------------------------------------------------------------------------------
// Q4_K GEMM with every operand by LDS DMA (the per-call dequant route for Q4_K weights).
//
// The weight stays in its Q4_K HBM layout (144-byte blocks of 256 values: d, dmin, 12 bytes of
// 6-bit scales and mins, 128 bytes of nibbles). Per 64-deep K stage a 256-row weight tile needs
// 32 bytes of nibbles a row (sub-blocks 2j and 2j+1 of the block, j = stage % 4) and, per block,
// its 16-byte header. Three LDS rings are filled by global_load_lds_dwordx4:
//   A  the row-scaled fp16 activations, two stages;
//   Q  the nibbles, three stages: thread t owns 16 bytes (row t/2, half t%2), landing at t*16;
//   H  the headers, two blocks: lanes 0-31 of wave w fetch rows 32w..32w+31, the rows its
//      threads decode.
// Q and H are private to the wave that fetches them, so only A needs the block's barrier. Each
// thread decodes its 32 values (rounding exactly as ggml's dequantizer) from Q and H into a
// double-buffered fp16 tile B; A and B use the 8-chunk XOR swizzle of the fp16 kernels, so the
// MFMA fragment reads are theirs. HBM and L2 traffic per weight is the Q4_K size, 0.5625 bytes
// (a resident fp16 copy moves 2).
//
// Per stage s (fragments of K step 0 already in registers; loop unrolled by 4, so s % 4 and
// with it every wait count below is a compile-time constant):
//   - the MFMAs of s, the fragments of the next K step read under each step's MFMAs;
//   - at one K step, a wait for the nibbles (and header) of s+1, issued two stages earlier, and
//     their decode into the free B buffer. Waves 4-7 decode two K steps after waves 0-3: the
//     waves that share a SIMD (w and w+4) take turns, one decoding while the other multiplies;
//   - after the first MFMA of the last K step: a wait for the activations of s+1 and this wave's
//     LDS writes, one barrier, the first fragments of s+1, then the DMA of the activations of
//     s+2, the nibbles of s+3 and, when s % 4 == 1, the header of the next block; the rest of the
//     step's MFMAs run under these.
// DMA instructions retire in order, so each wait counts the ones issued after its target (QD =
// the quant DMA instructions a thread issues per stage, 1 for Q4_K):
//   before the decode in stage s:  PA + QD, or PA + QD + 1 when s % 4 == 2 (a header was issued last)
//   at the end of stage s:         QD, or QD + 1 when s % 4 == 2.
// K % 256 == 0; a K split (args.ksplit) divides whole blocks. Past the last stage the last one
// is fetched and decoded again into the free buffers, so every stage issues the same DMA.
//
// The same pipeline takes Q8_0 weights in their split layout (int8 quants [rows][K], then fp16 d
// [rows][K/32]): a thread's 32 values are 32 quant bytes (QD = 2 instructions, the Q ring twice as
// wide) and the "header" of 256 values is the row's 8 block scales, 16 bytes as for Q4_K. The
// decode is Q8_0's packed one (exact: the int8 code under 1024, less the offset, times d rounds
// the exact product once). The wider Q ring leaves room for the 128 x 256 tile only.
// ---------------------------------------------------------------------------------------------
template <int WT, int BM, int WGM, int WGN>
struct Q4kCfg {
    static constexpr int BN = 256, NW = WGM * WGN, THREADS = WAVE * NW;
    static constexpr int TM = BM / WGM, TN = BN / WGN, MI = TM / 32, NJ = TN / 32;
    static constexpr int DK = 64, RB = 128;                         // 8 chunks of 16 bytes a row
    static constexpr int QD = WT == T_Q8_0 ? 2 : 1;                 // quant DMA per thread and stage
    static constexpr int A_BYTES = BM * RB, B_BYTES = BN * RB;
    static constexpr int Q_BYTES = BN * 32 * QD, H_BYTES = BN * 16;
    static constexpr int OFF_B = 2 * A_BYTES, OFF_Q = OFF_B + 2 * B_BYTES, OFF_H = OFF_Q + 3 * Q_BYTES;
    static constexpr int LDS = OFF_H + 2 * H_BYTES;
    static constexpr int PA = A_BYTES / (THREADS * 16);             // activation DMA per wave
    static_assert(WT == T_Q4_K || WT == T_Q8_0, "weight type");
    static_assert(NW == 8 && THREADS == 2 * BN, "one (row, half) item per thread");
    static_assert(MI >= 1 && NJ >= 1 && TM % 32 == 0 && TN % 32 == 0, "wave tile");
    static_assert(PA >= 1 && PA * THREADS * 16 == A_BYTES, "DMA split");
    static_assert(LDS <= 160 * 1024, "LDS");
};

// s_waitcnt with vmcnt(N) only (expcnt and lgkmcnt at their maximum): gfx9 encoding.
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N <= 63, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

template <int WT, int BM, int WGM, int WGN>
__global__ void __launch_bounds__(WAVE * WGM * WGN)
__attribute__((amdgpu_waves_per_eu(2, 2)))
gemm_q4k_kernel(GemmArgs args) {
    using C = Q4kCfg<WT, BM, WGM, WGN>;
    extern __shared__ __align__(16) uint8_t smem[];
    const int t = threadIdx.x, lane = t % WAVE, wave = t / WAVE;
    const int wm = wave / WGN, wn = wave % WGN;

    const int ks = args.ksplit > 1 ? args.ksplit : 1;
    int tile = xcd_tile(blockIdx.x, gridDim.x);
    const int split = tile % ks;
    tile /= ks;
    const int mt = tile % args.m_tiles, nt = tile / args.m_tiles;
    int g = 0;
#pragma unroll
    for (int i = 1; i < GEMM_MAX_GROUPS; i++)
        if (i < args.ng && nt >= args.g[i].ntile_begin) g = i;
    const uint8_t * W = (const uint8_t *)args.g[0].W;
    int64_t row0 = args.g[0].row0, rows_total = args.g[0].rows_total;
    int N = args.g[0].N, ntb = args.g[0].ntile_begin;
    float * Cp = args.g[0].C;
    int64_t ldc = args.g[0].ldc;
#pragma unroll
    for (int i = 1; i < GEMM_MAX_GROUPS; i++)
        if (i == g) {
            W = (const uint8_t *)args.g[i].W; row0 = args.g[i].row0; N = args.g[i].N;
            ntb = args.g[i].ntile_begin; Cp = args.g[i].C; ldc = args.g[i].ldc;
            rows_total = args.g[i].rows_total;
        }
    split_target(args, g, split, Cp, ldc);
    const int n0 = (nt - ntb) * C::BN, m0 = mt * BM;
    const int M = args.M, K = args.K;
    const int nsb = K / 256;                                   // 256-value blocks a row
    const int per = (nsb + ks - 1) / ks;
    const int sb0 = split * per;
    const int nk = 4 * max(0, min(nsb, sb0 + per) - sb0);      // stages of this split

    // activation DMA: one 16-byte chunk of a row per instruction, the chunk that belongs at the
    // lane's LDS slot under the swizzle; rows past M read the last row (never stored)
    const uint16_t * asrc[C::PA];
#pragma unroll
    for (int q = 0; q < C::PA; q++) {
        const int slot = (q * C::NW + wave) * WAVE + lane;
        const int r = slot / 8, c = (slot % 8) ^ ((r / 2) & 7);
        asrc[q] = args.A + (int64_t)min(m0 + r, M - 1) * args.lda + (int64_t)sb0 * 256 + 8 * c;
    }
    // weight DMA: the quants of item t (row t/2, half t%2) and, for lanes 0-31, the header of
    // row 32 * wave + lane; rows past N read the last row (their outputs are never stored).
    // Q4_K: per block qs_blk bytes apart, the header at the block's start, the nibbles of
    // quarter j at 16 + 32 j; Q8_0: the quants at 64 bytes a stage, the 8 scales of a block
    // 16 bytes apart in the scale plane.
    const int64_t qrow = row0 + min(n0 + t / 2, N - 1), hrow = row0 + min(n0 + 32 * wave + lane % 32, N - 1);
    const uint8_t * qsrc;
    const uint8_t * hsrc;
    if constexpr (WT == T_Q4_K) {
        const int64_t rowb = (int64_t)(K / 256) * 144;
        qsrc = W + qrow * rowb + (int64_t)sb0 * 144 + 16 + 16 * (t % 2);
        hsrc = W + hrow * rowb + (int64_t)sb0 * 144;
    } else {
        qsrc = W + qrow * K + (int64_t)sb0 * 256 + 32 * (t % 2);
        hsrc = W + rows_total * K + (hrow * (K / 32) + (int64_t)sb0 * 8) * 2;
    }
    const int wave_s = __builtin_amdgcn_readfirstlane(wave);

    auto issue_a = [&](int s) {
        uint8_t * st = smem + (s & 1) * C::A_BYTES;
        const int64_t off = (int64_t)min(s, nk - 1) * C::DK;
#pragma unroll
        for (int q = 0; q < C::PA; q++) dma16(asrc[q] + off, st + (q * C::NW + wave_s) * 1024);
    };
    // the quant DMA of item t lands at (q * THREADS + t) * 16 of its Q stage, q < QD
    auto issue_q = [&](int s) {
        const int sc = min(s, nk - 1);
        const uint8_t * src = WT == T_Q4_K ? qsrc + (sc / 4) * 144 + 32 * (sc % 4) : qsrc + (int64_t)sc * 64;
#pragma unroll
        for (int q = 0; q < C::QD; q++)
            dma16(src + 16 * q, smem + C::OFF_Q + (s % 3) * C::Q_BYTES + (q * C::NW + wave_s) * 1024);
    };
    auto issue_h = [&](int b) {
        const int bc = min(b, nk / 4 - 1);
        if (lane < 32)
            dma16(hsrc + (WT == T_Q4_K ? bc * 144 : bc * 16), smem + C::OFF_H + (b & 1) * C::H_BYTES + wave_s * 512);
    };
    // decode the item of stage s (J = s % 4) into B buffer s & 1
    auto decode = [&](int s, auto Jc) {
        constexpr int J = decltype(Jc)::value;
        const u32x4 hdr = *(const u32x4 *)(smem + C::OFF_H + ((s / 4) & 1) * C::H_BYTES + (t / 2) * 16);
        const uint8_t * qs = smem + C::OFF_Q + (s % 3) * C::Q_BYTES + t * 16;
        u32x4 out[4];
        int run0, run1;
        if constexpr (WT == T_Q4_K) {
            WLoad<T_Q4_K> w;
            w.hdr = hdr;
            w.qs = *(const u32x4 *)qs;
            w.j = J;
            w.ok = true;
            w.decode(t % 2, out, run0, run1);
        } else {
            // block 2 J + half of the 256 values: its scale is half (t % 2) of word J
            WLoad<T_Q8_0> w;
            w.q[0] = *(const u32x4 *)qs;
            w.q[1] = *(const u32x4 *)(qs + C::THREADS * 16);
            w.d = (uint16_t)(hdr[J] >> (16 * (t % 2)));
            w.ok = true;
            w.decode_fast(t % 2, out, run0, run1);
        }
        uint8_t * bs = smem + C::OFF_B + (s & 1) * C::B_BYTES;
        const int r = t / 2;
        *(u32x4 *)(bs + swz<8>(r, run0 / 8)) = out[0];
        *(u32x4 *)(bs + swz<8>(r, run0 / 8 + 1)) = out[1];
        *(u32x4 *)(bs + swz<8>(r, run1 / 8)) = out[2];
        *(u32x4 *)(bs + swz<8>(r, run1 / 8 + 1)) = out[3];
    };

    float16v acc[C::MI][C::NJ];
#pragma unroll
    for (int i = 0; i < C::MI; i++)
#pragma unroll
        for (int j = 0; j < C::NJ; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

    const int lr = lane % 32, lg = lane / 32, x = (lr / 2) & 7;
    const int a_off = (wm * C::TM + lr) * C::RB, b_off = C::OFF_B + (wn * C::TN + lr) * C::RB;
    struct Frags {
        half8 a[C::MI], b[C::NJ];
    };
    auto read_frags = [&](int s, int kstep, Frags & f) {
        const uint8_t * as = smem + (s & 1) * C::A_BYTES;
        const uint8_t * bs = smem + (s & 1) * C::B_BYTES;
        const int co = ((2 * kstep + lg) ^ x) * 16;
#pragma unroll
        for (int i = 0; i < C::MI; i++) f.a[i] = *(const half8 *)(as + a_off + i * 32 * C::RB + co);
#pragma unroll
        for (int j = 0; j < C::NJ; j++) f.b[j] = *(const half8 *)(bs + b_off + j * 32 * C::RB + co);
    };
    // the MFMAs of one 16-deep K step; `part` 0 = only the first, 1 = all but the first
    auto mma = [&](const Frags & f, int part) {
#pragma unroll
        for (int i = 0; i < C::MI; i++)
#pragma unroll
            for (int j = 0; j < C::NJ; j++)
                if ((part == 0) == (i == 0 && j == 0)) acc[i][j] = mfma32(f.a[i], f.b[j], acc[i][j]);
    };
    constexpr int KST = C::DK / 16;
    const int kd = wave_s >= 4 ? 2 : 0;   // the K step at which this wave decodes
    Frags f0, f1;
    // stage s, J = s % 4
    auto stage = [&](int s, auto Jc) {
        constexpr int J = decltype(Jc)::value;
#pragma unroll
        for (int kstep = 0; kstep < KST; kstep++) {
            Frags & F = (kstep % 2 == 0) ? f0 : f1;
            Frags & G = (kstep % 2 == 0) ? f1 : f0;
            mma(F, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (kstep + 1 < KST) {
                read_frags(s, kstep + 1, G);
                __builtin_amdgcn_sched_barrier(0);
            }
            if (kstep == kd) {
                wait_vm<C::PA + C::QD + (J == 2 ? 1 : 0)>();
                decode(s + 1, std::integral_constant<int, (J + 1) % 4>());
                __builtin_amdgcn_sched_barrier(0);
            }
            if (kstep + 1 == KST) {
                wait_vm_lgkm0<C::QD + (J == 2 ? 1 : 0)>();
                __builtin_amdgcn_s_barrier();
                read_frags(s + 1, 0, G);
                __builtin_amdgcn_sched_barrier(0);
                issue_a(s + 2);
                issue_q(s + 3);
                if (J == 1) issue_h(s / 4 + 1);   // the next block: its first decode is two stages on
                __builtin_amdgcn_sched_barrier(0);
            }
            mma(F, 1);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    if (nk > 0) {
        // prologue: stage 0 decoded, then the DMA in the order the steady state has in flight
        // at the start of stage 0: nibbles of 1, activations of 1, nibbles of 2
        issue_h(0);
        issue_q(0);
        issue_a(0);
        wait_vm<0>();
        decode(0, std::integral_constant<int, 0>());
        __builtin_amdgcn_sched_barrier(0);
        issue_q(1);
        issue_a(1);
        issue_q(2);
        __builtin_amdgcn_sched_barrier(0);
        wait_vm_lgkm0<C::PA + 2 * C::QD>();   // this wave's LDS writes; the DMA stays in flight
        __builtin_amdgcn_s_barrier();
        read_frags(0, 0, f0);
        __builtin_amdgcn_sched_barrier(0);
        for (int s = 0; s < nk; s += 4) {
            stage(s, std::integral_constant<int, 0>());
            stage(s + 1, std::integral_constant<int, 1>());
            stage(s + 2, std::integral_constant<int, 2>());
            stage(s + 3, std::integral_constant<int, 3>());
        }
        wait_vm_lgkm0<0>();   // no DMA may still be writing this block's LDS when it exits
    }

    // epilogue: C = scale[m] * acc
    scale_rows(acc, args.scales, m0 + wm * C::TM, lg, M);
#pragma unroll
    for (int i = 0; i < C::MI; i++) {
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int r = m0 + wm * C::TM + i * 32 + 8 * (e / 4) + 4 * lg + (e % 4);
            if (r >= M) continue;
            float * crow = Cp + (int64_t)r * ldc;
#pragma unroll
            for (int j = 0; j < C::NJ; j++) {
                const int n = n0 + wn * C::TN + j * 32 + lr;
                if (n < N) {
                    if (ks == 1 || args.part) crow[n] = acc[i][j][e];
                    else unsafeAtomicAdd(crow + n, acc[i][j][e]);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Skinny GEMM with the weight staged by LDS DMA (M <= 128; Q4_K, Q8_0 and Q6_K weights).
//
// The register-staged skinny kernel above keeps one K group of weight in flight per wave beside
// the one it multiplies, so a block that owns a few groups pays an HBM round trip for nearly each
// of them. Here the bytes go from HBM into LDS by global_load_lds_dwordx4, which holds them
// without registers: a ring of NS stages, each one K group (CH 64-deep chunks) of the activation
// slice and of the weight, NS - 1 groups requested ahead of the one multiplied. A lane's weight
// item (decoder item g of chunk c of weight row r, as in the register kernel) arrives as NP
// 16-byte pieces, each DMA'd by the lane that decodes it, to LDS slot
// ((c * NP + p) * NW + wave) * 1 KB + 16 * lane, so the weight ring is private to its wave; the
// few bytes of an item that are not 16-byte pieces (a Q8_0 block's scale, a Q6_K block's scales
// and d) come as the aligned 16 bytes of their plane that hold them, so no register ring (whose
// loads the compiler would wait for in full at the loop's back edge) is needed. The activation slice is shared by the
// block's waves and lands XOR-swizzled as in the register kernel: each lane fetches the chunk
// that belongs at its slot. Per group: wait for this wave's DMA of the group (every group issues
// the same count, past the block's last group the last one is fetched again, so the count is a
// constant), one barrier (the slice is complete, and every wave is done with the stage about to
// be refilled), the DMA of group + NS - 1, then the group's decode and MFMAs.
// Same decoders, same fp16 products and the same K order per output as the register kernel.
// ---------------------------------------------------------------------------------------------
template <int WT> struct SkPieces;

// The aligned 16 bytes of a plane of 2-byte values that hold value `idx` (a plane starts 16-byte
// aligned and, with N % 16 == 0, spans a whole number of 16-byte chunks, so the chunk is inside
// it), and the value from that chunk.
__device__ __forceinline__ const uint8_t * chunk_of16(const uint8_t * plane, int64_t idx) {
    return plane + ((2 * idx) & ~(int64_t)15);
}
// word i (0..3) of c by selects: a runtime index into a vector would go through scratch memory
__device__ __forceinline__ uint32_t word_of(const u32x4 & c, int i) {
    const uint32_t lo = (i & 1) ? c[1] : c[0], hi = (i & 1) ? c[3] : c[2];
    return (i & 2) ? hi : lo;
}
__device__ __forceinline__ uint16_t half_in_chunk(const u32x4 & c, int64_t idx) {
    const int o = (int)((2 * idx) & 15);
    return (uint16_t)(word_of(c, o >> 2) >> (8 * (o & 3)));
}

template <> struct SkPieces<T_Q4_K> {   // the block header and this item's 16 bytes of nibbles
    static constexpr int NP = 2;
    __device__ static const uint8_t * piece(const uint8_t * W, int64_t rows, int64_t K, int64_t row, int64_t k0,
                                            int u, int p) {
        const uint8_t * b = W + (row * (K / 256) + k0 / 256) * 144;
        return p == 0 ? b : b + 16 + 32 * ((k0 % 256) / 64) + 16 * u;
    }
    __device__ static void item(WLoad<T_Q4_K> & w, const u32x4 (&pc)[NP], int64_t, int64_t, int64_t row, int64_t k0,
                                int, bool ok) {
        w.hdr = pc[0];
        w.qs = pc[1];
        w.j = (int)((k0 % 256) / 64);
        w.ok = ok;
    }
};

template <> struct SkPieces<T_Q8_0> {   // the item's 32 quants and the chunk holding its scale
    static constexpr int NP = 3;
    // the item's first value, k0 + 32 u, clamped to 0 past K (the item is then masked)
    __device__ static int64_t kk(int64_t K, int64_t k0, int u) {
        const int64_t k = k0 + 32 * u;
        return k < K ? k : 0;
    }
    __device__ static const uint8_t * piece(const uint8_t * W, int64_t rows, int64_t K, int64_t row, int64_t k0,
                                            int u, int p) {
        if (p < 2) return W + row * K + kk(K, k0, u) + 16 * p;
        return chunk_of16(W + rows * K, row * (K / 32) + kk(K, k0, u) / 32);
    }
    __device__ static void item(WLoad<T_Q8_0> & w, const u32x4 (&pc)[NP], int64_t rows, int64_t K, int64_t row,
                                int64_t k0, int u, bool ok) {
        w.q[0] = pc[0];
        w.q[1] = pc[1];
        w.d = half_in_chunk(pc[2], row * (K / 32) + kk(K, k0, u) / 32);
        w.ok = ok;
    }
};

template <> struct SkPieces<T_Q6_K> {   // ql (two runs), qh, the block's 16 scales, the chunk holding d
    static constexpr int NP = 5;
    __device__ static const uint8_t * piece(const uint8_t * W, int64_t rows, int64_t K, int64_t row, int64_t k0,
                                            int u, int p) {
        const int64_t blk = k0 / 256;
        const int h = (int)((k0 % 256) / 64) >> 1, l0 = 16 * u;
        if (p < 2) return W + row * (K / 2) + blk * 128 + 64 * h + l0 + 32 * p;
        if (p == 2) return W + rows * (K / 2) + row * (K / 4) + blk * 64 + 32 * h + l0;
        const uint8_t * sc = W + rows * (K / 2) + rows * (K / 4);
        if (p == 3) return sc + row * (K / 16) + blk * 16;
        return chunk_of16(sc + rows * (K / 16), row * (K / 256) + blk);
    }
    __device__ static void item(WLoad<T_Q6_K> & w, const u32x4 (&pc)[NP], int64_t rows, int64_t K, int64_t row,
                                int64_t k0, int u, bool ok) {
        const int64_t blk = k0 / 256;
        const int q4 = (int)((k0 % 256) / 64), h = q4 >> 1, hi = q4 & 1;
        w.qla = pc[0];
        w.qlb = pc[1];
        w.qh = pc[2];
        // scales 8h + u + 4hi and that + 2 of the block (sub-blocks (l/16) + {0,2} or + {4,6})
        const int i0 = 8 * h + u + 4 * hi;
        const uint32_t s0 = (word_of(pc[3], i0 >> 2) >> (8 * (i0 & 3))) & 0xFFu;
        const uint32_t s1 = (word_of(pc[3], (i0 + 2) >> 2) >> (8 * ((i0 + 2) & 3))) & 0xFFu;
        w.sc = s0 | (s1 << 8);
        w.d = half_in_chunk(pc[4], row * (K / 256) + blk);
        w.hi = hi;
        w.ok = ok;
    }
};

template <int WT, int MT, int CH, int NS>
struct SkDmaCfg {
    static constexpr int NW = SK_NW, THREADS = NW * WAVE;
    static constexpr int NP = SkPieces<WT>::NP;
    static constexpr int CPR = 8 * CH;                    // 16-byte chunks per activation row of the slice
    static constexpr int A_BYTES = 32 * MT * CPR * 16;    // the slice [32 MT][64 CH] fp16
    static constexpr int PA = A_BYTES / (THREADS * 16);   // activation DMA per wave per group
    static constexpr int W_BYTES = CH * NP * NW * 1024;   // every wave's pieces of the group
    static constexpr int STAGE = A_BYTES + W_BYTES;
    static constexpr int LDS = NS * STAGE;
    static constexpr int PER = PA + CH * NP;              // DMA per wave per group
    static_assert(PA >= 1 && PA * THREADS * 16 == A_BYTES, "slice split");
    static_assert(NS >= 2 && NS <= 4 && LDS <= 160 * 1024, "LDS");
};

// One block a CU (its ring takes most of the LDS), so one wave a SIMD: the whole register file is
// the wave's.
template <int WT, int MT, int CH, int NS>
__global__ void __launch_bounds__(SK_NW * WAVE)
__attribute__((amdgpu_waves_per_eu(1, 1)))
gemm_skinny_dma_kernel(GemmArgs args, int groups_per_block) {
    using C = SkDmaCfg<WT, MT, CH, NS>;
    using P = SkPieces<WT>;
    constexpr int NW = C::NW, CPR = C::CPR, NP = C::NP;
    extern __shared__ __align__(16) uint8_t smem[];

    const int t = threadIdx.x, lane = t % WAVE, wave = t / WAVE;
    const int wave_s = __builtin_amdgcn_readfirstlane(wave);
    const int lr = lane % 32, lg = lane / 32;
    const int ks = args.ksplit;
    const int split = blockIdx.x % ks;
    const int nt = blockIdx.x / ks;
    int g = 0;
#pragma unroll
    for (int i = 1; i < GEMM_MAX_GROUPS; i++)
        if (i < args.ng && nt >= args.g[i].ntile_begin) g = i;
    GemmGroup G;
    G.W = args.g[0].W; G.rows_total = args.g[0].rows_total; G.row0 = args.g[0].row0; G.N = args.g[0].N;
    G.C = args.g[0].C; G.ldc = args.g[0].ldc; G.ntile_begin = args.g[0].ntile_begin;
#pragma unroll
    for (int i = 1; i < GEMM_MAX_GROUPS; i++)
        if (i == g) {
            G.W = args.g[i].W; G.rows_total = args.g[i].rows_total; G.row0 = args.g[i].row0; G.N = args.g[i].N;
            G.C = args.g[i].C; G.ldc = args.g[i].ldc; G.ntile_begin = args.g[i].ntile_begin;
        }
    split_target(args, g, split, G.C, G.ldc);
    const int n = (nt - G.ntile_begin) * (32 * NW) + 32 * wave + lr;   // this lane's weight row
    const bool okn = n < G.N;
    const int64_t row = G.row0 + (okn ? n : G.N - 1);
    const int K = args.K;
    const int nchunks = (K + 63) / 64;
    const int ngroups = (nchunks + CH - 1) / CH;
    const int gb = split * groups_per_block;
    const int gn = max(0, min(ngroups, gb + groups_per_block) - gb);
    const int glast = gb + max(gn, 1) - 1;
    const uint8_t * W = (const uint8_t *)G.W;

    // activation DMA sources: slot q of the slice holds row q / CPR, logical chunk
    // (q % CPR) ^ (row & 7); rows past M read the last row and k past K the row's first chunk
    // (finite values, multiplied by zero weights or never stored)
    const uint16_t * asrc[C::PA];
    int acol[C::PA];
#pragma unroll
    for (int i = 0; i < C::PA; i++) {
        const int q = (i * NW + wave) * WAVE + lane;
        const int r = q / CPR, c = (q % CPR) ^ (r & 7);
        asrc[i] = args.A + (int64_t)min(r, args.M - 1) * args.lda;
        acol[i] = 8 * c;
    }
    // group grp (clamped to the block's last) into stage st
    auto issue = [&](int grp, int st) __attribute__((always_inline)) {
        const int gg = min(grp, glast);
        uint8_t * base = smem + st * C::STAGE;
        const int64_t kb = (int64_t)gg * CH * 64;
#pragma unroll
        for (int i = 0; i < C::PA; i++) {
            const int64_t k = kb + acol[i];
            dma16(asrc[i] + (k < K ? k : 0), base + (i * NW + wave_s) * 1024);
        }
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const int cc = min(gg * CH + c, nchunks - 1);
            const int64_t k0 = (int64_t)cc * 64;
#pragma unroll
            for (int p = 0; p < NP; p++)
                dma16(P::piece(W, G.rows_total, K, row, k0, lg, p),
                      base + C::A_BYTES + ((c * NP + p) * NW + wave_s) * 1024);
        }
    };

    float16v acc[MT][1];
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[i][0][e] = 0.0f;
    auto compute = [&](int grp, int st) __attribute__((always_inline)) {
        const uint8_t * base = smem + st * C::STAGE;
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const int cc = grp * CH + c;
            u32x4 pc[NP];
#pragma unroll
            for (int p = 0; p < NP; p++)
                pc[p] = *(const u32x4 *)(base + C::A_BYTES + ((c * NP + p) * NW + wave) * 1024 + 16 * lane);
            WLoad<WT> w;
            P::item(w, pc, G.rows_total, K, row, (int64_t)min(cc, nchunks - 1) * 64, lg,
                    okn && cc < nchunks && (WT != T_Q8_0 || (int64_t)cc * 64 + 32 * lg < K));
            u32x4 b[4];
            int run0, run1;
            w.decode_fast(lg, b, run0, run1);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int ch = 8 * c + (q < 2 ? run0 + 8 * q : run1 + 8 * (q - 2)) / 8;   // slice chunk
                const half8 bf = __builtin_bit_cast(half8, b[q]);
#pragma unroll
                for (int i = 0; i < MT; i++) {
                    const int r = 32 * i + lr;
                    const half8 af = *(const half8 *)(base + (r * CPR + (ch ^ (r & 7))) * 16);
                    acc[i][0] = mfma32(af, bf, acc[i][0]);
                }
            }
        }
    };

    if (gn > 0) {
#pragma unroll
        for (int q = 0; q < NS - 1; q++) issue(gb + q, q);
        // step j: group gb + j from stage j % NS; the DMA of group gb + j + NS - 1 into the stage
        // group gb + j - 1 used. Unrolled by NS so the register ring's indices are constants.
        auto step = [&](int j, auto Sc) __attribute__((always_inline)) {
            constexpr int S = decltype(Sc)::value;
            wait_vm_lgkm0<(NS - 2) * C::PER>();
            __builtin_amdgcn_s_barrier();
            issue(gb + j + NS - 1, (S + NS - 1) % NS);
            compute(gb + j, S);
        };
        int j = 0;
        for (; j + NS <= gn; j += NS) {
            step(j, std::integral_constant<int, 0>());
            step(j + 1, std::integral_constant<int, 1>());
            if constexpr (NS > 2) step(j + 2, std::integral_constant<int, 2 % NS>());
            if constexpr (NS > 3) step(j + 3, std::integral_constant<int, 3 % NS>());
        }
        const int left = gn - j;
        if (left > 0) step(j, std::integral_constant<int, 0>());
        if (left > 1) step(j + 1, std::integral_constant<int, 1 % NS>());
        if constexpr (NS > 2) if (left > 2) step(j + 2, std::integral_constant<int, 2 % NS>());
        wait_vm_lgkm0<0>();   // no DMA may still be writing this block's LDS when it exits
    }

    scale_rows(acc, args.scales, 0, lg, args.M);
    if (!okn || gn == 0) return;
#pragma unroll
    for (int i = 0; i < MT; i++) {
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int r = i * 32 + 8 * (e / 4) + 4 * lg + (e % 4);
            if (r >= args.M) continue;
            float * p = G.C + (int64_t)r * G.ldc + n;
            if (ks == 1 || args.part) *p = acc[i][0][e];
            else unsafeAtomicAdd(p, acc[i][0][e]);
        }
    }
}

// The K-split partials summed in split order, C_g[r][n] = P[0][r][pcol_g + n] + P[1][..] + ...:
// one thread per 4 columns of a partial row (every group's N and pcol are multiples of 16).
__global__ void __launch_bounds__(256) reduce_splits_kernel(GemmArgs a, int ks) {
    const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t per_row = a.ldp / 4;
    if (q >= (int64_t)a.M * per_row) return;
    const int64_t r = q / per_row, c = 4 * (q % per_row);
    int g = 0;
#pragma unroll
    for (int i = 1; i < GEMM_MAX_GROUPS; i++)
        if (i < a.ng && c >= a.g[i].pcol) g = i;
    float * C = a.g[0].C;
    int64_t ldc = a.g[0].ldc, pcol = a.g[0].pcol;
#pragma unroll
    for (int i = 1; i < GEMM_MAX_GROUPS; i++)
        if (i == g) { C = a.g[i].C; ldc = a.g[i].ldc; pcol = a.g[i].pcol; }
    const int64_t slab = (int64_t)a.M * a.ldp;
    const float * p = a.part + r * a.ldp + c;
    float4v s = *(const float4v *)p;
    // loads in batches of 8 (all in flight at once), added in split order
    for (int k0 = 1; k0 < ks; k0 += 8) {
        float4v v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = k0 + j < ks ? *(const float4v *)(p + (k0 + j) * slab) : float4v{0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (k0 + j < ks)
#pragma unroll
                for (int e = 0; e < 4; e++) s[e] += v[j][e];
    }
    float * o = C + r * ldc + (c - pcol);
    if ((reinterpret_cast<uintptr_t>(o) & 15) == 0) {
        *(float4v *)o = s;
    } else {
#pragma unroll
        for (int e = 0; e < 4; e++) o[e] = s[e];
    }
}

__global__ void __launch_bounds__(256) zero_rows_kernel(GemmArgs args) {
    const GemmGroup & G = args.g[blockIdx.y];
    float * row = G.C + (int64_t)blockIdx.x * G.ldc;
    const int N = G.N;
    int c0 = 0;
    if ((reinterpret_cast<uintptr_t>(row) & 15) == 0) {
        for (int c = 4 * threadIdx.x; c + 3 < N; c += 4 * blockDim.x) *(float4v *)(row + c) = float4v{0, 0, 0, 0};
        c0 = N & ~3;
    }
    for (int c = c0 + threadIdx.x; c < N; c += blockDim.x) row[c] = 0.0f;
}

// ---------------------------------------------------------------------------------------------
// dequant to fp16 and the weight re-layout
// ---------------------------------------------------------------------------------------------

// One thread per (row, 32-value half of a 64-wide slab): the same decoders the GEMM uses.
// TL: write the tiled layout (tiled_index); every 16-value run stays inside one 32-wide slab.
template <int WT, bool TL>
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
    if (TL) {
        *(u32x4 *)(out + tiled_index(row, k0 + run0, K)) = o[0];
        *(u32x4 *)(out + tiled_index(row, k0 + run0 + 8, K)) = o[1];
        *(u32x4 *)(out + tiled_index(row, k0 + run1, K)) = o[2];
        *(u32x4 *)(out + tiled_index(row, k0 + run1 + 8, K)) = o[3];
        return;
    }
    uint16_t * d = out + row * K + k0;
    *(u32x4 *)(d + run0) = o[0];
    *(u32x4 *)(d + run0 + 8) = o[1];
    *(u32x4 *)(d + run1) = o[2];
    *(u32x4 *)(d + run1 + 8) = o[3];
}

// F32 or BF16 values -> fp16 (round to nearest even): the resident form of an F32 / BF16 weight,
// as rocket_weight_to_fp16 makes it (ggml-rocket.cpp:3855-3890).
__global__ void convert_f16_kernel(int type, const void * __restrict__ src, int64_t n, uint16_t * __restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float f;
    if (type == T_F32) f = ((const float *)src)[i];
    else f = __builtin_bit_cast(float, (uint32_t)((const uint16_t *)src)[i] << 16);
    dst[i] = f2h_bits(f);
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

// ggml MXFP4 -> split planes. One thread per 17-byte block.
__global__ void pack_mxfp4_kernel(const uint8_t * __restrict__ src, int64_t rows, int64_t K,
                                  uint8_t * __restrict__ dst) {
    const int64_t nb = K / 32;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * nb) return;
    const int64_t row = i / nb, b = i % nb;
    const uint8_t * s = src + i * 17;
    uint8_t * qs = dst + row * (K / 2) + b * 16;
    for (int l = 0; l < 16; l++) qs[l] = s[1 + l];
    dst[rows * (K / 2) + row * nb + b] = s[0];
}

// ggml Q4_0 -> split planes. One thread per block.
__global__ void pack_q4_0_kernel(const uint8_t * __restrict__ src, int64_t rows, int64_t K,
                                 uint8_t * __restrict__ dst) {
    const int64_t nb = K / 32;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * nb) return;
    const int64_t row = i / nb, b = i % nb;
    const uint8_t * s = src + i * 18;
    uint8_t * qs = dst + row * (K / 2) + b * 16;
    for (int l = 0; l < 16; l++) qs[l] = s[2 + l];
    uint8_t * d = dst + rows * (K / 2) + (row * nb + b) * 2;
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
                           float * scales, hipStream_t st, float * zc, int64_t ldzc, int zn) {
    if (M <= 0) return hipSuccess;
    constexpr int RPB = PACK_THREADS / WAVE;   // rows a block of the wave form
    if (K <= pack_wave_k())
        hipLaunchKernelGGL(pack_act_wave_kernel<false>, dim3((M + RPB - 1) / RPB), dim3(PACK_THREADS), 0, st, X, ldx,
                           M, K, A16, lda, scales, zc, ldzc, zn);
    else
        hipLaunchKernelGGL(pack_act_kernel<false>, dim3(M), dim3(PACK_THREADS), 0, st, X, ldx, M, K, A16, lda, scales,
                           zc, ldzc, zn);
    return hipGetLastError();
}

hipError_t launch_pack_act_tiled(const float * X, int64_t ldx, int M, int K, uint16_t * A16, float * scales,
                                 hipStream_t st, float * zc, int64_t ldzc, int zn) {
    if (M <= 0) return hipSuccess;
    constexpr int RPB = PACK_THREADS / WAVE;
    if (K <= pack_wave_k())
        hipLaunchKernelGGL(pack_act_wave_kernel<true>, dim3((M + RPB - 1) / RPB), dim3(PACK_THREADS), 0, st, X, ldx,
                           M, K, A16, (int64_t)K, scales, zc, ldzc, zn);
    else
        hipLaunchKernelGGL(pack_act_kernel<true>, dim3(M), dim3(PACK_THREADS), 0, st, X, ldx, M, K, A16, (int64_t)K,
                           scales, zc, ldzc, zn);
    return hipGetLastError();
}

// Tile configurations. The launcher picks one per call (choose_cfg); MI355X_GEMM_CFG=<id>
// forces one (for tuning and for the tests, which run every configuration).
//   0-3  register-staged kernel with the weight decoded into LDS: every weight type.
//   4-15 LDS-DMA kernel: fp16 weights only (row-major or tiled); 15 has wave columns of two
//        widths (gemm_f16_cols_kernel), 21 and 22 are that tile with 32-deep stages, three or
//        four of them in flight where 15 has one of 64 (the 256 x 224 tile's DMA waits are
//        what bounds it); 23 and 24 are 8 and 14 with eight 32-deep stages.
//   16-19 Q4_K with every operand by DMA (gemm_q4k_kernel), K % 256 == 0; 18 and 19 split K
//        (q4k_split). 20 is the skinny kernel's id (use_skinny), not a tile configuration.
// choose_cfg prices a launch from two rates: a block's own pace, rounds * (ov_us + MFMA work
// of a block / tf_cu) (pipeline fill and epilogue, then its per-CU MFMA rate), and the
// aggregate rate at which the L2s feed the CUs for that tile shape, L2->CU bytes of all blocks
// / bw (bigger tiles fetch less per FLOP but keep fewer bytes in flight per CU). The two
// overlap, so the estimate is their 4-norm (pace^4 + feed^4)^(1/4), which follows the measured
// transition between the regimes better than the max; a split-K launch adds zc microseconds per
// MB of output (the zero fill and the second addend's atomics). The four were fitted per
// configuration to measurements on tiled weights at M = 128-2048, N = 1024-28672,
// K = 2880-14336, each launch on a weight panel no earlier launch left in the caches: mean
// error 2-9% per configuration, and over 50 shapes the chosen configurations cost 0.6% more
// than the best measured ones.
enum CfgKind { REG = 0, DMA = 1, Q4KDMA = 2, NONE = 3 };
struct CfgDesc {
    int kind;        // REG: gemm_kernel, DMA: gemm_f16_kernel / _cols, Q4KDMA: gemm_q4k_kernel
    int bm, bn, ksplit;
    int dk;          // K per LDS stage (0 for the register-staged kernel)
    double tf_cu;    // TFLOP/s per CU
    double ov_us;    // fixed microseconds per block
    double bw;       // aggregate L2 -> CU TB/s
    double zc;       // split-K: microseconds per MB of output
};
static constexpr CfgDesc kCfgs[] = {
    {REG, 128, 128, 1, 0, 0.0, 0.0, 0.0, 0.0},        // 0: 4 waves of 64x64
    {REG, 128, 128, 2, 0, 0.0, 0.0, 0.0, 0.0},        // 1: same, K split (launcher-sized, >= 2)
    {REG, 256, 128, 1, 0, 0.0, 0.0, 0.0, 0.0},        // 2: 4 waves of 128x64
    {REG, 128, 256, 1, 0, 0.0, 0.0, 0.0, 0.0},        // 3: 4 waves of 64x128
    {DMA, 256, 256, 1, 64, 6.30, 6.0, 8.05, 0.00},   // 4: 8 waves of 64x128, 2 stages of 64
    {DMA, 128, 128, 1, 64, 4.03, 0.0, 13.00, 0.00},  // 5: 8 waves of 32x64, 4 stages of 64
    {DMA, 64, 128, 1, 128, 2.75, 5.0, 16.32, 0.00},  // 6: 4 waves of 32x64, 3 stages of 128
    {DMA, 128, 64, 1, 128, 2.92, 5.9, 16.88, 0.00},  // 7: 4 waves of 64x32, 3 stages of 128
    {DMA, 128, 128, 2, 64, 3.52, 0.0, 25.17, 1.76},  // 8: as 5, K split in two
    {DMA, 64, 128, 2, 128, 2.50, 6.3, 40.00, 0.69},  // 9: as 6, K split in two
    {DMA, 128, 128, 1, 32, 4.43, 0.0, 13.05, 0.00},  // 10: 8 waves of 32x64, 4 stages of 32 (any K)
    {DMA, 128, 128, 1, 32, 4.35, 0.0, 13.10, 0.00},  // 11: 8 waves of 32x64, 8 stages of 32
    {DMA, 256, 128, 1, 64, 5.62, 8.6, 10.70, 0.00},  // 12: 8 waves of 64x64, 3 stages of 64
    {DMA, 128, 256, 1, 64, 5.33, 6.9, 10.85, 0.00},  // 13: 8 waves of 64x64, 3 stages of 64
    {DMA, 64, 128, 1, 64, 2.60, 2.3, 17.23, 0.00},   // 14: 4 waves of 32x64, 6 stages of 64
    {DMA, 256, 224, 1, 64, 5.70, 0.0, 8.88, 0.00},   // 15: 8 waves of 64x128 and 64x96, 2 stages of 64
    {Q4KDMA, 256, 256, 1, 64, 0.0, 0.0, 0.0, 0.0}, // 16: Q4_K by DMA, 8 waves of 64x128
    {Q4KDMA, 128, 256, 1, 64, 0.0, 0.0, 0.0, 0.0}, // 17: Q4_K by DMA, 8 waves of 64x64
    {Q4KDMA, 256, 256, 2, 64, 0.0, 0.0, 0.0, 0.0}, // 18: as 16, K split (launcher-sized, >= 2)
    {Q4KDMA, 128, 256, 2, 64, 0.0, 0.0, 0.0, 0.0}, // 19: as 17, K split (launcher-sized, >= 2)
    {NONE, 0, 0, 1, 0, 0.0, 0.0, 0.0, 0.0},        // 20: the skinny kernel (not a tile configuration)
    {DMA, 256, 224, 1, 32, 7.07, 10.7, 9.00, 0.00},   // 21: as 15, 4 stages of 32
    {DMA, 256, 224, 1, 32, 6.78, 10.1, 8.73, 0.00},   // 22: as 15, 5 stages of 32
    {DMA, 128, 128, 2, 32, 3.59, 0.0, 17.89, 1.65},   // 23: as 8, 8 stages of 32
    {DMA, 64, 128, 1, 32, 2.70, 1.4, 17.12, 0.00},    // 24: as 14, 8 stages of 32
};
constexpr int FIRST_DMA_CFG = 4;
constexpr int N_CFGS = sizeof(kCfgs) / sizeof(kCfgs[0]);

template <int WT, int BM, int BN, int WM, int WN, int R, int KS>
static hipError_t launch_one(const GemmArgs & a, int nblocks, hipStream_t st) {
    using C = GemmCfg<BM, BN, WM, WN, R>;
    auto kern = gemm_kernel<WT, BM, BN, WM, WN, R, KS>;
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS);
        if (e != hipSuccess) return e;
        attr = true;
    }
    hipLaunchKernelGGL(kern, dim3(nblocks), dim3(GEMM_THREADS), C::LDS, st, a);
    return hipGetLastError();
}

template <int BM, int BN, int WGM, int WGN, int DK, int NS, int KS, bool TL>
static hipError_t launch_f16(const GemmArgs & a, int nblocks, hipStream_t st) {
    using C = F16Cfg<BM, BN, WGM, WGN, DK, NS>;
    auto kern = gemm_f16_kernel<BM, BN, WGM, WGN, DK, NS, KS, TL>;
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS);
        if (e != hipSuccess) return e;
        attr = true;
    }
    hipLaunchKernelGGL(kern, dim3(nblocks), dim3(C::THREADS), C::LDS, st, a);
    return hipGetLastError();
}

template <int BM, int BN0, int BN1, int DK, int NS, bool TL>
static hipError_t launch_cols(const GemmArgs & a, int nblocks, hipStream_t st) {
    using C = ColsCfg<BM, BN0, BN1, DK, NS>;
    auto kern = gemm_f16_cols_kernel<BM, BN0, BN1, DK, NS, TL>;
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS);
        if (e != hipSuccess) return e;
        attr = true;
    }
    hipLaunchKernelGGL(kern, dim3(nblocks), dim3(C::THREADS), C::LDS, st, a);
    return hipGetLastError();
}

template <int WT, int BM, int WGM, int WGN>
static hipError_t launch_q4k(const GemmArgs & a, int nblocks, hipStream_t st) {
    using C = Q4kCfg<WT, BM, WGM, WGN>;
    auto kern = gemm_q4k_kernel<WT, BM, WGM, WGN>;
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS);
        if (e != hipSuccess) return e;
        attr = true;
    }
    hipLaunchKernelGGL(kern, dim3(nblocks), dim3(C::THREADS), C::LDS, st, a);
    return hipGetLastError();
}

template <bool TL>
static hipError_t launch_dma_cfg(int cfg, const GemmArgs & a, int nblocks, hipStream_t st) {
    switch (cfg) {
        case 15: return launch_cols<256, 128, 96, 64, 2, TL>(a, nblocks, st);
        case 21: return launch_cols<256, 128, 96, 32, 4, TL>(a, nblocks, st);
        case 22: return launch_cols<256, 128, 96, 32, 5, TL>(a, nblocks, st);
        case 23: return launch_f16<128, 128, 4, 2, 32, 8, 2, TL>(a, nblocks, st);
        case 24: return launch_f16<64, 128, 2, 2, 32, 8, 1, TL>(a, nblocks, st);
        case 4: return launch_f16<256, 256, 4, 2, 64, 2, 1, TL>(a, nblocks, st);
        case 5: return launch_f16<128, 128, 4, 2, 64, 4, 1, TL>(a, nblocks, st);
        case 6: return launch_f16<64, 128, 2, 2, 128, 3, 1, TL>(a, nblocks, st);
        case 7: return launch_f16<128, 64, 2, 2, 128, 3, 1, TL>(a, nblocks, st);
        case 8: return launch_f16<128, 128, 4, 2, 64, 4, 2, TL>(a, nblocks, st);
        case 9: return launch_f16<64, 128, 2, 2, 128, 3, 2, TL>(a, nblocks, st);
        case 10: return launch_f16<128, 128, 4, 2, 32, 4, 1, TL>(a, nblocks, st);
        case 11: return launch_f16<128, 128, 4, 2, 32, 8, 1, TL>(a, nblocks, st);
        case 12: return launch_f16<256, 128, 4, 2, 64, 3, 1, TL>(a, nblocks, st);
        case 13: return launch_f16<128, 256, 2, 4, 64, 3, 1, TL>(a, nblocks, st);
        case 14: return launch_f16<64, 128, 2, 2, 64, 6, 1, TL>(a, nblocks, st);
        default: return hipErrorInvalidValue;
    }
}

template <int WT>
static hipError_t launch_cfg(int cfg, const GemmArgs & a, int nblocks, hipStream_t st) {
    if (kCfgs[cfg].kind == Q4KDMA) {
        if constexpr (WT == T_Q4_K) {
            switch (cfg) {
                case 16: case 18: return launch_q4k<T_Q4_K, 256, 4, 2>(a, nblocks, st);
                case 17: case 19: return launch_q4k<T_Q4_K, 128, 2, 4>(a, nblocks, st);
                default: return hipErrorInvalidValue;
            }
        } else if constexpr (WT == T_Q8_0) {
            switch (cfg) {
                case 17: case 19: return launch_q4k<T_Q8_0, 128, 2, 4>(a, nblocks, st);
                default: return hipErrorInvalidValue;
            }
        } else {
            return hipErrorInvalidValue;
        }
    }
    if (kCfgs[cfg].kind == DMA) {
        if (WT != T_F16 && WT != T_F16T) return hipErrorInvalidValue;
        return launch_dma_cfg<WT == T_F16T>(cfg, a, nblocks, st);
    }
    if constexpr (WT == T_F16T) return hipErrorInvalidValue;
    else switch (cfg) {
        case 0: return launch_one<WT, 128, 128, 2, 2, 2, 1>(a, nblocks, st);
        case 1: return launch_one<WT, 128, 128, 2, 2, 2, 0>(a, nblocks, st);   // split a.ksplit ways
        case 2: return launch_one<WT, 256, 128, 2, 2, 2, 1>(a, nblocks, st);
        case 3: return launch_one<WT, 128, 256, 2, 2, 2, 1>(a, nblocks, st);
        default: return hipErrorInvalidValue;
    }
}

static int cu_count() {
    static int n = 0;
    if (n == 0) {
        int dev = 0;
        hipDeviceProp_t p;
        n = (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&p, dev) == hipSuccess) ? p.multiProcessorCount : 256;
    }
    return n;
}

static int tiles_of(const GemmArgs & a, int bm, int bn) {
    int nt = 0;
    for (int i = 0; i < a.ng; i++) nt += (a.g[i].N + bn - 1) / bn;
    return nt * ((a.M + bm - 1) / bm);
}

static int64_t tiles_n_cols(const GemmArgs & a) {
    int64_t n = 0;
    for (int i = 0; i < a.ng; i++) n += a.g[i].N;
    return n;
}

// The K split of the register-staged split configuration (1). Fitted to the fastest split
// measured for Q4_K and Q8_0 at M 32-512, N 3072-14336, K 3072-8192 (1% over the best in
// total): ~6.65 K^0.75 / sqrt(M N). A wider output has more elements to add atomically per
// split, a deeper K more work to share. At least 2 ways, at most 16 and at least 4 K slabs per
// split. MI355X_GEMM_KSPLIT=<n> forces n (for tuning).
static double reg_split_est(const GemmArgs & a) {
    return 6.65 * std::pow((double)a.K, 0.75) / std::sqrt((double)a.M * (double)tiles_n_cols(a));
}
static int reg_split(const GemmArgs & a, int cap) {
    const int nk = (a.K + BK - 1) / BK;
    if (const char * e = getenv("MI355X_GEMM_KSPLIT")) {
        const int v = atoi(e);
        if (v >= 2 && v <= nk) return std::min(v, cap);
    }
    int ks = (int)std::lround(reg_split_est(a));
    const int most = std::min(nk / 4 < 16 ? nk / 4 : 16, cap);
    if (ks > most) ks = most;
    return ks < 2 ? 2 : ks;
}

// The K split of the Q4_K DMA split configurations (18, 19): about one block per CU, in whole
// Q4_K blocks of K, at least 2 ways and at least 2 blocks (8 stages) a split.
// MI355X_GEMM_KSPLIT=<n> forces n (for tuning).
static int q4k_split(const GemmArgs & a, int bm, int bn, int cap) {
    const int nsb = a.K / 256;
    const int most = std::min(std::max(2, nsb / 2), cap);
    int ks = 0;
    if (const char * e = getenv("MI355X_GEMM_KSPLIT")) ks = atoi(e);
    if (ks < 2) ks = (int)std::lround((double)cu_count() / tiles_of(a, bm, bn));
    ks = std::min(std::max(ks, 2), most);
    // equal splits of whole blocks: the count that leaves no split empty
    const int per = (nsb + ks - 1) / ks;
    return (nsb + per - 1) / per;
}

static bool cfg_fits(int c, int wt, int K) {
    const CfgDesc & d = kCfgs[c];
    if (d.kind == NONE) return false;
    if (d.kind == REG) return wt != T_F16T;
    if (d.kind == Q4KDMA) return (wt == T_Q4_K || (wt == T_Q8_0 && d.bm == 128)) && K % 256 == 0;
    if ((wt != T_F16 && wt != T_F16T) || K % d.dk) return false;
    return d.ksplit == 1 || K / d.dk >= 2;
}

// fp16 weights: the DMA configuration with the least estimated time (the CfgDesc model; every
// DMA block has a CU to itself, so a launch runs in ceil(blocks / CUs) rounds).
// Q4_K weights (K % 256 == 0): the all-DMA kernel where it fills the chip (below).
// Other weights: split K when the output is skinny for its depth (reg_split), otherwise the
// unsplit register-staged tile with the best grid fill times its relative per-CU efficiency
// (bigger wave tiles read LDS less per MFMA).
static int choose_cfg(int wt, const GemmArgs & a) {
    if (const char * e = getenv("MI355X_GEMM_CFG")) {
        if (*e) {
            const int c = atoi(e);
            if (c >= 0 && c < N_CFGS && cfg_fits(c, wt, a.K)) return c;
        }
    }
    const int cus = cu_count();
    if (wt == T_F16 || wt == T_F16T) {
        int best = -1;
        double best_us = 0.0;
        for (int c = FIRST_DMA_CFG; c < N_CFGS; c++) {
            if (kCfgs[c].kind != DMA || !cfg_fits(c, wt, a.K)) continue;
            const CfgDesc & d = kCfgs[c];
            // the model was fitted on tiled weights; on row-major ones a 32-deep stage reads half
            // cache lines per row (qkv at M 512: 496 against 613 TFLOP/s for 64-deep stages), so
            // it is left to the K % 64 != 0 shapes that nothing else takes
            if (wt == T_F16 && d.dk == 32 && a.K % 64 == 0) continue;
            const int blocks = tiles_of(a, d.bm, d.bn) * d.ksplit;
            const int rounds = (blocks + cus - 1) / cus;
            const double kb = (double)a.K / d.ksplit;
            const double pace = rounds * (d.ov_us + 2.0 * d.bm * d.bn * kb / (d.tf_cu * 1e6));
            const double feed = (double)blocks * (d.bm + d.bn) * kb * 2.0 / (d.bw * 1e6);
            const double p2 = pace * pace, f2 = feed * feed;
            double us = std::sqrt(std::sqrt(p2 * p2 + f2 * f2));
            if (d.ksplit > 1) us += d.zc * (double)a.M * tiles_n_cols(a) * 4.0 / 1e6;
            if (best < 0 || us < best_us - 1e-9) { best = c; best_us = us; }
        }
        if (best >= 0) return best;
    }
    // Q4_K with whole blocks: the all-DMA kernel where its tiles fill the chip in one round or
    // more (a 256 x 256 block runs a 64-deep stage in about 2.2 us, a 128 x 256 one in 1.3 us),
    // and its K split where K is deep for the output width. Measured on Q4_K at M 256-2048 for
    // the four projections of an 8B model (qkv 6144 x 4096, o 4096 x 4096, gate/up 28672 x 4096,
    // down 4096 x 14336), these picks are the fastest configuration or within 4% of it, and
    // 1.2-1.4x faster than the register-staged kernel where they apply.
    if (wt == T_Q4_K && a.K % 256 == 0) {
        const int fill = (cus * 7 + 9) / 10;
        if ((int64_t)a.K >= 2 * tiles_n_cols(a)) return a.M <= 1024 ? 19 : 18;
        if (tiles_of(a, 256, 256) >= fill) return 16;
        if (tiles_of(a, 128, 256) >= fill) return 17;
    }
    // Q8_0 with whole blocks: the all-DMA kernel on its 128 x 256 tiles, K split where K is deep
    // for the output width or the tiles fill less than half the chip. Measured at M 512 and 2048
    // for N x K in {3072, 8192} x {3072, 8192} and the 8B shapes 14336 x 4096 / 4096 x 14336, the
    // pick is the faster of the two, and 1.1-1.6x faster than the register-staged kernel.
    if (wt == T_Q8_0 && a.K % 256 == 0) {
        const int fill = (cus * 7 + 9) / 10;
        if (((int64_t)a.K >= 2 * tiles_n_cols(a) && a.M <= 1024) || tiles_of(a, 128, 256) < fill / 2) return 19;
        return 17;
    }
    // a skinny output: split K (see reg_split); otherwise the unsplit tile with the best fill
    if (reg_split_est(a) >= 1.5 && (a.K / BK) >= 8) return 1;
    const double tile_eff[FIRST_DMA_CFG] = {1.0, 0.97, 1.25, 1.25};
    int best = 0;
    double best_score = -1.0;
    for (int c = 0; c < FIRST_DMA_CFG; c++) {
        if (kCfgs[c].ksplit > 1) continue;
        const int tiles = tiles_of(a, kCfgs[c].bm, kCfgs[c].bn);
        const int blocks = tiles * kCfgs[c].ksplit;
        const int waves = (blocks + cus - 1) / cus;
        const double fill = (double)blocks / ((double)waves * cus);
        const double score = fill * tile_eff[c];
        if (score > best_score + 1e-9) { best_score = score; best = c; }
    }
    return best;
}

__global__ void zero_rows_kernel(GemmArgs args);

// The skinny kernel (configuration 20 for MI355X_GEMM_CFG): every weight format but the tiled
// fp16 one, M <= SK_MAX_M. Chunk depth CH by M tiles (LDS 32 KB per block, double-buffered). The
// K split aims at ~240 blocks, about one per CU: fewer leave weight bytes unrequested, more add
// atomic traffic (the fastest splits measured for Q4_K / Q8_0 at M 32-128, N 3072-14336,
// K 3072-14336 launch 144-256 blocks).
constexpr int SKINNY_CFG = 20;
static_assert(kCfgs[SKINNY_CFG].kind == NONE, "the skinny kernel's id");

// Row-major fp16 weights also have the DMA kernels: past M = 32 those win unless K is deep for
// the output width (measured at M 32-128; at M 128, K 14336 x N 4096: 50 us skinny, 60 us DMA;
// N 14336 x K 4096: 51 us skinny, 44 us DMA).
static bool use_skinny(int wt, const GemmArgs & a) {
    if (wt == T_F16T || a.M > SK_MAX_M) return false;
    if (const char * e = getenv("MI355X_GEMM_CFG"))
        if (*e) return atoi(e) == SKINNY_CFG;
    if (wt == T_F16 && a.M > 32 && (int64_t)a.K < 2 * tiles_n_cols(a)) return false;
    return true;
}

static int skinny_ch(int M) { return M <= 64 ? 4 : 2; }

// The LDS-DMA skinny kernel (Q4_K, Q8_0, Q6_K): chunk depth CH and ring depth NS per weight type
// and 32-row M tile, the deepest ring of whole groups that fits in LDS (MI355X_SKINNY_DMA=0
// selects the register-staged kernel, for comparison).
// Where it is faster (measured at N 3072-8192, K 3072-8192 on MI355X): Q6_K at every M (M 128:
// 39.4 against 43.2 us at 8192 x 3072) and Q8_0 past 64 rows; Q4_K, and Q8_0 up to 64 rows, keep
// the register kernel, which is as fast or faster there (Q4_K M 32: 19.1 against 21.8 us), being
// bound by its decode and address VALU work rather than by the weight bytes in flight.
// MI355X_SKINNY_DMA=1 forces this kernel for the three types, 0 the register one (tests).
// The scale chunks it reads stay inside their planes when every panel's row count is a multiple
// of 16 (the planes then span whole 16-byte chunks); other panels take the register kernel.
static bool skinny_dma(int wt, const GemmArgs & a) {
    if (!(wt == T_Q4_K || wt == T_Q8_0 || wt == T_Q6_K)) return false;
    const char * e = getenv("MI355X_SKINNY_DMA");
    const int force = (e && *e) ? atoi(e) : -1;
    if (force == 0) return false;
    if (force < 0 && !(wt == T_Q6_K || (wt == T_Q8_0 && a.M > 64))) return false;
    for (int i = 0; i < a.ng; i++)
        if (a.g[i].rows_total % 16 != 0) return false;
    return true;
}
static int skinny_dma_ch(int wt, int M) {
    const int mt = (M + 31) / 32;
    if (wt == T_Q6_K) return mt <= 1 ? 2 : 1;
    if (wt == T_Q8_0) return mt <= 2 ? 2 : 1;
    return mt <= 1 ? 4 : 2;
}
static int skinny_chunk_depth(int wt, const GemmArgs & a) {
    return skinny_dma(wt, a) ? skinny_dma_ch(wt, a.M) : skinny_ch(a.M);
}

template <int WT, int MT, int CH, int NS>
static hipError_t launch_skinny_dma1(const GemmArgs & a, int nblocks, int gpb, hipStream_t st) {
    using C = SkDmaCfg<WT, MT, CH, NS>;
    auto kern = gemm_skinny_dma_kernel<WT, MT, CH, NS>;
    static bool attr = false;
    if (!attr) {
        const hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS);
        if (e != hipSuccess) return e;
        attr = true;
    }
    hipLaunchKernelGGL(kern, dim3(nblocks), dim3(C::THREADS), C::LDS, st, a, gpb);
    return hipGetLastError();
}

template <int WT>
static hipError_t launch_skinny_dma(const GemmArgs & a, int nblocks, int gpb, hipStream_t st) {
    const int mt = (a.M + 31) / 32;
    if constexpr (WT == T_Q6_K) {
        if (mt == 1) return launch_skinny_dma1<WT, 1, 2, 3>(a, nblocks, gpb, st);
        if (mt == 2) return launch_skinny_dma1<WT, 2, 1, 4>(a, nblocks, gpb, st);
        return launch_skinny_dma1<WT, 4, 1, 4>(a, nblocks, gpb, st);
    } else if constexpr (WT == T_Q8_0) {
        if (mt == 1) return launch_skinny_dma1<WT, 1, 2, 4>(a, nblocks, gpb, st);
        if (mt == 2) return launch_skinny_dma1<WT, 2, 2, 3>(a, nblocks, gpb, st);
        return launch_skinny_dma1<WT, 4, 1, 4>(a, nblocks, gpb, st);
    } else {
        if (mt == 1) return launch_skinny_dma1<WT, 1, 4, 3>(a, nblocks, gpb, st);
        if (mt == 2) return launch_skinny_dma1<WT, 2, 2, 4>(a, nblocks, gpb, st);
        return launch_skinny_dma1<WT, 4, 2, 3>(a, nblocks, gpb, st);
    }
}

static int skinny_ntiles(const GemmArgs & a) {
    int nt = 0;
    for (int i = 0; i < a.ng; i++) nt += (a.g[i].N + 32 * SK_NW - 1) / (32 * SK_NW);
    return nt;
}

// K groups per block (the split count is ceil(groups / that)), at most `cap` splits
static int skinny_gpb(int wt, const GemmArgs & a, int cap) {
    const int ch = skinny_chunk_depth(wt, a);
    const int ngroups = ((a.K + 63) / 64 + ch - 1) / ch;
    double blocks = 240.0;
    if (const char * e = getenv("MI355X_SKINNY_BLOCKS")) {   // tuning override
        const int v = atoi(e);
        if (v > 0) blocks = v;
    }
    const double target = blocks / skinny_ntiles(a);
    const int ks = std::min(std::max(1, (int)std::lround(target)), cap);
    return (ngroups + ks - 1) / ks;
}

template <int WT>
static hipError_t launch_skinny(const GemmArgs & a, int nblocks, int gpb, hipStream_t st) {
    const int mt = (a.M + 31) / 32;
    if (mt == 1) hipLaunchKernelGGL((gemm_skinny_kernel<WT, 1, 4>), dim3(nblocks), dim3(SK_NW * WAVE), 0, st, a, gpb);
    else if (mt == 2) hipLaunchKernelGGL((gemm_skinny_kernel<WT, 2, 4>), dim3(nblocks), dim3(SK_NW * WAVE), 0, st, a, gpb);
    else hipLaunchKernelGGL((gemm_skinny_kernel<WT, 4, 2>), dim3(nblocks), dim3(SK_NW * WAVE), 0, st, a, gpb);
    return hipGetLastError();
}

// A launch's configuration and K split. The split is at most `cap` ways: the number of partial
// slabs [M][sum of N] the caller's workspace holds, and at least 2.
struct GemmPlan {
    bool skinny;
    int cfg;    // kCfgs index (unused for the skinny kernel)
    int ks;     // K split
    int gpb;    // skinny kernel: K groups per block
};

static int64_t total_cols(const GemmArgs & a) {
    int64_t n = 0;
    for (int i = 0; i < a.ng; i++) n += a.g[i].N;
    return n;
}

static int split_cap(const GemmArgs & a, size_t part_bytes) {
    const size_t slab = (size_t)a.M * (size_t)total_cols(a) * sizeof(float);
    const size_t n = slab ? part_bytes / slab : 0;
    return (int)std::max<size_t>(2, std::min<size_t>(n, 64));
}

static GemmPlan plan_gemm(int wt, const GemmArgs & a, int cap) {
    GemmPlan p{};
    if (use_skinny(wt, a)) {
        p.skinny = true;
        p.cfg = SKINNY_CFG;
        p.gpb = skinny_gpb(wt, a, cap);
        const int ch = skinny_chunk_depth(wt, a);
        const int ngroups = ((a.K + 63) / 64 + ch - 1) / ch;
        p.ks = (ngroups + p.gpb - 1) / p.gpb;
        return p;
    }
    p.cfg = choose_cfg(wt, a);
    const CfgDesc & d = kCfgs[p.cfg];
    p.ks = p.cfg == 1 ? reg_split(a, cap)
         : (d.kind == Q4KDMA && d.ksplit > 1) ? q4k_split(a, d.bm, d.bn, cap) : d.ksplit;
    return p;
}

// Q8_0 at M < 1024 with whole 256-value blocks runs the all-DMA kernel (choose_cfg) faster than
// the decode-first form (the whole weight decoded to tiled fp16, then the fp16 GEMM) except where
// N >= K, the weight has more than 2^24 values and its 128 x 256 tiles leave more than 30% of the
// chip idle (8192 x 3072 at M 512: 71.2 against 66.0 us); at M >= 1024 the decode-first form is
// as fast or faster (its weight decoded once, against once per 128-row M tile), e.g. 14336 x 4096
// at M 2048: 296 against 366 us.
bool q8_0_decode_first(int64_t M, int64_t N, int64_t K) {
    if (M >= 1024) return true;
    if (K % 256) return N >= K;
    const int64_t tiles = ((M + 127) / 128) * ((N + 255) / 256);
    return N >= K && N * K > ((int64_t)1 << 24) && tiles < (cu_count() * 7 + 9) / 10;
}

size_t gemm_split_bytes(int wt, const GemmArgs & a) {
    const GemmPlan p = plan_gemm(wt, a, 64);
    return p.ks > 2 ? (size_t)p.ks * (size_t)a.M * (size_t)total_cols(a) * sizeof(float) : 0;
}

bool gemm_accumulates(int wt, const GemmArgs & a, size_t part_bytes) {
    return plan_gemm(wt, a, split_cap(a, part_bytes)).ks == 2;
}

hipError_t launch_gemm(int wt, const GemmArgs & a_in, int /*unused*/, hipStream_t st, bool c_zeroed, float * part,
                       size_t part_bytes) {
    GemmArgs a = a_in;
    const GemmPlan p = plan_gemm(wt, a, part ? split_cap(a, part_bytes) : 2);
    const int bn = p.skinny ? 32 * SK_NW : kCfgs[p.cfg].bn;
    int nt = 0;
    int64_t pcol = 0;
    for (int i = 0; i < a.ng; i++) {
        a.g[i].ntile_begin = nt;
        nt += (a.g[i].N + bn - 1) / bn;
        a.g[i].pcol = pcol;
        pcol += a.g[i].N;
    }
    a.m_tiles = p.skinny ? 1 : (a.M + kCfgs[p.cfg].bm - 1) / kCfgs[p.cfg].bm;
    a.ksplit = p.ks;
    a.part = p.ks > 2 ? part : nullptr;
    a.ldp = pcol;
    const int nblocks = nt * a.m_tiles * a.ksplit;
    if (nblocks <= 0) return hipSuccess;
    if (p.ks == 2 && !c_zeroed) {
        hipLaunchKernelGGL(zero_rows_kernel, dim3(a.M, a.ng), dim3(256), 0, st, a);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    hipError_t e = hipErrorInvalidValue;
    if (p.skinny) {
        switch (wt) {
            case T_F16: e = launch_skinny<T_F16>(a, nblocks, p.gpb, st); break;
            case T_Q8_0: e = skinny_dma(wt, a) ? launch_skinny_dma<T_Q8_0>(a, nblocks, p.gpb, st)
                                            : launch_skinny<T_Q8_0>(a, nblocks, p.gpb, st); break;
            case T_Q4_0: e = launch_skinny<T_Q4_0>(a, nblocks, p.gpb, st); break;
            case T_Q4_K: e = skinny_dma(wt, a) ? launch_skinny_dma<T_Q4_K>(a, nblocks, p.gpb, st)
                                            : launch_skinny<T_Q4_K>(a, nblocks, p.gpb, st); break;
            case T_Q5_K: e = launch_skinny<T_Q5_K>(a, nblocks, p.gpb, st); break;
            case T_Q6_K: e = skinny_dma(wt, a) ? launch_skinny_dma<T_Q6_K>(a, nblocks, p.gpb, st)
                                            : launch_skinny<T_Q6_K>(a, nblocks, p.gpb, st); break;
            case T_MXFP4: e = launch_skinny<T_MXFP4>(a, nblocks, p.gpb, st); break;
            default: break;
        }
    } else {
        switch (wt) {
            case T_F16: e = launch_cfg<T_F16>(p.cfg, a, nblocks, st); break;
            case T_F16T: e = launch_cfg<T_F16T>(p.cfg, a, nblocks, st); break;
            case T_Q8_0: e = launch_cfg<T_Q8_0>(p.cfg, a, nblocks, st); break;
            case T_Q4_0: e = launch_cfg<T_Q4_0>(p.cfg, a, nblocks, st); break;
            case T_Q4_K: e = launch_cfg<T_Q4_K>(p.cfg, a, nblocks, st); break;
            case T_Q5_K: e = launch_cfg<T_Q5_K>(p.cfg, a, nblocks, st); break;
            case T_Q6_K: e = launch_cfg<T_Q6_K>(p.cfg, a, nblocks, st); break;
            case T_MXFP4: e = launch_cfg<T_MXFP4>(p.cfg, a, nblocks, st); break;
            default: break;
        }
    }
    if (e != hipSuccess || !a.part) return e;
    const int64_t threads = (int64_t)a.M * (a.ldp / 4);
    hipLaunchKernelGGL(reduce_splits_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, a, a.ksplit);
    return hipGetLastError();
}

template <bool TL>
static hipError_t launch_dequant(int wt, const void * W, int64_t rows, int64_t K, uint16_t * out, hipStream_t st) {
    const int64_t items = rows * (K / 32);
    if (items <= 0) return hipSuccess;
    const dim3 grid((unsigned)((items + 255) / 256));
    const uint8_t * w = (const uint8_t *)W;
    switch (wt) {
        case T_F16: hipLaunchKernelGGL((dequant_f16_kernel<T_F16, TL>), grid, dim3(256), 0, st, w, rows, K, out); break;
        case T_Q8_0: hipLaunchKernelGGL((dequant_f16_kernel<T_Q8_0, TL>), grid, dim3(256), 0, st, w, rows, K, out); break;
        case T_Q4_0: hipLaunchKernelGGL((dequant_f16_kernel<T_Q4_0, TL>), grid, dim3(256), 0, st, w, rows, K, out); break;
        case T_Q4_K: hipLaunchKernelGGL((dequant_f16_kernel<T_Q4_K, TL>), grid, dim3(256), 0, st, w, rows, K, out); break;
        case T_Q5_K: hipLaunchKernelGGL((dequant_f16_kernel<T_Q5_K, TL>), grid, dim3(256), 0, st, w, rows, K, out); break;
        case T_Q6_K: hipLaunchKernelGGL((dequant_f16_kernel<T_Q6_K, TL>), grid, dim3(256), 0, st, w, rows, K, out); break;
        case T_MXFP4: hipLaunchKernelGGL((dequant_f16_kernel<T_MXFP4, TL>), grid, dim3(256), 0, st, w, rows, K, out); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_dequant_f16(int wt, const void * W, int64_t rows, int64_t K, uint16_t * out, hipStream_t st) {
    return launch_dequant<false>(wt, W, rows, K, out, st);
}

hipError_t launch_f16_tiled(int wt, const void * W, int64_t rows, int64_t K, uint16_t * out, hipStream_t st) {
    return launch_dequant<true>(wt, W, rows, K, out, st);
}

hipError_t launch_convert_f16(int type, const void * src, int64_t n, uint16_t * dst, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(convert_f16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, type, src, n, dst);
    return hipGetLastError();
}

hipError_t launch_pack_weight(int wt, const void * src, int64_t rows, int64_t K, void * dst, hipStream_t st) {
    const uint8_t * s = (const uint8_t *)src;
    uint8_t * d = (uint8_t *)dst;
    switch (wt) {
        case T_F16:
        case T_Q4_K:
        case T_Q5_K: {
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
        case T_Q4_0: {
            const int64_t n = rows * (K / 32);
            if (n <= 0) return hipSuccess;
            hipLaunchKernelGGL(pack_q4_0_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, s, rows, K, d);
            return hipGetLastError();
        }
        case T_MXFP4: {
            const int64_t n = rows * (K / 32);
            if (n <= 0) return hipSuccess;
            hipLaunchKernelGGL(pack_mxfp4_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, s, rows, K, d);
            return hipGetLastError();
        }
        default: return hipErrorInvalidValue;
    }
}

}  // namespace mx
