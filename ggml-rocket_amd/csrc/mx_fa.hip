// SPDX-License-Identifier: MIT
// FLASH_ATTN_EXT prefill for gfx950: online softmax in fp32 registers, K and V streamed into LDS
// by DMA, V^T read from the row-major V tile by gfx950's transposing LDS load.
//
// Semantics (ggml-rocket.cpp:5444-5691 and its reference rocket_fa_ref_f32, 5392-5442):
//   O[t,h,:] = softmax_j( cap(scale * q[h,t].k[hk,j]) + mask[t,j] ) . v[hk,j,:],  hk = h / (H/HK)
// where cap(s) = softcap * tanh(s / softcap) when softcap != 0. A row whose every key is masked
// is written as zeros. Q is converted to fp16 with the scale folded in (the reference's
// ROCKET_FA_QSCALE fold, 5462-5465); a row whose scaled Q does not fit fp16 is divided by a
// per-row factor f that multiplies the scores back, so no range fallback is needed. The scores
// never leave fp32 registers (there is no fp16 score surface to overflow), P is rounded to fp16
// for the P.V MFMA, both contractions accumulate in fp32.
//
// One op is two launches (one when the caller says the workspace already holds the classes of
// this mask, e.g. for every layer after the first of a micro-batch, which all share one mask):
//   fa_prep   the mask tile classes (per 32-query x 64-key tile: every key masked / no key
//             masked / mixed), and 16 zero bytes (the K and V source of padded head dims).
//   fa        a block is 4 tasks, each 32 query rows of one head, all 4 on one KV head (GQA
//             reuse of the LDS tiles); two waves per task take alternate key tiles and merge at
//             the end (one wave per task, alone on its SIMD, for DV 256, whose O tile takes 128
//             accumulators). Per 64-key tile: K [64][DK] and V [64][DV], both row-major as in
//             the cache, arrive in LDS by global_load_lds (a 4-deep ring, two tiles landing while
//             two are used; 2-deep when four stages do not fit, for DK 192 and 256);
//             tiles whose mask is -inf for all the block's queries are skipped, tiles with
//             no mask entry read no mask. Scores are computed transposed, S^T = K . Q^T, so each
//             lane owns one query: the row max and sum need one exchange with the partner lane
//             (l ^ 32), and O^T = V^T . P^T keeps the same ownership, so the rescale by
//             exp(m_old - m_new) is lane-local. The V^T operand of that product is read from the
//             V tile by ds_read_b64_tr_b16, which transposes 4 x 16 blocks of fp16 across lanes.
// Head dims between the built ones (mx_fa_dims.h) run on the next larger build: K chunks past dk
// are fetched from 16 zero bytes of the workspace (row stride 0), Q columns past dk and V columns
// past dv are read as zero, output columns past dv are not stored.
// The KV range may be split across blocks; every split writes an unnormalised partial O with
// its (max, sum), and a third launch, fa_combine, merges them.

#include "mx_common.h"
#include "mx_fa_dims.h"
#include "mx_kernels_impl.h"

namespace mx {

constexpr int FA_BKV = 64;      // keys per tile
constexpr int FA_QW = 32;       // query rows per wave task
// Wave tasks (head, 32-query tile) per block, FaArgs::tasks (fa_tasks_ok): 4 (two waves a task, taking
// alternate key tiles; one wave a task for DV 256) or, for DV <= 128, 2 (four waves a task: each
// of the two tile parities split again into the tile's two 32-key halves). Two tasks make twice
// the blocks for the same work, so the chip fills without splitting the key range, and their
// key tiles serve half as many queries; four tasks do twice the MFMA work per step and LDS
// fill, which pays off once the key range is long enough to split (the launcher's choice).
constexpr int FA_LDS_MAX = 160 * 1024;
constexpr int FA_CLS_RESERVE = 2048;   // LDS kept beside the ring for the class rows (KV <= 32768)
constexpr float FA_LAZY = 8.0f / 1.4426950408889634f;   // ln(2^8): how far a score may pass the running max


// DK: the Q.K contraction (Q and K head dim), DV: the V and output head dim (DK > DV for the
// non-absorbed MLA of DeepSeek-style models, 192 / 128).
template <int DK, int DV, int NTASK = 4>
struct FaCfg {
    static constexpr int KCH = DK / 8;                       // 16-byte chunks per K row
    // K rows swizzle their chunks by XOR when KCH is a power of two (conflict free), else by a
    // rotation of one chunk per row
    static constexpr bool KXOR = (KCH & (KCH - 1)) == 0;
    static constexpr int KRPW = KCH >= 16 ? 1 : 16 / KCH;    // K rows per 256-byte bank window
    static constexpr int K_BYTES = FA_BKV * DK * 2;          // [64 keys][DK]
    static constexpr int VCH = DV / 8;                       // 16-byte chunks per V row
    static constexpr int VRB = DV * 2;                       // bytes per V row
    static constexpr int V_BYTES = FA_BKV * DV * 2;          // [64 keys][DV]
    static constexpr int STAGE = K_BYTES + V_BYTES;
    // ring depth: two tiles land while two are used, when four stages fit; else two stages and
    // the next pair is fetched between the steps
    static constexpr int NS = 4 * STAGE + FA_CLS_RESERVE <= FA_LDS_MAX - 64 ? 4 : 2;
    static constexpr int LDS = NS * STAGE;
    // waves per task: two taking alternate key tiles (merged at the end), or for DV > 128 one
    // wave taking every tile, alone on its SIMD so the 128 accumulators of its O tile fit
    static constexpr int PAR = DV > 128 ? 1 : 2;
    // and, with two tasks a block, two waves per tile, each taking one 32-key half of it
    static constexpr int TASKS = NTASK;
    static constexpr int HALF = TASKS == 2 ? 2 : 1;
    static_assert(fa_tasks_ok(DV, TASKS), "tasks");
    static constexpr int WAVES = TASKS * PAR * HALF;
    static_assert(WAVES == 4 || WAVES == 8, "waves");
    static constexpr int THREADS = WAVES * WAVE;
    static constexpr int PK = K_BYTES / (THREADS * 16);   // DMA instructions per wave
    static constexpr int PV = V_BYTES / (THREADS * 16);
    static constexpr int PER = PK + PV;
    static_assert(PK >= 1 && PV >= 1 && PK * THREADS * 16 == K_BYTES && PV * THREADS * 16 == V_BYTES, "DMA split");
    static_assert(DK % 64 == 0 && DV % 64 == 0, "head dims");
    static_assert(NS * STAGE + FA_CLS_RESERVE <= FA_LDS_MAX - 64, "LDS");
    // physical 16-byte chunk of logical chunk c in K row r
    __device__ static __forceinline__ int kchunk(int r, int c) {
        if constexpr (KXOR) return c ^ ((r / KRPW) & (KCH - 1));
        else return (c + r) % KCH;
    }
    // logical chunk stored at physical chunk p of K row r
    __device__ static __forceinline__ int kchunk_inv(int r, int p) {
        if constexpr (KXOR) return p ^ ((r / KRPW) & (KCH - 1));
        else return (p + KCH - r % KCH) % KCH;
    }
    // V rows swizzle their chunks by XOR with vswz(r), a multiple of 4 chunks (64 bytes): the
    // transposing reads take 64 bytes (32 dims) from each of 4 consecutive keys per 32 lanes, and
    // the swizzle puts those four segments in different quarters of the 256-byte bank window
    // (V rows of 128 bytes share a window two at a time, hence r / 2 there)
    __device__ static __forceinline__ int vswz(int r) {
        return (4 * (VRB >= 256 ? r : r / 2)) & (VCH - 1) & ~3;
    }
};

typedef const void __attribute__((address_space(1))) * fa_gptr_t;
typedef void __attribute__((address_space(3))) * fa_lptr_t;

__device__ __forceinline__ void fa_dma16(const void * g, void * l) {
    __builtin_amdgcn_global_load_lds((fa_gptr_t)g, (fa_lptr_t)l, 16, 0, 0);
}

// s_waitcnt with vmcnt(N), expcnt(7) (no wait), lgkmcnt(0): gfx9 encoding.
template <int N>
__device__ __forceinline__ void fa_wait_vm_lgkm0() {
    static_assert(N >= 0 && N <= 63, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | ((N >> 4) << 14));
}

// V^T fragments by transposing LDS reads: NF fragments of two ds_read_b64_tr_b16 each (keys
// k..k+3 at the address, k+8..k+11 at 8 rows of VRB bytes further) and a wait for them, in one
// statement. The intrinsic form makes the compiler wait for every K/V DMA in flight first (it
// cannot tell these reads from the DMA's LDS writes), which would serialize each tile behind
// the prefetch of the next; here the results are complete when the statement ends, so no
// instruction can see the registers before their data.
typedef int v2i __attribute__((ext_vector_type(2)));
template <int NF, int VRB>
__device__ __forceinline__ void fa_tr_read(const uint32_t (&a)[NF], v2i (&r)[2 * NF]);
template <> __device__ __forceinline__ void fa_tr_read<2, 128>(const uint32_t (&a)[2], v2i (&r)[4]) {
    asm volatile(
        "ds_read_b64_tr_b16 %0, %4\n"
        "ds_read_b64_tr_b16 %1, %4 offset:1024\n"
        "ds_read_b64_tr_b16 %2, %5\n"
        "ds_read_b64_tr_b16 %3, %5 offset:1024\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])
        : "v"(a[0]), "v"(a[1]));
}
template <> __device__ __forceinline__ void fa_tr_read<4, 128>(const uint32_t (&a)[4], v2i (&r)[8]) {
    asm volatile(
        "ds_read_b64_tr_b16 %0, %8\n"
        "ds_read_b64_tr_b16 %1, %8 offset:1024\n"
        "ds_read_b64_tr_b16 %2, %9\n"
        "ds_read_b64_tr_b16 %3, %9 offset:1024\n"
        "ds_read_b64_tr_b16 %4, %10\n"
        "ds_read_b64_tr_b16 %5, %10 offset:1024\n"
        "ds_read_b64_tr_b16 %6, %11\n"
        "ds_read_b64_tr_b16 %7, %11 offset:1024\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]), "=&v"(r[7])
        : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]));
}
template <> __device__ __forceinline__ void fa_tr_read<4, 256>(const uint32_t (&a)[4], v2i (&r)[8]) {
    asm volatile(
        "ds_read_b64_tr_b16 %0, %8\n"
        "ds_read_b64_tr_b16 %1, %8 offset:2048\n"
        "ds_read_b64_tr_b16 %2, %9\n"
        "ds_read_b64_tr_b16 %3, %9 offset:2048\n"
        "ds_read_b64_tr_b16 %4, %10\n"
        "ds_read_b64_tr_b16 %5, %10 offset:2048\n"
        "ds_read_b64_tr_b16 %6, %11\n"
        "ds_read_b64_tr_b16 %7, %11 offset:2048\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]), "=&v"(r[7])
        : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]));
}
template <> __device__ __forceinline__ void fa_tr_read<8, 256>(const uint32_t (&a)[8], v2i (&r)[16]) {
    asm volatile(
        "ds_read_b64_tr_b16 %0, %16\n"
        "ds_read_b64_tr_b16 %1, %16 offset:2048\n"
        "ds_read_b64_tr_b16 %2, %17\n"
        "ds_read_b64_tr_b16 %3, %17 offset:2048\n"
        "ds_read_b64_tr_b16 %4, %18\n"
        "ds_read_b64_tr_b16 %5, %18 offset:2048\n"
        "ds_read_b64_tr_b16 %6, %19\n"
        "ds_read_b64_tr_b16 %7, %19 offset:2048\n"
        "ds_read_b64_tr_b16 %8, %20\n"
        "ds_read_b64_tr_b16 %9, %20 offset:2048\n"
        "ds_read_b64_tr_b16 %10, %21\n"
        "ds_read_b64_tr_b16 %11, %21 offset:2048\n"
        "ds_read_b64_tr_b16 %12, %22\n"
        "ds_read_b64_tr_b16 %13, %22 offset:2048\n"
        "ds_read_b64_tr_b16 %14, %23\n"
        "ds_read_b64_tr_b16 %15, %23 offset:2048\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]), "=&v"(r[7]), "=&v"(r[8]), "=&v"(r[9]), "=&v"(r[10]), "=&v"(r[11]), "=&v"(r[12]), "=&v"(r[13]), "=&v"(r[14]), "=&v"(r[15])
        : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7]));
}
template <> __device__ __forceinline__ void fa_tr_read<8, 512>(const uint32_t (&a)[8], v2i (&r)[16]) {
    asm volatile(
        "ds_read_b64_tr_b16 %0, %16\n"
        "ds_read_b64_tr_b16 %1, %16 offset:4096\n"
        "ds_read_b64_tr_b16 %2, %17\n"
        "ds_read_b64_tr_b16 %3, %17 offset:4096\n"
        "ds_read_b64_tr_b16 %4, %18\n"
        "ds_read_b64_tr_b16 %5, %18 offset:4096\n"
        "ds_read_b64_tr_b16 %6, %19\n"
        "ds_read_b64_tr_b16 %7, %19 offset:4096\n"
        "ds_read_b64_tr_b16 %8, %20\n"
        "ds_read_b64_tr_b16 %9, %20 offset:4096\n"
        "ds_read_b64_tr_b16 %10, %21\n"
        "ds_read_b64_tr_b16 %11, %21 offset:4096\n"
        "ds_read_b64_tr_b16 %12, %22\n"
        "ds_read_b64_tr_b16 %13, %22 offset:4096\n"
        "ds_read_b64_tr_b16 %14, %23\n"
        "ds_read_b64_tr_b16 %15, %23 offset:4096\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]), "=&v"(r[7]), "=&v"(r[8]), "=&v"(r[9]), "=&v"(r[10]), "=&v"(r[11]), "=&v"(r[12]), "=&v"(r[13]), "=&v"(r[14]), "=&v"(r[15])
        : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7]));
}

// ---------------------------------------------------------------------------------------------
// prep: the mask classes
// ---------------------------------------------------------------------------------------------
enum : uint8_t { FA_TILE_SKIP = 0, FA_TILE_FULL = 1, FA_TILE_MIXED = 2 };

// The value of lane i ^ 32 (the lane holding the same query's other 16 scores): gfx950's
// v_permlane32_swap exchanges lanes 32-63 of its first operand with lanes 0-31 of its second, so
// with both operands = x, lanes 0-31 find the partner in the second result and lanes 32-63 in the
// first. A VALU exchange: no LDS round trip and no wait on the LDS reads in flight.
__device__ __forceinline__ float fa_partner(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

__global__ void __launch_bounds__(256) fa_prep_kernel(FaArgs a) {
    const int t = threadIdx.x;
    const int nkt = a.kvp / FA_BKV;
    const int b = blockIdx.x;
    if (b == 0 && t < 8) a.kzero[t] = 0;   // the K and V source of the padded columns
    const int nqt = (a.T + FA_QW - 1) / FA_QW;
    const int nct = nqt * a.cls_stride;   // rows padded to cls_stride entries (padding: skip)
    const int cb = b;
    if (cb * 4 < nct) {
        // one wave per (query tile, key tile): lane l scans row l/2, keys 32*(l%2) .. +31
        const int wave = t / WAVE, lane = t % WAVE;
        const int ct = cb * 4 + wave;
        if (ct >= nct) return;
        const int qt = ct / a.cls_stride, kt = ct % a.cls_stride;
        bool vis = false, nz = false;
        if (kt >= nkt) {
            vis = false;                              // padding entry
        } else if (a.mask) {
            const int tq = qt * FA_QW + lane / 2;
            const int jb = kt * FA_BKV + 32 * (lane % 2);
            if (tq < a.T) {
                const uint16_t * mr = a.mask + (int64_t)tq * a.mask_nb1 + jb;
                if (jb + 32 <= a.KV) {
                    // 8 independent 8-byte loads (rows are 8-byte aligned)
                    u32x2 w[8];
#pragma unroll
                    for (int i = 0; i < 8; i++) w[i] = *(const u32x2 *)(mr + 4 * i);
#pragma unroll
                    for (int i = 0; i < 8; i++)
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            const float m = h2f_bits((uint16_t)((w[i][e / 2] >> (16 * (e % 2))) & 0xFFFFu));
                            vis |= (m != -INFINITY);
                            nz |= (m != 0.0f);
                        }
                } else {
                    for (int j = 0; j < 32; j++) {
                        if (jb + j < a.KV) {
                            const float m = h2f_bits(mr[j]);
                            vis |= (m != -INFINITY);
                            nz |= (m != 0.0f);
                        }
                    }
                }
            }
        } else {
            vis = true;
        }
        const bool any_vis = __any(vis), any_nz = __any(nz);
        if (lane == 0) a.cls[ct] = !any_vis ? FA_TILE_SKIP : (any_nz ? FA_TILE_MIXED : FA_TILE_FULL);
        return;
    }
}

// ---------------------------------------------------------------------------------------------
// main kernel
// ---------------------------------------------------------------------------------------------
template <int DK, int DV, int NTASK, bool SOFTCAP>
__global__ void __launch_bounds__((FaCfg<DK, DV, NTASK>::THREADS))
__attribute__((amdgpu_waves_per_eu(FaCfg<DK, DV, NTASK>::PAR, FaCfg<DK, DV, NTASK>::PAR)))
fa_kernel(FaArgs a) {
    using C = FaCfg<DK, DV, NTASK>;
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int FA_NS = C::NS;
    constexpr int KSTEPS = DK / 16;  // QK contraction steps
    constexpr int DBLK = DV / 32;    // output row blocks of O^T

    const int t = threadIdx.x, lane = t % WAVE, wave = t / WAVE;
    const int lq = lane % 32, lg = lane / 32;
    const int wave_s = __builtin_amdgcn_readfirstlane(wave);
    constexpr int TASKS = C::TASKS;
    // wave = task + TASKS (half + HALF par): the two waves of a SIMD (w, w + 4) are one task's
    // two parities, which take alternate key tiles
    const int slot_task = wave % TASKS, half = (wave / TASKS) % C::HALF, par = wave / (TASKS * C::HALF);
    constexpr int KB = 2 / C::HALF;          // 32-key blocks of a tile per wave
    const int kb0 = C::HALF == 2 ? half : 0;  // the first of them

    // block -> (kv head, group of 4 wave tasks, kv split); two waves per task. Logical ids are
    // kv-head major and spread so that each XCD takes a contiguous run of them: the blocks of a
    // kv head read its K and V through one L2.
    const int g = a.H / a.HK;
    const int n_ttiles = (a.T + FA_QW - 1) / FA_QW;
    const int tasks = g * n_ttiles;
    const int bph = (tasks + TASKS - 1) / TASKS;   // blocks per kv head
    int b = xcd_tile(blockIdx.x, gridDim.x);
    const int split = b % a.nsplit;
    b /= a.nsplit;
    const int hk = b / bph;
    const int task0 = (b % bph) * TASKS;
    const int task = task0 + slot_task;
    const bool active = task < tasks;
    const int h = hk * g + (active ? task % g : 0);
    const int qt = active ? task / g : 0;
    const int tq = qt * FA_QW + lq;                      // this lane's query token
    const bool qok = active && tq < a.T;
    const int nkt = a.kvp / FA_BKV;

    // Q is converted once per task: its first wave loads it and, where the ring has room (four
    // stages), hands the fp16 form to the task's other waves through LDS
    constexpr bool QSHARE = C::PAR == 2 && FA_NS == 4;
    const bool lead = par == 0 && half == 0;   // the task's first wave
    const bool qload = !QSHARE || lead;

    // the block's key tiles: the union of its tasks' non-skipped ranges (a cooperative scan of
    // the class rows, 16 entries per load; at most one load per thread for KV within
    // fa_max_kv), then this split's share. The class loads are issued before Q's; Q is converted
    // right after the scan, which by then has waited for the loads in flight.
    const int qt_first = task0 / g, qt_last = min(tasks - 1, task0 + TASKS - 1) / g;
    const int nchunk = a.cls_stride / 16;
    const int items = (qt_last - qt_first + 1) * nchunk;
    u32x4 cw = {0, 0, 0, 0};
    if (t < items) cw = *(const u32x4 *)(a.cls + (int64_t)(qt_first + t / nchunk) * a.cls_stride + 16 * (t % nchunk));

    float4v qraw[KSTEPS][2];
    {
        const float * q = a.q + (int64_t)h * a.q_nb2 + (int64_t)(qok ? tq : 0) * a.q_nb1;
#pragma unroll
        for (int s = 0; s < KSTEPS; s++) {
            const int d = 16 * s + 8 * lg;   // < DK
            qraw[s][0] = float4v{0, 0, 0, 0};
            qraw[s][1] = float4v{0, 0, 0, 0};
            if (qload && qok && d < a.dk) {
                qraw[s][0] = *(const float4v *)(q + d);
                qraw[s][1] = *(const float4v *)(q + d + 4);
            }
        }
    }
    // DMA sources: K and V rows (keys, clamped to the last key); chunks past dk / dv, padding,
    // read the zero bytes for every key (row stride 0)
    const uint16_t * ksrc[C::PK];
    uint32_t kreal = 0, vreal = 0;   // bit q: source q is a real column (else the zero bytes)
    const uint16_t * vsrc[C::PV];
#pragma unroll
    for (int q = 0; q < C::PK; q++) {
        const int slot = (q * C::WAVES + wave) * WAVE + lane;
        const int r = slot / C::KCH, c = C::kchunk_inv(r, slot % C::KCH);
        const bool real = 8 * c < a.dk;
        kreal |= (uint32_t)real << q;
        ksrc[q] = real ? a.k + (int64_t)hk * a.k_nb2 + 8 * c + (int64_t)r * a.k_nb1 : a.kzero;   // + key offset per tile
    }
#pragma unroll
    for (int q = 0; q < C::PV; q++) {
        const int slot = (q * C::WAVES + wave) * WAVE + lane;
        const int r = slot / C::VCH, c = (slot % C::VCH) ^ C::vswz(r);
        const bool real = 8 * c < a.dv;
        vreal |= (uint32_t)real << q;
        vsrc[q] = real ? a.v + (int64_t)hk * a.v_nb2 + 8 * c + (int64_t)r * a.v_nb1 : a.kzero;   // + key offset per tile
    }
    const int kv_last = max(a.KV - 1, 0);
    // tile i of the range starting at key tile dma_t0 (dma_nt tiles) into ring buffer i % FA_NS;
    // past the last tile the last one is fetched again into the buffer just freed (nobody reads
    // it), so every step issues the same DMA count
    int dma_t0 = 0, dma_nt = 2;
    auto issue = [&](int i) {
        uint8_t * st = smem + (i % FA_NS) * C::STAGE;
        i = min(i, max(dma_nt - 1, 0));
        const int j0 = (dma_t0 + i) * FA_BKV;
        if (j0 + FA_BKV <= a.KV) {
            // every key of the tile exists: one scalar row offset for the whole wave, added to
            // the real sources only
            const int64_t ko = (int64_t)j0 * a.k_nb1, vo = (int64_t)j0 * a.v_nb1;
#pragma unroll
            for (int q = 0; q < C::PK; q++)
                fa_dma16(ksrc[q] + ((kreal >> q) & 1u ? ko : 0), st + (q * C::WAVES + wave_s) * 1024);
#pragma unroll
            for (int q = 0; q < C::PV; q++)
                fa_dma16(vsrc[q] + ((vreal >> q) & 1u ? vo : 0), st + C::K_BYTES + (q * C::WAVES + wave_s) * 1024);
            return;
        }
#pragma unroll
        for (int q = 0; q < C::PK; q++) {
            const int slot = (q * C::WAVES + wave) * WAVE + lane;
            const int r = slot / C::KCH;
            const int64_t jr = (int64_t)min(j0 + r, kv_last) - r;
            fa_dma16(ksrc[q] + ((kreal >> q) & 1u ? jr * a.k_nb1 : 0), st + (q * C::WAVES + wave_s) * 1024);
        }
#pragma unroll
        for (int q = 0; q < C::PV; q++) {
            const int slot = (q * C::WAVES + wave) * WAVE + lane;
            const int r = slot / C::VCH;
            const int64_t jr = (int64_t)min(j0 + r, kv_last) - r;
            fa_dma16(vsrc[q] + ((vreal >> q) & 1u ? jr * a.v_nb1 : 0), st + C::K_BYTES + (q * C::WAVES + wave_s) * 1024);
        }
    };

    // The first two key tiles are requested now, before the mask classes say where the block's
    // range starts: with one KV split the range almost always starts at key tile 0 (a causal
    // mask hides no leading key from any query), and then the tiles' HBM round trip runs under
    // the class scan and the Q conversion instead of after them. Stages 0 and 1 are free (the Q
    // hand-over uses 2 and 3, the class rows sit behind the ring). A guess that turns out wrong
    // waits for these tiles to land and requests the real ones.
    const bool spec = a.nsplit == 1 && a.KV >= 1;
    if (spec) {
        issue(0);
        issue(1);
    }
    // Parity-0 waves issue first on their SIMD: both waves of a SIMD reach each step's score
    // MFMAs together, and the priority lets one run them while the other waits, so afterwards
    // one wave's softmax overlaps the other's MFMAs instead of both competing for each unit.
    if (par == 0) __builtin_amdgcn_s_setprio(1);

    // The barriers wait for LDS work only (lgkmcnt), never for global loads in flight.
    __shared__ int range_lo, range_hi;
    if (t == 0) { range_lo = nkt; range_hi = 0; }
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    {
        int mylo = nkt, myhi = 0;
        for (int it = t; it < items; it += C::THREADS) {
            const int q = qt_first + it / nchunk, c = it % nchunk;
            const u32x4 w = it == t ? cw : *(const u32x4 *)(a.cls + (int64_t)q * a.cls_stride + 16 * c);
            *(u32x4 *)(smem + C::LDS + (q - qt_first) * a.cls_stride + 16 * c) = w;   // kept for the loop
#pragma unroll
            for (int e = 0; e < 16; e++)
                if ((w[e / 4] >> (8 * (e % 4))) & 0xFFu) {
                    mylo = min(mylo, 16 * c + e);
                    myhi = max(myhi, 16 * c + e + 1);
                }
        }
        if (mylo < nkt) atomicMin(&range_lo, mylo);
        if (myhi > 0) atomicMax(&range_hi, myhi);
    }
    // ---- Q: scaled, range-guarded, converted to fp16 in the B-operand layout while the scan's
    // atomics land. Where the ring has room the task's first wave hands the fp16 form to the
    // task's other waves through ring stages 2 and 3 (no tile is requested yet), published by
    // the barrier that publishes the range: per task [KSTEPS][64 lanes] half8, then the 64
    // lanes' range factors ----
    half8 qf[KSTEPS];
    float qfac = 1.0f;
    if (qload) {
        float amax = 0.0f;
        float qv[KSTEPS][8];
#pragma unroll
        for (int s = 0; s < KSTEPS; s++) {
            const float4v x0 = qraw[s][0], x1 = qraw[s][1];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                qv[s][e] = x0[e] * a.scale;
                qv[s][4 + e] = x1[e] * a.scale;
                amax = fmaxf(amax, fmaxf(fabsf(qv[s][e]), fabsf(qv[s][4 + e])));
            }
        }
        amax = fmaxf(amax, __shfl_xor(amax, 32, WAVE));
        // 65504 is the largest finite fp16; a row past it is divided by f = amax / 32768
        if (amax > 65504.0f) qfac = amax / 32768.0f;
        const float inv = 1.0f / qfac;
#pragma unroll
        for (int s = 0; s < KSTEPS; s++)
#pragma unroll
            for (int e = 0; e < 8; e++) qf[s][e] = (_Float16)(qfac == 1.0f ? qv[s][e] : qv[s][e] * inv);
    }
    uint8_t * const qx = smem + 2 * C::STAGE + slot_task * (KSTEPS * 1024 + 256);
    if constexpr (QSHARE) {
        if (lead) {
#pragma unroll
            for (int s = 0; s < KSTEPS; s++) *(half8 *)(qx + s * 1024 + lane * 16) = qf[s];
            *(float *)(qx + KSTEPS * 1024 + lane * 4) = qfac;
        }
    }
    static_assert(!QSHARE || TASKS * (KSTEPS * 1024 + 256) <= 2 * C::STAGE, "Q hand-over space");
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    // block-uniform: read into SGPRs, so the tile indices and the per-tile DMA offsets below are
    // scalar arithmetic
    const int lo = __builtin_amdgcn_readfirstlane(range_lo), hi = __builtin_amdgcn_readfirstlane(range_hi);
    const int span = max(0, hi - lo);
    const int per = (span + a.nsplit - 1) / a.nsplit;
    const int tile0 = lo + split * per;
    const int tile1 = min(hi, tile0 + per);
    const int ntl = max(0, tile1 - tile0);
    dma_t0 = tile0;
    dma_nt = ntl;
    // the guessed tiles are the real tiles 0 and 1 when the range starts at key tile 0 (a tile
    // past the range's end is never read); otherwise they land before their stages are refilled
    const bool spec_ok = spec && tile0 == 0;
    if (spec && !spec_ok) fa_wait_vm_lgkm0<0>();

    float16v o[DBLK];
#pragma unroll
    for (int i = 0; i < DBLK; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) o[i][e] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;
    const float inv_cap = SOFTCAP ? 1.0f / a.softcap : 0.0f;
    const float LOG2E = 1.4426950408889634f;
    const uint16_t * mrow = (a.mask && qok) ? a.mask + (int64_t)tq * a.mask_nb1 : nullptr;
    // this task's class row, copied into LDS behind the ring by the range scan above
    const uint8_t * cls_w = smem + C::LDS + (qt - qt_first) * a.cls_stride;

    // V^T fragments by ds_read_b64_tr_b16, which gives lane i of each 16-lane group element e =
    // element i % 4 of the group's source lane 4e + i / 4. Source lane s of group gq points at
    // 4 dims (32 db + 16 (gq % 2) + 4 (s % 4) ..) of key 16 s2 + 8 h + 4 lg + s / 4, so lane i
    // receives dim 32 db + 16 (gq % 2) + i (its row of the MFMA operand) of keys
    // 16 s2 + 8 h + 4 lg + 0..3: elements 4h..4h+3 of the fragment, the keys the P^T operand
    // holds there (the S^T accumulator layout). The lane's byte offset for db is
    // vbase + ((64 db) ^ vsw): the swizzle (a multiple of 4 chunks) only flips bits of db.
    int vbase, vsw;
    {
        const int sl = lane % 16, gq = lane / 16, y = sl / 4;
        const int x = 2 * (gq % 2) + (sl % 4) / 2;   // logical chunk within the 32 dims of db
        vsw = 16 * C::vswz(4 * lg + y);               // equals vswz of every key row it reads
        vbase = (4 * lg + y) * C::VRB + 16 * x + 8 * (sl % 2);
    }

    // Each step consumes two tiles: parity-0 waves take the even one, parity-1 waves the odd one
    // (the same query rows), and both land in the ring during the step before.
    const int nsteps = (ntl + 1) / 2;
    if (ntl > 0) {
        if (!spec_ok) {
            issue(0);
            issue(1);
        }
        if constexpr (!QSHARE)
#pragma unroll
            for (int p = 2; p < FA_NS; p++) issue(p);
    }
    if constexpr (QSHARE) {
        // the other waves take their task's Q; stages 2 and 3 are requested once every wave has
        // read it
        if (!lead) {
#pragma unroll
            for (int s = 0; s < KSTEPS; s++) qf[s] = *(const half8 *)(qx + s * 1024 + lane * 16);
            qfac = *(const float *)(qx + KSTEPS * 1024 + lane * 4);
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        if (ntl > 0) {
            issue(2);
            issue(3);
        }
    }
    const bool q_scaled = __any(qfac != 1.0f);   // a row of this wave needed the Q range factor
    if (ntl > 0) {
        fa_wait_vm_lgkm0<(FA_NS - 2) * C::PER>();
        __builtin_amdgcn_s_barrier();
    }
    for (int stp = 0; stp < nsteps; stp++) {
        // one tile of the step per wave when two share a task, both when one wave has the task
        for (int sub = 0; sub < 3 - C::PAR; sub++) {
            const int i = 2 * stp + (C::PAR == 2 ? par : sub);   // this wave's local tile
            const int tile = tile0 + i;
            const int j0 = tile * FA_BKV;
            const uint8_t * ks = smem + (i % FA_NS) * C::STAGE;
            const uint8_t * vt = ks + C::K_BYTES;   // V [64 keys][DV], rows swizzled by vswz
            // the class is the same in every lane of the wave: read it into an SGPR, so the branch
            // below is a scalar one
            const uint32_t cls = __builtin_amdgcn_readfirstlane(
                (active && i < ntl) ? (uint32_t)cls_w[tile] : (uint32_t)FA_TILE_SKIP);
            if (cls != FA_TILE_SKIP) {
                // ---- S^T = K . Q^T for this wave's 32-key blocks of the tile (kb0 .. kb0 + KB - 1) ----
                // Every K fragment read of the tile is issued before the first MFMA, so the LDS
                // latency is paid once per tile rather than once per MFMA; the scheduling barriers
                // keep the compiler from interleaving each read with the MFMA that consumes it.
                // (DK <= 128; the wider heads, whose fragments do not fit the register budget
                // twice over, read and multiply one 32-key block at a time.)
                float16v sacc[KB];
                auto kfrag = [&](int kb, int s2) {
                    return *(const half8 *)(ks + (kb * 32 + lq) * (DK * 2) + (C::kchunk(kb * 32 + lq, 2 * s2 + lg) << 4));
                };
                if constexpr (DK <= 128) {
                    half8 kf[KB][KSTEPS];
#pragma unroll
                    for (int kk = 0; kk < KB; kk++)
#pragma unroll
                        for (int s2 = 0; s2 < KSTEPS; s2++) kf[kk][s2] = kfrag(kb0 + kk, s2);
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int kk = 0; kk < KB; kk++) {
#pragma unroll
                        for (int e = 0; e < 16; e++) sacc[kk][e] = 0.0f;
#pragma unroll
                        for (int s2 = 0; s2 < KSTEPS; s2++) sacc[kk] = mfma32(kf[kk][s2], qf[s2], sacc[kk]);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                } else {
#pragma unroll
                    for (int kk = 0; kk < KB; kk++) {
                        half8 kf[KSTEPS];
#pragma unroll
                        for (int s2 = 0; s2 < KSTEPS; s2++) kf[s2] = kfrag(kb0 + kk, s2);
#pragma unroll
                        for (int e = 0; e < 16; e++) sacc[kk][e] = 0.0f;
#pragma unroll
                        for (int s2 = 0; s2 < KSTEPS; s2++) sacc[kk] = mfma32(kf[s2], qf[s2], sacc[kk]);
                    }
                }
                // the V^T fragments of the wave's first two 16-key P.V steps do not depend on the
                // softmax: issue their reads now, so they land while the scores are computed (DK,
                // DV <= 128; the wider builds have no registers to spare for them)
                constexpr bool EARLY_V = DK <= 128 && DV <= 128;
                // the fragments of NS2 consecutive 16-key steps from s2 on, for every db
                const uint32_t vt_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint8_t *)vt;
                auto vfrags = [&](int s2, auto & f) {
                    constexpr int NS2 = sizeof(f) / sizeof(f[0]);
                    uint32_t ad[NS2 * DBLK];
#pragma unroll
                    for (int i = 0; i < NS2; i++)
#pragma unroll
                        for (int db = 0; db < DBLK; db++)
                            ad[i * DBLK + db] = vt_lds + vbase + ((64 * db) ^ vsw) + 16 * (s2 + i) * C::VRB;
                    v2i r[2 * NS2 * DBLK];
                    fa_tr_read<NS2 * DBLK, C::VRB>(ad, r);
#pragma unroll
                    for (int i = 0; i < NS2; i++)
#pragma unroll
                        for (int db = 0; db < DBLK; db++) {
                            const v2i lo = r[2 * (i * DBLK + db)], hi = r[2 * (i * DBLK + db) + 1];
                            typedef int v4i __attribute__((ext_vector_type(4)));
                            f[i][db] = __builtin_bit_cast(half8, v4i{lo[0], lo[1], hi[0], hi[1]});
                        }
                };
                half8 vfa[EARLY_V ? 2 : 1][DBLK];
                if constexpr (EARLY_V) {
                    vfrags(2 * kb0, vfa);   // their wait overlaps the score MFMAs in flight
                    __builtin_amdgcn_sched_barrier(0);
                }
                // ---- scores: scale back, cap, mask, key bound (each a wave-uniform case) ----
                if (q_scaled) {
#pragma unroll
                    for (int kk = 0; kk < KB; kk++)
#pragma unroll
                        for (int ii = 0; ii < 16; ii++) sacc[kk][ii] *= qfac;
                }
                if (SOFTCAP) {
#pragma unroll
                    for (int kk = 0; kk < KB; kk++)
#pragma unroll
                        for (int ii = 0; ii < 16; ii++) sacc[kk][ii] = a.softcap * tanhf(sacc[kk][ii] * inv_cap);
                }
                if (cls == FA_TILE_MIXED) {
                    if (mrow) {
#pragma unroll
                        for (int kk = 0; kk < KB; kk++)
#pragma unroll
                            for (int q4 = 0; q4 < 4; q4++) {
                                const int jb = j0 + (kb0 + kk) * 32 + 8 * q4 + 4 * lg;   // first of 4 keys
                                float mk[4];
                                if (jb + 3 < a.KV) {
                                    const u32x2 mm = *(const u32x2 *)(mrow + jb);
                                    mk[0] = h2f_bits((uint16_t)(mm[0] & 0xFFFFu));
                                    mk[1] = h2f_bits((uint16_t)(mm[0] >> 16));
                                    mk[2] = h2f_bits((uint16_t)(mm[1] & 0xFFFFu));
                                    mk[3] = h2f_bits((uint16_t)(mm[1] >> 16));
                                } else {
#pragma unroll
                                    for (int e = 0; e < 4; e++) mk[e] = (jb + e < a.KV) ? h2f_bits(mrow[jb + e]) : 0.0f;
                                }
#pragma unroll
                                for (int e = 0; e < 4; e++) sacc[kk][4 * q4 + e] += mk[e];
                            }
                    }
                }
                if (j0 + FA_BKV > a.KV) {
#pragma unroll
                    for (int kk = 0; kk < KB; kk++)
#pragma unroll
                        for (int ii = 0; ii < 16; ii++)
                            if (j0 + (kb0 + kk) * 32 + 8 * (ii / 4) + 4 * lg + (ii % 4) >= a.KV) sacc[kk][ii] = -INFINITY;
                }
                float mt = -INFINITY;
#pragma unroll
                for (int kk = 0; kk < KB; kk++)
#pragma unroll
                    for (int ii = 0; ii < 16; ii++) mt = fmaxf(mt, sacc[kk][ii]);
                mt = fmaxf(mt, fa_partner(mt));
                // The running max moves only when a score passes it by more than FA_LAZY (2^8 in
                // P): P then stays below 256, well inside fp16 and the fp32 sums, and most tiles
                // skip the rescale of O. When it moves, every row of the wave takes its exact max.
                // No lane-divergent branch: the P.V MFMA reads every lane's operands, so a lane
                // whose keys are all masked so far must still supply finite P (zeros).
                if (__any(mt > m_run + FA_LAZY)) {   // false for a row with every key masked
                    const float m_new = fmaxf(m_run, mt);
                    const float alpha = (m_run == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f((m_run - m_new) * LOG2E);
                    m_run = m_new;
                    l_run *= alpha;
#pragma unroll
                    for (int db = 0; db < DBLK; db++)
#pragma unroll
                        for (int e = 0; e < 16; e++) o[db][e] *= alpha;
                }
                const float mb = (m_run == -INFINITY) ? 0.0f : m_run * LOG2E;
#pragma unroll
                for (int kk = 0; kk < KB; kk++)
#pragma unroll
                    for (int ii = 0; ii < 16; ii++)
                        // v_exp_f32: exp2(-inf) = 0; results below the fp32 normal range flush to 0
                        sacc[kk][ii] = __builtin_amdgcn_exp2f(fmaf(sacc[kk][ii], LOG2E, -mb));
                // ---- O^T += V^T . P^T, one step per 16 keys of the wave ----
                if constexpr (EARLY_V) {
                    half8 pf[2 * KB];
#pragma unroll
                    for (int s2 = 0; s2 < 2 * KB; s2++)
#pragma unroll
                        for (int e = 0; e < 8; e++) pf[s2][e] = (_Float16)sacc[s2 / 2][8 * (s2 % 2) + e];
                    // the row sum of the P that the MFMA multiplies (its fp16 values), two per
                    // v_dot2_f32_f16 with fp32 accumulation
                    float psum = 0.0f;
                    const half2v one2 = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
                    for (int s2 = 0; s2 < 2 * KB; s2++)
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            psum = __builtin_amdgcn_fdot2(half2v{pf[s2][2 * e], pf[s2][2 * e + 1]}, one2, psum, false);
                    l_run += psum;
#pragma unroll
                    for (int s2 = 0; s2 < 2; s2++)
#pragma unroll
                        for (int db = 0; db < DBLK; db++) o[db] = mfma32(vfa[s2][db], pf[s2], o[db]);
                    __builtin_amdgcn_sched_barrier(0);
                    if constexpr (KB == 2) {
                        // the last two steps' fragments are read while the first two steps multiply
                        half8 vfb[2][DBLK];
                        vfrags(2, vfb);
                        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                        for (int s2 = 0; s2 < 2; s2++)
#pragma unroll
                            for (int db = 0; db < DBLK; db++) o[db] = mfma32(vfb[s2][db], pf[2 + s2], o[db]);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                } else {
                    float psum = 0.0f;
#pragma unroll
                    for (int kk = 0; kk < KB; kk++)
#pragma unroll
                        for (int ii = 0; ii < 16; ii++) psum += sacc[kk][ii];
                    l_run += psum;
#pragma unroll
                    for (int j = 0; j < 2 * KB; j++) {
                        const int kk = j / 2, hs = j % 2;
                        half8 pf;
#pragma unroll
                        for (int e = 0; e < 8; e++) pf[e] = (_Float16)sacc[kk][8 * hs + e];
                        half8 vf[1][DBLK];
                        vfrags(2 * kb0 + j, vf);
#pragma unroll
                        for (int db = 0; db < DBLK; db++) o[db] = mfma32(vf[0][db], pf, o[db]);
                    }
                }
            }
        }
        // the next two tiles have landed for every wave, and every wave is done with these two
        fa_wait_vm_lgkm0<0>();
        __builtin_amdgcn_s_barrier();
        if (2 * stp + FA_NS < ntl) {   // block-uniform; the wait above counts nothing issued later
            issue(2 * stp + FA_NS);
            issue(2 * stp + FA_NS + 1);
            if constexpr (FA_NS == 2) {   // no tiles in flight behind these: wait for them here
                fa_wait_vm_lgkm0<0>();
                __builtin_amdgcn_s_barrier();
            }
        }
    }
    fa_wait_vm_lgkm0<0>();   // no DMA may still be writing LDS: the merge below reuses the ring
    __syncthreads();

    // ---- merge each task's waves (same rows, disjoint keys) through LDS: each parity-1 wave
    // into its parity-0 partner, then the parity-0 wave of the second key halves into the task's
    // first wave ----
    auto merge = [&](bool give, bool take, int slot) {
        float * ob = (float *)smem + (size_t)slot * (DBLK * 16 + 2) * WAVE;   // [DBLK*16 + 2][64]
        if (give) {
#pragma unroll
            for (int db = 0; db < DBLK; db++)
#pragma unroll
                for (int e = 0; e < 16; e++) ob[(db * 16 + e) * WAVE + lane] = o[db][e];
            ob[(DBLK * 16) * WAVE + lane] = m_run;
            ob[(DBLK * 16 + 1) * WAVE + lane] = l_run;
        }
        __syncthreads();
        if (take) {
            const float m1 = ob[(DBLK * 16) * WAVE + lane], l1 = ob[(DBLK * 16 + 1) * WAVE + lane];
            const float M = fmaxf(m_run, m1);
            const float a0 = (m_run == -INFINITY) ? 0.0f : __expf(m_run - M);
            const float a1 = (m1 == -INFINITY) ? 0.0f : __expf(m1 - M);
#pragma unroll
            for (int db = 0; db < DBLK; db++)
#pragma unroll
                for (int e = 0; e < 16; e++) o[db][e] = o[db][e] * a0 + ob[(db * 16 + e) * WAVE + lane] * a1;
            l_run = l_run * a0 + l1 * a1;
            m_run = M;
        }
    };
    static_assert(C::PAR == 1 || TASKS * C::HALF * (DBLK * 16 + 2) * WAVE * 4 <= C::LDS, "merge space");
    if constexpr (C::PAR == 2) merge(par == 1, par == 0, slot_task + TASKS * half);
    if constexpr (C::HALF == 2) {
        __syncthreads();   // the first merge's reads are done before its area is written again
        merge(par == 0 && half == 1, lead, slot_task);
    }

    const float l_tot = l_run + fa_partner(l_run);
    if (!lead) return;   // the task's first wave holds its merged result
    if (a.nsplit == 1) {
        if (!qok) return;
        const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
        float * dst = a.dst + (int64_t)tq * a.dst_nb2 + (int64_t)h * a.dst_nb1;
#pragma unroll
        for (int db = 0; db < DBLK; db++)
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) {
                const int d = db * 32 + 8 * q4 + 4 * lg;
                float4v v;
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] = o[db][4 * q4 + e] * inv;
                if (d < a.dv) *(float4v *)(dst + d) = v;
            }
        return;
    }

    // partial: O unnormalised [split][T][H][D], (m, l) [split][T][H]; fa_combine merges them
    if (!qok) return;
    const int64_t rows = (int64_t)a.T * a.H;
    const int64_t row = (int64_t)split * rows + (int64_t)tq * a.H + h;
    float * po = a.part_o + row * DV;
#pragma unroll
    for (int db = 0; db < DBLK; db++)
#pragma unroll
        for (int q4 = 0; q4 < 4; q4++) {
            const int d = db * 32 + 8 * q4 + 4 * lg;
            float4v v;
#pragma unroll
            for (int e = 0; e < 4; e++) v[e] = o[db][4 * q4 + e];
            *(float4v *)(po + d) = v;
        }
    if (lg == 0) {
        a.part_ml[2 * row] = m_run;
        a.part_ml[2 * row + 1] = l_tot;
    }
}

// Merge the nsplit partials of every (token, head) row:
// O = sum_s exp(m_s - M) O_s / sum_s exp(m_s - M) l_s. D/4 threads per row, a float4 each
// (D = DV, the output head dim).
template <int D>
__global__ void __launch_bounds__(256) fa_combine_kernel(FaArgs a) {
    constexpr int TPR = D / 4;
    const int64_t rows = (int64_t)a.T * a.H;
    const int64_t r = (int64_t)blockIdx.x * (256 / TPR) + threadIdx.x / TPR;
    if (r >= rows) return;
    const int c = threadIdx.x % TPR;
    float M = -INFINITY;
    for (int s = 0; s < a.nsplit; s++) M = fmaxf(M, a.part_ml[2 * ((int64_t)s * rows + r)]);
    float4v num = {0, 0, 0, 0};
    float den = 0.0f;
    if (M != -INFINITY) {
        for (int s = 0; s < a.nsplit; s++) {
            const int64_t pr = (int64_t)s * rows + r;
            const float ms = a.part_ml[2 * pr];
            if (ms == -INFINITY) continue;
            const float w = __expf(ms - M);
            den += w * a.part_ml[2 * pr + 1];
            const float4v v = *(const float4v *)(a.part_o + pr * D + 4 * c);
#pragma unroll
            for (int e = 0; e < 4; e++) num[e] += w * v[e];
        }
    }
    const float inv = den > 0.0f ? 1.0f / den : 0.0f;
    const int tq = (int)(r / a.H), h = (int)(r % a.H);
    float4v out;
#pragma unroll
    for (int e = 0; e < 4; e++) out[e] = num[e] * inv;
    if (4 * c < a.dv) *(float4v *)(a.dst + (int64_t)tq * a.dst_nb2 + (int64_t)h * a.dst_nb1 + 4 * c) = out;
}

int fa_blocks_per_split(const FaArgs & a) {
    const int g = a.H / a.HK;
    const int n_ttiles = (a.T + FA_QW - 1) / FA_QW;
    return a.HK * ((g * n_ttiles + a.tasks - 1) / a.tasks);
}

int fa_prep_blocks(const FaArgs & a) {
    const int nqt = (a.T + FA_QW - 1) / FA_QW;
    return max(1, (nqt * a.cls_stride + 3) / 4);
}

// the ring plus the class rows of up to `tasks` query tiles
static size_t fa_ring_bytes(int D, int DV) {
    if (D == 64 && DV == 64) return FaCfg<64, 64>::LDS;
    if (D == 128 && DV == 128) return FaCfg<128, 128>::LDS;
    if (D == 192 && DV == 128) return FaCfg<192, 128>::LDS;
    if (D == 256 && DV == 256) return FaCfg<256, 256>::LDS;
    return 0;
}
static size_t fa_lds_bytes(const FaArgs & a) { return fa_ring_bytes(a.D, a.DV) + (size_t)a.tasks * a.cls_stride; }

bool fa_dims_supported(int dk, int dv) {
    int D = 0, DV = 0;
    return fa_pad_dims(dk, dv, D, DV) && fa_ring_bytes(D, DV) != 0;
}

size_t fa_max_kv(int dk, int dv) {
    int D = 0, DV = 0;
    if (!fa_pad_dims(dk, dv, D, DV)) return 0;
    const size_t ring = fa_ring_bytes(D, DV);
    if (!ring) return 0;
    // class rows of up to 4 query tiles (one byte per 64-key tile, rows of a multiple of 16)
    return (size_t)(FA_LDS_MAX - ring - 64) / 4 / 16 * 16 * FA_BKV;
}

template <int DK, int DV, int NT, bool SC>
static hipError_t fa_launch_main(const FaArgs & a, int nb, hipStream_t st) {
    static bool done = false;
    if (!done) {
        hipError_t e = hipFuncSetAttribute((const void *)fa_kernel<DK, DV, NT, SC>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, FA_LDS_MAX - 64);
        if (e != hipSuccess) return e;
        done = true;
    }
    hipLaunchKernelGGL((fa_kernel<DK, DV, NT, SC>), dim3(nb), dim3(FaCfg<DK, DV, NT>::THREADS), fa_lds_bytes(a), st, a);
    return hipGetLastError();
}

template <int DK, int DV>
static hipError_t fa_launch_all(const FaArgs & a, int nb, bool prep, hipStream_t st) {
    hipError_t e = hipSuccess;
    if (prep) {
        hipLaunchKernelGGL(fa_prep_kernel, dim3(fa_prep_blocks(a)), dim3(256), 0, st, a);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    if constexpr (DV <= 128) {
        if (a.tasks == 2)
            e = a.softcap != 0.0f ? fa_launch_main<DK, DV, 2, true>(a, nb, st) : fa_launch_main<DK, DV, 2, false>(a, nb, st);
        else
            e = a.softcap != 0.0f ? fa_launch_main<DK, DV, 4, true>(a, nb, st) : fa_launch_main<DK, DV, 4, false>(a, nb, st);
    } else {
        e = a.softcap != 0.0f ? fa_launch_main<DK, DV, 4, true>(a, nb, st) : fa_launch_main<DK, DV, 4, false>(a, nb, st);
    }
    if (e != hipSuccess || a.nsplit == 1) return e;
    const int64_t rows = (int64_t)a.T * a.H;
    const int rpb = 256 / (DV / 4);
    hipLaunchKernelGGL(fa_combine_kernel<DV>, dim3((unsigned)((rows + rpb - 1) / rpb)), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_fa(const FaArgs & a, bool prep, hipStream_t st) {
    if (!fa_tasks_ok(a.DV, a.tasks)) return hipErrorInvalidValue;
    const int nb = fa_blocks_per_split(a) * a.nsplit;
    if (nb <= 0) return hipSuccess;
    if (a.D == 64 && a.DV == 64) return fa_launch_all<64, 64>(a, nb, prep, st);
    if (a.D == 128 && a.DV == 128) return fa_launch_all<128, 128>(a, nb, prep, st);
    if (a.D == 192 && a.DV == 128) return fa_launch_all<192, 128>(a, nb, prep, st);
    if (a.D == 256 && a.DV == 256) return fa_launch_all<256, 256>(a, nb, prep, st);
    return hipErrorInvalidValue;
}

}  // namespace mx
