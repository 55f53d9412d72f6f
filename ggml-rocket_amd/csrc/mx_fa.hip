// SPDX-License-Identifier: MIT
// FLASH_ATTN_EXT prefill for gfx950: one fused kernel, online softmax in fp32 registers.
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
// Work decomposition: a block is 4 waves; each wave owns 32 query rows of one head. The 4 waves
// of a block share one KV head, so each K/V tile staged in LDS serves all of them (GQA reuse).
// The scores are computed transposed, S^T = K . Q^T, so each lane owns one query: the row max
// and row sum need one exchange with the partner lane (l ^ 32) only, and O^T = V^T . P^T keeps
// the same ownership, so the rescale by exp(m_old - m_new) is lane-local.
// The KV range may be split across blocks; each split then writes an unnormalised partial O with
// its (max, sum), and a combine kernel merges them.

#include "mx_common.h"
#include "mx_kernels_impl.h"

namespace mx {

constexpr int FA_BKV = 64;         // keys per LDS tile
constexpr int FA_QW = 32;          // query rows per wave
constexpr int FA_WAVES = 4;
constexpr int FA_VT_STRIDE = 136;  // bytes per V^T row (64 keys * 2 B + 8 B pad)

template <int D>
struct FaSmem {
    static constexpr int K_BYTES = FA_BKV * D * 2;
    static constexpr int V_BYTES = D * FA_VT_STRIDE;
    static constexpr int STAGE = K_BYTES + V_BYTES;
    static constexpr int TOTAL = 2 * STAGE;
};

__device__ __forceinline__ float fa_cap(float s, float softcap, float inv_softcap) {
    return softcap != 0.0f ? softcap * tanhf(s * inv_softcap) : s;
}

// Stage keys [j0, j0+64) of K (row-major [key][D]) and V (transposed into [d][key]) into LDS.
template <int D>
__device__ __forceinline__ void fa_load_kv(const FaArgs & a, int hk, int j0, uint8_t * ks, uint8_t * vt, int t) {
    constexpr int KCH = D / 8;   // 16-byte chunks per K row
    const uint16_t * K = a.k + (int64_t)hk * a.k_nb2;
    const uint16_t * V = a.v + (int64_t)hk * a.v_nb2;
    // K: 64 rows x KCH chunks
#pragma unroll
    for (int i = 0; i < (FA_BKV * KCH) / (FA_WAVES * WAVE); i++) {
        const int c = t + i * FA_WAVES * WAVE;
        const int r = c / KCH, ch = c % KCH;
        const int j = j0 + r;
        u32x4 v = {0, 0, 0, 0};
        if (j < a.KV) v = *(const u32x4 *)(K + (int64_t)j * a.k_nb1 + ch * 8);
        *(u32x4 *)(ks + swz<KCH>(r, ch)) = v;
    }
    // V: thread takes 4 keys x 8 dims, writes 8 transposed 4-key runs
    constexpr int DCH = D / 8;
    constexpr int ITEMS = 16 * DCH;   // (key group, d chunk) pairs
#pragma unroll
    for (int i = 0; i < (ITEMS + FA_WAVES * WAVE - 1) / (FA_WAVES * WAVE); i++) {
        const int it = t + i * FA_WAVES * WAVE;
        if (it >= ITEMS) break;
        const int kg = it % 16, dc = it / 16;
        u32x4 rows[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int j = j0 + 4 * kg + r;
            rows[r] = u32x4{0, 0, 0, 0};
            if (j < a.KV) rows[r] = *(const u32x4 *)(V + (int64_t)j * a.v_nb1 + dc * 8);
        }
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int w = e / 2, sh = (e % 2) * 16;
            const uint32_t h0 = (rows[0][w] >> sh) & 0xFFFFu, h1 = (rows[1][w] >> sh) & 0xFFFFu;
            const uint32_t h2 = (rows[2][w] >> sh) & 0xFFFFu, h3 = (rows[3][w] >> sh) & 0xFFFFu;
            *(u32x2 *)(vt + (dc * 8 + e) * FA_VT_STRIDE + kg * 8) = u32x2{h0 | (h1 << 16), h2 | (h3 << 16)};
        }
    }
}

template <int D>
__global__ void __launch_bounds__(FA_WAVES * WAVE) fa_kernel(FaArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int KSTEPS = D / 16;   // QK contraction steps
    constexpr int DBLK = D / 32;     // output column blocks of the PV product

    const int t = threadIdx.x, lane = t % WAVE, wave = t / WAVE;
    const int lq = lane % 32, lg = lane / 32;

    // block -> (kv head, group of 4 wave tasks, kv split)
    const int g = a.H / a.HK;
    const int n_ttiles = (a.T + FA_QW - 1) / FA_QW;
    const int tasks = g * n_ttiles;
    const int bph = (tasks + FA_WAVES - 1) / FA_WAVES;   // blocks per kv head
    int b = blockIdx.x;
    const int split = b % a.nsplit;
    b /= a.nsplit;
    const int hk = b / bph;
    const int task = (b % bph) * FA_WAVES + wave;
    const bool active = task < tasks;
    const int h = hk * g + (active ? task % g : 0);
    const int t0 = (active ? task / g : 0) * FA_QW;
    const int tq = t0 + lq;               // this lane's query token
    const bool qok = active && tq < a.T;

    // KV range of this split, in whole tiles
    const int ntiles = (a.KV + FA_BKV - 1) / FA_BKV;
    const int per = (ntiles + a.nsplit - 1) / a.nsplit;
    const int tile0 = split * per;
    const int tile1 = min(ntiles, tile0 + per);

    // ---- Q: scaled, range-guarded, converted to fp16 in the B-operand layout ----
    half8 qf[KSTEPS];
    float qfac = 1.0f;
    {
        const float * q = a.q + (int64_t)h * a.q_nb2 + (int64_t)tq * a.q_nb1;
        float amax = 0.0f;
        float qv[KSTEPS][8];
#pragma unroll
        for (int s = 0; s < KSTEPS; s++) {
            const int d = 16 * s + 8 * lg;
            float4v x0 = {0, 0, 0, 0}, x1 = {0, 0, 0, 0};
            if (qok) {
                x0 = *(const float4v *)(q + d);
                x1 = *(const float4v *)(q + d + 4);
            }
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

    float16v o[DBLK];
#pragma unroll
    for (int i = 0; i < DBLK; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) o[i][e] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;
    const float inv_cap = a.softcap != 0.0f ? 1.0f / a.softcap : 0.0f;
    const float LOG2E = 1.4426950408889634f;
    const uint16_t * mrow = (a.mask && qok) ? a.mask + (int64_t)tq * a.mask_nb1 : nullptr;

    if (tile0 < tile1) {
        fa_load_kv<D>(a, hk, tile0 * FA_BKV, smem, smem + FaSmem<D>::K_BYTES, t);
    }
    __syncthreads();

    for (int tile = tile0; tile < tile1; tile++) {
        const int cur = (tile - tile0) & 1;
        uint8_t * ks = smem + cur * FaSmem<D>::STAGE;
        uint8_t * vt = ks + FaSmem<D>::K_BYTES;
        const int j0 = tile * FA_BKV;
        // stage the next tile into the other buffer while this one is consumed
        if (tile + 1 < tile1) {
            uint8_t * ks2 = smem + (cur ^ 1) * FaSmem<D>::STAGE;
            fa_load_kv<D>(a, hk, j0 + FA_BKV, ks2, ks2 + FaSmem<D>::K_BYTES, t);
        }
        if (active) {
            // ---- S^T = K . Q^T for 64 keys: two 32-key blocks ----
            float16v sacc[2];
#pragma unroll
            for (int kb = 0; kb < 2; kb++) {
#pragma unroll
                for (int e = 0; e < 16; e++) sacc[kb][e] = 0.0f;
#pragma unroll
                for (int s = 0; s < KSTEPS; s++) {
                    const half8 kf = *(const half8 *)(ks + swz<D / 8>(kb * 32 + lq, 2 * s + lg));
                    sacc[kb] = mfma32(kf, qf[s], sacc[kb]);
                }
            }
            // ---- scores: scale back, cap, mask, key bound ----
            float mt = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < 2; kb++) {
#pragma unroll
                for (int q4 = 0; q4 < 4; q4++) {
                    const int jb = j0 + kb * 32 + 8 * q4 + 4 * lg;   // first of 4 keys
                    float mk[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                    if (mrow && jb + 3 < a.KV) {
                        const u32x2 mm = *(const u32x2 *)(mrow + jb);
                        mk[0] = h2f_bits((uint16_t)(mm[0] & 0xFFFFu));
                        mk[1] = h2f_bits((uint16_t)(mm[0] >> 16));
                        mk[2] = h2f_bits((uint16_t)(mm[1] & 0xFFFFu));
                        mk[3] = h2f_bits((uint16_t)(mm[1] >> 16));
                    } else if (mrow) {
#pragma unroll
                        for (int e = 0; e < 4; e++) mk[e] = (jb + e < a.KV) ? h2f_bits(mrow[jb + e]) : 0.0f;
                    }
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const int i = 4 * q4 + e;
                        float s = fa_cap(sacc[kb][i] * qfac, a.softcap, inv_cap) + mk[e];
                        if (jb + e >= a.KV) s = -INFINITY;
                        sacc[kb][i] = s;
                        mt = fmaxf(mt, s);
                    }
                }
            }
            mt = fmaxf(mt, __shfl_xor(mt, 32, WAVE));
            const float m_new = fmaxf(m_run, mt);
            // No lane-divergent branch here: the P.V MFMA reads every lane's operands, so a
            // lane whose keys are all masked so far must still supply finite P (zeros).
            {
                const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;
                const float alpha = (m_run == -INFINITY) ? 0.0f : exp2f((m_run - m_use) * LOG2E);
                const float mb = m_use * LOG2E;
                float psum = 0.0f;
#pragma unroll
                for (int kb = 0; kb < 2; kb++)
#pragma unroll
                    for (int i = 0; i < 16; i++) {
                        const float p = exp2f(sacc[kb][i] * LOG2E - mb);   // exp(-inf) = 0
                        sacc[kb][i] = p;
                        psum += p;
                    }
                l_run = l_run * alpha + psum;
                m_run = m_new;
#pragma unroll
                for (int i = 0; i < DBLK; i++)
#pragma unroll
                    for (int e = 0; e < 16; e++) o[i][e] *= alpha;
                // ---- O^T += V^T . P^T, 4 steps of 16 keys ----
#pragma unroll
                for (int s = 0; s < 4; s++) {
                    const int kb = s / 2, hs = s % 2;
                    half8 pf;
#pragma unroll
                    for (int e = 0; e < 8; e++) pf[e] = (_Float16)sacc[kb][8 * hs + e];
                    const int kofs = (kb * 32 + 16 * hs + 4 * lg) * 2;   // bytes
#pragma unroll
                    for (int db = 0; db < DBLK; db++) {
                        const uint8_t * row = vt + (db * 32 + lq) * FA_VT_STRIDE;
                        const u32x2 lo = *(const u32x2 *)(row + kofs);
                        const u32x2 hi = *(const u32x2 *)(row + kofs + 16);
                        const u32x4 vv = {lo[0], lo[1], hi[0], hi[1]};
                        o[db] = mfma32(__builtin_bit_cast(half8, vv), pf, o[db]);
                    }
                }
            }
        }
        __syncthreads();
    }

    if (!qok) return;
    // ---- epilogue ----
    const float l_tot = l_run + __shfl_xor(l_run, 32, WAVE);
    if (a.nsplit == 1) {
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
                *(float4v *)(dst + d) = v;
            }
    } else {
        // partial: O unnormalised [split][T][H][D], (m, l) [split][T][H]
        const int64_t row = ((int64_t)split * a.T + tq) * a.H + h;
        float * po = a.part_o + row * D;
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
}

// Merge nsplit partials: O = sum_s exp(m_s - M) O_s / sum_s exp(m_s - M) l_s. One thread per
// output element, D threads per (t, h) row.
template <int D>
__global__ void __launch_bounds__(256) fa_combine_kernel(FaArgs a) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t rows = (int64_t)a.T * a.H;
    if (i >= rows * D) return;
    const int64_t r = i / D;
    const int d = (int)(i % D);
    const int tq = (int)(r / a.H), h = (int)(r % a.H);
    float M = -INFINITY;
    for (int s = 0; s < a.nsplit; s++) M = fmaxf(M, a.part_ml[2 * ((int64_t)s * rows + r)]);
    float num = 0.0f, den = 0.0f;
    if (M != -INFINITY) {
        for (int s = 0; s < a.nsplit; s++) {
            const int64_t pr = (int64_t)s * rows + r;
            const float ms = a.part_ml[2 * pr];
            if (ms == -INFINITY) continue;
            const float w = __expf(ms - M);
            num += w * a.part_o[pr * D + d];
            den += w * a.part_ml[2 * pr + 1];
        }
    }
    a.dst[(int64_t)tq * a.dst_nb2 + (int64_t)h * a.dst_nb1 + d] = den > 0.0f ? num / den : 0.0f;
}

int fa_blocks_per_split(const FaArgs & a) {
    const int g = a.H / a.HK;
    const int n_ttiles = (a.T + FA_QW - 1) / FA_QW;
    return a.HK * ((g * n_ttiles + FA_WAVES - 1) / FA_WAVES);
}

hipError_t launch_fa(const FaArgs & a, hipStream_t st) {
    const int nb = fa_blocks_per_split(a) * a.nsplit;
    if (nb <= 0) return hipSuccess;
    switch (a.D) {
        case 64:
            hipLaunchKernelGGL(fa_kernel<64>, dim3(nb), dim3(FA_WAVES * WAVE), FaSmem<64>::TOTAL, st, a);
            break;
        case 128:
            hipLaunchKernelGGL(fa_kernel<128>, dim3(nb), dim3(FA_WAVES * WAVE), FaSmem<128>::TOTAL, st, a);
            break;
        default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.nsplit == 1) return e;
    const int64_t n = (int64_t)a.T * a.H * a.D;
    const dim3 grid((unsigned)((n + 255) / 256));
    if (a.D == 64) hipLaunchKernelGGL(fa_combine_kernel<64>, grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL(fa_combine_kernel<128>, grid, dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace mx
