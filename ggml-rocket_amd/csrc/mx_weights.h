// SPDX-License-Identifier: MIT
// Weight formats in HBM and their on-the-fly decoders.
//
// A weight panel is `rows` rows of K values. The layouts are:
//   F16   [rows][K] fp16, the ggml payload unchanged (zero copy).
//   F16T  fp16 in 16 x 32 tiles of 1 KB (tiled_index, mx_common.h): the resident fp16 form the
//         LDS-DMA GEMM streams, one contiguous kilobyte per load instruction.
//   Q4_K  [rows][K/256] blocks of 144 B, the ggml payload unchanged: { fp16 d, fp16 dmin,
//         u8 scales[12], u8 qs[128] }. Every block starts on a 16-byte boundary.
//   Q8_0  split into two planes so every load is 16-byte aligned (a 34-byte ggml block is only
//         2-byte aligned): qs int8 [rows][K] at 0, then d fp16 [rows][K/32].
//   Q6_K  split into four planes for the same reason (a ggml block is 210 B): ql [rows][K/2]
//         at 0, qh [rows][K/4] at rows*K/2, scales int8 [rows][K/16] at rows*K*3/4, then
//         d fp16 [rows][K/256] at rows*K*13/16.
//   MXFP4 split into two planes (a ggml block is 17 B: { u8 e; u8 qs[16]; } per 32 values):
//         qs [rows][K/2] at 0 (16 bytes per block), then e [rows][K/32] at rows*K/2.
//   Q4_0  split into two planes (a ggml block is 18 B: { fp16 d; u8 qs[16]; } per 32 values):
//         qs [rows][K/2] at 0, then d fp16 [rows][K/32] at rows*K/2.
//   Q5_K  [rows][K/256] blocks of 176 B, the ggml payload unchanged: { fp16 d, fp16 dmin,
//         u8 scales[12], u8 qh[32], u8 qs[128] }. Every block starts on a 16-byte boundary.
// The split layouts hold exactly the ggml bytes, re-ordered; their size equals the ggml size.
//
// Decoding follows ggml's dequantizers value for value (the to_float contract the reference
// uses at ggml-rocket.cpp:3894-3906): Q8_0 y = d*q; Q4_0 y = d*(q-8); Q4_K and Q5_K
// y = (d*sc)*q - dmin*m (Q5_K's q has a fifth bit); Q6_K y = (d*sc)*(q-32); MXFP4 y = kvalues_mxfp4[code] * 2^(e-128) (E2M1 codes doubled to integers,
// the E8M0 scale halved: GGML_E8M0_TO_FP32_HALF), exact in f32. Each product and difference is
// rounded on its own, then the f32 result is rounded once to fp16 (ggml_fp32_to_fp16_row, 3907).
//
// Every loader issues its loads unconditionally from an address inside the panel (the caller
// passes a valid row; a K position past the end reads position 0 instead) and remembers whether
// the item is real. The zeroing of an unreal item happens in decode(), when the data is used, so
// a pipeline can keep all of a stage's loads in flight until then.
#pragma once

#include "mx_common.h"

namespace mx {

__host__ __device__ inline int64_t packed_weight_bytes(int wt, int64_t rows, int64_t K) {
    switch (wt) {
        case T_F16: return rows * K * 2;
        case T_F16T: return tiled_rows(rows) * K * 2;
        case T_Q8_0: return rows * K + rows * (K / 32) * 2;
        case T_Q4_K: return rows * (K / 256) * 144;
        case T_Q6_K: return rows * (K / 256) * 210;
        case T_MXFP4: return rows * (K / 32) * 17;
        case T_Q4_0: return rows * (K / 32) * 18;
        case T_Q5_K: return rows * (K / 256) * 176;
        case T_Q4_KX: return rows % 32 ? -1 : rows * (K / 256) * 144;
        case T_Q8_0X: return rows % 32 ? -1 : rows * K + rows * (K / 32) * 2;
        case T_MXFP4X: return rows % 32 ? -1 : rows * (K / 32) * 17;
        case T_Q6_KX: return rows % 32 ? -1 : rows * (K / 256) * 210;
        default: return -1;
    }
}

// The 6-bit (scale, min) pair j of a Q4_K block, from its 12 packed bytes held as three
// little-endian words s0 (bytes 0-3), s1 (4-7), s2 (8-11).
__device__ __forceinline__ void q4k_sm(int j, uint32_t s0, uint32_t s1, uint32_t s2, int & sc, int & mn) {
    // pairs 0-3: 6-bit fields in bytes j (scale) and j+4 (min); pairs 4-7: the low / high nibble
    // of byte j+4 under the top two bits of bytes j-4 (scale) and j (min). With r = j % 4 the
    // three bytes are byte r of each word, whichever half j is in. Selects, not branches: j is
    // uniform, and a branch here would split the caller's scheduling region.
    const int sh = 8 * (j & 3);
    const uint32_t lo = (s0 >> sh) & 0xFFu, mid = (s1 >> sh) & 0xFFu, hi = (s2 >> sh) & 0xFFu;
    const uint32_t first = 0u - (uint32_t)(j < 4);   // all ones for pairs 0-3
    sc = (int)(((lo & 63u) & first) | (((hi & 0x0Fu) | ((lo >> 6) << 4)) & ~first));
    mn = (int)(((mid & 63u) & first) | (((hi >> 4) | ((mid >> 6) << 4)) & ~first));
}

__device__ __forceinline__ void zero_out(bool ok, u32x4 out[4]) {
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) out[i][e] = ok ? out[i][e] : 0u;
}

// The E2M1 value of an MXFP4 code, doubled (kvalues_mxfp4 of ggml-common.h): bit 3 is the sign,
// the low 3 bits index 0 1 2 3 4 6 8 12.
__device__ __forceinline__ int mxfp4_code(uint32_t c) {
    const int mag = (int)((0xC8643210u >> (4 * (c & 7u))) & 15u);
    return (c & 8u) ? -mag : mag;
}

// Packed-fp16 decoding, for kernels whose decode VALU is the bound (the skinny GEMM): a small
// integer code c (0 <= c < 256) is placed under the fp16 exponent of 1024, whose mantissa step is
// 1, by one byte permute per pair (v_perm_b32: bytes {c0, 0x64, c1, 0x64} = {1024 + c0, 1024 +
// c1}); subtracting the offset is exact, and one packed FMA applies scale and bias. The scale
// and bias are rounded to fp16 before the product, so a value can differ from the exact decode
// by a few fp16 ulp; the dequant kernels keep the exact form.
__device__ __forceinline__ half2v h2_of(uint32_t u) { return __builtin_bit_cast(half2v, u); }
__device__ __forceinline__ uint32_t u_of(half2v h) { return __builtin_bit_cast(uint32_t, h); }
// bytes 0,1 (sel01) or 2,3 (sel23) of x, each < 256, as {1024 + x.b0, 1024 + x.b1} etc.
constexpr uint32_t PERM_B01 = 0x04010400u, PERM_B23 = 0x04030402u;
__device__ __forceinline__ half2v magic_pair(uint32_t x, uint32_t sel) {
    return h2_of(__builtin_amdgcn_perm(0x64646464u, x, sel));
}
__device__ __forceinline__ half2v splat_h(float v) {
    const _Float16 h = (_Float16)v;
    return half2v{h, h};
}

// Global-load stage of one thread's share of a BK=64 weight tile: 32 consecutive-in-format
// values of one row. `u` (0/1) selects which half of the row's 64 values the thread takes.
// decode() produces them as fp16 in two runs of 16, at K offsets run0 and run1 of the slab.
template <int WT> struct WLoad;

template <> struct WLoad<T_F16> {
    u32x4 v[4];   // 32 fp16 values, k = k0 + 32u + 0..31
    bool ok;
    __device__ __forceinline__ void load(const uint8_t * W, int64_t rows, int64_t K, int64_t row,
                                         int64_t k0, int u, bool ok_row) {
        const int64_t k = k0 + 32 * u;
        ok = ok_row && k < K;
        const u32x4 * p = (const u32x4 *)(W + (row * K + (k < K ? k : 0)) * 2);
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = p[i];
    }
    __device__ __forceinline__ void decode_fast(int u, u32x4 out[4], int & run0, int & run1) const {
        decode(u, out, run0, run1);
    }
    __device__ __forceinline__ void decode(int u, u32x4 out[4], int & run0, int & run1) const {
#pragma unroll
        for (int i = 0; i < 4; i++) out[i] = v[i];
        zero_out(ok, out);
        run0 = 32 * u;
        run1 = 32 * u + 16;
    }
};

template <> struct WLoad<T_Q8_0> {
    u32x4 q[2];
    uint16_t d;
    bool ok;
    __device__ __forceinline__ void load(const uint8_t * W, int64_t rows, int64_t K, int64_t row,
                                         int64_t k0, int u, bool ok_row) {
        int64_t k = k0 + 32 * u;   // one 32-value block
        ok = ok_row && k < K;
        k = k < K ? k : 0;
        const u32x4 * p = (const u32x4 *)(W + row * K + k);
        const uint16_t * dp = (const uint16_t *)(W + rows * K) + row * (K / 32) + k / 32;
        q[0] = p[0];
        q[1] = p[1];
        d = *dp;
    }
    __device__ __forceinline__ void decode(int u, u32x4 out[4], int & run0, int & run1) const {
        const float df = h2f_bits(d);
        uint32_t o[16];
#pragma unroll
        for (int w = 0; w < 8; w++) {
            const uint32_t word = q[w / 4][w % 4];
            float f[4];
#pragma unroll
            for (int b = 0; b < 4; b++) f[b] = mul_rn(df, (float)(int8_t)((word >> (8 * b)) & 0xFFu));
            o[2 * w] = pack2h(f[0], f[1]);
            o[2 * w + 1] = pack2h(f[2], f[3]);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) out[i] = u32x4{o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]};
        zero_out(ok, out);
        run0 = 32 * u;
        run1 = 32 * u + 16;
    }
    // packed: a signed byte b as 1024 + (b ^ 0x80) = 1152 + b, less 1152, times d (a zero scale
    // where the item is masked: a finite code times zero is zero, one select per item)
    __device__ __forceinline__ void decode_fast(int u, u32x4 out[4], int & run0, int & run1) const {
        const half2v D = h2_of(ok ? (uint32_t)d * 0x10001u : 0u);
        const half2v OFF = {(_Float16)-1152.0f, (_Float16)-1152.0f};
        uint32_t o[16];
#pragma unroll
        for (int w = 0; w < 8; w++) {
            const uint32_t x = q[w / 4][w % 4] ^ 0x80808080u;
            o[2 * w] = u_of((magic_pair(x, PERM_B01) + OFF) * D);
            o[2 * w + 1] = u_of((magic_pair(x, PERM_B23) + OFF) * D);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) out[i] = u32x4{o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]};
        run0 = 32 * u;
        run1 = 32 * u + 16;
    }
};

// MXFP4: one 32-value block per item (the same slab halves as Q8_0).
template <> struct WLoad<T_MXFP4> {
    u32x4 qs;    // 16 bytes: weight j in the low nibble of byte j, weight j + 16 in the high one
    uint8_t e;
    bool ok;
    __device__ __forceinline__ void load(const uint8_t * W, int64_t rows, int64_t K, int64_t row,
                                         int64_t k0, int u, bool ok_row) {
        int64_t k = k0 + 32 * u;
        ok = ok_row && k < K;
        k = k < K ? k : 0;
        qs = *(const u32x4 *)(W + row * (K / 2) + k / 2);
        e = W[rows * (K / 2) + row * (K / 32) + k / 32];
    }
    // packed: a code's three magnitude bits moved to fp16 bits 11-9 and its sign to bit 15 read
    // as fp16 are the doubled E2M1 value times 2^-15 exactly (0 and 1 land in the subnormals: 0
    // and 2^-15). Two packed multiplies by powers of two scale that by 2^(e-113) = 2^15 * 2^(e-128):
    // first by 2^a, a = clamp(e - 113, 0, 15), exact (a result of at most two significant bits
    // between 2^-15 and 12), then by 2^(e-113-a), which rounds the exact product once, as the exact
    // decode's f32 product and fp16 rounding do. So the values are the exact decode's for every
    // e < 144; a block scale of 2^16 or more (every nonzero weight past the fp16 range) gives
    // finite values instead of infinities. A masked item multiplies by zero.
    __device__ __forceinline__ void decode_fast(int u, u32x4 out[4], int & run0, int & run1) const {
        const int s = (int)e - 113;
        const int a = s < 0 ? 0 : (s > 15 ? 15 : s);
        const int b = s - a;                           // -113 .. 127
        const uint32_t ha = (uint32_t)(a + 15) << 10;  // 2^a, a normal fp16
        // 2^b: normal for b >= -14, subnormal down to -24, below that a zero (as the product
        // would round to); b > 15 only for e >= 144, held at 2^15
        const uint32_t hb = !ok ? 0u
                          : b >= -14 ? (uint32_t)((b > 15 ? 15 : b) + 15) << 10
                          : b >= -24 ? 1u << (b + 24) : 0u;
        const half2v DA = h2_of(ha * 0x10001u), DB = h2_of(hb * 0x10001u);
        uint32_t o[16];
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const uint32_t x = qs[w];
            // per byte: magnitude << 1 in bits 3-1 and the sign in bit 7 (the fp16 high byte)
            const uint32_t lo = ((x << 1) & 0x0E0E0E0Eu) | ((x << 4) & 0x80808080u);
            const uint32_t hi = ((x >> 3) & 0x0E0E0E0Eu) | (x & 0x80808080u);
            o[2 * w] = u_of(h2_of(__builtin_amdgcn_perm(0u, lo, 0x010C000Cu)) * DA * DB);       // 4w, 4w+1
            o[2 * w + 1] = u_of(h2_of(__builtin_amdgcn_perm(0u, lo, 0x030C020Cu)) * DA * DB);   // 4w+2, 4w+3
            o[8 + 2 * w] = u_of(h2_of(__builtin_amdgcn_perm(0u, hi, 0x010C000Cu)) * DA * DB);   // 16+4w ...
            o[8 + 2 * w + 1] = u_of(h2_of(__builtin_amdgcn_perm(0u, hi, 0x030C020Cu)) * DA * DB);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) out[i] = u32x4{o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]};
        run0 = 32 * u;
        run1 = 32 * u + 16;
    }
    __device__ __forceinline__ void decode(int u, u32x4 out[4], int & run0, int & run1) const {
        // 2^(e-128) from its bits: a subnormal for e < 2
        const uint32_t eb = e < 2 ? (0x00200000u << e) : ((uint32_t)(e - 1) << 23);
        const float d = __builtin_bit_cast(float, eb);
        uint32_t o[16];
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const uint32_t word = qs[w];
            float lo[4], hi[4];
#pragma unroll
            for (int b = 0; b < 4; b++) {
                lo[b] = mul_rn(d, (float)mxfp4_code((word >> (8 * b)) & 15u));
                hi[b] = mul_rn(d, (float)mxfp4_code((word >> (8 * b + 4)) & 15u));
            }
            o[2 * w] = pack2h(lo[0], lo[1]);          // weights 4w .. 4w+3
            o[2 * w + 1] = pack2h(lo[2], lo[3]);
            o[8 + 2 * w] = pack2h(hi[0], hi[1]);      // weights 16 + 4w .. 16 + 4w+3
            o[8 + 2 * w + 1] = pack2h(hi[2], hi[3]);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) out[i] = u32x4{o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]};
        zero_out(ok, out);
        run0 = 32 * u;
        run1 = 32 * u + 16;
    }
};

// Q4_0: one 32-value block per item, as MXFP4.
template <> struct WLoad<T_Q4_0> {
    u32x4 qs;    // weight j in the low nibble of byte j, weight j + 16 in the high one
    uint16_t d;
    bool ok;
    __device__ __forceinline__ void load(const uint8_t * W, int64_t rows, int64_t K, int64_t row,
                                         int64_t k0, int u, bool ok_row) {
        int64_t k = k0 + 32 * u;
        ok = ok_row && k < K;
        k = k < K ? k : 0;
        qs = *(const u32x4 *)(W + row * (K / 2) + k / 2);
        d = *((const uint16_t *)(W + rows * (K / 2)) + row * (K / 32) + k / 32);
    }
    __device__ __forceinline__ void decode_fast(int u, u32x4 out[4], int & run0, int & run1) const {
        decode(u, out, run0, run1);
    }
    __device__ __forceinline__ void decode(int u, u32x4 out[4], int & run0, int & run1) const {
        const float df = h2f_bits(d);
        uint32_t o[16];
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const uint32_t word = qs[w];
            float lo[4], hi[4];
#pragma unroll
            for (int b = 0; b < 4; b++) {
                // (q - 8) * d: a 4-bit integer times an fp16 value, exact in f32
                lo[b] = mul_rn(df, (float)((int)((word >> (8 * b)) & 15u) - 8));
                hi[b] = mul_rn(df, (float)((int)((word >> (8 * b + 4)) & 15u) - 8));
            }
            o[2 * w] = pack2h(lo[0], lo[1]);
            o[2 * w + 1] = pack2h(lo[2], lo[3]);
            o[8 + 2 * w] = pack2h(hi[0], hi[1]);
            o[8 + 2 * w + 1] = pack2h(hi[2], hi[3]);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) out[i] = u32x4{o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]};
        zero_out(ok, out);
        run0 = 32 * u;
        run1 = 32 * u + 16;
    }
};

// Q5_K: as Q4_K, plus 16 bytes of fifth bits per item (qh[16u .. 16u+15], bits 2j and 2j+1).
template <> struct WLoad<T_Q5_K> {
    u32x4 hdr;   // d, dmin, scales[12]
    u32x4 qh;    // fifth bits of weights l = 16u .. 16u+15 of every sub-block
    u32x4 qs;    // 16 bytes of nibbles
    int j;       // quarter of the block (0..3)
    bool ok;
    __device__ __forceinline__ void load(const uint8_t * W, int64_t rows, int64_t K, int64_t row,
                                         int64_t k0, int u, bool ok_row) {
        const int64_t blk = k0 / 256;
        j = (int)((k0 % 256) / 64);
        ok = ok_row;
        const uint8_t * b = W + (row * (K / 256) + blk) * 176;
        hdr = *(const u32x4 *)b;
        qh = *(const u32x4 *)(b + 16 + 16 * u);
        qs = *(const u32x4 *)(b + 48 + 32 * j + 16 * u);
    }
    // Byte b of qs is q[32j + 16u + b]: its low nibble is weight 64j + 16u + b (sub-block 2j)
    // with fifth bit 2j of qh byte b, its high nibble weight 64j + 32 + 16u + b (sub-block
    // 2j+1) with bit 2j+1.
    __device__ __forceinline__ void decode_fast(int u, u32x4 out[4], int & run0, int & run1) const {
        decode(u, out, run0, run1);
    }
    __device__ __forceinline__ void decode(int u, u32x4 out[4], int & run0, int & run1) const {
        const float d = h2f_bits((uint16_t)(hdr[0] & 0xFFFFu));
        const float dmin = h2f_bits((uint16_t)(hdr[0] >> 16));
        int s0, m0, s1, m1;
        q4k_sm(2 * j, hdr[1], hdr[2], hdr[3], s0, m0);
        q4k_sm(2 * j + 1, hdr[1], hdr[2], hdr[3], s1, m1);
        // d * sc has at most 17 significant bits and d * sc * q at most 22: exact in f32, so one
        // fma rounds d*sc*q - dmin*m as the CPU's rounded product followed by the difference
        const float d0 = d * (float)s0, mm0 = dmin * (float)m0;
        const float d1 = d * (float)s1, mm1 = dmin * (float)m1;
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int w = 0; w < 4; w++) {
            // the fifth bits as 0x10 per byte, for the low and the high nibbles
            const uint32_t b0 = ((qh[w] >> (2 * j)) & 0x01010101u) << 4;
            const uint32_t b1 = ((qh[w] >> (2 * j + 1)) & 0x01010101u) << 4;
            uint32_t l5 = (qs[w] & 0x0F0F0F0Fu) | b0, h5 = ((qs[w] >> 4) & 0x0F0F0F0Fu) | b1;
            asm("" : "+v"(l5), "+v"(h5));
            float fl[4], fh[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                fl[i] = fma_rn(d0, (float)((l5 >> (8 * i)) & 0xFFu), -mm0);
                fh[i] = fma_rn(d1, (float)((h5 >> (8 * i)) & 0xFFu), -mm1);
            }
            lo[2 * w] = pack2h(fl[0], fl[1]);
            lo[2 * w + 1] = pack2h(fl[2], fl[3]);
            hi[2 * w] = pack2h(fh[0], fh[1]);
            hi[2 * w + 1] = pack2h(fh[2], fh[3]);
        }
        out[0] = u32x4{lo[0], lo[1], lo[2], lo[3]};
        out[1] = u32x4{lo[4], lo[5], lo[6], lo[7]};
        out[2] = u32x4{hi[0], hi[1], hi[2], hi[3]};
        out[3] = u32x4{hi[4], hi[5], hi[6], hi[7]};
        zero_out(ok, out);
        run0 = 16 * u;
        run1 = 32 + 16 * u;
    }
};

template <> struct WLoad<T_Q4_K> {
    u32x4 hdr;   // d, dmin, scales[12]
    u32x4 qs;    // 16 bytes of nibbles
    int j;       // quarter of the block (0..3)
    bool ok;
    __device__ __forceinline__ void load(const uint8_t * W, int64_t rows, int64_t K, int64_t row,
                                         int64_t k0, int u, bool ok_row) {
        const int64_t blk = k0 / 256;
        j = (int)((k0 % 256) / 64);
        ok = ok_row;
        const uint8_t * b = W + (row * (K / 256) + blk) * 144;
        hdr = *(const u32x4 *)b;
        qs = *(const u32x4 *)(b + 16 + 32 * j + 16 * u);
    }
    // Byte b of qs (b = 0..15) is q[32j + 16u + b]: its low nibble is weight 64j + 16u + b
    // (sub-block 2j), its high nibble weight 64j + 32 + 16u + b (sub-block 2j+1).
    __device__ __forceinline__ void decode(int u, u32x4 out[4], int & run0, int & run1) const {
        const float d = h2f_bits((uint16_t)(hdr[0] & 0xFFFFu));
        const float dmin = h2f_bits((uint16_t)(hdr[0] >> 16));
        int s0, m0, s1, m1;
        q4k_sm(2 * j, hdr[1], hdr[2], hdr[3], s0, m0);
        q4k_sm(2 * j + 1, hdr[1], hdr[2], hdr[3], s1, m1);
        // d * sc and dmin * m have at most 17 significant bits and d * sc * q at most 21: all
        // exact in f32, so one fma rounds d*sc*q - dmin*m exactly as the CPU's rounded product
        // followed by the difference does
        const float d0 = d * (float)s0, mm0 = dmin * (float)m0;
        const float d1 = d * (float)s1, mm1 = dmin * (float)m1;
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int w = 0; w < 4; w++) {
            uint32_t l4 = qs[w] & 0x0F0F0F0Fu, h4 = (qs[w] >> 4) & 0x0F0F0F0Fu;   // nibbles as bytes
            // opaque to the compiler, so each byte converts with one v_cvt_f32_ubyteN instead of
            // a 4-bit extract folded from the mask plus a conversion
            asm("" : "+v"(l4), "+v"(h4));
            float fl[4], fh[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                fl[i] = fma_rn(d0, (float)((l4 >> (8 * i)) & 0xFFu), -mm0);
                fh[i] = fma_rn(d1, (float)((h4 >> (8 * i)) & 0xFFu), -mm1);
            }
            lo[2 * w] = pack2h(fl[0], fl[1]);
            lo[2 * w + 1] = pack2h(fl[2], fl[3]);
            hi[2 * w] = pack2h(fh[0], fh[1]);
            hi[2 * w + 1] = pack2h(fh[2], fh[3]);
        }
        out[0] = u32x4{lo[0], lo[1], lo[2], lo[3]};
        out[1] = u32x4{lo[4], lo[5], lo[6], lo[7]};
        out[2] = u32x4{hi[0], hi[1], hi[2], hi[3]};
        out[3] = u32x4{hi[4], hi[5], hi[6], hi[7]};
        zero_out(ok, out);
        run0 = 16 * u;
        run1 = 32 + 16 * u;
    }
    // packed: (1024 + q - 1024) * fp16(d*sc) + fp16(-dmin*m)
    __device__ __forceinline__ void decode_fast(int u, u32x4 out[4], int & run0, int & run1) const {
        const float d = h2f_bits((uint16_t)(hdr[0] & 0xFFFFu));
        const float dmin = h2f_bits((uint16_t)(hdr[0] >> 16));
        int s0, m0, s1, m1;
        q4k_sm(2 * j, hdr[1], hdr[2], hdr[3], s0, m0);
        q4k_sm(2 * j + 1, hdr[1], hdr[2], hdr[3], s1, m1);
        // a masked item decodes to zero through zero scales
        const float z = ok ? 1.0f : 0.0f;
        const half2v S0 = splat_h(z * (d * (float)s0)), B0 = splat_h(z * -(dmin * (float)m0));
        const half2v S1 = splat_h(z * (d * (float)s1)), B1 = splat_h(z * -(dmin * (float)m1));
        const half2v OFF = {(_Float16)-1024.0f, (_Float16)-1024.0f};
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const uint32_t l4 = qs[w] & 0x0F0F0F0Fu, h4 = (qs[w] >> 4) & 0x0F0F0F0Fu;
            lo[2 * w] = u_of((magic_pair(l4, PERM_B01) + OFF) * S0 + B0);
            lo[2 * w + 1] = u_of((magic_pair(l4, PERM_B23) + OFF) * S0 + B0);
            hi[2 * w] = u_of((magic_pair(h4, PERM_B01) + OFF) * S1 + B1);
            hi[2 * w + 1] = u_of((magic_pair(h4, PERM_B23) + OFF) * S1 + B1);
        }
        out[0] = u32x4{lo[0], lo[1], lo[2], lo[3]};
        out[1] = u32x4{lo[4], lo[5], lo[6], lo[7]};
        out[2] = u32x4{hi[0], hi[1], hi[2], hi[3]};
        out[3] = u32x4{hi[4], hi[5], hi[6], hi[7]};
        run0 = 16 * u;
        run1 = 32 + 16 * u;
    }
};

// Q4_K regrouped by 32 rows (T_Q4_KX): per (32-row group, 256-value block) 4608 bytes, the 32
// headers (16 B each, row order) then per 64-value quarter j the 32 rows' 32 nibble bytes. The
// same decode as Q4_K; lanes that take consecutive rows read consecutive bytes.
constexpr int Q4KX_GROUP = 32;
__host__ __device__ inline int64_t q4kx_block(int64_t row, int64_t blk, int64_t nblk) {
    return ((row / Q4KX_GROUP) * nblk + blk) * (Q4KX_GROUP * 144);
}
// The regrouped layouts are loaded through a Lane, the loop-invariant part of a lane's loads:
// the expert's first group-block in each plane (block-uniform, so it lives in scalar registers)
// and the 32-bit byte offsets of the lane's pieces from there (an expert is whole 32-row groups,
// and the host keeps an expert's share of a plane under 2^31 bytes). A slab's load then adds a
// block-uniform slab offset to the base and the fixed lane offset, with no per-lane address
// arithmetic in the loop. `row0` is the expert's first row, `nloc` the lane's row inside it.
template <> struct WLoad<T_Q4_KX> : WLoad<T_Q4_K> {
    struct Lane {
        const uint8_t * base;
        uint32_t oh, oq;   // the row's header and its quant bytes of quarter 0, half u
    };
    __device__ __forceinline__ static Lane lane(const uint8_t * W, int64_t rows, int64_t K, int64_t row0, int nloc,
                                                int u) {
        const int64_t nblk = K / 256;
        const uint32_t g = (uint32_t)(nloc / Q4KX_GROUP) * (uint32_t)nblk * (uint32_t)(Q4KX_GROUP * 144);
        const int r = nloc % Q4KX_GROUP;
        return {W + q4kx_block(row0, 0, nblk), g + 16u * r, g + 16u * Q4KX_GROUP + 32u * r + 16u * u};
    }
    __device__ __forceinline__ void load(const Lane & L, int64_t K, int64_t k0, bool ok_row) {
        j = (int)((k0 % 256) / 64);
        ok = ok_row;
        const uint8_t * b = L.base + (k0 / 256) * (Q4KX_GROUP * 144);
        hdr = *(const u32x4 *)(b + L.oh);
        qs = *(const u32x4 *)((b + 32 * Q4KX_GROUP * j) + L.oq);
    }
};

// Q8_0 and MXFP4 regrouped by 32 rows (T_Q8_0X, T_MXFP4X): the two planes of the split layouts,
// each ordered by (32-row group, 32-value block) and, inside, by row: per group and block the 32
// rows' quants (Q8_0: 32 bytes each, 1 KiB; MXFP4: 16 bytes each, 512 B), and in the second plane
// the 32 rows' scales (Q8_0: fp16, 64 B; MXFP4: the E8M0 byte, 32 B). The same decode as the
// split layouts; lanes that take consecutive rows read consecutive bytes.
__host__ __device__ inline int64_t x32_index(int64_t row, int64_t blk, int64_t nblk) {
    return ((row / 32) * nblk + blk) * 32 + row % 32;
}
// A lane's item is block k0 / 32 + u; in the last slab of a K that is an odd number of blocks
// the u = 1 item lies past K: it reads block k0 / 32 of its row (lane offsets o*0) and decodes to
// zero.
template <> struct WLoad<T_Q8_0X> : WLoad<T_Q8_0> {
    struct Lane {
        const uint8_t * qb, * sb;   // the expert's first group-block of quants and of scales
        uint32_t oq, os, oq0, os0;
        int u;
    };
    __device__ __forceinline__ static Lane lane(const uint8_t * W, int64_t rows, int64_t K, int64_t row0, int nloc,
                                                int u) {
        const int64_t nblk = K / 32, x0 = x32_index(row0, 0, nblk);
        const uint32_t gb = (uint32_t)(nloc / 32) * (uint32_t)nblk, r = (uint32_t)(nloc % 32);
        const uint32_t oq0 = (gb * 32 + r) * 32, os0 = (gb * 32 + r) * 2;
        return {W + x0 * 32, W + rows * K + x0 * 2, oq0 + 1024u * u, os0 + 64u * u, oq0, os0, u};
    }
    __device__ __forceinline__ void load(const Lane & L, int64_t K, int64_t k0, bool ok_row) {
        ok = ok_row && k0 + 32 * L.u < K;
        const int64_t b0 = k0 / 32;
        const u32x4 * p = (const u32x4 *)((L.qb + b0 * 1024) + (ok ? L.oq : L.oq0));
        q[0] = p[0];
        q[1] = p[1];
        d = *(const uint16_t *)((L.sb + b0 * 64) + (ok ? L.os : L.os0));
    }
};
template <> struct WLoad<T_MXFP4X> : WLoad<T_MXFP4> {
    struct Lane {
        const uint8_t * qb, * sb;
        uint32_t oq, os, oq0, os0;
        int u;
    };
    __device__ __forceinline__ static Lane lane(const uint8_t * W, int64_t rows, int64_t K, int64_t row0, int nloc,
                                                int u) {
        const int64_t nblk = K / 32, x0 = x32_index(row0, 0, nblk);
        const uint32_t gb = (uint32_t)(nloc / 32) * (uint32_t)nblk, r = (uint32_t)(nloc % 32);
        const uint32_t oq0 = (gb * 32 + r) * 16, os0 = gb * 32 + r;
        return {W + x0 * 16, W + rows * (K / 2) + x0, oq0 + 512u * u, os0 + 32u * u, oq0, os0, u};
    }
    __device__ __forceinline__ void load(const Lane & L, int64_t K, int64_t k0, bool ok_row) {
        ok = ok_row && k0 + 32 * L.u < K;
        const int64_t b0 = k0 / 32;
        qs = *(const u32x4 *)((L.qb + b0 * 512) + (ok ? L.oq : L.oq0));
        e = *((L.sb + b0 * 32) + (ok ? L.os : L.os0));
    }
};

template <> struct WLoad<T_Q6_K> {
    u32x4 qla, qlb, qh;   // ql[l], ql[l+32], qh[l] for the thread's 16 l
    uint32_t sc;          // the 4 int8 scales it needs, packed
    uint16_t d;
    int hi;               // 0: weights l, l+32 of the half; 1: l+64, l+96
    bool ok;
    __device__ __forceinline__ void load(const uint8_t * W, int64_t rows, int64_t K, int64_t row,
                                         int64_t k0, int u, bool ok_row) {
        const int64_t blk = k0 / 256;
        const int q4 = (int)((k0 % 256) / 64);
        const int h = q4 >> 1;
        hi = q4 & 1;
        ok = ok_row;
        const int l0 = 16 * u;
        const uint8_t * ql = W + row * (K / 2) + blk * 128 + 64 * h + l0;
        const uint8_t * qhp = W + rows * (K / 2) + row * (K / 4) + blk * 64 + 32 * h + l0;
        const int8_t * scp = (const int8_t *)(W + rows * (K / 2) + rows * (K / 4)) + row * (K / 16) + blk * 16 + 8 * h;
        const uint16_t * dp = (const uint16_t *)(W + rows * (K / 2) + rows * (K / 4) + rows * (K / 16)) + row * (K / 256) + blk;
        qla = *(const u32x4 *)ql;
        qlb = *(const u32x4 *)(ql + 32);
        qh = *(const u32x4 *)qhp;
        // scales for sub-blocks (l/16) + {0,2} (hi=0) or + {4,6} (hi=1), l/16 = u
        const int i0 = u + 4 * hi;
        sc = (uint32_t)(uint8_t)scp[i0] | ((uint32_t)(uint8_t)scp[i0 + 2] << 8);
        d = *dp;
    }
    // packed: the 6-bit codes assembled four bytes at a time (nibble of ql, two bits of qh),
    // each placed under 1024 (magic_pair), less 1024 + 32, times the sub-block scale d * sc
    // rounded to fp16 (zero where the item is masked)
    __device__ __forceinline__ void decode_fast(int u, u32x4 out[4], int & run0, int & run1) const {
        const float df = h2f_bits(d);
        const half2v DA = splat_h(ok ? df * (float)(int8_t)(sc & 0xFFu) : 0.0f);
        const half2v DB = splat_h(ok ? df * (float)(int8_t)((sc >> 8) & 0xFFu) : 0.0f);
        const half2v OFF = {(_Float16)-1056.0f, (_Float16)-1056.0f};
        const int sn = 4 * hi;
        uint32_t a[8], b[8];
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const uint32_t va = ((qla[w] >> sn) & 0x0F0F0F0Fu) | (((qh[w] >> sn) & 0x03030303u) << 4);
            const uint32_t vb = ((qlb[w] >> sn) & 0x0F0F0F0Fu) | (((qh[w] >> (sn + 2)) & 0x03030303u) << 4);
            a[2 * w] = u_of((magic_pair(va, PERM_B01) + OFF) * DA);
            a[2 * w + 1] = u_of((magic_pair(va, PERM_B23) + OFF) * DA);
            b[2 * w] = u_of((magic_pair(vb, PERM_B01) + OFF) * DB);
            b[2 * w + 1] = u_of((magic_pair(vb, PERM_B23) + OFF) * DB);
        }
        out[0] = u32x4{a[0], a[1], a[2], a[3]};
        out[1] = u32x4{a[4], a[5], a[6], a[7]};
        out[2] = u32x4{b[0], b[1], b[2], b[3]};
        out[3] = u32x4{b[4], b[5], b[6], b[7]};
        run0 = 16 * u;
        run1 = 32 + 16 * u;
    }
    __device__ __forceinline__ void decode(int u, u32x4 out[4], int & run0, int & run1) const {
        const float df = h2f_bits(d);
        const float da = mul_rn(df, (float)(int8_t)(sc & 0xFFu));
        const float db = mul_rn(df, (float)(int8_t)((sc >> 8) & 0xFFu));
        const int sn = 4 * hi;   // nibble of ql
        const int sh = 4 * hi;   // bit pair base in qh
        uint32_t a[8], b[8];
#pragma unroll
        for (int w = 0; w < 4; w++) {
#pragma unroll
            for (int p = 0; p < 2; p++) {
                float fa[2], fb[2];
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const int bi = 2 * p + e;   // byte within the word
                    const uint32_t la = (qla[w] >> (8 * bi)) & 0xFFu;
                    const uint32_t lb = (qlb[w] >> (8 * bi)) & 0xFFu;
                    const uint32_t hh = (qh[w] >> (8 * bi)) & 0xFFu;
                    const int qa = (int)(((la >> sn) & 15u) | (((hh >> sh) & 3u) << 4)) - 32;
                    const int qb = (int)(((lb >> sn) & 15u) | (((hh >> (sh + 2)) & 3u) << 4)) - 32;
                    fa[e] = mul_rn(da, (float)qa);
                    fb[e] = mul_rn(db, (float)qb);
                }
                a[2 * w + p] = pack2h(fa[0], fa[1]);
                b[2 * w + p] = pack2h(fb[0], fb[1]);
            }
        }
        out[0] = u32x4{a[0], a[1], a[2], a[3]};
        out[1] = u32x4{a[4], a[5], a[6], a[7]};
        out[2] = u32x4{b[0], b[1], b[2], b[3]};
        out[3] = u32x4{b[4], b[5], b[6], b[7]};
        zero_out(ok, out);
        run0 = 16 * u;
        run1 = 32 + 16 * u;
    }
};

// Q6_K regrouped by 32 rows (T_Q6_KX): the four planes of the split layout, each ordered by
// (32-row group, 256-value block) and, inside, so that the 32 rows' pieces a wave loads together
// are consecutive: ql as [16-byte chunk (8)][row (32)] (4 KiB a group-block), qh as [chunk (4)]
// [row] (2 KiB), scales as [row][16 bytes] (512 B), d as [row] (64 B). The same decode as Q6_K.
struct Q6kxPlanes {
    int64_t ql, qh, sc, d;   // byte offsets of the row's group-block in each plane
    int r;
};
__host__ __device__ inline Q6kxPlanes q6kx_planes(int64_t rows, int64_t K, int64_t row, int64_t blk) {
    const int64_t gb = (row / 32) * (K / 256) + blk;
    return {gb * 4096, rows * (K / 2) + gb * 2048, rows * (K / 2) + rows * (K / 4) + gb * 512,
            rows * (K / 2) + rows * (K / 4) + rows * (K / 16) + gb * 64, (int)(row % 32)};
}
template <> struct WLoad<T_Q6_KX> : WLoad<T_Q6_K> {
    struct Lane {
        const uint8_t * ql, * qh, * sc, * d;   // the expert's first group-block in each plane
        uint32_t oql, oqh, osc, od;
        uint32_t sel;   // byte permute taking scale bytes u and u + 2 of a scale word
    };
    __device__ __forceinline__ static Lane lane(const uint8_t * W, int64_t rows, int64_t K, int64_t row0, int nloc,
                                                int u) {
        const Q6kxPlanes p = q6kx_planes(rows, K, row0, 0);
        const uint32_t gb = (uint32_t)(nloc / 32) * (uint32_t)(K / 256), r = (uint32_t)(nloc % 32);
        return {W + p.ql, W + p.qh, W + p.sc, W + p.d, gb * 4096 + (32u * u + r) * 16, gb * 2048 + (32u * u + r) * 16,
                gb * 512 + r * 16, gb * 64 + 2 * r, 0x0C0C0000u | ((uint32_t)(u + 2) << 8) | (uint32_t)u};
    }
    __device__ __forceinline__ void load(const Lane & L, int64_t K, int64_t k0, bool ok_row) {
        const int64_t blk = k0 / 256;
        const int q4 = (int)((k0 % 256) / 64);
        const int h = q4 >> 1;
        hi = q4 & 1;
        ok = ok_row;
        const uint8_t * pl = L.ql + blk * 4096 + h * 2048;
        qla = *(const u32x4 *)(pl + L.oql);
        qlb = *(const u32x4 *)((pl + 1024) + L.oql);
        qh = *(const u32x4 *)((L.qh + blk * 2048 + h * 1024) + L.oqh);
        // scales u + 4 hi and u + 4 hi + 2 of the half h: bytes u and u + 2 of one word
        const uint32_t sw = *(const uint32_t *)((L.sc + blk * 512 + 8 * h + 4 * hi) + L.osc);
        sc = __builtin_amdgcn_perm(0u, sw, L.sel);
        d = *(const uint16_t *)((L.d + blk * 64) + L.od);
    }
};

}  // namespace mx
