// SPDX-License-Identifier: MIT
// Device-side helpers shared by the gfx950 kernels: vector types, MFMA wrappers, the LDS
// swizzle, fp16 conversion and the exact-rounding arithmetic the weight decoders use.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mx {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int WAVE = 64;

// ggml type ids (ggml.h enum ggml_type) for the weight formats this path decodes, and layouts of
// this library's own, which are no ggml types: T_F16T, tiled fp16 (tiled_index below), and the
// expert-stack layouts regrouped by 32 rows, T_Q4_KX, T_Q8_0X, T_Q6_KX and T_MXFP4X
// (WLoad<T_Q4_KX> etc. in mx_weights.h).
enum : int { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_I32 = 26,
             T_BF16 = 30, T_MXFP4 = 39,
             T_F16T = 0x101, T_Q4_KX = 0x10C, T_Q8_0X = 0x108, T_Q6_KX = 0x10E, T_MXFP4X = 0x127 };

// The tiled fp16 layout of a [rows][K] matrix (K % 32 == 0): 16 x 32 tiles of 1 KB, row-major
// inside, tile (row / 16, k / 32) at ((row / 16) * (K / 32) + k / 32) * 512 values; rows padded to
// a multiple of 16 (the padding is never read). One 64-lane, 16-byte-per-lane load reads one
// tile: 1 KB of consecutive bytes, whatever K-slab width the reader stages, and each 16-row
// block of a matrix is one sequential run along K.
__host__ __device__ inline int64_t tiled_rows(int64_t rows) { return (rows + 15) & ~(int64_t)15; }

__host__ __device__ inline int64_t tiled_index(int64_t row, int64_t k, int64_t K) {
    return ((((row >> 4) * (K >> 5)) + (k >> 5)) << 9) + ((row & 15) << 5) + (k & 31);
}

// D(32x32, f32) += A(32x16, f16) . B(16x32, f16). Lane l holds A row (l % 32) and B column
// (l % 32), K slots 8*(l/32)+0..7. D: lane l, element i -> row 8*(i/4) + 4*(l/32) + (i%4),
// column l % 32.
__device__ __forceinline__ float16v mfma32(const half8 & a, const half8 & b, const float16v & c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Byte offset of the 16-byte chunk `c` of row `r` in an LDS tile whose rows hold CHUNKS 16-byte
// chunks (CHUNKS a power of two, 4..16). LDS has 64 banks of 4 bytes, so a 256-byte window
// holds 16 chunk slots and 16 / CHUNKS rows. The chunk index is XORed with the row's index
// within each group of CHUNKS windows, so 16 consecutive rows read at one logical chunk (what an
// MFMA fragment read does) land on 16 distinct slots: no bank conflict.
template <int CHUNKS>
__device__ __forceinline__ int swz(int r, int c) {
    constexpr int RPW = 16 / CHUNKS;   // rows per 256-byte window
    return r * (CHUNKS * 16) + ((c ^ ((r / RPW) & (CHUNKS - 1))) << 4);
}

__device__ __forceinline__ uint16_t f2h_bits(float f) {
    _Float16 h = (_Float16)f;   // v_cvt_f16_f32, round to nearest even
    return __builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ float h2f_bits(uint16_t b) {
    return (float)__builtin_bit_cast(_Float16, b);
}
typedef float float2v __attribute__((ext_vector_type(2)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
// two f32 -> packed fp16, each rounded to nearest even (one v_cvt_pk_f16_f32)
__device__ __forceinline__ uint32_t pack2h(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(float2v{a, b}, half2v));
}

// Separately rounded multiply and subtract: the decoders must not fuse d*q - m into one FMA,
// because the CPU dequantizer rounds the product before the subtraction, and a result that is
// then converted to fp16 must not be folded into the conversion: the backend turns
// fptrunc(a * b) into one v_fma_mix, which rounds once where the CPU rounds to f32 and then to
// fp16 (it does so even without the contract flag). The empty asm makes the rounded f32 value
// the only thing the next operation can see.
__device__ __forceinline__ float mul_rn(float a, float b) {
    float p;
    {
#pragma clang fp contract(off)
        p = a * b;
    }
    asm("" : "+v"(p));
    return p;
}
__device__ __forceinline__ float sub_rn(float a, float b) {
    float d;
    {
#pragma clang fp contract(off)
        d = a - b;
    }
    asm("" : "+v"(d));
    return d;
}
// a * b + c rounded once to f32, pinned there like mul_rn (no fold into an f16 conversion). Only
// for operands whose product is exact in f32, where it equals sub_rn(mul_rn(a, b), -c).
__device__ __forceinline__ float fma_rn(float a, float b, float c) {
    float r = __builtin_fmaf(a, b, c);
    asm("" : "+v"(r));
    return r;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}

// One activation row of up to PACK_WAVE_K values packed by one wave: x / s as fp16 and s = the
// row's max |x| (1 for a zero row), rounded as the block-per-row pack does (the product rounded
// to f32, then to fp16). The max comes from lane exchanges alone, with all of the row's loads in
// flight at once. Row-major output at A16 + m * lda, or (TL) the tiled layout over K.
constexpr int PACK_WAVE_VEC = 16;                       // float4 a lane
constexpr int PACK_WAVE_K = WAVE * PACK_WAVE_VEC * 4;   // 4096 values
template <bool TL>
__device__ __forceinline__ void pack_row_wave(const float * x, int m, int K, uint16_t * A16, int64_t lda,
                                              float * scales, int lane) {
    const int n4 = K / 4;
    float4v v[PACK_WAVE_VEC];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < PACK_WAVE_VEC; i++) {
        const int c = lane + i * WAVE;
        v[i] = c < n4 ? *(const float4v *)(x + 4 * c) : float4v{0, 0, 0, 0};
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[i][0]), fabsf(v[i][1])), fmaxf(fabsf(v[i][2]), fabsf(v[i][3]))));
    }
    amax = wave_max(amax);
    const float s = amax > 0.0f ? amax : 1.0f;
    const float inv = 1.0f / s;
#pragma unroll
    for (int i = 0; i < PACK_WAVE_VEC; i++) {
        const int c = lane + i * WAVE;
        if (c < n4) {
            u32x2 o;
            o[0] = pack2h(mul_rn(v[i][0], inv), mul_rn(v[i][1], inv));
            o[1] = pack2h(mul_rn(v[i][2], inv), mul_rn(v[i][3], inv));
            *(u32x2 *)(TL ? A16 + tiled_index(m, 4 * c, K) : A16 + (int64_t)m * lda + 4 * c) = o;
        }
    }
    if (lane == 0) scales[m] = s;
}

// Blocks are handed to the 8 XCDs round-robin by linear id. Renumber so that each XCD gets a
// contiguous run of logical ids (XCD x takes ids [x q + min(x, r), ...) of its q or q + 1
// blocks, q = n / 8, r = n % 8; a bijection for any n): work items that share an operand panel
// then share one XCD's L2.
__device__ __forceinline__ int xcd_tile(int bid, int nblocks) {
    const int q = nblocks / 8, r = nblocks % 8, x = bid % 8;
    return x * q + min(x, r) + bid / 8;
}

// Multiplies a wave's MI x NJ accumulator tiles (32x32 MFMA output layout: element e of tile
// row i is row base + 32 i + 8 (e / 4) + 4 lg + e % 4) by their row scales, loading every scale
// and applying it before the caller's first output store. Loads and stores retire through one
// in-order counter, so a scale loaded, or first used, between stores would wait for every
// store issued before it: one memory round trip per row, which a row-by-row epilogue costs.
template <int MI, int NJ, class Acc>
__device__ __forceinline__ void scale_rows(Acc (&acc)[MI][NJ], const float * scales, int base, int lg,
                                           int M) {
    float rs[MI][16];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int e = 0; e < 16; e++)
            rs[i][e] = scales[min(base + i * 32 + 8 * (e / 4) + 4 * lg + (e % 4), M - 1)];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] *= rs[i][e];
    // the empty asm keeps the products here: left alone, the compiler sinks each multiply into
    // the bounds-checked store that consumes it, after earlier stores
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) asm("" : "+v"(acc[i][j]));
    __builtin_amdgcn_sched_barrier(0);
}

}  // namespace mx
