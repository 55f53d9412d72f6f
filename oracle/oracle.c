/*
 * oracle.c -- CPU restatement of the prefill hot path, used ONLY as a checker.
 *
 * This file is test infrastructure. Only tests/, __graft_entry__.smoke() and the cpu_baseline
 * leg of bench.py load it, and only to check or time the HIP path. The product library
 * (libmi355x.so) never links, loads or calls it.
 *
 * What it restates, each from the reference file:line it follows:
 *   - fp16 <-> fp32 conversion, round-to-nearest-even (the semantics of ggml_fp32_to_fp16 that
 *     ggml-rocket.cpp:1473, 1516, 3860, 3907 rely on);
 *   - the splitmix64 fills of test-common.h:181-193 and a Box-Muller normal fill on top of them;
 *   - the Q8_0 / Q4_K / Q6_K / MXFP4 block decoders that ggml_get_type_traits(t)->to_float provides
 *     (ggml-rocket.cpp:3894-3906). ggml is an un-vendored third-party dependency of the
 *     reference (CMakeLists.txt:176-186, compatible range llama.cpp b10558-b11539 per
 *     README.md:380-391); the decoders here are written from ggml's published block formats;
 *   - a quantizer for synthetic weights (the reference quantizes with ggml_quantize_chunk,
 *     test-rocket-matmul.cpp:102; its exact bytes are not reproducible without ggml, and the
 *     parity tests do not need them because both sides decode the same bytes);
 *   - the fp64 GEMM of rocket_cpu_matmul_slice (ggml-rocket.cpp:4048-4084) and of the quant
 *     golden (test-rocket-matmul.cpp:343-351);
 *   - the full-precision attention reference rocket_fa_ref_f32 (ggml-rocket.cpp:5392-5442) and
 *     the test oracle ref_fa (test-rocket-fa.cpp:101-135), which rounds Q to fp16 first;
 *   - MUL_MAT_ID semantics (ggml-rocket.cpp:6654-6662) with the counting-sort bucketing of
 *     6706-6732.
 *
 * Built with -ffp-contract=off so that no multiply-add is fused: the dequantizers compute
 * d*sc, dmin*m, then y = d1*q - m1 as separate roundings, which the HIP decoders mirror.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

#define ORC_API __attribute__((visibility("default")))

/* ggml type ids (ggml.h enum ggml_type); the formats this path carries. */
enum { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_BF16 = 30,
       T_MXFP4 = 39 };

/* ------------------------------------------------------------------------------------------ */
/* fp16                                                                                        */
/* ------------------------------------------------------------------------------------------ */

ORC_API uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                       /* inf / nan */
        if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);   /* >= 65520 rounds to inf */
    if (ax >= 0x38800000u) {                        /* normal half: >= 2^-14 */
        const uint32_t r = ax + 0x0fffu + ((ax >> 13) & 1u);   /* nearest, ties to even */
        return (uint16_t)(sign | ((r - 0x38000000u) >> 13));
    }
    /* subnormal half or zero: units of 2^-24, scaled exactly, rounded to nearest even */
    float af;
    memcpy(&af, &ax, 4);
    const uint32_t m = (uint32_t)rintf(af * 16777216.0f);
    return (uint16_t)(sign | m);
}

ORC_API float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) { x = sign; }
        else {
            float f = (float)m * (1.0f / 16777216.0f);   /* m * 2^-24, exact */
            memcpy(&x, &f, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

ORC_API void orc_f32_to_f16_row(const float * src, uint16_t * dst, int64_t n) {
    for (int64_t i = 0; i < n; i++) dst[i] = orc_f32_to_f16(src[i]);
}
ORC_API void orc_f16_to_f32_row(const uint16_t * src, float * dst, int64_t n) {
    for (int64_t i = 0; i < n; i++) dst[i] = orc_f16_to_f32(src[i]);
}

static inline float bf16_to_f32(uint16_t b) {
    uint32_t x = (uint32_t)b << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* ------------------------------------------------------------------------------------------ */
/* fills (test-common.h:181-193)                                                               */
/* ------------------------------------------------------------------------------------------ */

static inline uint64_t rk_hash(uint64_t seed, uint64_t i) {
    uint64_t z = seed * 0x9E3779B97F4A7C15ull + i + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* uniform in [-amp, amp): the period-free splitmix64 fill of test-common.h:190-193 */
ORC_API void orc_fill_uniform(float * v, int64_t n, uint64_t seed, float amp) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++)
        v[i] = amp * (float)((double)(rk_hash(seed, (uint64_t)i) >> 11) * (2.0 / 9007199254740992.0) - 1.0);
}

/* N(mean, std): Box-Muller over two splitmix64 uniforms per element (index 2i, 2i+1). */
ORC_API void orc_fill_normal(float * v, int64_t n, uint64_t seed, float mean, float std) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) {
        const double u1 = ((double)(rk_hash(seed, 2 * (uint64_t)i) >> 11) + 1.0) / 9007199254740993.0;
        const double u2 = (double)(rk_hash(seed, 2 * (uint64_t)i + 1) >> 11) / 9007199254740992.0;
        const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
        v[i] = (float)(mean + std * z);
    }
}

/* ------------------------------------------------------------------------------------------ */
/* block formats (ggml's published layouts)                                                    */
/*   Q4_0: { fp16 d; u8 qs[16]; }                                          18 B / 32 weights     */
/*     (qs[j] low nibble = weight j, high nibble = weight j + 16; y = d * (q - 8))              */
/*   Q8_0: { fp16 d; int8 qs[32]; }                                       34 B / 32 weights     */
/*   Q4_K: { fp16 d; fp16 dmin; u8 scales[12]; u8 qs[128]; }             144 B / 256 weights    */
/*   Q5_K: { fp16 d; fp16 dmin; u8 scales[12]; u8 qh[32]; u8 qs[128]; } 176 B / 256 weights    */
/*     (Q4_K's scales and nibbles plus a fifth bit: weight 32 i + l of sub-block i takes bit i  */
/*     of qh[l], i.e. +16 before the scale)                                                    */
/*   Q6_K: { u8 ql[128]; u8 qh[64]; int8 scales[16]; fp16 d; }           210 B / 256 weights    */
/*   MXFP4: { u8 e; u8 qs[16]; }                                           17 B / 32 weights     */
/*     (the OCP microscaling FP4 block ggml stores for gpt-oss: an E8M0 power-of-two scale and  */
/*     32 E2M1 codes, qs[j] low nibble = weight j, high nibble = weight j + 16)                 */
/* ------------------------------------------------------------------------------------------ */

ORC_API int64_t orc_block_size(int type) {
    switch (type) {
        case T_F32: case T_F16: case T_BF16: return 1;
        case T_Q4_0: case T_Q8_0: case T_MXFP4: return 32;
        case T_Q4_K: case T_Q5_K: case T_Q6_K: return 256;
        default: return 0;
    }
}
ORC_API int64_t orc_type_size(int type) {
    switch (type) {
        case T_F32: return 4;
        case T_F16: case T_BF16: return 2;
        case T_Q4_0: return 18;
        case T_Q8_0: return 34;
        case T_Q4_K: return 144;
        case T_Q5_K: return 176;
        case T_Q6_K: return 210;
        case T_MXFP4: return 17;
        default: return 0;
    }
}
ORC_API int64_t orc_row_size(int type, int64_t K) {
    const int64_t bs = orc_block_size(type);
    if (bs <= 0 || K % bs) return -1;
    return K / bs * orc_type_size(type);
}

static inline uint16_t rd16(const uint8_t * p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline void wr16(uint8_t * p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

/* The 6-bit (scale, min) pair j of a Q4_K block's 12 packed bytes. */
static inline void q4k_scale_min(int j, const uint8_t * q, int * sc, int * mn) {
    if (j < 4) {
        *sc = q[j] & 63;
        *mn = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4);
        *mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

static void dequant_q8_0(const uint8_t * x, float * y, int64_t K) {
    for (int64_t b = 0; b < K / 32; b++, x += 34, y += 32) {
        const float d = orc_f16_to_f32(rd16(x));
        const int8_t * qs = (const int8_t *)(x + 2);
        for (int l = 0; l < 32; l++) y[l] = d * (float)qs[l];
    }
}

static void dequant_q4_0(const uint8_t * x, float * y, int64_t K) {
    for (int64_t b = 0; b < K / 32; b++, x += 18, y += 32) {
        const float d = orc_f16_to_f32(rd16(x));
        for (int j = 0; j < 16; j++) {
            y[j] = (float)((int)(x[2 + j] & 0x0F) - 8) * d;
            y[j + 16] = (float)((int)(x[2 + j] >> 4) - 8) * d;
        }
    }
}

/* Q5_K: per 64 weights j (sub-blocks 2j, 2j+1) the nibbles of qs[32j..32j+31], the fifth bits
 * 2j and 2j+1 of qh[0..31]; y = (d * sc) * q - dmin * m, the products rounded on their own. */
static void dequant_q5_k(const uint8_t * x, float * y, int64_t K) {
    for (int64_t b = 0; b < K / 256; b++, x += 176) {
        const float d = orc_f16_to_f32(rd16(x));
        const float dmin = orc_f16_to_f32(rd16(x + 2));
        const uint8_t * sc = x + 4;
        const uint8_t * qh = x + 16;
        const uint8_t * qs = x + 48;
        for (int j = 0; j < 4; j++) {
            int s0, m0, s1, m1;
            q4k_scale_min(2 * j, sc, &s0, &m0);
            q4k_scale_min(2 * j + 1, sc, &s1, &m1);
            const float d0 = d * (float)s0, mm0 = dmin * (float)m0;
            const float d1 = d * (float)s1, mm1 = dmin * (float)m1;
            for (int l = 0; l < 32; l++)
                *y++ = d0 * (float)((qs[32 * j + l] & 0x0F) + (((qh[l] >> (2 * j)) & 1) << 4)) - mm0;
            for (int l = 0; l < 32; l++)
                *y++ = d1 * (float)((qs[32 * j + l] >> 4) + (((qh[l] >> (2 * j + 1)) & 1) << 4)) - mm1;
        }
    }
}

static void dequant_q4_k(const uint8_t * x, float * y, int64_t K) {
    for (int64_t b = 0; b < K / 256; b++, x += 144) {
        const float d = orc_f16_to_f32(rd16(x));
        const float dmin = orc_f16_to_f32(rd16(x + 2));
        const uint8_t * sc = x + 4;
        const uint8_t * qs = x + 16;
        for (int j = 0; j < 4; j++) {           /* 64 weights per quarter */
            int s0, m0, s1, m1;
            q4k_scale_min(2 * j, sc, &s0, &m0);
            q4k_scale_min(2 * j + 1, sc, &s1, &m1);
            const float d0 = d * (float)s0, mm0 = dmin * (float)m0;
            const float d1 = d * (float)s1, mm1 = dmin * (float)m1;
            for (int l = 0; l < 32; l++) *y++ = d0 * (float)(qs[32 * j + l] & 0x0F) - mm0;
            for (int l = 0; l < 32; l++) *y++ = d1 * (float)(qs[32 * j + l] >> 4) - mm1;
        }
    }
}

static void dequant_q6_k(const uint8_t * x, float * y, int64_t K) {
    for (int64_t b = 0; b < K / 256; b++, x += 210) {
        const uint8_t * ql = x;
        const uint8_t * qh = x + 128;
        const int8_t * sc = (const int8_t *)(x + 192);
        const float d = orc_f16_to_f32(rd16(x + 208));
        for (int half = 0; half < 2; half++) {
            for (int l = 0; l < 32; l++) {
                const int is = l / 16;
                const int q1 = (int)((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int q2 = (int)((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                y[l + 0]  = d * (float)sc[is + 0] * (float)q1;
                y[l + 32] = d * (float)sc[is + 2] * (float)q2;
                y[l + 64] = d * (float)sc[is + 4] * (float)q3;
                y[l + 96] = d * (float)sc[is + 6] * (float)q4;
            }
            y += 128; ql += 64; qh += 32; sc += 8;
        }
    }
}

/* MXFP4: E2M1 values (kvalues_mxfp4 of ggml-common.h: 0 1 2 3 4 6 8 12 and their negatives,
 * doubled so they are integers) times the E8M0 scale 2^(e-128) (GGML_E8M0_TO_FP32_HALF: the
 * block exponent minus the bias 127, halved). Every product is exact in f32. */
static const int8_t MXFP4_K[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

static inline float e8m0_half(uint8_t e) {
    /* 2^(e-128) as f32 bits: a subnormal for e < 2 */
    const uint32_t bits = e < 2 ? (uint32_t)0x00200000u << e : (uint32_t)(e - 1) << 23;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static void dequant_mxfp4(const uint8_t * x, float * y, int64_t K) {
    for (int64_t b = 0; b < K / 32; b++, x += 17, y += 32) {
        const float d = e8m0_half(x[0]);
        for (int j = 0; j < 16; j++) {
            y[j] = (float)MXFP4_K[x[1 + j] & 0x0F] * d;
            y[j + 16] = (float)MXFP4_K[x[1 + j] >> 4] * d;
        }
    }
}

/* One [K] row of `type` to f32: the to_float contract of ggml-rocket.cpp:3894-3906. */
ORC_API int orc_dequant_row(int type, const void * src, float * dst, int64_t K) {
    const uint8_t * x = (const uint8_t *)src;
    switch (type) {
        case T_F32: memcpy(dst, src, (size_t)K * 4); return 0;
        case T_F16: for (int64_t i = 0; i < K; i++) dst[i] = orc_f16_to_f32(rd16(x + 2 * i)); return 0;
        case T_BF16: for (int64_t i = 0; i < K; i++) dst[i] = bf16_to_f32(rd16(x + 2 * i)); return 0;
        case T_Q4_0: if (K % 32) return -1; dequant_q4_0(x, dst, K); return 0;
        case T_Q8_0: if (K % 32) return -1; dequant_q8_0(x, dst, K); return 0;
        case T_Q4_K: if (K % 256) return -1; dequant_q4_k(x, dst, K); return 0;
        case T_Q5_K: if (K % 256) return -1; dequant_q5_k(x, dst, K); return 0;
        case T_Q6_K: if (K % 256) return -1; dequant_q6_k(x, dst, K); return 0;
        case T_MXFP4: if (K % 32) return -1; dequant_mxfp4(x, dst, K); return 0;
        default: return -1;
    }
}

/* nrows rows, each dequantized then rounded to fp16: the streamed weight of
 * rocket_weight_to_fp16 (ggml-rocket.cpp:3903-3909). */
ORC_API int orc_dequant_rows_f16(int type, const void * src, uint16_t * dst, int64_t nrows, int64_t K) {
    const int64_t rb = orc_row_size(type, K);
    if (rb < 0) return -1;
    int bad = 0;
    #pragma omp parallel for schedule(static) reduction(|:bad)
    for (int64_t n = 0; n < nrows; n++) {
        float * row = (float *)malloc((size_t)K * 4);
        bad |= orc_dequant_row(type, (const uint8_t *)src + n * rb, row, K) != 0;
        orc_f32_to_f16_row(row, dst + n * K, K);
        free(row);
    }
    return bad ? -1 : 0;
}

ORC_API int orc_dequant_rows_f32(int type, const void * src, float * dst, int64_t nrows, int64_t K) {
    const int64_t rb = orc_row_size(type, K);
    if (rb < 0) return -1;
    int bad = 0;
    #pragma omp parallel for schedule(static) reduction(|:bad)
    for (int64_t n = 0; n < nrows; n++)
        bad |= orc_dequant_row(type, (const uint8_t *)src + n * rb, dst + n * K, K) != 0;
    return bad ? -1 : 0;
}

/* ------------------------------------------------------------------------------------------ */
/* quantizers for synthetic weights (this build's own; not ggml's search)                      */
/* ------------------------------------------------------------------------------------------ */

static void quant_q8_0(const float * x, uint8_t * y, int64_t K) {
    for (int64_t b = 0; b < K / 32; b++, x += 32, y += 34) {
        float amax = 0.0f;
        for (int l = 0; l < 32; l++) amax = fmaxf(amax, fabsf(x[l]));
        const float d = amax / 127.0f;
        const float id = d > 0.0f ? 1.0f / d : 0.0f;
        wr16(y, orc_f32_to_f16(d));
        for (int l = 0; l < 32; l++) {
            float q = roundf(x[l] * id);
            q = q > 127.0f ? 127.0f : (q < -127.0f ? -127.0f : q);
            ((int8_t *)(y + 2))[l] = (int8_t)q;
        }
    }
}

static inline int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

static void quant_q4_0(const float * x, uint8_t * y, int64_t K) {
    for (int64_t b = 0; b < K / 32; b++, x += 32, y += 18) {
        float amax = 0.0f;
        for (int l = 0; l < 32; l++) amax = fmaxf(amax, fabsf(x[l]));
        const uint16_t dh = orc_f32_to_f16(amax / 7.0f);
        const float dq = orc_f16_to_f32(dh);
        wr16(y, dh);
        int q[32];
        for (int l = 0; l < 32; l++) q[l] = dq > 0.0f ? clampi((int)lrintf(x[l] / dq), -8, 7) + 8 : 8;
        for (int j = 0; j < 16; j++) y[2 + j] = (uint8_t)(q[j] | (q[j + 16] << 4));
    }
}

static void quant_q4_k(const float * x, uint8_t * y, int64_t K) {
    for (int64_t b = 0; b < K / 256; b++, x += 256, y += 144) {
        float scale[8], minv[8];
        float max_scale = 0.0f, max_min = 0.0f;
        for (int j = 0; j < 8; j++) {
            float lo = 0.0f, hi = 0.0f;
            for (int l = 0; l < 32; l++) { lo = fminf(lo, x[32 * j + l]); hi = fmaxf(hi, x[32 * j + l]); }
            scale[j] = (hi - lo) / 15.0f;
            minv[j] = -lo;                                  /* >= 0 */
            max_scale = fmaxf(max_scale, scale[j]);
            max_min = fmaxf(max_min, minv[j]);
        }
        const float d = max_scale / 63.0f, dmin = max_min / 63.0f;
        const uint16_t dh = orc_f32_to_f16(d), dmh = orc_f32_to_f16(dmin);
        const float dq = orc_f16_to_f32(dh), dmq = orc_f16_to_f32(dmh);
        int sc[8], mn[8];
        for (int j = 0; j < 8; j++) {
            sc[j] = dq > 0.0f ? clampi((int)lrintf(scale[j] / dq), 0, 63) : 0;
            mn[j] = dmq > 0.0f ? clampi((int)lrintf(minv[j] / dmq), 0, 63) : 0;
        }
        wr16(y, dh);
        wr16(y + 2, dmh);
        uint8_t * s = y + 4;
        for (int j = 0; j < 4; j++) {
            s[j]     = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
            s[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
            s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
        }
        uint8_t q[256];
        for (int j = 0; j < 8; j++) {
            const float dd = dq * (float)sc[j], mm = dmq * (float)mn[j];
            for (int l = 0; l < 32; l++)
                q[32 * j + l] = (uint8_t)(dd > 0.0f ? clampi((int)lrintf((x[32 * j + l] + mm) / dd), 0, 15) : 0);
        }
        uint8_t * qs = y + 16;
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 32; l++)
                qs[32 * j + l] = (uint8_t)(q[64 * j + l] | (q[64 * j + 32 + l] << 4));
    }
}

static void quant_q5_k(const float * x, uint8_t * y, int64_t K) {
    for (int64_t b = 0; b < K / 256; b++, x += 256, y += 176) {
        float scale[8], minv[8];
        float max_scale = 0.0f, max_min = 0.0f;
        for (int j = 0; j < 8; j++) {
            float lo = 0.0f, hi = 0.0f;
            for (int l = 0; l < 32; l++) { lo = fminf(lo, x[32 * j + l]); hi = fmaxf(hi, x[32 * j + l]); }
            scale[j] = (hi - lo) / 31.0f;
            minv[j] = -lo;
            max_scale = fmaxf(max_scale, scale[j]);
            max_min = fmaxf(max_min, minv[j]);
        }
        const uint16_t dh = orc_f32_to_f16(max_scale / 63.0f), dmh = orc_f32_to_f16(max_min / 63.0f);
        const float dq = orc_f16_to_f32(dh), dmq = orc_f16_to_f32(dmh);
        int sc[8], mn[8];
        for (int j = 0; j < 8; j++) {
            sc[j] = dq > 0.0f ? clampi((int)lrintf(scale[j] / dq), 0, 63) : 0;
            mn[j] = dmq > 0.0f ? clampi((int)lrintf(minv[j] / dmq), 0, 63) : 0;
        }
        wr16(y, dh);
        wr16(y + 2, dmh);
        uint8_t * s = y + 4;
        for (int j = 0; j < 4; j++) {
            s[j]     = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
            s[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
            s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
        }
        uint8_t q[256];
        for (int j = 0; j < 8; j++) {
            const float dd = dq * (float)sc[j], mm = dmq * (float)mn[j];
            for (int l = 0; l < 32; l++)
                q[32 * j + l] = (uint8_t)(dd > 0.0f ? clampi((int)lrintf((x[32 * j + l] + mm) / dd), 0, 31) : 0);
        }
        uint8_t * qh = y + 16;
        uint8_t * qs = y + 48;
        memset(qh, 0, 32);
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 32; l++) {
                const uint8_t a = q[64 * j + l], c = q[64 * j + 32 + l];
                qs[32 * j + l] = (uint8_t)((a & 15) | ((c & 15) << 4));
                qh[l] |= (uint8_t)(((a >> 4) << (2 * j)) | ((c >> 4) << (2 * j + 1)));
            }
    }
}

static void quant_q6_k(const float * x, uint8_t * y, int64_t K) {
    for (int64_t b = 0; b < K / 256; b++, x += 256, y += 210) {
        float sub[16], max_sub = 0.0f;
        for (int i = 0; i < 16; i++) {
            float amax = 0.0f;
            for (int l = 0; l < 16; l++) amax = fmaxf(amax, fabsf(x[16 * i + l]));
            sub[i] = amax / 31.0f;
            max_sub = fmaxf(max_sub, sub[i]);
        }
        const float d = max_sub / 127.0f;
        const uint16_t dh = orc_f32_to_f16(d);
        const float dq = orc_f16_to_f32(dh);
        int8_t sc[16];
        for (int i = 0; i < 16; i++) sc[i] = (int8_t)(dq > 0.0f ? clampi((int)lrintf(sub[i] / dq), -127, 127) : 0);
        uint8_t q[256];                                     /* q + 32, in 0..63 */
        for (int p = 0; p < 256; p++) {
            const float dd = dq * (float)sc[p / 16];
            const int v = dd != 0.0f ? clampi((int)lrintf(x[p] / dd), -32, 31) : 0;
            q[p] = (uint8_t)(v + 32);
        }
        uint8_t * ql = y;
        uint8_t * qh = y + 128;
        for (int half = 0; half < 2; half++) {
            const uint8_t * qq = q + 128 * half;
            for (int l = 0; l < 32; l++) {
                ql[64 * half + l]      = (uint8_t)((qq[l] & 15) | ((qq[l + 64] & 15) << 4));
                ql[64 * half + l + 32] = (uint8_t)((qq[l + 32] & 15) | ((qq[l + 96] & 15) << 4));
                qh[32 * half + l] = (uint8_t)((qq[l] >> 4) | ((qq[l + 32] >> 4) << 2) |
                                              ((qq[l + 64] >> 4) << 4) | ((qq[l + 96] >> 4) << 6));
            }
        }
        memcpy(y + 192, sc, 16);
        wr16(y + 208, dh);
    }
}

/* MXFP4 quantizer for synthetic weights (this repository's own: the smallest scale 2^(e-128)
 * with amax <= 6 * 2^(e-127), i.e. the largest code fits, then each value to the nearest code). */
static void quant_mxfp4(const float * x, uint8_t * y, int64_t K) {
    for (int64_t b = 0; b < K / 32; b++, x += 32, y += 17) {
        float amax = 0.0f;
        for (int l = 0; l < 32; l++) amax = fmaxf(amax, fabsf(x[l]));
        int e = 0;
        while (e < 254 && 12.0f * e8m0_half((uint8_t)e) < amax) e++;
        y[0] = (uint8_t)e;
        const float d = e8m0_half((uint8_t)e);
        uint8_t code[32];
        for (int l = 0; l < 32; l++) {
            int best = 0;
            float bd = INFINITY;
            for (int c = 0; c < 16; c++) {
                const float dv = fabsf((float)MXFP4_K[c] * d - x[l]);
                if (dv < bd) { bd = dv; best = c; }
            }
            code[l] = (uint8_t)best;
        }
        for (int j = 0; j < 16; j++) y[1 + j] = (uint8_t)(code[j] | (code[j + 16] << 4));
    }
}

ORC_API int orc_quantize_rows(int type, const float * src, void * dst, int64_t nrows, int64_t K) {
    const int64_t rb = orc_row_size(type, K);
    if (rb < 0) return -1;
    #pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < nrows; n++) {
        const float * x = src + n * K;
        uint8_t * y = (uint8_t *)dst + n * rb;
        switch (type) {
            case T_F32: memcpy(y, x, (size_t)K * 4); break;
            case T_F16: for (int64_t i = 0; i < K; i++) wr16(y + 2 * i, orc_f32_to_f16(x[i])); break;
            case T_Q4_0: quant_q4_0(x, y, K); break;
            case T_Q8_0: quant_q8_0(x, y, K); break;
            case T_Q4_K: quant_q4_k(x, y, K); break;
            case T_Q5_K: quant_q5_k(x, y, K); break;
            case T_Q6_K: quant_q6_k(x, y, K); break;
            case T_MXFP4: quant_mxfp4(x, y, K); break;
            default: break;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* fp64 GEMM: dst[m*N + n] = sum_k X[m*K + k] * W(n, k)                                         */
/* rocket_cpu_matmul_slice (ggml-rocket.cpp:4053-4084): weight decoded by its dequantizer,      */
/* the dot accumulated in double from the original F32 activations, rounded once to F32.       */
/* ------------------------------------------------------------------------------------------ */

ORC_API int orc_mul_mat(int wtype, const void * W, const float * X, float * dst,
                        int64_t M, int64_t N, int64_t K, int nthreads) {
    const int64_t rb = orc_row_size(wtype, K);
    if (rb < 0) return -1;
    if (nthreads > 0) omp_set_num_threads(nthreads);
    /* decode the weight once, in double, then a blocked fp64 GEMM */
    double * Wd = (double *)malloc((size_t)N * K * sizeof(double));
    double * Xd = (double *)malloc((size_t)M * K * sizeof(double));
    if (!Wd || !Xd) { free(Wd); free(Xd); return -2; }
    int bad = 0;
    #pragma omp parallel for schedule(static) reduction(|:bad)
    for (int64_t n = 0; n < N; n++) {
        float * row = (float *)malloc((size_t)K * 4);
        bad |= orc_dequant_row(wtype, (const uint8_t *)W + n * rb, row, K) != 0;
        for (int64_t k = 0; k < K; k++) Wd[n * K + k] = (double)row[k];
        free(row);
    }
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < M * K; i++) Xd[i] = (double)X[i];
    const int64_t MB = 8, NB = 64;
    #pragma omp parallel for collapse(2) schedule(dynamic)
    for (int64_t m0 = 0; m0 < M; m0 += MB)
        for (int64_t n0 = 0; n0 < N; n0 += NB) {
            const int64_t m1 = m0 + MB < M ? m0 + MB : M, n1 = n0 + NB < N ? n0 + NB : N;
            for (int64_t m = m0; m < m1; m++) {
                const double * xr = Xd + m * K;
                for (int64_t n = n0; n < n1; n++) {
                    const double * wr = Wd + n * K;
                    double a0 = 0, a1 = 0, a2 = 0, a3 = 0;
                    int64_t k = 0;
                    for (; k + 4 <= K; k += 4) {
                        a0 += xr[k] * wr[k];
                        a1 += xr[k + 1] * wr[k + 1];
                        a2 += xr[k + 2] * wr[k + 2];
                        a3 += xr[k + 3] * wr[k + 3];
                    }
                    for (; k < K; k++) a0 += xr[k] * wr[k];
                    dst[m * N + n] = (float)((a0 + a1) + (a2 + a3));
                }
            }
        }
    free(Wd);
    free(Xd);
    return bad ? -1 : 0;
}

/* ------------------------------------------------------------------------------------------ */
/* MUL_MAT_ID (ggml-rocket.cpp:6654-6662):                                                      */
/*   dst[t][e][:] = as[ids[t][e]] . b[t][e % ne11][:]                                           */
/* rows bucketed by expert with a counting sort (6706-6732); an id outside [0, n_expert) fails. */
/* ------------------------------------------------------------------------------------------ */

ORC_API int orc_mul_mat_id(int wtype, const void * as, int64_t K, int64_t N, int64_t n_expert,
                           const float * b, int64_t ne11, const int32_t * ids, int64_t n_used,
                           int64_t n_tokens, float * dst, int nthreads) {
    const int64_t rb = orc_row_size(wtype, K);
    if (rb < 0 || ne11 <= 0) return -1;
    if (nthreads > 0) omp_set_num_threads(nthreads);
    const int64_t R = n_used * n_tokens;
    int64_t * off = (int64_t *)calloc((size_t)n_expert + 1, sizeof(int64_t));
    int64_t * rows = (int64_t *)malloc((size_t)(R > 0 ? R : 1) * sizeof(int64_t));
    for (int64_t r = 0; r < R; r++) {
        const int32_t x = ids[r];
        if (x < 0 || x >= n_expert) { free(off); free(rows); return 1; }
        off[x + 1]++;
    }
    for (int64_t e = 0; e < n_expert; e++) off[e + 1] += off[e];
    int64_t * cur = (int64_t *)malloc((size_t)(n_expert > 0 ? n_expert : 1) * sizeof(int64_t));
    for (int64_t e = 0; e < n_expert; e++) cur[e] = off[e];
    for (int64_t r = 0; r < R; r++) rows[cur[ids[r]]++] = r;   /* r = t*n_used + slot */
    const size_t ebytes = (size_t)rb * N;
    #pragma omp parallel for schedule(dynamic)
    for (int64_t e = 0; e < n_expert; e++) {
        const int64_t r0 = off[e], r1 = off[e + 1];
        if (r0 == r1) continue;
        double * Wd = (double *)malloc((size_t)N * K * sizeof(double));
        float * row = (float *)malloc((size_t)K * 4);
        for (int64_t n = 0; n < N; n++) {
            orc_dequant_row(wtype, (const uint8_t *)as + e * ebytes + n * rb, row, K);
            for (int64_t k = 0; k < K; k++) Wd[n * K + k] = (double)row[k];
        }
        for (int64_t i = r0; i < r1; i++) {
            const int64_t r = rows[i], t = r / n_used, slot = r % n_used;
            const float * x = b + (t * ne11 + slot % ne11) * K;
            float * d = dst + (t * n_used + slot) * N;
            for (int64_t n = 0; n < N; n++) {
                const double * w = Wd + n * K;
                double acc = 0.0;
                for (int64_t k = 0; k < K; k++) acc += (double)x[k] * w[k];
                d[n] = (float)acc;
            }
        }
        free(row);
        free(Wd);
    }
    free(cur);
    free(rows);
    free(off);
    return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* FLASH_ATTN_EXT references. Layouts are the op's contiguous ggml ones:                       */
/*   q [H][T][D] F32, k [HK][KV][D] fp16, v [HK][KV][DV] fp16, mask [T][mask_stride] fp16,       */
/*   dst [T][H][DV] F32.                                                                         */
/* q_mode 0: Q rounded to fp16 before the dot, then scaled (test-rocket-fa.cpp:101-135);         */
/* q_mode 1: Q as F32 (rocket_fa_ref_f32, ggml-rocket.cpp:5392-5442).                           */
/* Soft-cap: s = softcap * tanh(scale*q.k / softcap), then the mask is added (5428-5430).        */
/* A row whose every key is masked is written as zeros (5395-5397, 5437-5439).                  */
/* ------------------------------------------------------------------------------------------ */

ORC_API int orc_flash_attn(const float * q, const uint16_t * k, const uint16_t * v,
                           const uint16_t * mask, int64_t mask_stride, float * dst,
                           int D, int DV, int T, int H, int KV, int HK,
                           float scale, float softcap, int q_mode, int nthreads) {
    if (HK <= 0 || H % HK) return -1;
    if (nthreads > 0) omp_set_num_threads(nthreads);
    const int g = H / HK;
    /* K and V decoded once (exact: every fp16 is a double) */
    double * Kd = (double *)malloc((size_t)HK * KV * D * sizeof(double));
    double * Vd = (double *)malloc((size_t)HK * KV * DV * sizeof(double));
    if (!Kd || !Vd) { free(Kd); free(Vd); return -2; }
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)HK * KV * D; i++) Kd[i] = (double)orc_f16_to_f32(k[i]);
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)HK * KV * DV; i++) Vd[i] = (double)orc_f16_to_f32(v[i]);
    #pragma omp parallel
    {
        double * qd = (double *)malloc((size_t)D * sizeof(double));
        double * sc = (double *)malloc((size_t)KV * sizeof(double));
        double * acc = (double *)malloc((size_t)DV * sizeof(double));
        #pragma omp for schedule(dynamic)
        for (int64_t r = 0; r < (int64_t)H * T; r++) {
            const int h = (int)(r / T), t = (int)(r % T), hk = h / g;
            const float * qr = q + ((size_t)h * T + t) * D;
            for (int c = 0; c < D; c++)
                qd[c] = q_mode ? (double)qr[c] : (double)orc_f16_to_f32(orc_f32_to_f16(qr[c]));
            const double * Kh = Kd + (size_t)hk * KV * D;
            const double * Vh = Vd + (size_t)hk * KV * DV;
            const uint16_t * mr = mask ? mask + (size_t)t * mask_stride : NULL;
            double mx = -INFINITY;
            for (int j = 0; j < KV; j++) {
                const double mv = mr ? (double)orc_f16_to_f32(mr[j]) : 0.0;
                if (mv == -INFINITY) { sc[j] = -INFINITY; continue; }
                const double * kr = Kh + (size_t)j * D;
                double dd = 0.0;
                for (int c = 0; c < D; c++) dd += qd[c] * kr[c];
                double s = dd * (double)scale;
                if (softcap != 0.0f) s = (double)softcap * tanh(s / (double)softcap);
                s += mv;
                sc[j] = s;
                if (s > mx) mx = s;
            }
            double sum = 0.0;
            for (int j = 0; j < KV; j++) {
                sc[j] = (mx == -INFINITY || sc[j] == -INFINITY) ? 0.0 : exp(sc[j] - mx);
                sum += sc[j];
            }
            for (int c = 0; c < DV; c++) acc[c] = 0.0;
            for (int j = 0; j < KV; j++) {
                if (sc[j] == 0.0) continue;
                const double * vr = Vh + (size_t)j * DV;
                for (int c = 0; c < DV; c++) acc[c] += sc[j] * vr[c];
            }
            const double inv = sum > 0.0 ? 1.0 / sum : 0.0;
            float * dr = dst + ((size_t)t * H + h) * DV;
            for (int c = 0; c < DV; c++) dr[c] = (float)(acc[c] * inv);
        }
        free(qd); free(sc); free(acc);
    }
    free(Kd);
    free(Vd);
    return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* activation pack (rk_pack_act_row, ggml-rocket.cpp:1451-1475): per row s = max|x| (1 when the */
/* row is zero), a16 = fp16(x * (1/s)) rounded to nearest even.                                */
/* ------------------------------------------------------------------------------------------ */

ORC_API void orc_pack_act(const float * x, int64_t M, int64_t K, uint16_t * a16, float * scales) {
    #pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; m++) {
        const float * r = x + m * K;
        float amax = 0.0f;
        for (int64_t k = 0; k < K; k++) { const float v = fabsf(r[k]); if (v > amax) amax = v; }
        const float s = amax > 0.0f ? amax : 1.0f;
        const float inv = 1.0f / s;
        for (int64_t k = 0; k < K; k++) a16[m * K + k] = orc_f32_to_f16(r[k] * inv);
        scales[m] = s;
    }
}

ORC_API int orc_max_threads(void) { return omp_get_max_threads(); }
