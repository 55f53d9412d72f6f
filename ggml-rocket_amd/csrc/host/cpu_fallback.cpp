// SPDX-License-Identifier: MIT
// The degraded path: an op whose device job failed is computed here, on the host, in fp64,
// from the op's original inputs (ggml-rocket.cpp:4048-4084 for MUL_MAT, 5392-5442 for
// FLASH_ATTN_EXT, 6927-6939 for an expert). Slow and rare by design: the route counters and
// cpu_fallbacks() say when it ran. Rows of the output are spread over a few host threads.

#include <math.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <thread>
#include <vector>

#include "host.h"

namespace mxh {

static float h2f(uint16_t h) {
    const uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) x = s;
        else {
            float f = (float)m * (1.0f / 16777216.0f);
            memcpy(&x, &f, 4);
            x |= s;
        }
    } else if (e == 31) {
        x = s | 0x7f800000u | (m << 13);
    } else {
        x = s | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}
static inline uint16_t rd16(const uint8_t * p) { return (uint16_t)(p[0] | (p[1] << 8)); }

// One row of n values of a weight type to f32, as ggml's dequantizers define them.
bool decode_row_f32(int type, const void * src, float * y, int64_t n) {
    const uint8_t * x = (const uint8_t *)src;
    switch (type) {
        case MI355X_TYPE_F32: memcpy(y, src, (size_t)n * 4); return true;
        case MI355X_TYPE_F16: for (int64_t i = 0; i < n; i++) y[i] = h2f(rd16(x + 2 * i)); return true;
        case MI355X_TYPE_BF16:
            for (int64_t i = 0; i < n; i++) {
                const uint32_t b = (uint32_t)rd16(x + 2 * i) << 16;
                memcpy(&y[i], &b, 4);
            }
            return true;
        case MI355X_TYPE_Q8_0:
            for (int64_t b = 0; b < n / 32; b++, x += 34) {
                const float d = h2f(rd16(x));
                for (int l = 0; l < 32; l++) *y++ = d * (float)(int8_t)x[2 + l];
            }
            return true;
        case MI355X_TYPE_Q4_0:   // dequantize_row_q4_0: d * (q - 8), low nibbles first
            for (int64_t b = 0; b < n / 32; b++, x += 18) {
                const float d = h2f(rd16(x));
                for (int l = 0; l < 16; l++) y[l] = (float)((x[2 + l] & 15) - 8) * d;
                for (int l = 0; l < 16; l++) y[16 + l] = (float)((x[2 + l] >> 4) - 8) * d;
                y += 32;
            }
            return true;
        case MI355X_TYPE_Q5_K:   // dequantize_row_q5_K: Q4_K's scales, a fifth bit from qh
            for (int64_t b = 0; b < n / 256; b++, x += 176) {
                const float d = h2f(rd16(x)), dmin = h2f(rd16(x + 2));
                const uint8_t * s = x + 4;
                const uint8_t * qh = x + 16;
                const uint8_t * q = x + 48;
                for (int j = 0; j < 8; j++) {
                    int sc, mn;
                    if (j < 4) { sc = s[j] & 63; mn = s[j + 4] & 63; }
                    else { sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4); mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4); }
                    const float dd = d * (float)sc, mm = dmin * (float)mn;
                    const uint8_t * qq = q + 32 * (j / 2);
                    const int sh = (j % 2) * 4;
                    for (int l = 0; l < 32; l++)
                        *y++ = dd * (float)(((qq[l] >> sh) & 15) | (((qh[l] >> j) & 1) << 4)) - mm;
                }
            }
            return true;
        case MI355X_TYPE_Q4_K:
            for (int64_t b = 0; b < n / 256; b++, x += 144) {
                const float d = h2f(rd16(x)), dmin = h2f(rd16(x + 2));
                const uint8_t * s = x + 4;
                const uint8_t * q = x + 16;
                for (int j = 0; j < 8; j++) {
                    int sc, mn;
                    if (j < 4) { sc = s[j] & 63; mn = s[j + 4] & 63; }
                    else { sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4); mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4); }
                    const float dd = d * (float)sc, mm = dmin * (float)mn;
                    const uint8_t * qq = q + 32 * (j / 2);
                    const int sh = (j % 2) * 4;
                    for (int l = 0; l < 32; l++) *y++ = dd * (float)((qq[l] >> sh) & 15) - mm;
                }
            }
            return true;
        case MI355X_TYPE_Q6_K:
            for (int64_t b = 0; b < n / 256; b++, x += 210) {
                const float d = h2f(rd16(x + 208));
                const int8_t * sc = (const int8_t *)(x + 192);
                for (int p = 0; p < 256; p++) {
                    const int half = p / 128, r = p % 128, quarter = r / 32, l = r % 32;
                    const uint8_t lq = x[64 * half + l + (quarter & 1) * 32];
                    const int lo = (quarter >= 2) ? (lq >> 4) : (lq & 15);
                    const int hi = (x[128 + 32 * half + l] >> (2 * quarter)) & 3;
                    *y++ = d * (float)sc[p / 16] * (float)((lo | (hi << 4)) - 32);
                }
            }
            return true;
        case MI355X_TYPE_MXFP4:   // kvalues_mxfp4 (E2M1 doubled) times 2^(e-128), ggml-common.h
            for (int64_t b = 0; b < n / 32; b++, x += 17) {
                static const int8_t kv[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
                const uint32_t eb = x[0] < 2 ? (0x00200000u << x[0]) : ((uint32_t)(x[0] - 1) << 23);
                float d;
                memcpy(&d, &eb, 4);
                for (int l = 0; l < 16; l++) y[l] = (float)kv[x[1 + l] & 15] * d;
                for (int l = 0; l < 16; l++) y[16 + l] = (float)kv[x[1 + l] >> 4] * d;
                y += 32;
            }
            return true;
        default:
            if (const mi355x_to_float_fn fn = host_to_float(type)) {   // ggml's own decoder
                fn(src, y, n);
                return true;
            }
            return false;
    }
}

template <class F>
static void parallel_rows(int64_t n, F && f) {
    const int nt = (int)std::max<int64_t>(1, std::min<int64_t>(8, n / 4));
    if (nt <= 1) { f((int64_t)0, n); return; }
    std::vector<std::thread> th;
    const int64_t per = (n + nt - 1) / nt;
    for (int i = 0; i < nt; i++) {
        const int64_t a = i * per, b = std::min(n, a + per);
        if (a < b) th.emplace_back([&f, a, b] { f(a, b); });
    }
    for (auto & t : th) t.join();
}

// dst[..., n] = sum_k src1[..., k] * W[n, k], the weight decoded row by row.
void cpu_mul_mat(const mi355x_tensor * dst) {
    const mi355x_tensor * a = dst->src[0];
    const mi355x_tensor * b = dst->src[1];
    const int64_t K = a->ne[0], N = a->ne[1];
    const int64_t rows = b->ne[1] * b->ne[2] * b->ne[3];
    const size_t rb = (size_t)row_bytes(a->type, K);
    std::vector<double> W((size_t)N * K);
    parallel_rows(N, [&](int64_t n0, int64_t n1) {
        std::vector<float> r((size_t)K);
        for (int64_t n = n0; n < n1; n++) {
            decode_row_f32(a->type, (const uint8_t *)a->data + n * rb, r.data(), K);
            for (int64_t k = 0; k < K; k++) W[n * K + k] = r[k];
        }
    });
    const float * X = (const float *)b->data;
    float * D = (float *)dst->data;
    parallel_rows(rows, [&](int64_t m0, int64_t m1) {
        for (int64_t m = m0; m < m1; m++)
            for (int64_t n = 0; n < N; n++) {
                double acc = 0.0;
                const double * w = &W[n * K];
                const float * x = X + m * K;
                for (int64_t k = 0; k < K; k++) acc += (double)x[k] * w[k];
                D[m * N + n] = (float)acc;
            }
    });
}

// Attention on the host in double precision, to the contract of ggml-rocket.cpp:5392-5442:
// Q read as F32, K and V as fp16, logits = scale * q.k, soft-capped when a cap is set, plus the
// mask; softmax in double; a query whose every key is masked gets a zero output row.
// Work is laid out per (token, KV head): the H / HK query heads that share a KV head are scored
// together, so each visible key and value row is widened to double once for all of them. The
// logits are kept per head, then turned into weights against that head's largest logit and
// folded into the value sum in key order.
void cpu_flash_attn(const mi355x_tensor * dst) {
    const mi355x_tensor * q = dst->src[0];
    const mi355x_tensor * k = dst->src[1];
    const mi355x_tensor * v = dst->src[2];
    const mi355x_tensor * m = dst->src[3];
    const int64_t dk = q->ne[0], n_tok = q->ne[1], n_head = q->ne[2];
    const int64_t n_key = k->ne[1], n_kvh = k->ne[2], dv = v->ne[0];
    const int64_t group = n_head / n_kvh;   // query heads per KV head
    float scale_f, cap_f;
    memcpy(&scale_f, &dst->op_params[0], 4);
    memcpy(&cap_f, &dst->op_params[2], 4);
    const double scale = scale_f, cap = cap_f;
    auto widen = [](const char * row, int64_t n, double * out) {
        for (int64_t c = 0; c < n; c++) out[c] = (double)h2f(rd16((const uint8_t *)row + 2 * c));
    };
    parallel_rows(n_tok * n_kvh, [&](int64_t w0, int64_t w1) {
        std::vector<double> queries((size_t)(group * dk)), logits((size_t)(group * n_key));
        std::vector<double> vsum((size_t)(group * dv)), top((size_t)group), total((size_t)group);
        std::vector<double> key((size_t)dk), val((size_t)dv);
        std::vector<int64_t> seen;   // keys the mask leaves visible, in order
        seen.reserve((size_t)n_key);
        for (int64_t w = w0; w < w1; w++) {
            const int64_t tok = w / n_kvh, kvh = w % n_kvh;
            for (int64_t i = 0; i < group; i++) {
                const char * src = (const char *)q->data + tok * q->nb[1] + (kvh * group + i) * q->nb[2];
                for (int64_t c = 0; c < dk; c++) queries[(size_t)(i * dk + c)] = *(const float *)(src + c * q->nb[0]);
            }
            std::fill(top.begin(), top.end(), -INFINITY);
            seen.clear();
            for (int64_t j = 0; j < n_key; j++) {
                double bias = 0.0;
                if (m) bias = (double)h2f(rd16((const uint8_t *)m->data + tok * m->nb[1] + j * 2));
                if (std::isinf(bias) && bias < 0) continue;
                seen.push_back(j);
                widen((const char *)k->data + j * k->nb[1] + kvh * k->nb[2], dk, key.data());
                for (int64_t i = 0; i < group; i++) {
                    const double * qi = &queries[(size_t)(i * dk)];
                    double dot = 0.0;
                    for (int64_t c = 0; c < dk; c++) dot += qi[c] * key[(size_t)c];
                    double x = dot * scale;
                    if (cap != 0.0) x = cap * tanh(x / cap);
                    x += bias;
                    logits[(size_t)(i * n_key + j)] = x;
                    if (x > top[(size_t)i]) top[(size_t)i] = x;
                }
            }
            std::fill(vsum.begin(), vsum.end(), 0.0);
            std::fill(total.begin(), total.end(), 0.0);
            for (const int64_t j : seen) {
                widen((const char *)v->data + j * v->nb[1] + kvh * v->nb[2], dv, val.data());
                for (int64_t i = 0; i < group; i++) {
                    const double x = logits[(size_t)(i * n_key + j)];
                    if (std::isinf(top[(size_t)i]) || std::isinf(x)) continue;
                    const double p = exp(x - top[(size_t)i]);
                    total[(size_t)i] += p;
                    double * acc = &vsum[(size_t)(i * dv)];
                    for (int64_t c = 0; c < dv; c++) acc[c] += p * val[(size_t)c];
                }
            }
            for (int64_t i = 0; i < group; i++) {
                const int64_t h = kvh * group + i;
                float * out = (float *)((char *)dst->data + h * dst->nb[1] + tok * dst->nb[2]);
                const double t = total[(size_t)i];
                for (int64_t c = 0; c < dv; c++) out[c] = t > 0.0 ? (float)(vsum[(size_t)(i * dv + c)] / t) : 0.0f;
            }
        }
    });
}

// dst[:, s, t] = as[:, :, ids[s, t]] . b[:, s % ne11, t]
bool cpu_mul_mat_id(const mi355x_tensor * dst) {
    const mi355x_tensor * as = dst->src[0];
    const mi355x_tensor * b = dst->src[1];
    const mi355x_tensor * ids = dst->src[2];
    const int64_t K = as->ne[0], N = as->ne[1], E = as->ne[2];
    const int64_t ne11 = b->ne[1], U = ids->ne[0], T = ids->ne[1];
    for (int64_t t = 0; t < T; t++)
        for (int64_t s = 0; s < U; s++) {
            const int32_t e = *(const int32_t *)((const char *)ids->data + t * ids->nb[1] + s * ids->nb[0]);
            if (e < 0 || e >= E) return false;
        }
    const size_t rb = (size_t)row_bytes(as->type, K);
    parallel_rows(T, [&](int64_t t0, int64_t t1) {
        std::vector<float> w((size_t)K);
        for (int64_t t = t0; t < t1; t++)
            for (int64_t s = 0; s < U; s++) {
                const int32_t e = *(const int32_t *)((const char *)ids->data + t * ids->nb[1] + s * ids->nb[0]);
                const float * x = (const float *)((const char *)b->data + t * b->nb[2] + (s % ne11) * b->nb[1]);
                float * d = (float *)((char *)dst->data + t * dst->nb[2] + s * dst->nb[1]);
                for (int64_t n = 0; n < N; n++) {
                    decode_row_f32(as->type, (const uint8_t *)as->data + e * as->nb[2] + n * rb, w.data(), K);
                    double acc = 0.0;
                    for (int64_t k = 0; k < K; k++) acc += (double)x[k] * (double)w[k];
                    d[n] = (float)acc;
                }
            }
    });
    return true;
}

}  // namespace mxh
