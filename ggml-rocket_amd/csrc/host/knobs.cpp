// SPDX-License-Identifier: MIT
// Configuration knobs, ggml type facts and logging for the backend's host layer.
//
// Knob semantics follow the reference (ggml-rocket.cpp:694-1152, API.md:14-145): every knob is
// read once per process; a variable that is set but empty counts as unset (698-724); each knob
// is looked up as MI355X_<name> first and then under the reference's ROCKET_<name> spelling, so
// a configuration written for the reference keeps its meaning here.

#include <ctype.h>
#include <errno.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>

#include "host.h"
#include "../../../include/mi355x_kernels.h"

namespace mxh {

// Log lines go to stderr unless a host installed a sink (the ggml adapter routes them to
// ggml's logger, which llama.cpp and whisper.cpp redirect or silence).
namespace {
std::atomic<mi355x_log_fn> g_log_fn{nullptr};
std::atomic<void *> g_log_user{nullptr};

void emit(int level, const char * prefix, const char * fmt, va_list ap) {
    char line[1024];
    const int n = snprintf(line, sizeof line, "[mi355x] %s", prefix);
    vsnprintf(line + n, sizeof line - (size_t)n, fmt, ap);
    const mi355x_log_fn fn = g_log_fn.load(std::memory_order_acquire);
    if (fn) fn(level, line, g_log_user.load(std::memory_order_acquire));
    else fputs(line, stderr);
}
}  // namespace

void set_log_sink(mi355x_log_fn fn, void * user) {
    g_log_user.store(user, std::memory_order_release);
    g_log_fn.store(fn, std::memory_order_release);
}

void logw(const char * fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    emit(MI355X_LOG_WARN, "warning: ", fmt, ap);
    va_end(ap);
}

void logi(const char * fmt, ...) {
    static const bool quiet = getenv("MI355X_QUIET") != nullptr;
    if (quiet) return;
    va_list ap;
    va_start(ap, fmt);
    emit(MI355X_LOG_INFO, "", fmt, ap);
    va_end(ap);
}

// ---- ggml type facts: block size and block bytes (ggml's published formats) ----------------
// Decoders registered for quantized types the kernels do not decode, with ggml's block facts.
namespace {
constexpr int N_TYPE_IDS = 64;
struct HostDecoder {
    std::atomic<mi355x_to_float_fn> fn{nullptr};
    std::atomic<int64_t> block{0}, bytes{0};
};
HostDecoder g_decoders[N_TYPE_IDS];
}  // namespace

mi355x_to_float_fn host_to_float(int t) {
    return (t >= 0 && t < N_TYPE_IDS) ? g_decoders[t].fn.load(std::memory_order_acquire) : nullptr;
}

int register_to_float(int t, int64_t block, int64_t bytes, mi355x_to_float_fn fn) {
    if (t < 0 || t >= N_TYPE_IDS || !fn || block <= 1 || bytes <= 0) return MI355X_E_ARG;
    if (device_weight_type(t)) return MI355X_OK;   // decoded on the device; nothing to add
    const int64_t b = type_block(t), s = type_bytes(t);
    if ((b > 0 && b != block) || (s > 0 && s != bytes)) return MI355X_E_ARG;
    g_decoders[t].block.store(block, std::memory_order_release);
    g_decoders[t].bytes.store(bytes, std::memory_order_release);
    g_decoders[t].fn.store(fn, std::memory_order_release);
    return MI355X_OK;
}

int64_t type_block(int t) {
    switch (t) {
        case MI355X_TYPE_F32: case MI355X_TYPE_F16: case MI355X_TYPE_BF16: case MI355X_TYPE_I8:
        case MI355X_TYPE_I16: case MI355X_TYPE_I32: case MI355X_TYPE_I64: case MI355X_TYPE_F64:
            return 1;
        case MI355X_TYPE_Q4_0: case MI355X_TYPE_Q4_1: case MI355X_TYPE_Q5_0: case MI355X_TYPE_Q5_1:
        case MI355X_TYPE_Q8_0: case MI355X_TYPE_Q8_1: case MI355X_TYPE_IQ4_NL: case MI355X_TYPE_MXFP4:
            return 32;
        case MI355X_TYPE_Q2_K: case MI355X_TYPE_Q3_K: case MI355X_TYPE_Q4_K: case MI355X_TYPE_Q5_K:
        case MI355X_TYPE_Q6_K: case MI355X_TYPE_Q8_K: case MI355X_TYPE_IQ2_XXS: case MI355X_TYPE_IQ2_XS:
        case MI355X_TYPE_IQ3_XXS: case MI355X_TYPE_IQ1_S: case MI355X_TYPE_IQ3_S: case MI355X_TYPE_IQ2_S:
        case MI355X_TYPE_IQ4_XS: case MI355X_TYPE_IQ1_M: case MI355X_TYPE_TQ1_0: case MI355X_TYPE_TQ2_0:
            return 256;
        default: return (t >= 0 && t < N_TYPE_IDS) ? g_decoders[t].block.load(std::memory_order_acquire) : 0;
    }
}

int64_t type_bytes(int t) {
    switch (t) {
        case MI355X_TYPE_F32: case MI355X_TYPE_I32: return 4;
        case MI355X_TYPE_F16: case MI355X_TYPE_BF16: case MI355X_TYPE_I16: return 2;
        case MI355X_TYPE_I8: return 1;
        case MI355X_TYPE_I64: case MI355X_TYPE_F64: return 8;
        case MI355X_TYPE_Q4_0: return 18;
        case MI355X_TYPE_Q4_1: return 20;
        case MI355X_TYPE_Q5_0: return 22;
        case MI355X_TYPE_Q5_1: return 24;
        case MI355X_TYPE_Q8_0: return 34;
        case MI355X_TYPE_Q8_1: return 36;
        case MI355X_TYPE_Q2_K: return 84;
        case MI355X_TYPE_Q3_K: return 110;
        case MI355X_TYPE_Q4_K: return 144;
        case MI355X_TYPE_Q5_K: return 176;
        case MI355X_TYPE_Q6_K: return 210;
        case MI355X_TYPE_Q8_K: return 292;
        case MI355X_TYPE_IQ4_NL: return 18;
        case MI355X_TYPE_MXFP4: return 17;
        default: return (t >= 0 && t < N_TYPE_IDS) ? g_decoders[t].bytes.load(std::memory_order_acquire) : 0;
    }
}

bool type_is_quantized(int t) {
    return type_block(t) > 1;
}

int64_t row_bytes(int t, int64_t n) {
    const int64_t b = type_block(t), s = type_bytes(t);
    if (b <= 0 || s <= 0 || n % b) return -1;
    return n / b * s;
}

int64_t nelements(const mi355x_tensor * t) {
    return t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3];
}

size_t nbytes(const mi355x_tensor * t) {
    // bytes spanned by the tensor's extent (what ggml_nbytes gives for a plain layout)
    const int64_t blk = type_block(t->type);
    if (blk <= 0) return 0;
    if (nelements(t) == 0) return 0;
    size_t n = (size_t)(t->ne[0] / blk) * t->nb[0];
    for (int i = 1; i < MI355X_MAX_DIMS; i++) n += (size_t)(t->ne[i] - 1) * t->nb[i];
    return n;
}

bool is_contiguous(const mi355x_tensor * t) {
    const int64_t blk = type_block(t->type);
    if (blk <= 0) return false;
    size_t next = (size_t)type_bytes(t->type);
    if (t->nb[0] != next) return false;
    next *= (size_t)(t->ne[0] / blk);
    for (int i = 1; i < MI355X_MAX_DIMS; i++) {
        if (t->ne[i] != 1 && t->nb[i] != next) return false;
        next *= (size_t)t->ne[i];
    }
    return true;
}

bool device_weight_type(int t) {
    return t == MI355X_TYPE_F16 || t == MI355X_TYPE_F32 || t == MI355X_TYPE_BF16 ||
           t == MI355X_TYPE_Q8_0 || t == MI355X_TYPE_Q4_0 || t == MI355X_TYPE_Q4_K || t == MI355X_TYPE_Q5_K ||
           t == MI355X_TYPE_Q6_K || t == MI355X_TYPE_MXFP4;
}

bool weight_type_ok(int t) {
    return device_weight_type(t) || (type_is_quantized(t) && host_to_float(t) != nullptr);
}

// ---- knobs -----------------------------------------------------------------------------------
const char * knob_env(const char * name) {
    char buf[128];
    snprintf(buf, sizeof buf, "MI355X_%s", name);
    const char * e = getenv(buf);
    if (e && *e) return e;
    snprintf(buf, sizeof buf, "ROCKET_%s", name);
    e = getenv(buf);
    return (e && *e) ? e : nullptr;
}

int knob_int(const char * name, int dflt) {
    const char * e = knob_env(name);
    return e ? atoi(e) : dflt;
}

bool knob_on(const char * name, bool dflt) {
    const char * e = knob_env(name);
    return e ? atoi(e) > 0 : dflt;
}

// Strict MB parser (ggml-rocket.cpp:7932-7964): optional surrounding blanks, then a whole
// non-negative decimal number and nothing else. "auto" is refused without a warning (callers that
// accept it resolve it themselves). Values are capped at 2^40 MB so the shift cannot overflow.
bool parse_mb(const char * e, size_t * out) {
    if (!e) return false;
    const char * p = e;
    while (isspace((unsigned char)*p)) p++;
    if (strncmp(p, "auto", 4) == 0) {
        const char * q = p + 4;
        while (isspace((unsigned char)*q)) q++;
        if (!*q) return false;
    }
    if (!isdigit((unsigned char)*p)) {
        if (*p) logw("\"%s\" is not a whole non-negative number of MB; the default stands\n", e);
        return false;
    }
    errno = 0;
    char * end = nullptr;
    const unsigned long long v = strtoull(p, &end, 10);
    const char * q = end;
    while (isspace((unsigned char)*q)) q++;
    // strtoll's range is the reference's: a value past LLONG_MAX is refused
    if (errno == ERANGE || *q || v > 9223372036854775807ULL) {
        logw("\"%s\" is not a whole non-negative number of MB; the default stands\n", e);
        return false;
    }
    const unsigned long long cap = 1ULL << 40;
    *out = (size_t)(v > cap ? cap : v) << 20;
    return true;
}

int min_m() {
    static const int v = [] { const int x = knob_int("MIN_M", 32); return x < 4 ? 4 : x; }();
    return v;
}
int min_m_quant() {
    static const int v = [] { const int x = knob_int("MIN_M_QUANT", 512); return x < min_m() ? min_m() : x; }();
    return v;
}
int moe_mode() {
    static const int v = [] {
        const char * e = knob_env("MOE");
        if (!e) return (int)MOE_AUTO;
        return atoi(e) > 0 ? (int)MOE_FORCED : (int)MOE_OFF;
    }();
    return v;
}
int moe_min_tokens() {
    static const int v = [] { const int x = knob_int("MOE_MIN_TOKENS", 512); return x < min_m() ? min_m() : x; }();
    return v;
}
bool moe_native_on() {
    static const bool v = knob_on("MOE_NATIVE", true);
    return v;
}
int moe_m_bucket() {
    static const int v = [] {
        int g = knob_int("MOE_M_BUCKET", 64);
        if (g < 4) g = 4;
        int q = 4;
        while (q < g && q < (1 << 20)) q <<= 1;
        return q;
    }();
    return v;
}
int moe_min_work_mmac() {
    static const int v = [] { const int x = knob_int("MOE_MIN_WORK", 340); return x < 0 ? 0 : x; }();
    return v;
}
bool flash_attn_on() {
    static const bool v = knob_int("FLASH_ATTN", 1) > 0;
    return v;
}
int flash_attn_min_t() {
    static const int v = [] { const int x = knob_int("FLASH_ATTN_MIN_T", 16); return x < 1 ? 1 : x; }();
    return v;
}
int flash_attn_min_kv() {
    static const int v = [] { const int x = knob_int("FLASH_ATTN_MIN_KV", 1024); return x < 1 ? 1 : x; }();
    return v;
}
bool flash_attn_unmasked() {
    static const bool v = knob_int("FLASH_ATTN_UNMASKED", 0) > 0;
    return v;
}
bool quant_resident_on() {
    static const bool v = [] {
        const char * e = knob_env("QUANT_RESIDENT");
        return e && (strcmp(e, "auto") == 0 || atoi(e) > 0);
    }();
    return v;
}
bool fusion_on() {
    static const bool v = knob_int("FUSE", 1) > 0;
    return v;
}

}  // namespace mxh

MI355X_API int mi355x_backend_set_to_float(int type, int64_t block_size, int64_t type_size, mi355x_to_float_fn fn) {
    return mxh::register_to_float(type, block_size, type_size, fn);
}
