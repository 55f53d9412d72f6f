// SPDX-License-Identifier: MIT
// Internal declarations of the backend's host layer (claim rules, knobs, weight identity, the
// MoE residency ledger, the CPU fallback).
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <string>

#include "../../../include/mi355x_backend.h"

namespace mxh {

// ---- ggml type facts ----------------------------------------------------------------------
int64_t type_block(int type);       // values per block (1 for plain types), 0 if unknown
int64_t type_bytes(int type);       // bytes per block, 0 if unknown
bool type_is_quantized(int type);
int64_t row_bytes(int type, int64_t n);   // bytes of n values, -1 if n is not whole blocks
bool is_contiguous(const mi355x_tensor * t);
int64_t nelements(const mi355x_tensor * t);
size_t nbytes(const mi355x_tensor * t);
// repacked-weight sources (claims.cpp): whether t's bytes are in a buffer no route reads, the
// registered original bytes for it (nullptr if none match), and how many are registered
bool tensor_needs_source(const mi355x_tensor * t);
const void * tensor_source(const mi355x_tensor * t);
size_t registered_sources();
// The weight types the device path decodes (HBM layouts of mx_weights.h, after a conversion to
// fp16 for F32 and BF16).
bool device_weight_type(int type);
// ggml's decoder of a quantized type registered by the plugin (mi355x_backend_set_to_float), or
// nullptr; such weights are decoded on the host into an fp16 image
mi355x_to_float_fn host_to_float(int type);
int register_to_float(int type, int64_t block, int64_t bytes, mi355x_to_float_fn fn);
// a weight type some route takes: decoded on the device, or on the host by a registered decoder
bool weight_type_ok(int type);

// ---- knobs (read once; MI355X_<name> first, then the reference's ROCKET_<name>) -----------
const char * knob_env(const char * name);   // set-but-empty counts as unset
int knob_int(const char * name, int dflt);
bool knob_on(const char * name, bool dflt);
bool parse_mb(const char * text, size_t * bytes);

int min_m();
int min_m_quant();
enum { MOE_OFF = 0, MOE_AUTO = 1, MOE_FORCED = 2 };
int moe_mode();
int moe_min_tokens();
bool moe_native_on();
int moe_m_bucket();
int moe_min_work_mmac();
bool flash_attn_on();
int flash_attn_min_t();
int flash_attn_min_kv();
bool flash_attn_unmasked();
bool quant_resident_on();
bool fusion_on();

// ---- precision declarations (ggml-rocket.cpp:7334-7404) ------------------------------------
enum : int32_t { PREC_UNDECLARED = 0, PREC_F32 = 10, PREC_BF16 = 15, PREC_F16 = 20, PREC_Q8 = 30, PREC_Q4 = 40 };
bool prec_declines(const mi355x_tensor * op);

// ---- weight identity ------------------------------------------------------------------------
std::string weight_key(const mi355x_tensor * t);

// ---- MoE residency ledger (process-wide; ggml-rocket.cpp:5983-6375) -----------------------
bool moe_preflight_admit(const std::string & key, size_t stack_bytes, const void * src_buf, size_t src_buf_bytes);
bool moe_preflight_decided(const std::string & key, bool * admitted);
enum { MOE_UNDECIDED = 0, MOE_CLAIMED = 1, MOE_REFUSED = 2 };
int moe_preflight_claim(const std::string & key);
void moe_preflight_release(const std::string & key);
void moe_preflight_open();
void moe_preflight_close();

// ---- CPU fallback (fp64; the degraded path after a device failure) -------------------------
void cpu_mul_mat(const mi355x_tensor * dst);
void cpu_flash_attn(const mi355x_tensor * dst);
bool cpu_mul_mat_id(const mi355x_tensor * dst);   // false on an out-of-range id
bool decode_row_f32(int type, const void * src, float * out, int64_t n);

// ---- logging -------------------------------------------------------------------------------
void set_log_sink(mi355x_log_fn fn, void * user);
void logw(const char * fmt, ...) __attribute__((format(printf, 1, 2)));
void logi(const char * fmt, ...) __attribute__((format(printf, 1, 2)));

}  // namespace mxh
