// SPDX-License-Identifier: MIT
// Placement: which ops the scheduler may hand this backend, the precision contract, the weight
// identity every cache keys on, and the process-wide MoE residency ledger.
//
// The rules are the reference's (ggml-rocket.cpp:7334-7772), row for row, with three
// MI355X-specific differences, each stated where it is applied:
//   * the accumulator declaration: this device accumulates in fp32 and writes F32, so an F32 or
//     BF16 accumulator declaration is met (the NPU route could not, 7372-7380);
//   * the weight types: the device decodes F16, F32, BF16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K and MXFP4;
//     any other ggml quant type is claimed once a host decoder (ggml's to_float) is registered
//     for it, which decodes it on the host into the fp16 weight cache, and declined otherwise;
//   * FLASH_ATTN_EXT: head dims up to 1024 (dk % 32, dv % 8), and the strides the kernels read.

#include <atomic>
#include <map>
#include <mutex>
#include <string.h>
#include <string>
#include <unordered_map>

#include <hip/hip_runtime.h>

#include "host.h"
#include "../mx_fa_dims.h"

namespace mxh {

static float op_param_f32(const mi355x_tensor * t, int i) {
    float f;
    memcpy(&f, &t->op_params[i], sizeof f);
    return f;
}

// ---- precision declarations ------------------------------------------------------------------
// op_params[0] accumulator (MUL_MAT, MUL_MAT_ID), [3] activation rank, [1] the Hadamard hint.
// The activation of every route here is converted to fp16 (MoE included: no int8 requant on
// this device), so a declared activation rank above F16 (F32 10, BF16 15) is declined.
bool prec_declines(const mi355x_tensor * op) {
    const int32_t src1 = op->op_params[3];
    if (src1 != PREC_UNDECLARED && src1 < PREC_F16) return true;
    // GGML_HINT_SRC0_IS_HADAMARD: the CPU evaluates it as a fast Walsh-Hadamard transform
    if (op->op == MI355X_OP_MUL_MAT && op->op_params[1] == 1) return true;
    return false;
}

// ---- repacked-weight sources (the contract of ggml-rocket.cpp:6965-7047, API.md:280-314) ---
// ggml-cpu's CPU_REPACK buffer holds a quantized weight in an interleaved layout no route here
// reads. A host that keeps the original bytes (its mapped GGUF range) registers them for the
// tensor; ops on it are then claimed and computed from those bytes while the CPU keeps its
// repacked copy for decode. Placement has no backend handle, so the table is process-wide.
// A registration belongs to the tensor's place in the repack buffer and stands only while the
// tensor there still has the registered name and byte size; a different weight put in that place
// finds nothing (the same model reloaded into it must be unregistered first, as the host does).
namespace {

class SourceTable {
public:
    void put(const mi355x_tensor * t, const void * bytes, size_t n) {
        std::lock_guard<std::mutex> g(lock_);
        const uintptr_t at = (uintptr_t)t->data;
        if (!bytes) rows_.erase(at);
        else rows_[at] = Row{bytes, n, std::string(t->name, strnlen(t->name, MI355X_MAX_NAME))};
        count_.store(rows_.size(), std::memory_order_release);
    }
    // the original bytes for `base` (a tensor that owns its bytes), or nullptr
    const char * find(const mi355x_tensor * base) const {
        std::lock_guard<std::mutex> g(lock_);
        const auto hit = rows_.find((uintptr_t)base->data);
        if (hit == rows_.end()) return nullptr;
        const Row & r = hit->second;
        const bool same_weight = r.n == nbytes(base) && r.name.size() == strnlen(base->name, MI355X_MAX_NAME) &&
                                 memcmp(r.name.data(), base->name, r.name.size()) == 0;
        return same_weight ? (const char *)r.bytes : nullptr;
    }
    size_t count() const { return count_.load(std::memory_order_acquire); }

private:
    struct Row {
        const void * bytes;
        size_t n;
        std::string name;
    };
    mutable std::mutex lock_;
    std::map<uintptr_t, Row> rows_;
    std::atomic<size_t> count_{0};
};

SourceTable & sources() {
    static SourceTable table;
    return table;
}

// A view op reads (part of) the bytes of the tensor it was made from.
bool reads_through(int op) {
    switch (op) {
        case MI355X_OP_VIEW: case MI355X_OP_RESHAPE: case MI355X_OP_PERMUTE: case MI355X_OP_TRANSPOSE: return true;
        default: return false;
    }
}

// The tensor that owns t's bytes (t itself unless t is a view), and t's byte offset in it.
const mi355x_tensor * owner_of(const mi355x_tensor * t, size_t & offset) {
    const mi355x_tensor * o = t;
    while (reads_through(o->op) && o->src[0] != nullptr) o = o->src[0];
    offset = (o->data != nullptr && t->data != nullptr) ? (size_t)((const char *)t->data - (const char *)o->data) : 0;
    return o;
}

}  // namespace

bool tensor_needs_source(const mi355x_tensor * t) {
    size_t offset = 0;
    const int kind = owner_of(t, offset)->buffer_kind;
    return kind == MI355X_BUF_REPACK || kind == MI355X_BUF_OTHER;
}

const void * tensor_source(const mi355x_tensor * t) {
    if (sources().count() == 0) return nullptr;
    size_t offset = 0;
    const mi355x_tensor * o = owner_of(t, offset);
    const char * orig = sources().find(o);
    if (!orig || offset + nbytes(t) > nbytes(o)) return nullptr;
    return orig + offset;
}

size_t registered_sources() { return sources().count(); }

// ---- weight identity (the contract of ggml-rocket.cpp:4124-4222) -------------------------------
// A weight is identified by its logical name and a sample of its bytes. The sample is sixteen
// 64-byte windows at evenly spaced offsets from the first to the last byte (the whole tensor when
// it holds no more than that), so replacing a weight's bytes changes its key. A repacked weight
// is sampled from its registered original bytes: placement sees its data in the repack buffer,
// compute sees the original, and both must produce one key.
namespace {

// 64-bit multiply-xorshift accumulation (a splitmix64-style finalizer per word)
struct WindowHash {
    uint64_t s;
    explicit WindowHash(uint64_t seed) : s(seed) {}
    void word(uint64_t w) {
        s += w + 0x9E3779B97F4A7C15ULL;
        uint64_t z = s;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
        s = z ^ (z >> 31);
    }
    // `len` bytes; a short tail is zero-padded to a word and tagged with its length
    void bytes(const unsigned char * p, size_t len) {
        const size_t whole = len / 8;
        for (size_t i = 0; i < whole; i++) {
            uint64_t w;
            memcpy(&w, p + 8 * i, 8);
            word(w);
        }
        const size_t rest = len % 8;
        if (rest) {
            uint64_t w = 0;
            memcpy(&w, p + 8 * whole, rest);
            word(w ^ ((uint64_t)rest << 59));
        }
    }
};

uint64_t content_sample(const mi355x_tensor * t) {
    const size_t n = nbytes(t);
    const void * orig = tensor_needs_source(t) ? tensor_source(t) : nullptr;
    const unsigned char * base = (const unsigned char *)(orig ? orig : t->data);
    WindowHash h(((uint64_t)n << 8) ^ (uint64_t)(uint32_t)t->type);
    constexpr size_t kWindows = 16, kWidth = 64;
    if (n <= kWindows * kWidth) {
        h.bytes(base, n);
    } else {
        for (size_t i = 0; i < kWindows; i++) h.bytes(base + i * (n - kWidth) / (kWindows - 1), kWidth);
    }
    return h.s;
}

bool all_digits(const char * p) {
    if (*p == 0) return false;
    for (; *p; p++)
        if (*p < '0' || *p > '9') return false;
    return true;
}

// The logical weight name. ggml-backend-sched names the input copies it makes for a backend
// "<backend>#<name>#<index>"; only this backend's copies are mapped back to <name>, with the
// index dropped when it survived the name-length limit. Other names are kept whole.
std::string logical_name(const char * raw) {
    static const char kMine[] = "MI355X#";
    const size_t mine = sizeof kMine - 1;
    if (strncmp(raw, kMine, mine) != 0 || raw[mine] == 0) return std::string(raw);
    std::string name(raw + mine);
    const size_t cut = name.find_last_of('#');
    if (cut != std::string::npos && cut > 0 && all_digits(name.c_str() + cut + 1)) name.erase(cut);
    return name;
}

// "leaf_<n>" / "node_<n>": ggml's names for unnamed tensors, positions in one graph, which
// several graphs of one host reuse for different weights
bool positional_name(const std::string & name) {
    for (const char * p : {"leaf_", "node_"})
        if (name.rfind(p, 0) == 0 && all_digits(name.c_str() + 5)) return true;
    return false;
}

}  // namespace

std::string weight_key(const mi355x_tensor * t) {
    if (!t || !t->name[0]) return std::string();
    char raw[MI355X_MAX_NAME + 1];
    memcpy(raw, t->name, MI355X_MAX_NAME);
    raw[MI355X_MAX_NAME] = 0;
    std::string key = logical_name(raw);
    if (positional_name(key)) return std::string();
    if (t->data) {
        // "@" and the sample as 16 hex digits
        const uint64_t v = content_sample(t);
        static const char kHex[] = "0123456789abcdef";
        key.push_back('@');
        for (int sh = 60; sh >= 0; sh -= 4) key.push_back(kHex[(v >> sh) & 15]);
    }
    return key;
}

// ---- expert-stack ledger (the contract of ggml-rocket.cpp:5983-6375, without the NPU's IOVA) ---
// Placement decides per expert stack, once, whether the whole stack fits in HBM: a stack that
// would only partly fit is declined rather than half ingested. The decision is remembered so a
// stack never moves between devices from one micro-batch to the next. Each live backend holds
// its own HBM copy of a placed stack: the placement decision reserves one spare copy, the first
// backend that runs the stack takes it, and a further backend needs a new copy charged against
// the budget (or streams the stack when it does not fit). Copies are returned when their backend
// is freed; the whole ledger is forgotten once no backend is live. The budget is MOE_CACHE_MB
// (0 = unlimited), by default the device's HBM less an 8 GiB reserve. Under
// MOE_CHARGE_ALL_SOURCE=1 each distinct host weight buffer is also charged once, in full.
namespace {

class ExpertLedger {
public:
    bool place(const std::string & key, size_t copy_bytes, const void * buf, size_t buf_bytes) {
        if (key.empty() || copy_bytes == 0) return false;
        std::lock_guard<std::mutex> g(lock_);
        const auto known = stacks_.find(key);
        if (known != stacks_.end()) return known->second.placed;
        resolve_budget();
        if (charge_buffers_ && buf != nullptr && buf_bytes != 0) buffers_.emplace(buf, buf_bytes);   // once per buffer
        Stack s;
        s.copy_bytes = copy_bytes;
        s.placed = fits(copy_bytes);
        s.spare = s.placed ? 1 : 0;
        stacks_.emplace(key, s);
        return s.placed;
    }
    bool lookup(const std::string & key, bool & placed) {
        if (key.empty()) return false;
        std::lock_guard<std::mutex> g(lock_);
        const auto known = stacks_.find(key);
        if (known == stacks_.end()) return false;
        placed = known->second.placed;
        return true;
    }
    int take(const std::string & key) {
        if (key.empty()) return MOE_UNDECIDED;
        std::lock_guard<std::mutex> g(lock_);
        const auto known = stacks_.find(key);
        if (known == stacks_.end() || !known->second.placed) return MOE_UNDECIDED;
        Stack & s = known->second;
        if (s.spare > 0) {
            s.spare--;
        } else {
            if (!fits(s.copy_bytes)) return MOE_REFUSED;
        }
        s.held++;
        return MOE_CLAIMED;
    }
    void give_back(const std::string & key) {
        std::lock_guard<std::mutex> g(lock_);
        const auto known = stacks_.find(key);
        if (known != stacks_.end() && known->second.held > 0) known->second.held--;
    }
    void attach() {
        std::lock_guard<std::mutex> g(lock_);
        if (live_++ == 0) {
            stacks_.clear();
            buffers_.clear();
            budget_resolved_ = false;
        }
    }
    void detach() {
        std::lock_guard<std::mutex> g(lock_);
        if (live_ > 0) live_--;
    }

private:
    struct Stack {
        bool placed = false;
        size_t copy_bytes = 0;
        int spare = 0;   // charged copies no backend has taken (the placement's reservation)
        int held = 0;    // copies live backends hold
    };
    // bytes charged now: every spare and held copy, and the charged host buffers
    size_t charged() const {
        size_t sum = 0;
        for (const auto & kv : stacks_) sum += (size_t)(kv.second.spare + kv.second.held) * kv.second.copy_bytes;
        for (const auto & kv : buffers_) sum += kv.second;
        return sum;
    }
    bool fits(size_t more) const { return budget_ == 0 || charged() + more <= budget_; }
    void resolve_budget() {
        if (budget_resolved_) return;
        budget_resolved_ = true;
        size_t b = 0;
        const char * text = knob_env("MOE_CACHE_MB");
        budget_ = (text && parse_mb(text, &b)) ? b : hbm_less_reserve();
        charge_buffers_ = knob_int("MOE_CHARGE_ALL_SOURCE", 0) != 0;
    }
    static size_t hbm_less_reserve() {
        const size_t reserve = (size_t)8 << 30;
        size_t free_b = 0, total_b = 0;
        int devices = 0;
        if (hipGetDeviceCount(&devices) != hipSuccess || devices <= 0 || hipMemGetInfo(&free_b, &total_b) != hipSuccess ||
            total_b == 0) {
            (void)hipGetLastError();
            return (size_t)4 << 30;   // no device to ask: a conservative figure
        }
        return total_b > reserve ? total_b - reserve : total_b / 2;
    }

    std::mutex lock_;
    std::unordered_map<std::string, Stack> stacks_;
    std::map<const void *, size_t> buffers_;   // host weight buffers charged under MOE_CHARGE_ALL_SOURCE
    size_t budget_ = 0;                        // 0 = unlimited
    bool budget_resolved_ = false;
    bool charge_buffers_ = false;
    int live_ = 0;
};

ExpertLedger & ledger() {
    static ExpertLedger l;
    return l;
}

}  // namespace

bool moe_preflight_admit(const std::string & key, size_t stack_bytes, const void * src_buf, size_t src_buf_bytes) {
    return ledger().place(key, stack_bytes, src_buf, src_buf_bytes);
}
bool moe_preflight_decided(const std::string & key, bool * admitted) { return ledger().lookup(key, *admitted); }
int moe_preflight_claim(const std::string & key) { return ledger().take(key); }
void moe_preflight_release(const std::string & key) { ledger().give_back(key); }
void moe_preflight_open() { ledger().attach(); }
void moe_preflight_close() { ledger().detach(); }

// ---- claim rules -----------------------------------------------------------------------------

static bool claim_mul_mat(const mi355x_tensor * op) {
    const mi355x_tensor * a = op->src[0];
    const mi355x_tensor * b = op->src[1];
    if (!a || !b) return false;
    const int64_t K = a->ne[0], N = a->ne[1], M = b->ne[1];
    const bool a_quant = type_is_quantized(a->type);
    if (prec_declines(op)) return false;
    return a->op == MI355X_OP_NONE                      // a static leaf weight (7434-7440)
        && weight_type_ok(a->type)
        && b->type == MI355X_TYPE_F32
        && op->type == MI355X_TYPE_F32
        && is_contiguous(a) && is_contiguous(b) && is_contiguous(op)
        && a->ne[0] == b->ne[0]
        && a->ne[2] == 1 && a->ne[3] == 1               // plain 2D weight
        && (!a_quant || K % type_block(a->type) == 0)
        && K % 32 == 0 && N % 16 == 0
        && K >= 64 && N >= 64
        && M >= (a_quant ? min_m_quant() : min_m());
}

static bool claim_mul_mat_id(const mi355x_tensor * op) {
    const int mode = moe_mode();
    if (mode == MOE_OFF) return false;
    const mi355x_tensor * a = op->src[0];
    const mi355x_tensor * b = op->src[1];
    const mi355x_tensor * id = op->src[2];
    if (!a || !b || !id) return false;
    if (prec_declines(op)) return false;
    const int64_t K = a->ne[0], N = a->ne[1], n_tokens = id->ne[1];
    const bool a_quant = type_is_quantized(a->type);
    const bool computable = a->op == MI355X_OP_NONE
        && weight_type_ok(a->type)
        && b->type == MI355X_TYPE_F32
        && id->type == MI355X_TYPE_I32
        && op->type == MI355X_TYPE_F32
        && is_contiguous(a) && is_contiguous(b) && is_contiguous(op)
        && a->ne[0] == b->ne[0]
        && a->ne[3] == 1
        && (!a_quant || K % type_block(a->type) == 0)
        && K % 32 == 0 && N % 16 == 0
        && K >= 64 && N >= 64
        && n_tokens >= moe_min_tokens();
    if (!computable) return false;
    if (mode == MOE_FORCED) return true;
    // AUTO (ggml-rocket.cpp:7560-7652): a quantized stack on the native route, K%32 and N%32,
    // at least the row granule per expert, at least the per-dispatch work floor, and the
    // whole stack admitted by the residency pre-flight.
    if (!a_quant || !moe_native_on()) return false;
    if (K % 32 || N % 32) return false;
    const int64_t n_used = id->ne[0], n_expert = a->ne[2];
    if (n_expert <= 0) return false;
    const int64_t m_e = n_tokens * n_used / n_expert;
    if (m_e < moe_m_bucket()) return false;
    if (m_e * K * N < (int64_t)moe_min_work_mmac() * 1000000) return false;
    const std::string key = weight_key(a);
    bool admitted = false;
    if (moe_preflight_decided(key, &admitted)) return admitted;
    // a host-decoded type is held as its fp16 image
    const size_t rb = device_weight_type(a->type) ? (size_t)row_bytes(a->type, K) : (size_t)K * 2;
    const size_t stack_bytes = rb * (size_t)N * (size_t)n_expert;
    return moe_preflight_admit(key, stack_bytes, a->buffer_id, a->buffer_size);
}

static bool claim_flash_attn(const mi355x_tensor * op) {
    const mi355x_tensor * q = op->src[0];
    const mi355x_tensor * k = op->src[1];
    const mi355x_tensor * v = op->src[2];
    const mi355x_tensor * m = op->src[3];
    if (!flash_attn_on() || !q || !k || !v) return false;
    if (!m && !flash_attn_unmasked()) return false;
    if (op->src[4]) return false;                         // attention sinks (7703-7721)
    const float max_bias = op_param_f32(op, 1);
    const int64_t head_dim = q->ne[0], n_tokens = q->ne[1], n_head = q->ne[2];
    const int64_t dv = v->ne[0], n_kv = k->ne[1], n_kv_heads = k->ne[2];
    const bool ref_rules = max_bias == 0.0f
        && q->type == MI355X_TYPE_F32 && k->type == MI355X_TYPE_F16 && v->type == MI355X_TYPE_F16
        && (!m || (m->type == MI355X_TYPE_F16 && is_contiguous(m)))
        && op->type == MI355X_TYPE_F32 && is_contiguous(op)
        && q->ne[3] == 1 && k->ne[3] == 1
        && k->ne[0] == head_dim && op->ne[0] == dv
        && v->ne[1] == n_kv && v->ne[2] == n_kv_heads
        && head_dim % 32 == 0 && dv % 16 == 0
        && n_kv_heads > 0 && n_head % n_kv_heads == 0
        && (!m || (m->ne[0] >= n_kv && m->ne[1] >= n_tokens))
        && n_tokens >= flash_attn_min_t()
        && n_kv >= flash_attn_min_kv();
    if (!ref_rules) return false;
    // what the kernels read: head dims the fused kernel holds zero-padded (dk, dv <= 256; built
    // for 64/64, 128/128, the MLA 192/128 and 256/256) or, past those, the two-GEMM path (dk % 32
    // == 0, dv % 8 == 0, both up to 1024: the absorbed MLA's 576 / 512); element strides;
    // 16-byte rows
    int dk_pad = 0, dv_pad = 0;
    const bool dims = (head_dim <= 256 && dv <= 256 && mx::fa_pad_dims((int)head_dim, (int)dv, dk_pad, dv_pad)) ||
                      mx::fa_wide_dims((int)head_dim, (int)dv);
    const bool q_ok = q->nb[0] == 4 && q->nb[1] % 16 == 0 && q->nb[2] % 16 == 0;
    const bool kv_ok = k->nb[0] == 2 && v->nb[0] == 2 && k->nb[1] % 16 == 0 && k->nb[2] % 16 == 0 &&
                       v->nb[1] % 16 == 0 && v->nb[2] % 16 == 0;
    const bool m_ok = !m || m->nb[1] % 8 == 0;
    return dims && q_ok && kv_ok && m_ok;
}

}  // namespace mxh

using namespace mxh;

extern "C" {

MI355X_API bool mi355x_backend_supports_op(const mi355x_tensor * op) {
    if (!op) return false;
    // a source in a buffer this backend cannot read as ggml blocks (CPU_REPACK, another device)
    // stays on the CPU unless its original bytes are registered (ggml-rocket.cpp:7036-7043)
    for (int i = 0; i < MI355X_MAX_SRC; i++)
        if (op->src[i] && tensor_needs_source(op->src[i]) && !tensor_source(op->src[i])) return false;
    switch (op->op) {
        case MI355X_OP_NONE:
        case MI355X_OP_RESHAPE:
        case MI355X_OP_VIEW:
        case MI355X_OP_PERMUTE:
        case MI355X_OP_TRANSPOSE:
            return true;
        case MI355X_OP_MUL_MAT: return claim_mul_mat(op);
        case MI355X_OP_MUL_MAT_ID: return claim_mul_mat_id(op);
        case MI355X_OP_FLASH_ATTN_EXT: return claim_flash_attn(op);
        default: return false;
    }
}

MI355X_API bool mi355x_backend_offload_op(const mi355x_tensor * op) {
    return op && (op->op == MI355X_OP_MUL_MAT || op->op == MI355X_OP_MUL_MAT_ID) &&
           mi355x_backend_supports_op(op);
}

MI355X_API bool mi355x_backend_supports_buft(int buffer_kind) {
    return buffer_kind == MI355X_BUF_HOST || buffer_kind == MI355X_BUF_REPACK;
}

MI355X_API void mi355x_backend_register_weight_source(const mi355x_tensor * t, const void * data, size_t nbytes) {
    if (t && t->data) sources().put(t, data, nbytes);
}

MI355X_API int mi355x_backend_weight_key(const mi355x_tensor * t, char * out, int cap) {
    const std::string k = weight_key(t);
    if (out && cap > 0) {
        const size_t n = k.size() < (size_t)(cap - 1) ? k.size() : (size_t)(cap - 1);
        memcpy(out, k.data(), n);
        out[n] = 0;
    }
    return (int)k.size();
}

MI355X_API void mi355x_backend_set_log_callback(mi355x_log_fn fn, void * user) { set_log_sink(fn, user); }

MI355X_API bool mi355x_backend_parse_mb(const char * text, size_t * bytes) {
    return parse_mb(text, bytes);
}

}  // extern "C"
