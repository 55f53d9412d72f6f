// SPDX-License-Identifier: MIT
// Placement: which ops the scheduler may hand this backend, the precision contract, the weight
// identity every cache keys on, and the process-wide MoE residency ledger.
//
// The rules are the reference's (ggml-rocket.cpp:7334-7772), row for row, with three
// MI355X-specific differences, each stated where it is applied:
//   * the accumulator declaration: this device accumulates in fp32 and writes F32, so an F32 or
//     BF16 accumulator declaration is met (the NPU route could not, 7372-7380);
//   * the weight types: the device decodes F16, F32, BF16, Q8_0, Q4_K, Q6_K and MXFP4; other ggml quant
//     types are declined rather than claimed and then computed on the host;
//   * FLASH_ATTN_EXT: head dims up to 256, and the strides the kernel reads.

#include <atomic>
#include <mutex>
#include <string.h>
#include <string>
#include <unordered_map>
#include <unordered_set>

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

// ---- repacked-weight sources (ggml-rocket.cpp:6965-7047, API.md:280-314) ----------------------
// ggml-cpu's CPU_REPACK buffer holds a quantized weight in an interleaved layout no route here
// reads. A host that keeps the original bytes (its mapped GGUF range) registers them for the
// tensor; ops on it are then claimed and computed from those bytes, and the CPU keeps its
// repacked copy for decode. The registry is process-wide, as placement has no backend handle.
// An entry is keyed by the tensor's own data address (its place in the repack buffer) and is
// used only while the tensor's name and byte size still match it, which catches a tensor struct
// reused for another weight, not the same model reloaded into it: the host unregisters first.
namespace {
struct WSrc {
    const void * src;
    size_t nbytes;
    std::string name;
};
std::mutex g_wsrc_mu;
std::unordered_map<const void *, WSrc> g_wsrc;
std::atomic<size_t> g_wsrc_count{0};

bool is_view_op(int op) {
    return op == MI355X_OP_VIEW || op == MI355X_OP_RESHAPE || op == MI355X_OP_PERMUTE || op == MI355X_OP_TRANSPOSE;
}

// the tensor a view reads, and the byte offset of the view in it
const mi355x_tensor * view_base(const mi355x_tensor * t, size_t * offs) {
    const mi355x_tensor * b = t;
    while (is_view_op(b->op) && b->src[0]) b = b->src[0];
    *offs = (b->data && t->data) ? (size_t)((const char *)t->data - (const char *)b->data) : 0;
    return b;
}

}  // namespace

bool tensor_needs_source(const mi355x_tensor * t) {
    size_t offs;
    const mi355x_tensor * b = view_base(t, &offs);
    return b->buffer_kind == MI355X_BUF_REPACK || b->buffer_kind == MI355X_BUF_OTHER;
}

const void * tensor_source(const mi355x_tensor * t) {
    if (g_wsrc_count.load(std::memory_order_acquire) == 0) return nullptr;
    size_t offs;
    const mi355x_tensor * b = view_base(t, &offs);
    std::lock_guard<std::mutex> lk(g_wsrc_mu);
    auto it = g_wsrc.find(b->data);
    if (it == g_wsrc.end()) return nullptr;
    if (it->second.nbytes != nbytes(b) || it->second.name != std::string(b->name, strnlen(b->name, MI355X_MAX_NAME)))
        return nullptr;
    if (offs + nbytes(t) > it->second.nbytes) return nullptr;
    return (const char *)it->second.src + offs;
}

size_t registered_sources() { return g_wsrc_count.load(std::memory_order_acquire); }

// ---- weight identity ---------------------------------------------------------------------------
// A sampled content fingerprint: sixteen 64-byte windows spread over the tensor (all of it when
// smaller), mixed with the byte size and type. Changes when a weight's bytes are replaced. A
// repacked weight is fingerprinted over its registered original bytes, so placement (data at the
// repacked copy) and compute (data pointed at the original) agree on its key.
static uint64_t fingerprint(const mi355x_tensor * t) {
    const size_t n = nbytes(t);
    const void * src = tensor_needs_source(t) ? tensor_source(t) : nullptr;
    const unsigned char * p = (const unsigned char *)(src ? src : t->data);
    uint64_t h = 0xcbf29ce484222325ULL ^ ((uint64_t)n * 0x9E3779B97F4A7C15ULL) ^ ((uint64_t)(uint32_t)t->type << 48);
    auto mix = [&h](uint64_t x) {
        h ^= x + 0x632BE59BD9B4E019ULL + (h << 6) + (h >> 2);
        h *= 0x100000001B3ULL;
    };
    auto span = [&](size_t off, size_t len) {
        size_t i = 0;
        for (; i + 8 <= len; i += 8) {
            uint64_t x;
            memcpy(&x, p + off + i, 8);
            mix(x);
        }
        for (; i < len; i++) mix(0x100u | p[off + i]);
    };
    const int NW = 16;
    const size_t W = 64;
    if (n <= (size_t)NW * W) span(0, n);
    else for (int w = 0; w < NW; w++) span((n - W) / (NW - 1) * (size_t)w, W);
    return h;
}

std::string weight_key(const mi355x_tensor * t) {
    if (!t || !t->name[0]) return std::string();
    char name[MI355X_MAX_NAME + 1];
    memcpy(name, t->name, MI355X_MAX_NAME);
    name[MI355X_MAX_NAME] = 0;
    // the scheduler's input-copy grammar "<backend>#<name>#<idx>", for this backend only
    static const char PREFIX[] = "MI355X#";
    const size_t plen = sizeof(PREFIX) - 1;
    const bool copy = strncmp(name, PREFIX, plen) == 0 && name[plen];
    std::string key(copy ? name + plen : name);
    if (copy) {
        const size_t h = key.rfind('#');
        if (h != std::string::npos && h > 0 && h + 1 < key.size() &&
            key.find_first_not_of("0123456789", h + 1) == std::string::npos)
            key.resize(h);
    }
    // ggml auto-names ("leaf_<n>", "node_<n>") are graph positions, not weight identities
    for (const char * pre : {"leaf_", "node_"}) {
        if (key.compare(0, 5, pre) == 0 && key.size() > 5 &&
            key.find_first_not_of("0123456789", 5) == std::string::npos)
            return std::string();
    }
    if (t->data) {
        char id[24];
        snprintf(id, sizeof id, "@%016llx", (unsigned long long)fingerprint(t));
        key += id;
    }
    return key;
}

// ---- MoE residency ledger ------------------------------------------------------------------
// A stack (one expert weight tensor) is admitted whole or not at all, before its first ingest:
// partial residency is what the pre-flight exists to avoid (ggml-rocket.cpp:6198-6289). The
// charge is the stack's HBM copy (its packed bytes, equal to the GGUF bytes), plus, under
// MOE_CHARGE_ALL_SOURCE=1, each distinct mapped source buffer once. The budget is
// MOE_CACHE_MB (0 = unlimited), by default the device's HBM less an 8 GiB reserve. The ledger is
// process-wide and cleared when the last backend instance is freed.
namespace {
struct Stack {
    bool admitted = false;
    size_t bytes = 0;
    int copies = 0;
    int claimed = 0;
};
struct Ledger {
    std::mutex mu;
    bool frozen = false;
    size_t budget = 0;    // 0 = unlimited
    size_t used = 0;
    size_t src_used = 0;
    bool all_src = false;
    int live = 0;
    std::unordered_set<const void *> src_bufs;
    std::unordered_map<std::string, Stack> stacks;
};
Ledger g_ledger;

size_t default_moe_budget() {
    size_t fr = 0, tot = 0;
    int n = 0;
    if (hipGetDeviceCount(&n) == hipSuccess && n > 0 && hipMemGetInfo(&fr, &tot) == hipSuccess && tot) {
        const size_t reserve = (size_t)8 << 30;
        return tot > reserve ? tot - reserve : tot / 2;
    }
    (void)hipGetLastError();
    return (size_t)4096 << 20;   // no device to ask: a conservative figure
}
}  // namespace

bool moe_preflight_admit(const std::string & key, size_t stack_bytes, const void * src_buf, size_t src_buf_bytes) {
    if (key.empty() || stack_bytes == 0) return false;
    std::lock_guard<std::mutex> lk(g_ledger.mu);
    auto it = g_ledger.stacks.find(key);
    if (it != g_ledger.stacks.end()) return it->second.admitted;
    if (!g_ledger.frozen) {
        size_t b = 0;
        const char * e = knob_env("MOE_CACHE_MB");
        g_ledger.budget = (e && parse_mb(e, &b)) ? b : default_moe_budget();
        g_ledger.all_src = knob_int("MOE_CHARGE_ALL_SOURCE", 0) != 0;
        g_ledger.frozen = true;
    }
    if (g_ledger.all_src && src_buf && src_buf_bytes && g_ledger.src_bufs.insert(src_buf).second)
        g_ledger.src_used += src_buf_bytes;
    Stack st;
    const bool fits = !g_ledger.budget || g_ledger.used + g_ledger.src_used + stack_bytes <= g_ledger.budget;
    if (fits) {
        st.admitted = true;
        st.bytes = stack_bytes;
        st.copies = 1;
        g_ledger.used += stack_bytes;
    }
    g_ledger.stacks[key] = st;
    return fits;
}

bool moe_preflight_decided(const std::string & key, bool * admitted) {
    if (key.empty()) return false;
    std::lock_guard<std::mutex> lk(g_ledger.mu);
    auto it = g_ledger.stacks.find(key);
    if (it == g_ledger.stacks.end()) return false;
    *admitted = it->second.admitted;
    return true;
}

int moe_preflight_claim(const std::string & key) {
    if (key.empty()) return MOE_UNDECIDED;
    std::lock_guard<std::mutex> lk(g_ledger.mu);
    auto it = g_ledger.stacks.find(key);
    if (it == g_ledger.stacks.end() || !it->second.admitted) return MOE_UNDECIDED;
    Stack & st = it->second;
    if (st.claimed < st.copies) {
        st.claimed++;
        return MOE_CLAIMED;
    }
    // a second live backend wants its own copy: charge it if it fits
    if (g_ledger.budget && g_ledger.used + g_ledger.src_used + st.bytes > g_ledger.budget) return MOE_REFUSED;
    g_ledger.used += st.bytes;
    st.copies++;
    st.claimed++;
    return MOE_CLAIMED;
}

void moe_preflight_release(const std::string & key) {
    std::lock_guard<std::mutex> lk(g_ledger.mu);
    auto it = g_ledger.stacks.find(key);
    if (it == g_ledger.stacks.end() || it->second.claimed <= 0) return;
    it->second.claimed--;
    it->second.copies--;
    g_ledger.used -= it->second.bytes;
}

void moe_preflight_open() {
    std::lock_guard<std::mutex> lk(g_ledger.mu);
    if (g_ledger.live == 0) {
        g_ledger.stacks.clear();
        g_ledger.src_bufs.clear();
        g_ledger.used = g_ledger.src_used = 0;
        g_ledger.frozen = false;
    }
    g_ledger.live++;
}

void moe_preflight_close() {
    std::lock_guard<std::mutex> lk(g_ledger.mu);
    if (g_ledger.live > 0) g_ledger.live--;
}

// ---- claim rules -----------------------------------------------------------------------------

static bool claim_mul_mat(const mi355x_tensor * op) {
    const mi355x_tensor * a = op->src[0];
    const mi355x_tensor * b = op->src[1];
    if (!a || !b) return false;
    const int64_t K = a->ne[0], N = a->ne[1], M = b->ne[1];
    const bool a_quant = type_is_quantized(a->type);
    if (prec_declines(op)) return false;
    return a->op == MI355X_OP_NONE                      // a static leaf weight (7434-7440)
        && device_weight_type(a->type)
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
        && device_weight_type(a->type)
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
    const size_t stack_bytes = (size_t)row_bytes(a->type, K) * (size_t)N * (size_t)n_expert;
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
    // what the kernel reads: head dims it holds zero-padded (dk, dv <= 256; the kernels are
    // built for 64/64, 128/128, the MLA 192/128 and 256/256); element strides; 16-byte rows
    int dk_pad = 0, dv_pad = 0;
    const bool dims = head_dim <= 256 && dv <= 256 && mx::fa_pad_dims((int)head_dim, (int)dv, dk_pad, dv_pad);
    const bool q_ok = q->nb[0] == 4 && q->nb[1] % 16 == 0 && q->nb[2] % 16 == 0;
    const bool kv_ok = k->nb[0] == 2 && v->nb[0] == 2 && k->nb[1] % 16 == 0 && k->nb[2] % 16 == 0 &&
                       v->nb[1] % 16 == 0 && v->nb[2] % 16 == 0;
    const bool m_ok = !m || m->nb[1] % 8 == 0;
    return dims && q_ok && kv_ok && m_ok;
}

}  // namespace mxh

using namespace mxh;

extern "C" {

MI355X_API bool ggml_backend_mi355x_supports_op(const mi355x_tensor * op) {
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

MI355X_API bool ggml_backend_mi355x_offload_op(const mi355x_tensor * op) {
    return op && (op->op == MI355X_OP_MUL_MAT || op->op == MI355X_OP_MUL_MAT_ID) &&
           ggml_backend_mi355x_supports_op(op);
}

MI355X_API bool ggml_backend_mi355x_supports_buft(int buffer_kind) {
    return buffer_kind == MI355X_BUF_HOST || buffer_kind == MI355X_BUF_REPACK;
}

MI355X_API void ggml_backend_mi355x_register_weight_source(const mi355x_tensor * t, const void * data, size_t nbytes) {
    if (!t || !t->data) return;
    std::lock_guard<std::mutex> lk(g_wsrc_mu);
    if (!data) g_wsrc.erase(t->data);
    else g_wsrc[t->data] = WSrc{data, nbytes, std::string(t->name, strnlen(t->name, MI355X_MAX_NAME))};
    g_wsrc_count.store(g_wsrc.size(), std::memory_order_release);
}

MI355X_API int ggml_backend_mi355x_weight_key(const mi355x_tensor * t, char * out, int cap) {
    const std::string k = weight_key(t);
    if (out && cap > 0) {
        const size_t n = k.size() < (size_t)(cap - 1) ? k.size() : (size_t)(cap - 1);
        memcpy(out, k.data(), n);
        out[n] = 0;
    }
    return (int)k.size();
}

MI355X_API bool ggml_backend_mi355x_parse_mb(const char * text, size_t * bytes) {
    return parse_mb(text, bytes);
}

}  // extern "C"
