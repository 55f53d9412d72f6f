// SPDX-License-Identifier: MIT
// The ggml plugin face of the MI355X backend: ggml's backend, device and registry vtables over
// libmi355x's host layer (include/mi355x_backend.h), the reference's public API under this
// backend's name (include/ggml-mi355x.h, replacing ggml-rocket.h:23-91) and the GGML_BACKEND_DL
// loader entry (replacing ggml-rocket.cpp:8219-8266). Slot for slot it fills what
// ggml-rocket.cpp:7233-7239 (backend), 7829-7842 (device) and 7848-7881 (registry) fill.
//
// It is compiled against the HOST's ggml -- its public headers (ggml/include) and the private
// ggml-backend-impl.h / ggml-impl.h (ggml/src) -- and linked into libggml-mi355x.so with the
// host layer and kernels and the host's libggml-base / libggml-cpu, so the registry it hands out
// lands in the host's own ggml instance:
//     make -C ggml-rocket_amd ggml HOST_GGML_DIR=<llama.cpp or whisper.cpp checkout>
//
// ggml tensors reach the host layer as mi355x_tensor descriptors built per call. Ops are
// matched by the NAME the host's ggml gives them (ggml_op_name), never by ordinal, so the
// mapping follows a host whose op enum moved; the loader entry still refuses a host whose op
// ordinals differ from the ones this file was compiled with, because that means a different
// ggml whose tensor layout this build cannot vouch for either.

#include <stdio.h>
#include <string.h>

#include <atomic>
#include <deque>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "ggml-backend-impl.h"
#include "ggml-backend.h"
#include "ggml-cpu.h"
#include "ggml-impl.h"
#include "ggml.h"

#include "../../include/ggml-mi355x.h"
#include "../../include/mi355x_backend.h"

// The vtables below are checked against GGML_BACKEND_API_VERSION 2 and 3 (version 3 added
// slots to ggml_backend_buffer_type_i only, which this backend never fills: it hands out the
// host's CPU buffer type). Designated initializers bind each function to its slot by name, so
// a slot ggml adds compiles to NULL (unimplemented) and a renamed one fails to compile.
// A version not yet checked warns; built with MI355X_STRICT_ABI (`make ggml STRICT_ABI=1`) it
// is an error instead, so a CI build cannot pass on an unchecked ggml.
#if GGML_BACKEND_API_VERSION != 2 && GGML_BACKEND_API_VERSION != 3
#if defined(MI355X_STRICT_ABI)
#error "ggml-mi355x: GGML_BACKEND_API_VERSION is not 2 or 3; check the three vtables against ggml-backend-impl.h and add the version"
#else
#warning "ggml-mi355x: the vtables are checked against GGML_BACKEND_API_VERSION 2 and 3; check ggml-backend-impl.h"
#endif
#endif

namespace {

// ---- ops and buffers, as the host's ggml names them ---------------------------------------------

struct NamedOp {
    const char * name;
    int op;
};
constexpr NamedOp kNamedOps[] = {
    {"NONE", MI355X_OP_NONE},       {"MUL_MAT", MI355X_OP_MUL_MAT},       {"MUL_MAT_ID", MI355X_OP_MUL_MAT_ID},
    {"FLASH_ATTN_EXT", MI355X_OP_FLASH_ATTN_EXT}, {"RESHAPE", MI355X_OP_RESHAPE}, {"VIEW", MI355X_OP_VIEW},
    {"PERMUTE", MI355X_OP_PERMUTE}, {"TRANSPOSE", MI355X_OP_TRANSPOSE},   {"ADD", MI355X_OP_ADD},
    {"SCALE", MI355X_OP_SCALE},
};

// ordinal -> host-layer op + 1 (0 = not looked up yet); the same answer every time, so racing
// writers store the same value
std::atomic<int> g_op_of_ordinal[256];

int host_layer_op(enum ggml_op op) {
    const unsigned ord = (unsigned)op;
    if (ord < 256) {
        const int known = g_op_of_ordinal[ord].load(std::memory_order_relaxed);
        if (known) return known - 1;
    }
    const char * name = ggml_op_name(op);
    int found = MI355X_OP_OTHER;
    for (const NamedOp & e : kNamedOps)
        if (name && strcmp(name, e.name) == 0) found = e.op;
    if (ord < 256) g_op_of_ordinal[ord].store(found + 1, std::memory_order_relaxed);
    return found;
}

bool buft_is_repack(ggml_backend_buffer_type_t buft) {
    const char * n = buft ? ggml_backend_buft_name(buft) : nullptr;
    return n && strcmp(n, "CPU_REPACK") == 0;
}

int buffer_kind_of(ggml_backend_buffer_t b) {
    if (!b) return MI355X_BUF_NONE;
    if (ggml_backend_buffer_is_host(b)) return MI355X_BUF_HOST;
    return buft_is_repack(ggml_backend_buffer_get_type(b)) ? MI355X_BUF_REPACK : MI355X_BUF_OTHER;
}

bool is_view(int op) {
    return op == MI355X_OP_VIEW || op == MI355X_OP_RESHAPE || op == MI355X_OP_PERMUTE || op == MI355X_OP_TRANSPOSE;
}

// ---- descriptors ----------------------------------------------------------------------------------
// One mi355x_tensor per distinct ggml_tensor of a call, so nodes that share a source share its
// descriptor (the host layer fuses MUL_MATs on that identity). A node of the call and every view
// get their sources described; any other source only itself (its own sources are earlier parts
// of the host's graph that the host layer never reads). Descriptors live as long as the Mirror.
class Mirror {
public:
    // a tensor the call computes: described with its sources
    mi355x_tensor * node(const ggml_tensor * t) { return describe(t, true); }
    // a tensor the call reads
    mi355x_tensor * source(const ggml_tensor * t) { return describe(t, false); }

private:
    struct Entry {
        mi355x_tensor * d;
        bool expanded;
    };

    mi355x_tensor * describe(const ggml_tensor * t, bool with_sources) {
        if (!t) return nullptr;
        auto it = seen_.find(t);
        if (it == seen_.end()) {
            store_.emplace_back();
            mi355x_tensor * d = &store_.back();
            fill(d, t);
            it = seen_.emplace(t, Entry{d, false}).first;
        }
        Entry & e = it->second;
        if (!e.expanded && (with_sources || is_view(e.d->op))) {
            e.expanded = true;
            for (int j = 0; j < GGML_MAX_SRC && j < MI355X_MAX_SRC; j++) e.d->src[j] = source(t->src[j]);
        }
        return e.d;
    }

    static void fill(mi355x_tensor * d, const ggml_tensor * t) {
        memset(d, 0, sizeof *d);
        d->type = (int32_t)t->type;
        d->op = host_layer_op(t->op);
        for (int i = 0; i < MI355X_MAX_DIMS; i++) {
            d->ne[i] = t->ne[i];
            d->nb[i] = t->nb[i];
        }
        static_assert(sizeof(t->op_params) >= sizeof(d->op_params), "ggml op_params smaller than the descriptor's");
        memcpy(d->op_params, t->op_params, sizeof d->op_params);
        d->data = t->data;
        static_assert(sizeof(t->name) <= MI355X_MAX_NAME, "ggml tensor names longer than the descriptor's");
        memcpy(d->name, t->name, sizeof t->name);
        const ggml_backend_buffer_t b = t->view_src ? t->view_src->buffer : t->buffer;
        d->buffer_kind = buffer_kind_of(b);
        d->buffer_id = b;
        d->buffer_size = b ? ggml_backend_buffer_get_size(b) : 0;
    }

    std::deque<mi355x_tensor> store_;   // stable addresses
    std::unordered_map<const ggml_tensor *, Entry> seen_;
};

// ---- log lines into ggml's logger -----------------------------------------------------------------
void to_ggml_log(int level, const char * text, void *) {
    ggml_log_internal(level == MI355X_LOG_WARN ? GGML_LOG_LEVEL_WARN : GGML_LOG_LEVEL_INFO, "%s", text);
}

// ---- backend (ggml_backend_i) -----------------------------------------------------------------------
mi355x_backend_t ctx_of(ggml_backend_t b) { return (mi355x_backend_t)b->context; }

const char * backend_get_name(ggml_backend_t) { return mi355x_backend_name(); }

void backend_free(ggml_backend_t b) {
    mi355x_backend_free(ctx_of(b));
    delete b;
}

// Synchronous: every dst is in host memory when this returns (the vtable has no async slots).
enum ggml_status backend_graph_compute(ggml_backend_t b, struct ggml_cgraph * g) {
    Mirror m;
    const int n = ggml_graph_n_nodes(g);
    std::vector<mi355x_tensor *> nodes((size_t)n);
    for (int i = 0; i < n; i++) nodes[(size_t)i] = m.node(ggml_graph_node(g, i));
    const int st = mi355x_backend_graph_compute(ctx_of(b), nodes.data(), n);
    return st == MI355X_STATUS_SUCCESS ? GGML_STATUS_SUCCESS : GGML_STATUS_FAILED;
}

#pragma GCC diagnostic push
#pragma GCC diagnostic ignored "-Wmissing-field-initializers"
const ggml_backend_i kBackendIface = {
    .get_name = backend_get_name,
    .free = backend_free,
    .graph_compute = backend_graph_compute,
};
#pragma GCC diagnostic pop

ggml_guid_t backend_guid() {
    // "MI355X" + "gfx950" + 4 bytes: a fixed identity for ggml_backend_is_mi355x
    static ggml_guid id = {0x4d, 0x49, 0x33, 0x35, 0x35, 0x58, 0x67, 0x66, 0x78, 0x39, 0x35, 0x30, 0x5f, 0x70, 0x66, 0x31};
    return &id;
}

// ---- device (ggml_backend_device_i) ---------------------------------------------------------------
const char * device_get_name(ggml_backend_dev_t) { return mi355x_backend_name(); }
const char * device_get_description(ggml_backend_dev_t) { return mi355x_backend_description(); }

// Host memory (MemAvailable / MemTotal), as the reference reports it: the device hands out the
// host's CPU buffer type, so the model's tensors live in host pages, and llama.cpp's device
// auto-fit sizes them against memory_free. HBM only holds the weight cache (a copy, with its own
// budget) and per-op operands, so reporting it would let the auto-fit place more than host
// memory holds.
void device_get_memory(ggml_backend_dev_t, size_t * free_b, size_t * total_b) {
    mi355x_backend_get_host_memory(free_b, total_b);
}

enum ggml_backend_dev_type device_get_type(ggml_backend_dev_t) { return GGML_BACKEND_DEVICE_TYPE_ACCEL; }

void device_get_props(ggml_backend_dev_t dev, struct ggml_backend_dev_props * p) {
    p->name = device_get_name(dev);
    p->description = device_get_description(dev);
    p->type = device_get_type(dev);
    device_get_memory(dev, &p->memory_free, &p->memory_total);
    // fields some ggml versions have and others lack, set where present
    [](auto & props) {
        if constexpr (requires { props.device_id; }) props.device_id = nullptr;
    }(*p);
    p->caps.async = false;
    p->caps.host_buffer = false;
    p->caps.buffer_from_host_ptr = true;   // weights are read from the host's own (mmapped) buffers
    p->caps.events = false;
    [](auto & caps) {
        if constexpr (requires { caps.mmap_support; }) caps.mmap_support = true;
    }(p->caps);
}

ggml_backend_t device_init_backend(ggml_backend_dev_t, const char *) { return ggml_backend_mi355x_init(); }

ggml_backend_buffer_type_t device_get_buffer_type(ggml_backend_dev_t) { return ggml_backend_cpu_buffer_type(); }

ggml_backend_buffer_t device_buffer_from_host_ptr(ggml_backend_dev_t, void * ptr, size_t size, size_t) {
    return ggml_backend_cpu_buffer_from_ptr(ptr, size);
}

bool device_supports_op(ggml_backend_dev_t, const struct ggml_tensor * op) {
    Mirror m;
    return mi355x_backend_supports_op(m.node(op));
}

bool device_supports_buft(ggml_backend_dev_t, ggml_backend_buffer_type_t buft) {
    const int kind = ggml_backend_buft_is_host(buft) ? MI355X_BUF_HOST
                   : buft_is_repack(buft)           ? MI355X_BUF_REPACK
                                                    : MI355X_BUF_OTHER;
    return mi355x_backend_supports_buft(kind);
}

bool device_offload_op(ggml_backend_dev_t, const struct ggml_tensor * op) {
    Mirror m;
    return mi355x_backend_offload_op(m.node(op));
}

#pragma GCC diagnostic push
#pragma GCC diagnostic ignored "-Wmissing-field-initializers"
const ggml_backend_device_i kDeviceIface = {
    .get_name = device_get_name,
    .get_description = device_get_description,
    .get_memory = device_get_memory,
    .get_type = device_get_type,
    .get_props = device_get_props,
    .init_backend = device_init_backend,
    .get_buffer_type = device_get_buffer_type,
    .buffer_from_host_ptr = device_buffer_from_host_ptr,
    .supports_op = device_supports_op,
    .supports_buft = device_supports_buft,
    .offload_op = device_offload_op,
};
#pragma GCC diagnostic pop

// ---- registry (ggml_backend_reg_i) ----------------------------------------------------------------
const char * reg_get_name(ggml_backend_reg_t) { return mi355x_backend_name(); }
size_t reg_get_device_count(ggml_backend_reg_t) { return 1; }

ggml_backend_dev_t reg_get_device(ggml_backend_reg_t reg, size_t index) {
    GGML_ASSERT(index == 0);
    static ggml_backend_device device = {
        .iface = kDeviceIface,
        .reg = reg,
        .context = nullptr,
    };
    return &device;
}

// The registered-source hook (API.md:280-314): the original bytes of a weight whose tensor sits
// in CPU_REPACK; data == NULL unregisters. Described as placement sees the tensor.
void register_weight_source(const struct ggml_tensor * t, const void * data, size_t nbytes) {
    if (!t) return;
    Mirror m;
    mi355x_backend_register_weight_source(m.source(t), data, nbytes);
}

void * reg_get_proc_address(ggml_backend_reg_t, const char * name) {
    if (!name) return nullptr;
    // under the reference's name too, so a host written for ggml-rocket finds it unchanged
    if (strcmp(name, "ggml_backend_mi355x_register_weight_source") == 0 ||
        strcmp(name, "ggml_backend_rocket_register_weight_source") == 0)
        return (void *)register_weight_source;
    return nullptr;
}

#pragma GCC diagnostic push
#pragma GCC diagnostic ignored "-Wmissing-field-initializers"
const ggml_backend_reg_i kRegIface = {
    .get_name = reg_get_name,
    .get_device_count = reg_get_device_count,
    .get_device = reg_get_device,
    .get_proc_address = reg_get_proc_address,
};
#pragma GCC diagnostic pop

}  // namespace

// ---- public API (include/ggml-mi355x.h) ------------------------------------------------------------
extern "C" {

ggml_backend_reg_t ggml_backend_mi355x_reg(void) {
    static ggml_backend_reg reg = {
        .api_version = GGML_BACKEND_API_VERSION,
        .iface = kRegIface,
        .context = nullptr,
    };
    static std::once_flag routed;
    std::call_once(routed, [] {
        mi355x_backend_set_log_callback(to_ggml_log, nullptr);
        // every quantized type ggml can decode: the kernels keep theirs (Q4_0, Q8_0, Q4_K, Q5_K,
        // Q6_K, MXFP4), the rest are decoded on the host by ggml's own to_float into fp16 images, as the
        // reference decodes every quant type (ggml-rocket.cpp:3894-3909)
        for (int t = 0; t < GGML_TYPE_COUNT; t++) {
            const ggml_type_traits * tr = ggml_get_type_traits((ggml_type)t);
            if (tr && tr->to_float && ggml_is_quantized((ggml_type)t))
                (void)mi355x_backend_set_to_float(t, tr->blck_size, (int64_t)tr->type_size,
                                                  (mi355x_to_float_fn)tr->to_float);
        }
    });
    return &reg;
}

ggml_backend_t ggml_backend_mi355x_init(void) {
    mi355x_backend_t ctx = mi355x_backend_init();
    if (!ctx) return nullptr;
    return new ggml_backend{
        .guid = backend_guid(),
        .iface = kBackendIface,
        .device = ggml_backend_reg_dev_get(ggml_backend_mi355x_reg(), 0),
        .context = ctx,
    };
}

bool ggml_backend_is_mi355x(ggml_backend_t backend) {
    return backend != nullptr && ggml_guid_matches(backend->guid, backend_guid());
}

void ggml_backend_mi355x_set_n_threads(ggml_backend_t backend, int n_threads) {
    GGML_ASSERT(ggml_backend_is_mi355x(backend));
    mi355x_backend_set_n_threads(ctx_of(backend), n_threads);
}

void ggml_backend_mi355x_moe_stats(ggml_backend_t backend, long * n_resident, long * n_streamed) {
    GGML_ASSERT(ggml_backend_is_mi355x(backend));
    mi355x_backend_moe_stats(ctx_of(backend), n_resident, n_streamed);
}

long ggml_backend_mi355x_route_ops(ggml_backend_t backend, const char * route) {
    GGML_ASSERT(ggml_backend_is_mi355x(backend));
    return mi355x_backend_route_ops(ctx_of(backend), route);
}

long ggml_backend_mi355x_cpu_fallbacks(ggml_backend_t backend) {
    GGML_ASSERT(ggml_backend_is_mi355x(backend));
    return mi355x_backend_cpu_fallbacks(ctx_of(backend));
}

}  // extern "C"

// ---- the loader entry (GGML_BACKEND_DL) --------------------------------------------------------------
#ifdef GGML_BACKEND_DL
namespace {

// The ordinals this file was compiled with must name the same ops in the host's ggml: a
// mismatch means the .so was built against another ggml (ggml 1.0.0 moved MUL_MAT 29 -> 28 and
// FLASH_ATTN_EXT 74 -> 71), whose ggml_tensor this build cannot vouch for. ggml_op_name reads
// the host's own name table; every ordinal asked about here is below 80, inside every host's
// table.
bool compiled_against_this_host() {
    const struct {
        enum ggml_op op;
        const char * name;
    } checked[] = {
        {GGML_OP_NONE, "NONE"},       {GGML_OP_MUL_MAT, "MUL_MAT"}, {GGML_OP_MUL_MAT_ID, "MUL_MAT_ID"},
        {GGML_OP_RESHAPE, "RESHAPE"}, {GGML_OP_VIEW, "VIEW"},       {GGML_OP_PERMUTE, "PERMUTE"},
        {GGML_OP_TRANSPOSE, "TRANSPOSE"}, {GGML_OP_FLASH_ATTN_EXT, "FLASH_ATTN_EXT"},
    };
    bool same = true;
    for (const auto & c : checked) {
        const char * host = ggml_op_name(c.op);
        if (!host || strcmp(host, c.name) != 0) {
            GGML_LOG_ERROR("ggml-mi355x: op %d is %s here and %s in the host's ggml\n", (int)c.op, c.name,
                           host ? host : "(null)");
            same = false;
        }
    }
    return same;
}

ggml_backend_reg_t mi355x_dl_entry() {
    if (!compiled_against_this_host()) {
        GGML_LOG_ERROR("ggml-mi355x: built against a different ggml than the host loading it; rebuild with "
                       "HOST_GGML_DIR set to this host's checkout\n");
        return nullptr;   // the loader unloads the .so and the host runs without this device
    }
    return ggml_backend_mi355x_reg();
}

}  // namespace

GGML_BACKEND_DL_IMPL(mi355x_dl_entry)
#endif
