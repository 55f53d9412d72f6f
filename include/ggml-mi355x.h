/* SPDX-License-Identifier: MIT
 *
 * ggml-mi355x.h -- the ggml backend for one AMD Instinct MI355X (gfx950), the drop-in for
 * ggml-rocket's public header (ggml-rocket.h:23-91) with "rocket" read as "mi355x".
 *
 * The backend claims GGML_OP_MUL_MAT, GGML_OP_FLASH_ATTN_EXT and GGML_OP_MUL_MAT_ID under the
 * reference's claim rules and computes them on the GPU; the CPU backend computes every op it
 * declines. Weights stay in the host's buffers and are cached in HBM on first use. A host loads
 * it as libggml-mi355x.so through GGML_BACKEND_PATH / ggml_backend_load (the ggml_backend_init
 * entry of GGML_BACKEND_DL), or links it and calls ggml_backend_mi355x_reg().
 *
 * Implemented by ggml-rocket_amd/ggml/ggml-mi355x.cpp over libmi355x's host layer
 * (include/mi355x_backend.h); built against the host's ggml (make -C ggml-rocket_amd ggml
 * HOST_GGML_DIR=<llama.cpp or whisper.cpp checkout>).
 */
#ifndef GGML_MI355X_H
#define GGML_MI355X_H

#include "ggml.h"
#include "ggml-backend.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Replaces ggml_backend_rocket_init (ggml-rocket.h:23-24): creates a backend instance. It hands
 * out the host's CPU buffer type, so weights stay in host buffers; nothing touches the GPU
 * before the first graph_compute. */
GGML_BACKEND_API ggml_backend_t ggml_backend_mi355x_init(void);

/* Replaces ggml_backend_is_rocket (ggml-rocket.h:26-27): true if `backend` is an instance of
 * this backend (GUID match). */
GGML_BACKEND_API bool ggml_backend_is_mi355x(ggml_backend_t backend);

/* Replaces ggml_backend_rocket_set_n_threads (ggml-rocket.h:29-37): the host threads (1-8,
 * clamped with a warning) that fill and drain the pinned staging of the host <-> device copies.
 * Call before the first graph_compute; a later call warns and changes nothing. */
GGML_BACKEND_API void ggml_backend_mi355x_set_n_threads(ggml_backend_t backend, int n_threads);

/* Replaces ggml_backend_rocket_moe_stats (ggml-rocket.h:39-57): distinct MoE experts held in the
 * HBM expert cache, and distinct experts run from a per-call upload, over the backend's life.
 * Either pointer may be NULL. */
GGML_BACKEND_API void ggml_backend_mi355x_moe_stats(ggml_backend_t backend, long * n_resident,
                                                    long * n_streamed);

/* Replace ggml_backend_rocket_route_ops / _cpu_fallbacks (ggml-rocket.h:59-88): ops completed
 * per route ("mt", "prepacked", "prepacked-q", "fused", "fused-resident", "moe", "fa"; NULL =
 * all), and ops recomputed on the CPU after a device failure. Cumulative. */
GGML_BACKEND_API long ggml_backend_mi355x_route_ops(ggml_backend_t backend, const char * route);
GGML_BACKEND_API long ggml_backend_mi355x_cpu_fallbacks(ggml_backend_t backend);

/* Replaces ggml_backend_rocket_reg (ggml-rocket.h:90-91): the registry entry ggml's loader and
 * device enumeration use. Its get_proc_address also answers
 * "ggml_backend_rocket_register_weight_source" and "ggml_backend_mi355x_register_weight_source"
 * with void (*)(const struct ggml_tensor *, const void * data, size_t nbytes) (API.md:280-314). */
GGML_BACKEND_API ggml_backend_reg_t ggml_backend_mi355x_reg(void);

#ifdef __cplusplus
}
#endif

#endif /* GGML_MI355X_H */
