/*
 * ggml-mi355x.h - public interface of the MI355X (gfx950) ggml backend.
 *
 * The backend registers as device "MI355X<i>" (selected with
 * GGML_BACKEND=MI355X0, src/backend.h:109-121) and implements the ggml-backend
 * plug-in interface: buffer types (device, pinned host), buffers,
 * supports_op and graph_compute.  These entry points mirror the shape of
 * ggml's per-backend headers (ggml_backend_<name>_init / _reg / _buffer_type
 * / _host_buffer_type / _get_device_count), which src/backend.h reaches
 * through ggml_backend_load_all() / ggml_backend_init_by_name()
 * (src/backend.h:106-123).  A dynamically loaded build also exports
 * ggml_backend_init() and ggml_backend_score().
 */
#pragma once

#include "ggml-backend.h"

#ifdef __cplusplus
extern "C" {
#endif

#define GGML_MI355X_NAME "MI355X"

/* Registry of the backend: one device per visible gfx950 GPU. */
GGML_API ggml_backend_reg_t ggml_backend_mi355x_reg(void);

/* Backend on device `device` (one HIP stream of default priority). */
GGML_API ggml_backend_t ggml_backend_mi355x_init(int device);
GGML_API bool           ggml_backend_is_mi355x(ggml_backend_t backend);
GGML_API int            ggml_backend_mi355x_get_device_count(void);

/* Device memory; quantized tensors (Q8_0, Q4_K, Q6_K) are stored in the
 * row-grouped layout (same size as GGUF rows) and converted on set/get. */
GGML_API ggml_backend_buffer_type_t ggml_backend_mi355x_buffer_type(int device);
/* Pinned host memory (used for the CPU side of the scheduler,
 * src/backend.h:179-181). */
GGML_API ggml_backend_buffer_type_t ggml_backend_mi355x_host_buffer_type(void);

/* Number of graph_compute calls served by replaying a captured HIP graph, and
 * by eager launches (diagnostics for tests and the benchmark). */
GGML_API void ggml_backend_mi355x_graph_stats(ggml_backend_t backend, int64_t * replays, int64_t * eager);
/* The backend's graph cache: graphs it keeps (at most 8, least recently used
 * replaced first), how many of them hold a captured HIP graph, and captures
 * made so far.  Diagnostics, no counterpart in the reference. */
GGML_API void ggml_backend_mi355x_graph_cache_info(ggml_backend_t backend, int64_t * n_entries, int64_t * n_captured,
                                                   int64_t * n_captures);
/* GPU time of this backend's graph_compute calls so far, from HIP events
 * recorded on its stream around each call (waits for the last call to
 * finish); reset != 0 clears the totals.  Backend-specific, no counterpart in
 * the reference (used to report kernel-side time next to wall-clock). */
GGML_API void ggml_backend_mi355x_gpu_time(ggml_backend_t backend, double * total_ms, int64_t * n_calls, int reset);
/* Bytes of f16 weight copies the backend holds for its token-count GEMMs:
 * made, within GGML_MI355X_F16_WEIGHTS_MB (default 32768), for the quantised
 * weights that a graph computed three or more times multiplies at more than 16
 * tokens (the DiT's, once per diffusion step).  Diagnostics, no counterpart in
 * the reference. */
GGML_API size_t ggml_backend_mi355x_f16_weight_bytes(void);

#ifdef __cplusplus
}
#endif
