// ggml-mi355x.cpp - the MI355X ggml backend: registry, device, buffer types,
// buffers and the backend (graph_compute), dispatching every supported node
// to the gfx950 kernels of libmmhip (include/mmhip.h).
//
// Boundary with the reference: src/backend.h:93-190 selects a backend by name
// and builds the scheduler; src/static-graph.h:31-58 allocates graphs with
// gallocr and runs ggml_backend_graph_compute directly when supports_op
// holds for every node; weights are uploaded with ggml_backend_tensor_set
// (src/gguf-weights.h:161-203, src/weight-ctx.h:53-68).
//
// graph_compute runs a graph eagerly the first time it sees it; when the same
// graph (same nodes, same data addresses, src/graph-arena.h:1-6) comes back,
// the launches are captured into a HIP graph once and replayed from then on.
// Host inputs change between decode steps only through tensor data
// (positions, kv_rows, mask: src/qwen3-lm.h:895-920), never through topology.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "ggml-backend-impl.h"
#include "ggml-mi355x.h"
#include "mmhip.h"

#define MI_LOG(...) fprintf(stderr, "[ggml-mi355x] " __VA_ARGS__)

#define HIP_OK(call)                                                                    \
    ([&]() -> bool {                                                                    \
        hipError_t e_ = (call);                                                         \
        if (e_ != hipSuccess) {                                                         \
            MI_LOG("%s failed: %s (%s:%d)\n", #call, hipGetErrorString(e_), __FILE__, __LINE__); \
            return false;                                                               \
        }                                                                               \
        return true;                                                                    \
    }())

namespace {

// ---------------------------------------------------------------------------
// device / registry state

// Pinned staging for small host -> device tensor writes (per-step inputs of
// the decode graph): the data is copied into a slot on the host and sent with
// an asynchronous copy on the null stream, which the backends' blocking
// streams order after; a slot is reused only once its copy has completed.
// The caller sees ggml's synchronous tensor_set: its buffer is free on return.
struct mi_staging {
    static constexpr int    SLOTS     = 32;
    static constexpr size_t SLOT_SIZE = 256 << 10;
    std::mutex              mu;
    char *                  host = nullptr;
    hipEvent_t              ev[SLOTS]{};
    bool                    used[SLOTS]{};
    int                     next = 0;
    bool                    failed = false;
};

// Streams of freed backends are kept per device and handed to the next
// backend (after a synchronize), so creating and freeing backends in one
// process does not create and destroy HIP streams each time.
struct mi_device {
    int                             id;
    std::string                     name;
    std::string                     desc;
    struct ggml_backend_buffer_type buft;
    mi_staging                      staging;
    std::mutex                      stream_mu;
    std::vector<hipStream_t>        idle_streams;
};

// Buffers whose set_tensor / get_tensor failed: graph_compute refuses graphs
// that touch them (ggml's buffer interface has no error return there).
std::atomic<int> g_poisoned_buffers{ 0 };

struct mi_registry {
    std::vector<mi_device *>                 devs;
    std::vector<struct ggml_backend_device> gdevs;
    struct ggml_backend_reg                  reg;
    struct ggml_backend_buffer_type          host_buft;
};

mi_registry * g_reg = nullptr;
std::mutex    g_reg_mu;

bool is_repacked(enum ggml_type t) {
    return t == GGML_TYPE_Q8_0 || t == GGML_TYPE_Q4_K || t == GGML_TYPE_Q5_K || t == GGML_TYPE_Q6_K;
}

mmhip_view view_of(const struct ggml_tensor * t) {
    mmhip_view v;
    v.data = t->data;
    for (int i = 0; i < 4; i++) {
        v.ne[i] = t->ne[i];
        v.nb[i] = (int64_t) t->nb[i];
    }
    return v;
}

// ---------------------------------------------------------------------------
// device buffers

// An f16 copy of a quantised weight in the buffer (rows [N][K], the GEMM's
// exact dequantisation), registered with the kernel library so the
// token-count GEMMs read it instead of converting per call.
struct mi_f16_copy {
    const void * w;      // the quantised weight (its tensor's data)
    void *       wh;     // the copy
    size_t       bytes;  // of the copy
    size_t       wbytes; // of the quantised weight
    int          type;
    int64_t      N, K, rs;
};

struct mi_buffer {
    int                      device;
    void *                   ptr;
    bool                     poisoned = false;  // a set_tensor / get_tensor on it failed
    std::vector<mi_f16_copy> f16;               // f16 weight copies made for its tensors
};

// f16 weight copies, process-wide: their total size (bounded by
// GGML_MI355X_F16_WEIGHTS_MB, default 32768; 0 makes none) and a generation
// that moves whenever copies appear or go, so that captured HIP graphs, which
// hold the addresses the GEMMs read, are captured again.
std::atomic<size_t>   g_f16_bytes{ 0 };
std::atomic<uint64_t> g_f16_gen{ 0 };

size_t f16_limit() {
    static const size_t lim = [] {
        const char * e = getenv("GGML_MI355X_F16_WEIGHTS_MB");
        return (e ? (size_t) strtoull(e, nullptr, 10) : (size_t) 32768) << 20;
    }();
    return lim;
}

void poison(mi_buffer * c) {
    if (!c->poisoned) {
        c->poisoned = true;
        g_poisoned_buffers.fetch_add(1);
    }
}

// Work queued on any stream of the device may still read the buffer (a
// replayed HIP graph holds its addresses): wait for the device before freeing.
void buf_free(ggml_backend_buffer_t b) {
    mi_buffer * c = (mi_buffer *) b->context;
    hipSetDevice(c->device);
    HIP_OK(hipDeviceSynchronize());
    for (const mi_f16_copy & f : c->f16) {
        (void) mmhip_unregister_weights_f16(f.w);
        (void) hipFree(f.wh);
        g_f16_bytes.fetch_sub(f.bytes);
    }
    if (!c->f16.empty()) {
        g_f16_gen.fetch_add(1);
    }
    (void) hipFree(c->ptr);
    if (c->poisoned) {
        g_poisoned_buffers.fetch_sub(1);
    }
    delete c;
}

void * buf_base(ggml_backend_buffer_t b) {
    return ((mi_buffer *) b->context)->ptr;
}

enum ggml_status buf_init_tensor(ggml_backend_buffer_t b, struct ggml_tensor * t) {
    (void) b;
    (void) t;
    return GGML_STATUS_SUCCESS;
}

void refresh_f16_copies(mi_buffer * c, const char * lo, const char * hi);

// A constant byte fill is the same in the GGUF and the row-grouped layout.
void buf_memset(ggml_backend_buffer_t b, struct ggml_tensor * t, uint8_t value, size_t offset, size_t size) {
    mi_buffer * c = (mi_buffer *) b->context;
    hipSetDevice(c->device);
    if (!HIP_OK(hipMemset((char *) t->data + offset, value, size))) {
        poison(c);
    }
    refresh_f16_copies(c, (const char *) t->data + offset, (const char *) t->data + offset + size);
}

// Quantized rows are converted between GGUF bytes (host side) and the
// row-grouped device layout.  Whole-row transfers go straight through a device
// staging buffer; partial rows are read, patched and written back.
bool quant_rows_io(const struct ggml_tensor * t, size_t offset, size_t size, const void * src_host, void * dst_host) {
    const size_t  rs = ggml_row_size(t->type, t->ne[0]);
    const int64_t K  = t->ne[0];
    if (t->nb[1] != rs || !ggml_is_contiguous(t)) {
        MI_LOG("quantized tensor %s is not row-contiguous\n", t->name);
        return false;
    }
    const size_t r0    = offset / rs;
    const size_t r1    = (offset + size + rs - 1) / rs;
    const size_t nrows = r1 - r0;
    char *       dev   = (char *) t->data + r0 * rs;
    void *       stage = nullptr;
    if (!HIP_OK(hipMalloc(&stage, nrows * rs))) {
        return false;
    }
    bool ok = true;
    if (src_host) {
        if (offset % rs == 0 && size % rs == 0) {
            ok = HIP_OK(hipMemcpy(stage, src_host, size, hipMemcpyHostToDevice));
        } else {
            std::vector<char> host(nrows * rs);
            ok = mmhip_unpack_rows(t->type, dev, stage, (int64_t) nrows, K, nullptr) == MMHIP_OK &&
                 HIP_OK(hipMemcpy(host.data(), stage, host.size(), hipMemcpyDeviceToHost));
            if (ok) {
                memcpy(host.data() + (offset - r0 * rs), src_host, size);
                ok = HIP_OK(hipMemcpy(stage, host.data(), host.size(), hipMemcpyHostToDevice));
            }
        }
        ok = ok && mmhip_repack_rows(t->type, stage, dev, (int64_t) nrows, K, nullptr) == MMHIP_OK &&
             HIP_OK(hipDeviceSynchronize());
    } else {
        std::vector<char> host(nrows * rs);
        ok = mmhip_unpack_rows(t->type, dev, stage, (int64_t) nrows, K, nullptr) == MMHIP_OK &&
             HIP_OK(hipMemcpy(host.data(), stage, host.size(), hipMemcpyDeviceToHost));
        if (ok) {
            memcpy(dst_host, host.data() + (offset - r0 * rs), size);
        }
    }
    if (!ok) {
        MI_LOG("quantized transfer of %s failed: %s\n", t->name, mmhip_last_error());
    }
    (void) hipFree(stage);
    return ok;
}

mi_device * device_by_id(int id);

// Small write through the device's pinned staging ring; false when not taken.
bool staged_write(int device, void * dst, const void * src, size_t size) {
    mi_device * d = device_by_id(device);
    if (!d || size > mi_staging::SLOT_SIZE) {
        return false;
    }
    mi_staging &                g = d->staging;
    std::lock_guard<std::mutex> lk(g.mu);
    if (g.failed) {
        return false;
    }
    if (!g.host) {
        if (!HIP_OK(hipHostMalloc((void **) &g.host, (size_t) mi_staging::SLOTS * mi_staging::SLOT_SIZE, 0))) {
            g.failed = true;
            g.host   = nullptr;
            return false;
        }
        for (int i = 0; i < mi_staging::SLOTS; i++) {
            if (!HIP_OK(hipEventCreateWithFlags(&g.ev[i], hipEventDisableTiming))) {
                g.failed = true;
                return false;
            }
        }
    }
    const int i = g.next;
    g.next      = (g.next + 1) % mi_staging::SLOTS;
    if (g.used[i] && !HIP_OK(hipEventSynchronize(g.ev[i]))) {
        return false;
    }
    char * slot = g.host + (size_t) i * mi_staging::SLOT_SIZE;
    memcpy(slot, src, size);
    if (!HIP_OK(hipMemcpyAsync(dst, slot, size, hipMemcpyHostToDevice, nullptr)) ||
        !HIP_OK(hipEventRecord(g.ev[i], nullptr))) {
        return false;
    }
    g.used[i] = true;
    return true;
}

// A write into a weight that has an f16 copy (set_tensor, memset_tensor,
// cpy_tensor, clear) converts the copy again, in place (captured graphs keep
// its address), before the write returns.
void refresh_f16_copies(mi_buffer * c, const char * lo, const char * hi) {
    for (const mi_f16_copy & f : c->f16) {
        const char * w = (const char *) f.w;
        if (lo < w + f.wbytes && w < hi) {
            if (mmhip_weights_to_f16(f.type, f.w, f.N, f.K, f.rs, f.wh, nullptr) != MMHIP_OK ||
                !HIP_OK(hipDeviceSynchronize())) {
                MI_LOG("set_tensor: refreshing an f16 weight copy failed (%s): the buffer is marked failed\n",
                       mmhip_last_error());
                poison(c);
            }
        }
    }
}

void buf_set_tensor(ggml_backend_buffer_t b, struct ggml_tensor * t, const void * data, size_t offset, size_t size) {
    mi_buffer * c = (mi_buffer *) b->context;
    hipSetDevice(c->device);
    if (is_repacked(t->type)) {
        if (!quant_rows_io(t, offset, size, data, nullptr)) {
            MI_LOG("set_tensor %s failed: the buffer is marked failed, graphs using it are refused\n", t->name);
            poison(c);
        }
        refresh_f16_copies(c, (const char *) t->data + offset, (const char *) t->data + offset + size);
        return;
    }
    if (staged_write(c->device, (char *) t->data + offset, data, size)) {
        return;
    }
    if (!HIP_OK(hipMemcpy((char *) t->data + offset, data, size, hipMemcpyHostToDevice))) {
        poison(c);
    }
}

// On failure the destination is filled with 0xff bytes (NaN for f32 / f16)
// so a caller that ignores the log does not read plausible stale values.
void buf_get_tensor(ggml_backend_buffer_t b, const struct ggml_tensor * t, void * data, size_t offset, size_t size) {
    mi_buffer * c = (mi_buffer *) b->context;
    hipSetDevice(c->device);
    bool ok;
    if (is_repacked(t->type)) {
        ok = quant_rows_io(t, offset, size, nullptr, data);
    } else {
        ok = HIP_OK(hipMemcpy(data, (const char *) t->data + offset, size, hipMemcpyDeviceToHost));
    }
    if (!ok) {
        MI_LOG("get_tensor %s failed: the buffer is marked failed, graphs using it are refused\n", t->name);
        memset(data, 0xff, size);
        poison(c);
    }
}

// Is any tensor of the graph (nodes and their sources) in a poisoned buffer?
bool graph_poisoned(struct ggml_cgraph * g) {
    auto bad = [](const struct ggml_tensor * t) {
        const struct ggml_tensor * base = t->view_src ? t->view_src : t;
        ggml_backend_buffer_t      b    = base->buffer;
        return b && b->iface.free_buffer == buf_free && ((mi_buffer *) b->context)->poisoned;
    };
    for (int i = 0; i < ggml_graph_n_nodes(g); i++) {
        const struct ggml_tensor * n = ggml_graph_node(g, i);
        if (bad(n)) {
            return true;
        }
        for (int s = 0; s < GGML_MAX_SRC; s++) {
            if (n->src[s] && bad(n->src[s])) {
                return true;
            }
        }
    }
    return false;
}

bool buf_cpy_tensor(ggml_backend_buffer_t b, const struct ggml_tensor * src, struct ggml_tensor * dst) {
    // same layout on both sides: device-to-device copy of the bytes
    ggml_backend_buffer_t sb = src->view_src ? src->view_src->buffer : src->buffer;
    if (!sb || sb->iface.free_buffer != buf_free || src->type != dst->type) {
        return false;
    }
    mi_buffer * c = (mi_buffer *) b->context;
    hipSetDevice(c->device);
    if (!HIP_OK(hipMemcpy(dst->data, src->data, ggml_nbytes(src), hipMemcpyDeviceToDevice))) {
        return false;
    }
    refresh_f16_copies(c, (const char *) dst->data, (const char *) dst->data + ggml_nbytes(dst));
    return true;
}

void buf_clear(ggml_backend_buffer_t b, uint8_t value) {
    mi_buffer * c = (mi_buffer *) b->context;
    hipSetDevice(c->device);
    HIP_OK(hipMemset(c->ptr, value, b->size));
    HIP_OK(hipDeviceSynchronize());
    refresh_f16_copies(c, (const char *) c->ptr, (const char *) c->ptr + b->size);
}

const struct ggml_backend_buffer_i k_buf_iface = {
    /* free_buffer   */ buf_free,
    /* get_base      */ buf_base,
    /* init_tensor   */ buf_init_tensor,
    /* memset_tensor */ buf_memset,
    /* set_tensor    */ buf_set_tensor,
    /* get_tensor    */ buf_get_tensor,
    /* cpy_tensor    */ buf_cpy_tensor,
    /* clear         */ buf_clear,
    /* reset         */ nullptr,
};

const char * buft_name(ggml_backend_buffer_type_t buft) {
    return ((mi_device *) buft->context)->name.c_str();
}

ggml_backend_buffer_t buft_alloc(ggml_backend_buffer_type_t buft, size_t size) {
    mi_device * d = (mi_device *) buft->context;
    hipSetDevice(d->id);
    void * p = nullptr;
    if (!HIP_OK(hipMalloc(&p, size ? size : 256))) {
        return nullptr;
    }
    return ggml_backend_buffer_init(buft, k_buf_iface, new mi_buffer{ d->id, p }, size);
}

size_t buft_alignment(ggml_backend_buffer_type_t) {
    return 256;
}

size_t buft_max_size(ggml_backend_buffer_type_t) {
    return SIZE_MAX;
}

size_t buft_alloc_size(ggml_backend_buffer_type_t, const struct ggml_tensor * t) {
    return ggml_nbytes(t);
}

bool buft_is_host(ggml_backend_buffer_type_t) {
    return false;
}

// ---------------------------------------------------------------------------
// pinned host buffers

void hbuf_free(ggml_backend_buffer_t b) {
    (void) hipHostFree(b->context);
}

void * hbuf_base(ggml_backend_buffer_t b) {
    return b->context;
}

void hbuf_memset(ggml_backend_buffer_t, struct ggml_tensor * t, uint8_t v, size_t off, size_t size) {
    memset((char *) t->data + off, v, size);
}

void hbuf_set(ggml_backend_buffer_t, struct ggml_tensor * t, const void * data, size_t off, size_t size) {
    memcpy((char *) t->data + off, data, size);
}

void hbuf_get(ggml_backend_buffer_t, const struct ggml_tensor * t, void * data, size_t off, size_t size) {
    memcpy(data, (const char *) t->data + off, size);
}

void hbuf_clear(ggml_backend_buffer_t b, uint8_t v) {
    memset(b->context, v, b->size);
}

const struct ggml_backend_buffer_i k_hbuf_iface = {
    hbuf_free, hbuf_base, nullptr, hbuf_memset, hbuf_set, hbuf_get, nullptr, hbuf_clear, nullptr,
};

const char * hbuft_name(ggml_backend_buffer_type_t) {
    return GGML_MI355X_NAME "_Host";
}

ggml_backend_buffer_t hbuft_alloc(ggml_backend_buffer_type_t buft, size_t size) {
    void * p = nullptr;
    if (!HIP_OK(hipHostMalloc(&p, size ? size : 64, hipHostMallocDefault))) {
        return nullptr;
    }
    return ggml_backend_buffer_init(buft, k_hbuf_iface, p, size);
}

size_t hbuft_alignment(ggml_backend_buffer_type_t) {
    return 64;
}

bool hbuft_is_host(ggml_backend_buffer_type_t) {
    return true;
}

// ---------------------------------------------------------------------------
// backend

struct graph_plan;

// One graph the backend has seen: its signature (every node's identity,
// op, op_params, shape, strides, data address and sources: anything a launch
// takes by value), its execution plan and, from its second sight on, the
// instantiated HIP graph of its launches.  The reference alternates several
// graphs on one backend (the depth decoder's frame graph and the LM's decode
// graph every frame, src/pipeline.cpp:458, :545-547, one shared backend
// src/backend.h:21-23), so the backend keeps several, least recently used
// first out.
struct mi_graph_entry {
    const void *                graph   = nullptr;  // pre-key: the cgraph, its node count, first / last node
    int                         n_nodes = 0;
    const void *                first   = nullptr;
    const void *                last    = nullptr;
    std::vector<uint64_t>       sig;
    std::shared_ptr<graph_plan> plan;
    hipGraphExec_t              exec       = nullptr;
    int                         sights     = 0;
    bool                        no_capture = false;  // capture failed once: stay eager
    uint64_t                    stamp      = 0;
    uint64_t                    f16_gen    = 0;      // g_f16_gen when captured
};

struct mi_backend {
    static constexpr int GRAPH_ENTRIES = 8;
    mi_device *    dev;
    hipStream_t    stream = nullptr;
    void *         ws     = nullptr;
    size_t         ws_size = 0;
    void *         slot      = nullptr;  // quantised activation slots of the execution plan
    size_t         slot_size = 0;
    bool           capturing = false;
    bool           use_graphs = true;
    std::vector<mi_graph_entry> graphs;
    std::vector<uint64_t>       sig_buf;  // signature of the call being looked up
    uint64_t                    clock = 0;
    int64_t        n_replays = 0;
    int64_t        n_eager   = 0;
    int64_t        n_captures = 0;
    // GPU time of graph_compute calls: events recorded on the stream around
    // each call, read back at the next call (or on query)
    hipEvent_t     ev0 = nullptr, ev1 = nullptr;
    bool           ev_pending = false;
    double         gpu_ms     = 0.0;
    int64_t        gpu_n      = 0;
};

// Fold the previous call's event pair into the totals (waits for it).
void collect_time(mi_backend * c) {
    if (!c->ev_pending) {
        return;
    }
    c->ev_pending = false;
    float ms      = 0.0f;
    if (HIP_OK(hipEventSynchronize(c->ev1)) && HIP_OK(hipEventElapsedTime(&ms, c->ev0, c->ev1))) {
        c->gpu_ms += ms;
        c->gpu_n++;
    }
}

const char * be_name(ggml_backend_t b) {
    return ((mi_backend *) b->context)->dev->name.c_str();
}

// Teardown in dependency order: the stream's queued work (which may be a
// replay reading the workspace, the slots and graph tensors) finishes first,
// then the HIP graphs that launch into those buffers go, then the buffers;
// the stream goes back to the device for the next backend.
void be_free(ggml_backend_t b) {
    mi_backend * c = (mi_backend *) b->context;
    hipSetDevice(c->dev->id);
    const bool synced = HIP_OK(hipStreamSynchronize(c->stream));
    for (mi_graph_entry & e : c->graphs) {
        if (e.exec) {
            (void) hipGraphExecDestroy(e.exec);
            e.exec = nullptr;
        }
    }
    c->graphs.clear();
    if (c->ws) {
        (void) hipFree(c->ws);
    }
    if (c->slot) {
        (void) hipFree(c->slot);
    }
    if (c->ev0) {
        (void) hipEventDestroy(c->ev0);
        (void) hipEventDestroy(c->ev1);
    }
    if (synced) {
        std::lock_guard<std::mutex> lk(c->dev->stream_mu);
        c->dev->idle_streams.push_back(c->stream);
    } else {
        (void) hipStreamDestroy(c->stream);
    }
    delete c;
    delete b;
}

void be_sync(ggml_backend_t b) {
    mi_backend * c = (mi_backend *) b->context;
    HIP_OK(hipStreamSynchronize(c->stream));
}

// Workspace large enough for `need` bytes; returns nullptr when it would have
// to grow during a capture (the caller then abandons the capture).
// A captured graph holds the addresses of the workspace and the activation
// slots: when either moves, every capture is dropped (the graphs are captured
// again on their next sight).  The caller has synchronised the stream.
void drop_captured(mi_backend * c) {
    for (mi_graph_entry & e : c->graphs) {
        if (e.exec) {
            (void) hipGraphExecDestroy(e.exec);
            e.exec   = nullptr;
            e.sights = 1;
        }
    }
}

void * workspace(mi_backend * c, size_t need) {
    if (need <= c->ws_size) {
        return c->ws;
    }
    if (c->capturing) {
        return nullptr;
    }
    HIP_OK(hipStreamSynchronize(c->stream));
    if (c->ws) {
        (void) hipFree(c->ws);
        drop_captured(c);
    }
    c->ws      = nullptr;
    c->ws_size = 0;
    size_t sz  = need + need / 2 + (1 << 20);
    if (!HIP_OK(hipMalloc(&c->ws, sz))) {
        return nullptr;
    }
    c->ws_size = sz;
    return c->ws;
}

// the weight of a [K, N] 2-D quantized src0 and the activation rows of src1
bool mm_collapsible(const struct ggml_tensor * x) {
    return x->nb[0] == sizeof(float) && x->nb[2] == x->nb[1] * (size_t) x->ne[1] &&
           x->nb[3] == x->nb[2] * (size_t) x->ne[2] && x->nb[1] % sizeof(float) == 0;
}

bool supports_mul_mat(const struct ggml_tensor * op) {
    const struct ggml_tensor * w = op->src[0];
    const struct ggml_tensor * x = op->src[1];
    if (!is_repacked(w->type) || x->type != GGML_TYPE_F32 || op->type != GGML_TYPE_F32) {
        return false;
    }
    if (w->ne[2] != 1 || w->ne[3] != 1 || !ggml_is_contiguous(w)) {
        return false;
    }
    if (w->ne[0] % 256 != 0 || !mm_collapsible(x) || !ggml_is_contiguous(op)) {
        return false;
    }
    const size_t rs = ggml_row_size(w->type, w->ne[0]);
    // GEMM path: 16-byte rows; GEMV path handles 2-byte aligned Q6_K rows
    return rs % 16 == 0 || (w->type == GGML_TYPE_Q6_K && x->ne[1] * x->ne[2] * x->ne[3] <= 8);
}

bool supports_fa(const struct ggml_tensor * op) {
    const struct ggml_tensor *q = op->src[0], *k = op->src[1], *v = op->src[2], *m = op->src[3];
    float max_bias, softcap;
    memcpy(&max_bias, &op->op_params[1], sizeof(float));
    memcpy(&softcap, &op->op_params[2], sizeof(float));
    if (max_bias != 0.0f || softcap != 0.0f || op->src[4] != nullptr) {
        return false;
    }
    if (q->type != GGML_TYPE_F32 || k->type != GGML_TYPE_F16 || v->type != GGML_TYPE_F16) {
        return false;
    }
    if (m && m->type != GGML_TYPE_F16) {
        return false;
    }
    const int64_t D = q->ne[0];
    if (!(D == 64 || D == 128 || D == 256) || k->ne[0] != D || v->ne[0] != D) {
        return false;
    }
    // D = 256 runs only on the decode kernels (at most 16 query rows per KV
    // head); the MFMA prefill kernel takes D 64 / 128
    if (D == 256 && (k->ne[2] <= 0 || q->ne[2] % k->ne[2] != 0 || q->ne[1] * (q->ne[2] / k->ne[2]) > 16)) {
        return false;
    }
    return q->nb[0] == 4 && k->nb[0] == 2 && v->nb[0] == 2 && k->nb[1] % 16 == 0 && v->nb[1] % 16 == 0 &&
           k->nb[2] % 16 == 0 && v->nb[2] % 16 == 0 && k->nb[3] % 16 == 0 && v->nb[3] % 16 == 0;
}

bool supports_rope(const struct ggml_tensor * op) {
    const int mode = op->op_params[2];
    float     freq_scale, ext_factor, attn_factor;
    memcpy(&freq_scale, &op->op_params[6], sizeof(float));
    memcpy(&ext_factor, &op->op_params[7], sizeof(float));
    memcpy(&attn_factor, &op->op_params[8], sizeof(float));
    return mode == GGML_ROPE_TYPE_NEOX && freq_scale == 1.0f && ext_factor == 0.0f && attn_factor == 1.0f &&
           op->src[2] == nullptr && op->src[0]->type == GGML_TYPE_F32 && op->src[0]->nb[0] == 4 &&
           op->src[1]->type == GGML_TYPE_I32 && ggml_is_contiguous(op->src[1]) && op->src[1]->ne[0] == op->src[0]->ne[2];
}

bool is_f32_or_f16(enum ggml_type t) {
    return t == GGML_TYPE_F32 || t == GGML_TYPE_F16;
}

// 16-byte aligned data: the address once allocated, the view offset before
bool aligned16(const struct ggml_tensor * t) {
    return (uintptr_t) t->data % 16 == 0 && (t->view_src == nullptr || t->view_offs % 16 == 0);
}

bool supports(const struct ggml_tensor * op) {
    switch (op->op) {
        case GGML_OP_NONE:
        case GGML_OP_RESHAPE:
        case GGML_OP_VIEW:
        case GGML_OP_PERMUTE:
        case GGML_OP_TRANSPOSE:
            return true;
        case GGML_OP_MUL_MAT:
            if (op->src[0]->type == GGML_TYPE_BF16) {
                // BF16 weights: the GEMV up to 16 tokens (K % 8 == 0), the
                // 16-bit DMA GEMM above (K % 32 == 0); both make 16-byte loads,
                // so rows and bases are 16-byte aligned (also checked before
                // allocation, through the view offsets)
                const struct ggml_tensor * w = op->src[0];
                const struct ggml_tensor * x = op->src[1];
                const int64_t              M = x->ne[1] * x->ne[2] * x->ne[3];
                return w->nb[0] == 2 && w->ne[2] == 1 && w->ne[3] == 1 && w->ne[0] % (M <= 16 ? 8 : 32) == 0 &&
                       w->nb[1] % 16 == 0 && x->type == GGML_TYPE_F32 && mm_collapsible(x) && x->nb[1] % 16 == 0 &&
                       aligned16(x) && aligned16(w) && op->type == GGML_TYPE_F32 && ggml_is_contiguous(op);
            }
            if (op->src[0]->type == GGML_TYPE_F32) {  // activation x activation
                return op->src[1]->type == GGML_TYPE_F32 && op->src[0]->nb[0] == 4 && op->src[1]->nb[0] == 4 &&
                       op->type == GGML_TYPE_F32 && ggml_is_contiguous(op);
            }
            return supports_mul_mat(op);
        case GGML_OP_FLASH_ATTN_EXT:
            return supports_fa(op);
        case GGML_OP_SOFT_MAX: {
            float scale, max_bias;
            memcpy(&scale, &op->op_params[0], sizeof(float));
            memcpy(&max_bias, &op->op_params[1], sizeof(float));
            return op->src[1] == nullptr && scale == 1.0f && max_bias == 0.0f && op->src[0]->type == GGML_TYPE_F32 &&
                   op->type == GGML_TYPE_F32 && ggml_is_contiguous(op);
        }
        case GGML_OP_DIAG_MASK_INF:
            return op->src[0]->type == GGML_TYPE_F32 && op->type == GGML_TYPE_F32 && ggml_is_contiguous(op);
        case GGML_OP_ARGSORT:
            return op->src[0]->type == GGML_TYPE_F32 && op->op_params[0] == GGML_SORT_ORDER_DESC &&
                   op->src[0]->ne[0] <= 4096 && op->type == GGML_TYPE_I32 && ggml_is_contiguous(op);
        case GGML_OP_CUMSUM:
        case GGML_OP_SUM:
            return op->src[0]->type == GGML_TYPE_F32 && op->type == GGML_TYPE_F32 && ggml_is_contiguous(op);
        case GGML_OP_UNARY:
            return op->op_params[0] == GGML_UNARY_OP_STEP && op->src[0]->type == GGML_TYPE_F32 &&
                   op->type == GGML_TYPE_F32 && ggml_is_contiguous(op);
        case GGML_OP_ADD:
        case GGML_OP_SUB:
        case GGML_OP_MUL:
            return op->type == GGML_TYPE_F32 && op->src[0]->type == GGML_TYPE_F32 &&
                   op->src[1]->type == GGML_TYPE_F32 && ggml_is_contiguous(op);
        case GGML_OP_RMS_NORM:
            return op->src[0]->type == GGML_TYPE_F32 && op->src[0]->nb[0] == 4 && ggml_is_contiguous(op);
        case GGML_OP_ROPE:
            return supports_rope(op);
        case GGML_OP_CPY:
        case GGML_OP_CONT:
            if (op->type == GGML_TYPE_I32) {  // ggml_cast to I32 (the sampler's pick), CONT of the top-k view
                return (op->src[0]->type == GGML_TYPE_F32 || op->src[0]->type == GGML_TYPE_I32) &&
                       ggml_is_contiguous(op);
            }
            if (op->src[0]->type == GGML_TYPE_I32) {  // the top-k indices as F32
                return op->type == GGML_TYPE_F32 && ggml_is_contiguous(op);
            }
            return is_f32_or_f16(op->src[0]->type) && is_f32_or_f16(op->type);
        case GGML_OP_GET_ROWS:
            if (op->src[0]->type == GGML_TYPE_I32) {  // rows of indices (the sampler's gathers)
                return op->src[1]->type == GGML_TYPE_I32 && op->type == GGML_TYPE_I32 && ggml_is_contiguous(op);
            }
            return (is_f32_or_f16(op->src[0]->type) || is_repacked(op->src[0]->type)) &&
                   op->src[1]->type == GGML_TYPE_I32 && op->type == GGML_TYPE_F32 && ggml_is_contiguous(op);
        case GGML_OP_SET_ROWS:
            return op->src[0]->type == GGML_TYPE_F32 && is_f32_or_f16(op->type) &&
                   (op->src[1]->type == GGML_TYPE_I64 || op->src[1]->type == GGML_TYPE_I32);
        case GGML_OP_GLU:
            return op->op_params[0] == GGML_GLU_OP_SWIGLU && op->src[0]->type == GGML_TYPE_F32 &&
                   ggml_is_contiguous(op);
        case GGML_OP_SCALE:
            return op->src[0]->type == GGML_TYPE_F32 && ggml_is_contiguous(op);
        case GGML_OP_NORM:
            return op->src[0]->type == GGML_TYPE_F32 && op->type == GGML_TYPE_F32 && ggml_is_contiguous(op);
        case GGML_OP_CONCAT:
            return op->src[0]->type == GGML_TYPE_F32 && op->src[1]->type == GGML_TYPE_F32 &&
                   op->type == GGML_TYPE_F32 && ggml_is_contiguous(op);
        case GGML_OP_CLAMP:
            return op->src[0]->type == GGML_TYPE_F32 && ggml_is_contiguous(op->src[0]) && ggml_is_contiguous(op);
        default:
            return false;
    }
}

// ---- node execution ----

bool fail(const struct ggml_tensor * n, int rc) {
    MI_LOG("node %s (%s) failed: %d %s\n", n->name, ggml_op_name(n->op), rc, mmhip_last_error());
    return false;
}

bool run_mul_mat(mi_backend * c, const struct ggml_tensor * n) {
    const struct ggml_tensor * w  = n->src[0];
    const struct ggml_tensor * x  = n->src[1];
    const int64_t              N  = w->ne[1], K = w->ne[0];
    const int64_t              M  = x->ne[1] * x->ne[2] * x->ne[3];
    const size_t               ws = mmhip_mul_mat_workspace(w->type, N, K, M);
    void *                     wp = ws ? workspace(c, ws) : nullptr;
    if (ws && !wp) {
        return false;
    }
    const int rc = mmhip_mul_mat(w->type, w->data, N, K, (int64_t) w->nb[1], (const float *) x->data,
                                 (int64_t) (x->nb[1] / sizeof(float)), M, (float *) n->data, N, wp, ws, c->stream);
    return rc == MMHIP_OK || fail(n, rc);
}

bool run_fa(mi_backend * c, const struct ggml_tensor * n) {
    mmhip_view q = view_of(n->src[0]), k = view_of(n->src[1]), v = view_of(n->src[2]);
    mmhip_view m;
    const bool has_m = n->src[3] != nullptr;
    if (has_m) {
        m = view_of(n->src[3]);
    }
    float scale;
    memcpy(&scale, &n->op_params[0], sizeof(float));
    const size_t ws = mmhip_flash_attn_workspace(&q, &k, &v);
    void *       wp = ws ? workspace(c, ws) : nullptr;
    if (ws && !wp) {
        return false;
    }
    const int rc = mmhip_flash_attn_ext(&q, &k, &v, has_m ? &m : nullptr, scale, (float *) n->data, wp, ws, c->stream);
    return rc == MMHIP_OK || fail(n, rc);
}

int run_node(mi_backend * c, const struct ggml_tensor * n) {
    hipStream_t s  = c->stream;
    int         rc = MMHIP_OK;
    switch (n->op) {
        case GGML_OP_NONE:
        case GGML_OP_RESHAPE:
        case GGML_OP_VIEW:
        case GGML_OP_PERMUTE:
        case GGML_OP_TRANSPOSE:
            return MMHIP_OK;
        case GGML_OP_MUL_MAT:
            if (n->src[0]->type == GGML_TYPE_BF16 && n->src[1]->ne[1] * n->src[1]->ne[2] * n->src[1]->ne[3] > 16) {
                return run_mul_mat(c, n) ? MMHIP_OK : -1;  // the GEMM, with its bf16 activation copy
            }
            if (n->src[0]->type == GGML_TYPE_BF16) {
                const struct ggml_tensor * w = n->src[0];
                const struct ggml_tensor * x = n->src[1];
                rc = mmhip_mul_mat_bf16(w->data, w->ne[1], w->ne[0], (int64_t) (w->nb[1] / 2), (const float *) x->data,
                                        (int64_t) (x->nb[1] / 4), x->ne[1] * x->ne[2] * x->ne[3], (float *) n->data,
                                        w->ne[1], s);
                break;
            }
            if (n->src[0]->type == GGML_TYPE_F32) {
                mmhip_view a = view_of(n->src[0]), b = view_of(n->src[1]);
                rc           = mmhip_mul_mat_f32(&a, &b, (float *) n->data, s);
                break;
            }
            return run_mul_mat(c, n) ? MMHIP_OK : -1;
        case GGML_OP_FLASH_ATTN_EXT:
            return run_fa(c, n) ? MMHIP_OK : -1;
        case GGML_OP_ADD:
        case GGML_OP_SUB:
        case GGML_OP_MUL: {
            mmhip_view a = view_of(n->src[0]), b = view_of(n->src[1]);
            rc = mmhip_binary(n->op == GGML_OP_ADD ? 0 : n->op == GGML_OP_SUB ? 1 : 2, &a, &b, (float *) n->data, s);
            break;
        }
        case GGML_OP_RMS_NORM: {
            float eps;
            memcpy(&eps, &n->op_params[0], sizeof(float));
            mmhip_view x = view_of(n->src[0]);
            rc           = mmhip_rms_norm(&x, nullptr, eps, (float *) n->data, s);
            break;
        }
        case GGML_OP_ROPE: {
            const int n_dims = n->op_params[1];
            float     base;
            memcpy(&base, &n->op_params[5], sizeof(float));
            const float theta_scale = powf(base, -2.0f / (float) n_dims);
            mmhip_view  x           = view_of(n->src[0]);
            rc = mmhip_rope_neox(&x, (const int32_t *) n->src[1]->data, n_dims, theta_scale, (float *) n->data, s);
            break;
        }
        case GGML_OP_CPY:
        case GGML_OP_CONT: {
            if (n->type == GGML_TYPE_I32 && n->src[0]->type == GGML_TYPE_I32) {
                // 4-byte words moved as they are (the f32 copy path does no arithmetic)
                mmhip_view src = view_of(n->src[0]), dst = view_of(n);
                rc             = mmhip_cpy(&src, GGML_TYPE_F32, &dst, GGML_TYPE_F32, s);
                break;
            }
            if (n->type == GGML_TYPE_I32) {
                mmhip_view a = view_of(n->src[0]);
                rc           = mmhip_cast_i32(&a, (int32_t *) n->data, s);
                break;
            }
            if (n->src[0]->type == GGML_TYPE_I32) {
                mmhip_view a = view_of(n->src[0]);
                rc           = mmhip_cast_f32_of_i32(&a, (float *) n->data, s);
                break;
            }
            mmhip_view src = view_of(n->src[0]), dst = view_of(n);
            rc = mmhip_cpy(&src, n->src[0]->type, &dst, n->type, s);
            break;
        }
        case GGML_OP_GET_ROWS: {
            mmhip_view src = view_of(n->src[0]), ids = view_of(n->src[1]);
            rc = mmhip_get_rows(n->src[0]->type, &src, &ids, (float *) n->data, s);
            break;
        }
        case GGML_OP_SET_ROWS: {
            mmhip_view src = view_of(n->src[0]), ids = view_of(n->src[1]), dst = view_of(n);
            rc = mmhip_set_rows(&src, &ids, n->src[1]->type, &dst, n->type, s);
            break;
        }
        case GGML_OP_GLU: {
            mmhip_view a = view_of(n->src[0]);
            mmhip_view b;
            if (n->src[1]) {
                b = view_of(n->src[1]);
            }
            rc = mmhip_swiglu(&a, n->src[1] ? &b : nullptr, n->op_params[1], (float *) n->data, s);
            break;
        }
        case GGML_OP_SCALE: {
            float sc, bias;
            memcpy(&sc, &n->op_params[0], sizeof(float));
            memcpy(&bias, &n->op_params[1], sizeof(float));
            mmhip_view a = view_of(n->src[0]);
            rc           = mmhip_scale(&a, sc, bias, (float *) n->data, s);
            break;
        }
        case GGML_OP_NORM: {
            float eps;
            memcpy(&eps, &n->op_params[0], sizeof(float));
            mmhip_view x = view_of(n->src[0]);
            rc           = mmhip_norm(&x, eps, (float *) n->data, s);
            break;
        }
        case GGML_OP_CONCAT: {
            mmhip_view a = view_of(n->src[0]);
            mmhip_view b = view_of(n->src[1]);
            rc           = mmhip_concat(&a, &b, n->op_params[0], (float *) n->data, s);
            break;
        }
        case GGML_OP_CLAMP: {
            float lo, hi;
            memcpy(&lo, &n->op_params[0], sizeof(float));
            memcpy(&hi, &n->op_params[1], sizeof(float));
            mmhip_view a = view_of(n->src[0]);
            rc           = mmhip_clamp(&a, lo, hi, (float *) n->data, s);
            break;
        }
        case GGML_OP_SOFT_MAX: {
            mmhip_view a = view_of(n->src[0]);
            rc           = mmhip_soft_max(&a, (float *) n->data, s);
            break;
        }
        case GGML_OP_ARGSORT: {
            mmhip_view a = view_of(n->src[0]);
            rc           = mmhip_argsort_desc(&a, (int32_t *) n->data, s);
            break;
        }
        case GGML_OP_CUMSUM: {
            mmhip_view a = view_of(n->src[0]);
            rc           = mmhip_cumsum(&a, (float *) n->data, s);
            break;
        }
        case GGML_OP_SUM: {
            mmhip_view a = view_of(n->src[0]);
            rc           = mmhip_sum(&a, (float *) n->data, s);
            break;
        }
        case GGML_OP_UNARY: {
            mmhip_view a = view_of(n->src[0]);
            rc           = mmhip_step(&a, (float *) n->data, s);
            break;
        }
        case GGML_OP_DIAG_MASK_INF: {
            mmhip_view a = view_of(n->src[0]);
            rc           = mmhip_diag_mask_inf(&a, n->op_params[0], (float *) n->data, s);
            break;
        }
        default:
            MI_LOG("unsupported node %s (%s)\n", n->name, ggml_op_name(n->op));
            return -1;
    }
    return rc == MMHIP_OK ? MMHIP_OK : (fail(n, rc), -1);
}

// ---- execution plan ----
//
// The graph's nodes in order, with these chains fused into single steps.
// A fused step runs at the position of the chain's last node, so every input
// it reads has been produced; the chain's other nodes must have exactly one
// consumer (the next chain node) and not be graph outputs.
//   NORM      RMS_NORM -> MUL(w): one row kernel; when every consumer is a
//             GEMV MUL_MAT of one activation type, the rows are also
//             quantised into an activation slot those MUL_MATs read.
//   SWIGLU_Q  GLU SwiGLU whose consumers are GEMV MUL_MATs: quantised into a
//             slot as well.
//   HEAD      CONT(view) -> RESHAPE -> [RMS_NORM -> MUL] -> [ROPE] -> [CONT]
//             -> [RESHAPE -> SET_ROWS]: the per-head Q / K / V rows of the
//             attention block in one launch; also RESHAPE(rows) -> ... ->
//             SET_ROWS, a projection's own output (the V of the "_M" files'
//             layers whose V weight has its own type, src/qwen3-lm.h:749-757).
//   MM_GLU    a norm-fused gate_up GEMV MUL_MAT whose only consumer is a
//             SwiGLU feeding Q8_0 GEMVs: the SwiGLU and its quantisation into
//             those GEMVs' slot run in the gate_up GEMV's epilogue.
//   MM_ADD    a GEMV MUL_MAT whose only consumer is an ADD with a same-shape
//             residual: the ADD is done in the GEMV's store.
//   SATTN     CONT(PERMUTE(MUL_MAT(CONT(TRANSPOSE(v)), SOFT_MAX(DIAG_MASK_INF(
//             SCALE(MUL_MAT(k, q))))))): the depth decoder's manual causal
//             attention (src/depth-decoder.h:214-221) in one launch.
//   ROPE_H    CPY(PERMUTE(ROPE(x))) to F16 (the DiT's K cast,
//             src/dit.h:207-220): the rotation stores f16 straight into the
//             cast's rows.
// MUL_MATs reading a slot skip their activation quantisation.

enum step_kind { ST_NODE, ST_NORM, ST_SWIGLU_Q, ST_HEAD, ST_MM, ST_FA_Q, ST_GEMM, ST_LN, ST_GLU_V, ST_SATTN, ST_ROPE_H };

struct plan_step {
    int                  kind = ST_NODE;
    int                  node = -1;      // node executed / whose output is written
    int                  src  = -1;      // NORM: the RMS_NORM node
    int                  add  = -1;      // MM: the fused ADD node
    int                  add_res = -1;   // MM: index 0/1 of the ADD's residual source
    int                  norm    = -1;   // MM: the RMS_NORM node whose norm runs in the GEMV's prologue
    int                  norm_mul = -1;  // MM: the MUL by the norm weight (the GEMV's src1)
    int                  glu      = -1;  // MM: the SWIGLU node whose SwiGLU runs in the GEMV's prologue
    int                  glu_epi  = -1;  // MM / GEMM: the SWIGLU node computed in the GEMV's / GEMM's epilogue
    int                  glu_swapped = 0;  // GEMM: the gate rows are the first half
    int                  multi[2]    = { -1, -1 };  // GEMM: further MUL_MATs of the same activations in this launch
    int                  mm       = -1;  // GEMM: the MUL_MAT node
    int                  bias     = -1;  // GEMM: the bias ADD node / LN: the ADD of the LayerNorm bias
    int                  bias_src = -1;  // index 0/1 of that ADD's vector operand
    int                  mul      = -1;  // LN: the MUL by the LayerNorm weight
    int64_t              slot_out = -1;  // byte offset of the quantised slot written (NORM / SWIGLU_Q)
    int64_t              slot_in  = -1;  // byte offset of the slot read (MM)
    int                  vec_wtype = 0;  // weight type the slot is quantised for
    bool                 write_f32 = true;
    mmhip_head_rows_args head[4]{};  // HEAD: the chains run by this step (FA_Q: the fused Q, K, V chains)
    int                  head_end[4]{ -1, -1, -1, -1 };  // the chains' last nodes
    const struct ggml_tensor * head_in[4]{};               // the chains' source rows
    int                  n_head = 0;
};

struct graph_info {
    int                                          nn = 0;
    std::vector<int>                             uses;
    std::vector<int>                             cons;  // last consumer (the only one when uses == 1)
    std::vector<std::vector<int>>                consumers;
    std::unordered_map<const ggml_tensor *, int> index;
};

bool is_noop(enum ggml_op op) {
    return op == GGML_OP_NONE || op == GGML_OP_RESHAPE || op == GGML_OP_VIEW || op == GGML_OP_PERMUTE ||
           op == GGML_OP_TRANSPOSE;
}

bool is_output(const struct ggml_tensor * t) {
    return (t->flags & GGML_TENSOR_FLAG_OUTPUT) != 0;
}

// node index of t, or -1 for leafs / tensors outside the graph
int node_index(const graph_info & gi, const struct ggml_tensor * t) {
    auto it = gi.index.find(t);
    return it == gi.index.end() ? -1 : it->second;
}

// Would mmhip_mul_mat run this MUL_MAT as an activation-quantised GEMV?
// The operand index (0/1) of `add` (an ADD reading n) that is an f32
// contiguous vector of n->ne[0] elements broadcast over n's rows, else -1.
int add_row_vector(const struct ggml_tensor * add, const struct ggml_tensor * n) {
    if (add->op != GGML_OP_ADD && add->op != GGML_OP_MUL) {
        return -1;
    }
    const int oth = add->src[0] == n ? 1 : add->src[1] == n ? 0 : -1;
    if (oth < 0 || add->src[oth] == n) {
        return -1;
    }
    const struct ggml_tensor * v = add->src[oth];
    const bool ok = v->type == GGML_TYPE_F32 && ggml_is_contiguous(v) && v->ne[0] == n->ne[0] && v->ne[1] == 1 &&
                    v->ne[2] == 1 && v->ne[3] == 1 && ggml_are_same_shape(add, n) && add->type == GGML_TYPE_F32;
    return ok ? oth : -1;
}

// BF16 weights at 1-2 columns: the persistent BF16 decode GEMV (activations
// read as f32, no quantised slot)
bool mm_is_bf16_dec(const struct ggml_tensor * n) {
    const struct ggml_tensor * w = n->src[0];
    const struct ggml_tensor * x = n->src[1];
    const int64_t              M = x->ne[1] * x->ne[2] * x->ne[3];
    return n->op == GGML_OP_MUL_MAT && w->type == GGML_TYPE_BF16 && w->ne[2] == 1 && w->ne[3] == 1 &&
           x->type == GGML_TYPE_F32 && mm_collapsible(x) && x->nb[1] % 16 == 0 && ((uintptr_t) x->data) % 16 == 0 &&
           w->nb[1] % 16 == 0 && ((uintptr_t) w->data) % 16 == 0 && ggml_is_contiguous(n) &&
           mmhip_mul_mat_bf16_dec_supported(w->ne[1], w->ne[0], M, 0) && !getenv("GGML_MI355X_DISABLE_BF16_DEC");
}

bool mm_is_gemv(const struct ggml_tensor * n) {
    const struct ggml_tensor * x = n->src[1];
    const int64_t              M = x->ne[1] * x->ne[2] * x->ne[3];
    return n->op == GGML_OP_MUL_MAT && M >= 1 && M <= 16 &&
           (mmhip_act_bytes(n->src[0]->type, n->src[0]->ne[0], M) > 0 || mm_is_bf16_dec(n));
}

int act_vec_type(int wtype) {
    return wtype == GGML_TYPE_Q8_0 ? GGML_TYPE_Q8_0 : GGML_TYPE_Q8_K;
}

// All consumers of node p are GEMV MUL_MATs reading p as src1 with weights
// of one activation type; returns that weight type (0 if not).
int gemv_consumer_type(struct ggml_cgraph * g, const graph_info & gi, int p) {
    if (gi.consumers[(size_t) p].empty()) {
        return 0;
    }
    int wt = 0;
    for (int ci : gi.consumers[(size_t) p]) {
        const struct ggml_tensor * m = ggml_graph_node(g, ci);
        if (m->op != GGML_OP_MUL_MAT || m->src[1] != ggml_graph_node(g, p) || m->src[0] == m->src[1] ||
            !mm_is_gemv(m) || m->src[0]->type == GGML_TYPE_BF16) {
            return 0;  // BF16 GEMVs read f32 activations: no slot
        }
        if (wt && act_vec_type(wt) != act_vec_type(m->src[0]->type)) {
            return 0;
        }
        wt = m->src[0]->type;
    }
    return wt;
}

bool is_f32_vector(const struct ggml_tensor * w, int64_t n) {
    return w->type == GGML_TYPE_F32 && w->ne[0] == n && w->ne[1] == 1 && w->ne[2] == 1 && w->ne[3] == 1 &&
           w->nb[0] == sizeof(float);
}

bool rows_contiguous_f32(const struct ggml_tensor * t) {
    return t->type == GGML_TYPE_F32 && ggml_is_contiguous(t) && ((uintptr_t) t->data) % 16 == 0;
}

bool overlaps(const struct ggml_tensor * a, const struct ggml_tensor * b) {
    const uintptr_t a0 = (uintptr_t) a->data, b0 = (uintptr_t) b->data;
    return a0 && b0 && a0 < b0 + ggml_nbytes(b) && b0 < a0 + ggml_nbytes(a);
}

// Can every consumer of the norm-weight MUL j (after RMS_NORM i) be a GEMV
// that recomputes the norm itself (mmhip_rms_norm_mul_mat)?  The raw rows
// must then stay intact until the last of them ran: no node executed in
// between (or an ADD fused into one of them) may write over them.
bool norm_into_gemvs(struct ggml_cgraph * g, const graph_info & gi, int i, int j) {
    const struct ggml_tensor * n = ggml_graph_node(g, i);
    const struct ggml_tensor * m = ggml_graph_node(g, j);
    const struct ggml_tensor * x = n->src[0];
    const int64_t              K = x->ne[0], M = ggml_nrows(x);
    if (is_output(m) || gi.consumers[(size_t) j].empty() || x->type != GGML_TYPE_F32 || !mm_collapsible(x) ||
        ((uintptr_t) x->data | x->nb[1]) % 16 != 0 || !is_f32_vector(m->src[1], K) ||
        ((uintptr_t) m->src[1]->data) % 16 != 0) {
        return false;
    }
    int last = j;
    for (int ci : gi.consumers[(size_t) j]) {
        const struct ggml_tensor * mm = ggml_graph_node(g, ci);
        const bool bf = mm->src[0]->type == GGML_TYPE_BF16;
        if (mm->op != GGML_OP_MUL_MAT || mm->src[1] != m || mm->src[0] == m || !mm_is_gemv(mm) ||
            !(bf ? mmhip_mul_mat_bf16_dec_supported(mm->src[0]->ne[1], K, M, 0)
                 : mmhip_rms_norm_mul_mat_supported(mm->src[0]->type, mm->src[0]->ne[1], K, M))) {
            return false;
        }
        last = std::max(last, gi.uses[(size_t) ci] == 1 ? std::max(ci, gi.cons[(size_t) ci]) : ci);
    }
    for (int t = j + 1; t <= last; t++) {
        const struct ggml_tensor * nt = ggml_graph_node(g, t);
        if (!is_noop(nt->op) && overlaps(nt, x)) {
            return false;
        }
    }
    return true;
}

// The gate and up rows of a SWIGLU node (fused: the two halves of src0,
// swapped by op_params[1]; split: src0 and src1), each M rows of a uniform
// stride.  False when the layout is not one the SwiGLU GEMV reads.
bool glu_rows(const struct ggml_tensor * n, const float *& gate, int64_t & ldg, const float *& up, int64_t & ldu) {
    const struct ggml_tensor * a = n->src[0];
    const struct ggml_tensor * b = n->src[1];
    const int64_t              F = n->ne[0];
    auto rows_ok = [&](const struct ggml_tensor * t) {
        return t->type == GGML_TYPE_F32 && mm_collapsible(t) && ggml_nrows(t) == ggml_nrows(n) &&
               ((uintptr_t) t->data | t->nb[1]) % 16 == 0;
    };
    if (!rows_ok(a) || (b && (!rows_ok(b) || b->ne[0] != F)) || (!b && a->ne[0] != 2 * F)) {
        return false;
    }
    const bool swapped = n->op_params[1] != 0;
    gate = (const float *) a->data + (!b && swapped ? F : 0);
    up   = b ? (const float *) b->data : (const float *) a->data + (swapped ? 0 : F);
    ldg  = (int64_t) (a->nb[1] / 4);
    ldu  = b ? (int64_t) (b->nb[1] / 4) : ldg;
    return true;
}

// Can every consumer of SWIGLU node i be a GEMV that recomputes the SwiGLU
// itself (mmhip_swiglu_mul_mat)?  Its inputs must then stay intact until the
// last of them ran.
bool glu_into_gemvs(struct ggml_cgraph * g, const graph_info & gi, int i) {
    const struct ggml_tensor * n = ggml_graph_node(g, i);
    const float *              gp;
    const float *              up;
    int64_t                    ldg, ldu;
    if (is_output(n) || gi.consumers[(size_t) i].empty() || !glu_rows(n, gp, ldg, up, ldu)) {
        return false;
    }
    const int64_t K = n->ne[0], M = ggml_nrows(n);
    int           last = i;
    for (int ci : gi.consumers[(size_t) i]) {
        const struct ggml_tensor * mm = ggml_graph_node(g, ci);
        if (mm->op != GGML_OP_MUL_MAT || mm->src[1] != n || mm->src[0] == n || !mm_is_gemv(mm) ||
            !mmhip_swiglu_mul_mat_supported(mm->src[0]->type, mm->src[0]->ne[1], K, M)) {
            return false;
        }
        last = std::max(last, gi.uses[(size_t) ci] == 1 ? std::max(ci, gi.cons[(size_t) ci]) : ci);
    }
    for (int t = i + 1; t <= last; t++) {
        const struct ggml_tensor * nt = ggml_graph_node(g, t);
        if (!is_noop(nt->op) && (overlaps(nt, n->src[0]) || (n->src[1] && overlaps(nt, n->src[1])))) {
            return false;
        }
    }
    return true;
}

// Try the HEAD chain starting at CONT node i; fills st and marks absorbed nodes.
// The depth decoder's manual attention chain ending at CONT node i
// (src/depth-decoder.h:214-221): CONT(PERMUTE_0213(m2)), m2 = MUL_MAT(vt, sm),
// vt = CONT(TRANSPOSE(v)), sm = SOFT_MAX(dm) (no mask, scale 1), dm =
// DIAG_MASK_INF(sc), sc = SCALE(m1), m1 = MUL_MAT(k, q), all f32 and each
// intermediate read only by the next; S_q, S_kv <= 16, D <= 256.  Every node executed
// between the chain's first and last node must be one of its own (views
// otherwise), and the output must not overlap q, k or v (read until the end).
// The f16 view a ROPE_H step writes: the rope's shape, and per rope dim the
// stride of the cast's destination dim it lands in (ggml_permute sends
// source dim a to position op_params[a]).
mmhip_view rope_h_dst(const struct ggml_tensor * cpy) {
    const struct ggml_tensor * pm = cpy->src[0];
    const struct ggml_tensor * r  = pm->src[0];
    mmhip_view                 v{};
    v.data = cpy->data;
    for (int a = 0; a < 4; a++) {
        v.ne[a] = r->ne[a];
        v.nb[a] = (int64_t) cpy->nb[pm->op_params[a]];
    }
    return v;
}

// CPY(PERMUTE(ROPE(x))) into a contiguous F16 tensor, the rope and the
// permutation read by nothing else, only views between the rope and the CPY
// (so the rope's input is still intact at the CPY's position), and the
// shapes the position-parallel rope kernel takes.
bool plan_rope_h(struct ggml_cgraph * g, const graph_info & gi, int i, const std::vector<int> & step_at,
                 const std::vector<char> & absorbed) {
    const struct ggml_tensor * n  = ggml_graph_node(g, i);
    const struct ggml_tensor * pm = n->src[0];
    if (getenv("GGML_MI355X_DISABLE_ROPE_F16") || n->type != GGML_TYPE_F16 || !ggml_is_contiguous(n) || !pm ||
        pm->op != GGML_OP_PERMUTE || !pm->src[0] || pm->src[0]->op != GGML_OP_ROPE) {
        return false;
    }
    const struct ggml_tensor * r  = pm->src[0];
    const int                  ri = node_index(gi, r), pi = node_index(gi, pm);
    if (ri < 0 || pi < 0 || ri >= i || gi.uses[(size_t) ri] != 1 || gi.uses[(size_t) pi] != 1 || is_output(r) ||
        is_output(pm) || step_at[(size_t) ri] >= 0 || absorbed[(size_t) ri] || r->type != GGML_TYPE_F32 ||
        !supports_rope(r)) {
        return false;
    }
    for (int t = ri + 1; t < i; t++) {
        if (!is_noop(ggml_graph_node(g, t)->op)) {
            return false;
        }
    }
    const struct ggml_tensor * x      = r->src[0];
    const int                  n_dims = r->op_params[1];
    const mmhip_view           d      = rope_h_dst(n);
    // the fused launch reads x while it writes n: an allocator that reused
    // x's memory for the cast's output (x is dead after the rope in the
    // unfused order) would have n overlap x
    bool ok = !overlaps(n, x) && x->type == GGML_TYPE_F32 && ggml_are_same_shape(x, r) && n_dims > 0 && n_dims <= 256 &&
              (n_dims / 2) % 4 == 0 && x->ne[0] % 4 == 0 && x->nb[0] == 4 && ((uintptr_t) x->data) % 16 == 0 &&
              ((uintptr_t) n->data) % 8 == 0 && d.nb[0] == 2;
    for (int a = 1; a < 4; a++) {
        ok = ok && x->nb[a] % 16 == 0 && d.nb[a] % 8 == 0;
    }
    return ok;
}

bool plan_small_attn(struct ggml_cgraph * g, const graph_info & gi, int i, plan_step & st,
                     std::vector<char> & absorbed) {
    static const bool dbg = getenv("GGML_MI355X_PLAN_DEBUG") != nullptr;
#define SATTN_NO(why)                                                         \
    do {                                                                      \
        if (dbg) {                                                            \
            fprintf(stderr, "small_attn at node %d (%s): %s\n", i, n->name, why); \
        }                                                                     \
        return false;                                                         \
    } while (0)
    const struct ggml_tensor * n  = ggml_graph_node(g, i);
    const struct ggml_tensor * pm = n->src[0];
    if (n->type != GGML_TYPE_F32 || !ggml_is_contiguous(n) || !pm || pm->op != GGML_OP_PERMUTE ||
        pm->op_params[0] != 0 || pm->op_params[1] != 2 || pm->op_params[2] != 1 || pm->op_params[3] != 3) {
        return false;
    }
    const struct ggml_tensor * m2 = pm->src[0];
    if (!m2 || m2->op != GGML_OP_MUL_MAT) {
        return false;
    }
    const struct ggml_tensor * vt = m2->src[0];
    const struct ggml_tensor * sm = m2->src[1];
    if (vt->op != GGML_OP_CONT || !vt->src[0] || vt->src[0]->op != GGML_OP_TRANSPOSE || sm->op != GGML_OP_SOFT_MAX ||
        sm->src[1] != nullptr) {
        return false;
    }
    float sm_scale, sm_bias;
    memcpy(&sm_scale, &sm->op_params[0], sizeof(float));
    memcpy(&sm_bias, &sm->op_params[1], sizeof(float));
    const struct ggml_tensor * dm = sm->src[0];
    if (sm_scale != 1.0f || sm_bias != 0.0f || dm->op != GGML_OP_DIAG_MASK_INF) {
        return false;
    }
    const struct ggml_tensor * sc = dm->src[0];
    if (sc->op != GGML_OP_SCALE) {
        return false;
    }
    const struct ggml_tensor * m1 = sc->src[0];
    if (m1->op != GGML_OP_MUL_MAT) {
        return false;
    }
    const struct ggml_tensor * q = m1->src[1];
    const struct ggml_tensor * k = m1->src[0];
    const struct ggml_tensor * v = vt->src[0]->src[0];
    for (const struct ggml_tensor * t : { q, k, v }) {
        if (t->type != GGML_TYPE_F32 || t->nb[0] != 4 || t->ne[0] != q->ne[0]) {
            return false;
        }
    }
    if (q->ne[1] > 16 || k->ne[1] > 16 || q->ne[0] > 256 || k->ne[1] != v->ne[1] || q->ne[1] <= 0 || k->ne[1] <= 0 ||
        k->ne[2] <= 0 || v->ne[2] <= 0 || k->ne[3] <= 0 || v->ne[3] <= 0 || q->ne[2] % k->ne[2] != 0 ||
        q->ne[3] % k->ne[3] != 0 || q->ne[2] % v->ne[2] != 0 || q->ne[3] % v->ne[3] != 0 ||
        n->ne[0] != q->ne[0] || n->ne[1] != q->ne[2] || n->ne[2] != q->ne[1] || n->ne[3] != q->ne[3]) {
        SATTN_NO("shapes");
    }
    if (overlaps(n, q) || overlaps(n, k) || overlaps(n, v)) {
        SATTN_NO("output overlaps q / k / v");
    }
    // the chain's nodes: each read only by the next, none a graph output
    const struct ggml_tensor * chain[] = { m1, sc, dm, sm, vt->src[0], vt, m2, pm };
    int                        idx[8];
    int                        lo = i;
    for (int c = 0; c < 8; c++) {
        idx[c] = node_index(gi, chain[c]);
        if (idx[c] < 0 || idx[c] >= i || gi.uses[(size_t) idx[c]] != 1 || is_output(chain[c]) || absorbed[(size_t) idx[c]]) {
            SATTN_NO(absorbed[(size_t) std::max(idx[c], 0)] ? "a chain node is in another fused step" : "chain node uses");
        }
        lo = std::min(lo, idx[c]);
    }
    // nodes run between the chain's first node and i (the graph's other
    // branches, e.g. the q / k projections after CONT(TRANSPOSE(v))) must not
    // write over an input produced before them: the allocator, which planned
    // for the unfused order, may reuse an input's memory once its last
    // (absorbed) reader has run
    const struct ggml_tensor * ins[3] = { q, k, v };
    int                        prod[3];
    for (int x = 0; x < 3; x++) {
        const struct ggml_tensor * b = ins[x];
        while (b->view_src) {
            b = b->view_src;
        }
        prod[x] = node_index(gi, b);  // -1: a leaf, produced before the graph
    }
    for (int t = lo + 1; t < i; t++) {
        const struct ggml_tensor * nt  = ggml_graph_node(g, t);
        const bool                 own = std::find(std::begin(idx), std::end(idx), t) != std::end(idx);
        if (own || is_noop(nt->op)) {
            continue;
        }
        for (int x = 0; x < 3; x++) {
            if (prod[x] < t && overlaps(nt, ins[x])) {
                SATTN_NO("a node inside the chain writes over an input");
            }
        }
    }
#undef SATTN_NO
    if (dbg) {
        fprintf(stderr, "small_attn at node %d (%s): fused\n", i, n->name);
    }
    st.kind = ST_SATTN;
    st.node = i;
    st.mm   = idx[0];  // m1: k = src0, q = src1
    st.mul  = idx[1];  // SCALE
    st.bias = idx[2];  // DIAG_MASK_INF
    st.src  = idx[5];  // vt: v = its TRANSPOSE's source
    for (int c : { 0, 1, 2, 3, 5, 6 }) {
        absorbed[(size_t) idx[c]] = 1;
    }
    return true;
}

bool plan_head(struct ggml_cgraph * g, const graph_info & gi, int i, plan_step & st, std::vector<char> & absorbed) {
    const struct ggml_tensor * n0 = ggml_graph_node(g, i);
    const struct ggml_tensor * v  = n0->src[0];
    // entry: CONT of a 2-D view, then RESHAPE [D, H, T]; or a RESHAPE
    // [D, H, T] of 2-D rows (whose chain must then end in the cache write)
    const bool from_rows = n0->op == GGML_OP_RESHAPE;
    if (!(n0->op == GGML_OP_CONT || from_rows) || n0->type != GGML_TYPE_F32 || !v || v->type != GGML_TYPE_F32 ||
        v->nb[0] != 4 || v->ne[2] != 1 || v->ne[3] != 1 || v->nb[1] % 4 != 0) {
        return false;
    }
    std::vector<int> chain{ i };
    auto             next = [&](int k) -> int {
        if (gi.uses[(size_t) k] != 1 || is_output(ggml_graph_node(g, k))) {
            return -1;
        }
        return gi.cons[(size_t) k];
    };
    int j = i;
    if (!from_rows) {
        j = next(i);
        if (j < 0) {
            return false;
        }
    }
    const struct ggml_tensor * r1 = ggml_graph_node(g, j);
    const int64_t              D  = r1->ne[0], H = r1->ne[1], T = r1->ne[2];
    if (r1->op != GGML_OP_RESHAPE || (!from_rows && r1->src[0] != n0) || r1->ne[3] != 1 || D * H != v->ne[0] ||
        T != v->ne[1] || !(D == 64 || D == 128 || D == 256)) {
        return false;
    }
    if (!from_rows) {
        chain.push_back(j);
    }
    mmhip_head_rows_args a{};
    a.src      = v->data;
    a.src_nb_h = D * 4;
    a.src_nb_t = (int64_t) v->nb[1];
    a.D        = (int) D;
    a.H        = (int) H;
    a.T        = (int) T;
    a.dst_type = 0;
    int cur    = j;  // last node of the chain so far
    int end    = -1;
    auto input_ok = [&](const struct ggml_tensor * t) { return node_index(gi, t) < i; };

    int k = next(cur);
    if (k >= 0 && ggml_graph_node(g, k)->op == GGML_OP_RMS_NORM && ggml_graph_node(g, k)->src[0] ==
                                                                         ggml_graph_node(g, cur)) {
        memcpy(&a.eps, &ggml_graph_node(g, k)->op_params[0], sizeof(float));
        a.norm = 1;
        chain.push_back(k);
        cur = end = k;
        k         = next(cur);
        if (k >= 0) {
            const struct ggml_tensor * m = ggml_graph_node(g, k);
            if (m->op == GGML_OP_MUL && m->src[0] == ggml_graph_node(g, cur) && is_f32_vector(m->src[1], D) &&
                input_ok(m->src[1])) {
                a.norm_w = (const float *) m->src[1]->data;
                chain.push_back(k);
                cur = end = k;
                k         = next(cur);
            }
        }
    }
    if (k >= 0) {
        const struct ggml_tensor * r = ggml_graph_node(g, k);
        if (r->op == GGML_OP_ROPE && r->src[0] == ggml_graph_node(g, cur) && supports_rope(r) && r->op_params[1] == D &&
            r->src[1]->ne[0] == T && input_ok(r->src[1])) {
            float base;
            memcpy(&base, &r->op_params[5], sizeof(float));
            a.pos         = (const int32_t *) r->src[1]->data;
            a.theta_scale = powf(base, -2.0f / (float) D);
            chain.push_back(k);
            cur = end = k;
            k         = next(cur);
        }
    }
    if (k >= 0) {
        const struct ggml_tensor * c2 = ggml_graph_node(g, k);
        if (c2->op == GGML_OP_CONT && c2->type == GGML_TYPE_F32 && c2->src[0] == ggml_graph_node(g, cur)) {
            chain.push_back(k);
            cur = end = k;
            k         = next(cur);
        }
    }
    // [RESHAPE [D, 1, H, T] -> SET_ROWS]
    if (k >= 0) {
        const struct ggml_tensor * r2 = ggml_graph_node(g, k);
        const int                  sk = r2->op == GGML_OP_RESHAPE ? next(k) : -1;
        if (sk >= 0 && r2->src[0] == ggml_graph_node(g, cur) && r2->ne[0] == D && r2->ne[1] == 1 && r2->ne[2] == H &&
            r2->ne[3] == T) {
            const struct ggml_tensor * sr  = ggml_graph_node(g, sk);
            const struct ggml_tensor * ids = sr->src[1];
            const size_t               es  = sr->type == GGML_TYPE_F16 ? 2 : 4;
            if (sr->op == GGML_OP_SET_ROWS && sr->src[0] == r2 && (sr->type == GGML_TYPE_F16 || sr->type == GGML_TYPE_F32) &&
                (ids->type == GGML_TYPE_I64 || ids->type == GGML_TYPE_I32) && ids->ne[0] == 1 && ids->ne[3] == 1 &&
                H % ids->ne[1] == 0 && T % ids->ne[2] == 0 && sr->ne[0] == D && sr->nb[0] == es && sr->ne[2] == H &&
                sr->ne[3] == T && input_ok(ids)) {
                a.ids       = ids->data;
                a.ids_type  = ids->type;
                a.ids_nb1   = (int64_t) ids->nb[1];
                a.ids_nb2   = (int64_t) ids->nb[2];
                a.ids_ne1   = ids->ne[1];
                a.ids_ne2   = ids->ne[2];
                a.dst       = sr->data;
                a.dst_type  = sr->type == GGML_TYPE_F16 ? 1 : 0;
                a.dst_nb1   = (int64_t) sr->nb[1];
                a.dst_nb2   = (int64_t) sr->nb[2];
                a.dst_nb3   = (int64_t) sr->nb[3];
                chain.push_back(k);
                chain.push_back(sk);
                end = sk;
            }
        }
    }
    if (end < 0 || (from_rows && !a.ids)) {
        return false;  // nothing but a copy: the plain CONT is as good
    }
    const struct ggml_tensor * e = ggml_graph_node(g, end);
    if (!a.ids) {
        if (!rows_contiguous_f32(e) || e->ne[0] != D || e->ne[1] != H || e->ne[2] != T) {
            return false;
        }
        a.dst = e->data;
    }
    st.kind    = ST_HEAD;
    st.node    = end;
    st.head[0]     = a;
    st.head_end[0] = end;
    st.head_in[0]  = v;
    st.n_head      = 1;
    for (int x : chain) {
        absorbed[(size_t) x] = 1;
    }
    return true;
}

// Does node e feed only node fa, through no-op views?
bool feeds_only(struct ggml_cgraph * g, const graph_info & gi, int e, int fa, int depth = 0) {
    if (depth > 8 || is_output(ggml_graph_node(g, e)) || gi.consumers[(size_t) e].empty()) {
        return false;
    }
    for (int c : gi.consumers[(size_t) e]) {
        if (c != fa && !(is_noop(ggml_graph_node(g, c)->op) && feeds_only(g, gi, c, fa, depth + 1))) {
            return false;
        }
    }
    return true;
}

// May GEMV step s run before HEAD step h?  Its output must not overlap the
// chains' source rows or their outputs, its input rows not their outputs
// (no fused ADD: the residual would be another operand to check).
bool mm_commutes_with_head(struct ggml_cgraph * g, const plan_step & h, const plan_step & s) {
    if (s.kind != ST_MM || s.add >= 0 || s.glu >= 0 || s.glu_epi >= 0) {
        return false;
    }
    const struct ggml_tensor * mm = ggml_graph_node(g, s.node);
    const struct ggml_tensor * x  = s.norm >= 0 ? ggml_graph_node(g, s.norm)->src[0] : mm->src[1];
    for (int c = 0; c < h.n_head; c++) {
        const struct ggml_tensor * in  = h.head_in[c];
        const struct ggml_tensor * out = ggml_graph_node(g, h.head_end[c]);
        if (!in || overlaps(mm, in) || overlaps(mm, out) || overlaps(x, out)) {
            return false;
        }
    }
    return true;
}

// HEAD step h (three chains) + attention step a -> one FA_Q step f whose
// attention runs the chains in its prologue (mmhip_flash_attn_ext_head)
bool fa_head_fuse(struct ggml_cgraph * g, const graph_info & gi, const plan_step & h, const plan_step & a,
                  plan_step & f) {
    const int                  fi = a.node;
    const struct ggml_tensor * n  = ggml_graph_node(g, fi);
    if (n->op != GGML_OP_FLASH_ATTN_EXT || !(a.kind == ST_FA_Q || a.kind == ST_NODE) || !n->src[1] || !n->src[2]) {
        return false;
    }
    int qc = -1, kc = -1, vc = -1;
    for (int c = 0; c < 3; c++) {
        if (!h.head[c].ids) {
            qc = c;
        } else if (h.head[c].dst == n->src[1]->data) {
            kc = c;
        } else if (h.head[c].dst == n->src[2]->data) {
            vc = c;
        }
    }
    if (qc < 0 || kc < 0 || vc < 0 || h.head_end[qc] < 0 || !feeds_only(g, gi, h.head_end[qc], fi)) {
        return false;
    }
    const mmhip_view q = view_of(n->src[0]), k = view_of(n->src[1]), v = view_of(n->src[2]);
    if (!mmhip_flash_attn_ext_head_supported(&q, &k, &v)) {
        return false;
    }
    f = a;
    if (f.kind == ST_NODE) {
        f.kind     = ST_FA_Q;
        f.slot_out = -1;
    }
    f.head[0]     = h.head[qc];
    f.head[1]     = h.head[kc];
    f.head[2]     = h.head[vc];
    f.n_head      = 3;
    return true;
}

struct graph_plan {
    std::vector<plan_step> steps;
    size_t                 slot_bytes = 0;
};

graph_plan build_plan(struct ggml_cgraph * g) {
    graph_info gi;
    gi.nn = ggml_graph_n_nodes(g);
    gi.uses.assign((size_t) gi.nn, 0);
    gi.cons.assign((size_t) gi.nn, -1);
    gi.consumers.assign((size_t) gi.nn, {});
    gi.index.reserve((size_t) gi.nn * 2);
    for (int i = 0; i < gi.nn; i++) {
        struct ggml_tensor * n = ggml_graph_node(g, i);
        for (int s = 0; s < GGML_MAX_SRC; s++) {
            if (n->src[s]) {
                auto it = gi.index.find(n->src[s]);
                if (it != gi.index.end()) {
                    gi.uses[(size_t) it->second]++;
                    gi.cons[(size_t) it->second] = i;
                    gi.consumers[(size_t) it->second].push_back(i);
                }
            }
        }
        gi.index[n] = i;
    }
    const bool no_fuse = getenv("GGML_MI355X_DISABLE_FUSION") != nullptr;

    graph_plan               plan;
    std::vector<char>        absorbed((size_t) gi.nn, 0);
    std::vector<plan_step>   pending;                      // fused steps keyed by their execution node
    std::vector<int>         step_at((size_t) gi.nn, -1);  // index into pending
    std::vector<int64_t>     slot_of((size_t) gi.nn, -1);  // node -> quantised slot of its output
    std::vector<int>         slot_wtype((size_t) gi.nn, 0);
    std::vector<int64_t>     f16_slot_of((size_t) gi.nn, -1);  // node -> slot holding its rows in f16
    std::vector<int>         norm_of((size_t) gi.nn, -1);  // MUL node -> its RMS_NORM, norm done by the GEMVs
    const bool               no_norm_mm = getenv("GGML_MI355X_DISABLE_NORM_GEMV") != nullptr;
    std::vector<char>        glu_mm((size_t) gi.nn, 0);  // SWIGLU node done by its GEMVs
    const bool               no_glu_mm  = getenv("GGML_MI355X_DISABLE_SWIGLU_GEMV") != nullptr;
    const bool               no_glu_epi = getenv("GGML_MI355X_DISABLE_SWIGLU_EPILOGUE") != nullptr;
    const bool               no_sattn   = getenv("GGML_MI355X_DISABLE_SMALL_ATTN") != nullptr;
    auto add_pending = [&](const plan_step & st) {
        step_at[(size_t) st.node] = (int) pending.size();
        pending.push_back(st);
    };
    auto new_slot = [&](int wtype, int64_t K, int64_t M) -> int64_t {
        const size_t  bytes = mmhip_act_bytes(wtype, K, M);
        const int64_t off   = (int64_t) plan.slot_bytes;
        plan.slot_bytes += (bytes + 255) / 256 * 256;
        return off;
    };

    for (int i = 0; i < gi.nn && !no_fuse; i++) {
        if (absorbed[(size_t) i]) {
            continue;
        }
        struct ggml_tensor * n = ggml_graph_node(g, i);
        // Steps run at their last node: every node in between must be a view or
        // absorbed, so no other node can reuse a buffer the step still reads.
        auto quiet_between = [&](int a, int b, int s1, int s2) {
            for (int t = a + 1; t < b; t++) {
                if (t != s1 && t != s2 && !is_noop(ggml_graph_node(g, t)->op)) {
                    return false;
                }
            }
            return true;
        };
        if (n->op == GGML_OP_RMS_NORM && gi.uses[(size_t) i] == 1 && !is_output(n)) {
            const int j = gi.cons[(size_t) i];
            const struct ggml_tensor * m = ggml_graph_node(g, j);
            if (m->op == GGML_OP_MUL && m->src[0] == n && m->src[1]->type == GGML_TYPE_F32 &&
                ggml_are_same_shape(m, n) && node_index(gi, m->src[1]) < j) {
                if (!no_norm_mm && norm_into_gemvs(g, gi, i, j)) {
                    norm_of[(size_t) j]  = i;
                    absorbed[(size_t) i] = 1;
                    absorbed[(size_t) j] = 1;
                    continue;
                }
                plan_step st;
                st.kind = ST_NORM;
                st.node = j;
                st.src  = i;
                const struct ggml_tensor * x  = n->src[0];
                const int                  wt = gemv_consumer_type(g, gi, j);
                const bool row_ok = x->nb[0] == 4 && x->ne[0] % 256 == 0 && x->ne[0] <= 16384 &&
                                    is_f32_vector(m->src[1], x->ne[0]) && rows_contiguous_f32(m) &&
                                    ((uintptr_t) x->data | x->nb[1] | x->nb[2] | x->nb[3]) % 16 == 0;
                if (wt && row_ok) {
                    st.vec_wtype = wt;
                    st.slot_out  = new_slot(wt, x->ne[0], ggml_nrows(x));
                    st.write_f32 = is_output(m);
                    slot_of[(size_t) j]    = st.slot_out;
                    slot_wtype[(size_t) j] = wt;
                }
                absorbed[(size_t) i] = 1;
                absorbed[(size_t) j] = 1;
                add_pending(st);
                continue;
            }
        }
        if (n->op == GGML_OP_GLU && n->op_params[0] == GGML_GLU_OP_SWIGLU && rows_contiguous_f32(n) && !no_glu_epi) {
            // the SwiGLU (and the down GEMVs' activation quantisation) in the
            // epilogue of the norm-fused gate_up GEMV that produces its input
            const struct ggml_tensor * a = n->src[0];
            const int                  p = node_index(gi, a);
            const int64_t              F = n->ne[0], M = ggml_nrows(n);
            bool only_views = p >= 0 && p < i;  // the fused step runs at p and writes the SwiGLU's outputs then
            for (int t = p + 1; only_views && t < i; t++) {
                only_views = is_noop(ggml_graph_node(g, t)->op);
            }
            // BF16: every consumer a BF16 decode GEMV, the SwiGLU rows written in f32
            bool bf_cons = !gi.consumers[(size_t) i].empty() && n->op_params[1] == 0;
            for (int ci : gi.consumers[(size_t) i]) {
                const struct ggml_tensor * cm = ggml_graph_node(g, ci);
                bf_cons = bf_cons && cm->op == GGML_OP_MUL_MAT && cm->src[1] == n && cm->src[0] != n &&
                          mm_is_bf16_dec(cm);
            }
            if (!n->src[1] && only_views && step_at[(size_t) p] >= 0 && gi.uses[(size_t) p] == 1 && bf_cons &&
                !is_output(a) && a->op == GGML_OP_MUL_MAT && a->ne[0] == 2 * F && ggml_nrows(a) == M &&
                a->src[0]->type == GGML_TYPE_BF16) {
                plan_step & ms = pending[(size_t) step_at[(size_t) p]];
                if (ms.kind == ST_MM && ms.node == p && ms.norm >= 0 && ms.add < 0 && ms.glu < 0 &&
                    mmhip_mul_mat_bf16_dec_supported(a->ne[0], a->src[0]->ne[0], M, 1)) {
                    ms.glu_epi           = i;
                    ms.slot_out          = -1;
                    ms.write_f32         = true;
                    absorbed[(size_t) i] = 1;
                    continue;
                }
            }
            if (!n->src[1] && only_views && step_at[(size_t) p] >= 0 && gi.uses[(size_t) p] == 1 &&
                !is_output(a) && a->op == GGML_OP_MUL_MAT && a->ne[0] == 2 * F && ggml_nrows(a) == M &&
                gemv_consumer_type(g, gi, i) == GGML_TYPE_Q8_0) {
                plan_step & ms = pending[(size_t) step_at[(size_t) p]];
                if (ms.kind == ST_MM && ms.node == p && ms.norm >= 0 && ms.add < 0 && ms.glu < 0 &&
                    mmhip_rms_norm_mul_mat_glu_supported(a->src[0]->type, a->ne[0], a->src[0]->ne[0], M)) {
                    ms.glu_epi             = i;
                    ms.slot_out            = new_slot(GGML_TYPE_Q8_0, F, M);
                    ms.write_f32           = is_output(n);
                    slot_of[(size_t) i]    = ms.slot_out;
                    slot_wtype[(size_t) i] = GGML_TYPE_Q8_0;
                    absorbed[(size_t) i]   = 1;
                    continue;
                }
            }
        }
        if (n->op == GGML_OP_GLU && n->op_params[0] == GGML_GLU_OP_SWIGLU && rows_contiguous_f32(n) && !no_glu_mm &&
            glu_into_gemvs(g, gi, i)) {
            glu_mm[(size_t) i]   = 1;
            absorbed[(size_t) i] = 1;
            continue;
        }
        if (n->op == GGML_OP_GLU && n->op_params[0] == GGML_GLU_OP_SWIGLU && rows_contiguous_f32(n)) {
            const struct ggml_tensor * a  = n->src[0];
            const int                  wt = gemv_consumer_type(g, gi, i);
            const int64_t              F  = n->ne[0];
            const bool a_ok = a->nb[0] == 4 && a->nb[2] == a->nb[1] * (size_t) a->ne[1] &&
                              a->nb[3] == a->nb[2] * (size_t) a->ne[2] && a->nb[1] % 16 == 0 &&
                              ((uintptr_t) a->data) % 16 == 0;
            const struct ggml_tensor * b    = n->src[1];
            const bool                 b_ok = !b || (b->nb[0] == 4 && ggml_is_contiguous(b) && ((uintptr_t) b->data) % 16 == 0);
            if (wt && F % 256 == 0 && a_ok && b_ok) {
                plan_step st;
                st.kind      = ST_SWIGLU_Q;
                st.node      = i;
                st.vec_wtype = wt;
                st.slot_out  = new_slot(wt, F, ggml_nrows(n));
                st.write_f32 = is_output(n);
                slot_of[(size_t) i]    = st.slot_out;
                slot_wtype[(size_t) i] = wt;
                absorbed[(size_t) i]   = 1;
                add_pending(st);
                continue;
            }
        }
        // SWIGLU over the two halves of a bias GEMM's output (the DiT's ff_in,
        // src/dit.h:236-242): the CONTs of the halves and the SWIGLU run in the
        // GEMM's epilogue, the product itself is never written; when only GEMMs
        // read the SwiGLU rows they go out in f16 (their activation format)
        if (n->op == GGML_OP_GLU && n->op_params[0] == GGML_GLU_OP_SWIGLU && n->src[1] && rows_contiguous_f32(n) &&
            !no_glu_epi) {
            const int64_t              F    = n->ne[0];
            const struct ggml_tensor * view[2] = { nullptr, nullptr };  // gate, value
            int                        cont[2] = { -1, -1 };
            bool                       ok      = true;
            for (int k = 0; k < 2 && ok; k++) {
                const struct ggml_tensor * c  = n->src[k];
                const int                  ci = node_index(gi, c);
                ok = ci >= 0 && c->op == GGML_OP_CONT && gi.uses[(size_t) ci] == 1 && !is_output(c) &&
                     c->type == GGML_TYPE_F32 && ggml_are_same_shape(c, n);
                if (ok) {
                    const struct ggml_tensor * v  = c->src[0];
                    const int                  vi = node_index(gi, v);
                    ok = v->op == GGML_OP_VIEW && v->view_src && v->type == GGML_TYPE_F32 && v->nb[0] == 4 &&
                         ggml_are_same_shape(v, n) && (vi < 0 || (gi.uses[(size_t) vi] == 1 && !is_output(v)));
                    view[k] = v;
                    cont[k] = ci;
                }
            }
            const struct ggml_tensor * ff = ok ? view[0]->view_src : nullptr;
            const int                  fi = ff ? node_index(gi, ff) : -1;
            ok = ok && ff == view[1]->view_src && fi >= 0 && fi < i && step_at[(size_t) fi] >= 0 && !is_output(ff) &&
                 ff->type == GGML_TYPE_F32 && ggml_is_contiguous(ff) && ff->ne[0] == 2 * F &&
                 ggml_nrows(ff) == ggml_nrows(n) && view[0]->nb[1] == ff->nb[1] && view[1]->nb[1] == ff->nb[1] &&
                 view[0]->nb[2] == ff->nb[2] && view[1]->nb[2] == ff->nb[2] && view[0]->nb[3] == ff->nb[3] &&
                 view[1]->nb[3] == ff->nb[3] && gi.consumers[(size_t) fi].size() == 2;
            int swapped = 0;
            if (ok) {
                const size_t hb = (size_t) F * sizeof(float);
                ok = (view[0]->view_offs == hb && view[1]->view_offs == 0) ||
                     (view[0]->view_offs == 0 && view[1]->view_offs == hb);
                swapped = view[0]->view_offs == 0 ? 1 : 0;  // gate rows first
            }
            if (ok) {
                plan_step & gs = pending[(size_t) step_at[(size_t) fi]];
                ok = gs.kind == ST_GEMM && gs.node == fi && gs.add < 0 && gs.glu_epi < 0 &&
                     quiet_between(fi, i, cont[0], cont[1]);
                if (ok) {
                    const struct ggml_tensor * mmn = ggml_graph_node(g, gs.mm);
                    const struct ggml_tensor * x   = mmn->src[1];
                    const struct ggml_tensor * w   = mmn->src[0];
                    ok = w->ne[1] == 2 * F && !overlaps(n, w) && (gs.slot_in >= 0 || !overlaps(n, x)) &&
                         (gs.bias < 0 || !overlaps(n, ggml_graph_node(g, gs.bias)->src[gs.bias_src]));
                }
                if (ok) {
                    bool only_gemm = !is_output(n) && !gi.consumers[(size_t) i].empty() && F % 64 == 0;
                    for (int c : gi.consumers[(size_t) i]) {
                        const struct ggml_tensor * mm = ggml_graph_node(g, c);
                        only_gemm = only_gemm && mm->op == GGML_OP_MUL_MAT && mm->src[1] == n && mm->src[0] != n &&
                                    !mm_is_gemv(mm) && supports_mul_mat(mm) && ggml_is_contiguous(mm);
                    }
                    gs.glu_epi     = i;
                    gs.glu_swapped = swapped;
                    gs.write_f32   = !only_gemm;
                    if (only_gemm) {
                        gs.slot_out = (int64_t) plan.slot_bytes;
                        plan.slot_bytes += ((size_t) ggml_nelements(n) * 2 + 255) / 256 * 256;
                        f16_slot_of[(size_t) i] = gs.slot_out;
                    }
                    absorbed[(size_t) cont[0]] = 1;
                    absorbed[(size_t) cont[1]] = 1;
                    absorbed[(size_t) i]       = 1;
                    continue;
                }
            }
        }
        // SWIGLU reading its gate / value straight from the views the CONTs
        // before it copy (the DiT's value / gate halves of ff_in, src/dit.h:
        // 239-242): the CONTs are not run
        if (n->op == GGML_OP_GLU && n->op_params[0] == GGML_GLU_OP_SWIGLU && n->src[1] && ggml_is_contiguous(n)) {
            int cont_of[2] = { -1, -1 };
            for (int k = 0; k < 2; k++) {
                const struct ggml_tensor * c  = n->src[k];
                const int                  ci = node_index(gi, c);
                if (ci >= 0 && c->op == GGML_OP_CONT && gi.uses[(size_t) ci] == 1 && !is_output(c) &&
                    c->src[0]->type == GGML_TYPE_F32 && c->src[0]->nb[0] == 4 && !overlaps(n, c->src[0])) {
                    cont_of[k] = ci;
                }
            }
            const int lo = std::min(cont_of[0] >= 0 ? cont_of[0] : i, cont_of[1] >= 0 ? cont_of[1] : i);
            if ((cont_of[0] >= 0 || cont_of[1] >= 0) && quiet_between(lo, i, cont_of[0], cont_of[1])) {
                plan_step st;
                st.kind = ST_GLU_V;
                st.node = i;
                st.src  = cont_of[0];
                st.mul  = cont_of[1];
                for (int k = 0; k < 2; k++) {
                    if (cont_of[k] >= 0) {
                        absorbed[(size_t) cont_of[k]] = 1;
                    }
                }
                add_pending(st);
                continue;
            }
        }
        if (n->op == GGML_OP_CPY && plan_rope_h(g, gi, i, step_at, absorbed)) {
            plan_step st;
            st.kind = ST_ROPE_H;
            st.node = i;
            st.src  = node_index(gi, n->src[0]->src[0]);
            absorbed[(size_t) st.src] = 1;
            add_pending(st);
            continue;
        }
        if (n->op == GGML_OP_CONT) {
            plan_step st;
            if (!no_sattn && plan_small_attn(g, gi, i, st, absorbed)) {
                add_pending(st);
                continue;
            }
            if (plan_head(g, gi, i, st, absorbed)) {
                add_pending(st);
                continue;
            }
        }
        if (n->op == GGML_OP_RESHAPE && !absorbed[(size_t) i]) {
            plan_step st;
            if (plan_head(g, gi, i, st, absorbed)) {
                add_pending(st);
                continue;
            }
        }
        // LayerNorm with its weight MUL and bias ADD (dit_layer_norm): one kernel
        if (n->op == GGML_OP_NORM && gi.uses[(size_t) i] == 1 && !is_output(n) && rows_contiguous_f32(n)) {
            const int                  j  = gi.cons[(size_t) i];
            const struct ggml_tensor * m  = ggml_graph_node(g, j);
            const int                  wi = m->op == GGML_OP_MUL ? add_row_vector(m, n) : -1;
            if (wi >= 0 && node_index(gi, m->src[wi]) < j && gi.uses[(size_t) j] == 1 && !is_output(m)) {
                const int                  k  = gi.cons[(size_t) j];
                const struct ggml_tensor * a  = ggml_graph_node(g, k);
                const int                  bi = a->op == GGML_OP_ADD ? add_row_vector(a, m) : -1;
                if (bi >= 0 && node_index(gi, a->src[bi]) < k && ggml_is_contiguous(a) && quiet_between(i, k, j, -1)) {
                    plan_step st;
                    st.kind     = ST_LN;
                    st.node     = k;
                    st.src      = i;
                    st.mul      = j;
                    st.bias     = k;
                    st.bias_src = bi;
                    st.add_res  = wi;  // the MUL's weight operand
                    // feeding only GEMMs (the DiT's Q/K/V and ff_in projections): the
                    // rows go out in f16, the GEMMs' activation format, and not in f32
                    bool only_gemm = !is_output(a) && !gi.consumers[(size_t) k].empty() && (a->ne[0] % 64) == 0;
                    for (int c : gi.consumers[(size_t) k]) {
                        const struct ggml_tensor * mm = ggml_graph_node(g, c);
                        only_gemm = only_gemm && mm->op == GGML_OP_MUL_MAT && mm->src[1] == a && mm->src[0] != a &&
                                    !mm_is_gemv(mm) && supports_mul_mat(mm) && ggml_is_contiguous(mm);
                    }
                    if (only_gemm) {
                        st.slot_out  = (int64_t) plan.slot_bytes;
                        plan.slot_bytes += (ggml_nelements(a) * 2 + 255) / 256 * 256;
                        st.write_f32 = false;
                        f16_slot_of[(size_t) k] = st.slot_out;
                    }
                    absorbed[(size_t) i] = 1;
                    absorbed[(size_t) j] = 1;
                    absorbed[(size_t) k] = 1;
                    add_pending(st);
                    continue;
                }
            }
        }
        // GEMM with the bias ADD and / or residual ADD that follow it in its store
        if (n->op == GGML_OP_MUL_MAT && !mm_is_gemv(n) && supports_mul_mat(n) && ggml_is_contiguous(n)) {
            plan_step st;
            st.kind  = ST_GEMM;
            st.node  = i;
            st.mm    = i;
            int  cur = i;
            const int xp = node_index(gi, n->src[1]);
            if (xp >= 0 && f16_slot_of[(size_t) xp] >= 0) {
                st.slot_in = f16_slot_of[(size_t) xp];  // activations already in f16
            }
            auto single = [&](int t) { return gi.uses[(size_t) t] == 1 && !is_output(ggml_graph_node(g, t)); };
            if (single(cur)) {
                const int                  j  = gi.cons[(size_t) cur];
                const struct ggml_tensor * ad = ggml_graph_node(g, j);
                const int                  bi = ad->op == GGML_OP_ADD ? add_row_vector(ad, n) : -1;
                if (bi >= 0 && node_index(gi, ad->src[bi]) < j && ggml_is_contiguous(ad) && quiet_between(i, j, -1, -1)) {
                    st.bias     = j;
                    st.bias_src = bi;
                    cur         = j;
                }
            }
            if (single(cur)) {
                const int                  j   = gi.cons[(size_t) cur];
                const struct ggml_tensor * c_  = ggml_graph_node(g, cur);
                const struct ggml_tensor * ad  = ggml_graph_node(g, j);
                const int                  oth = ad->op == GGML_OP_ADD ? (ad->src[0] == c_ ? 1 : ad->src[1] == c_ ? 0 : -1) : -1;
                if (oth >= 0 && ad->src[oth] != c_) {
                    const struct ggml_tensor * r = ad->src[oth];
                    if (r->type == GGML_TYPE_F32 && ggml_are_same_shape(r, n) && ggml_are_same_shape(ad, n) &&
                        ggml_is_contiguous(ad) && mm_collapsible(r) && node_index(gi, r) < j &&
                        quiet_between(i, j, st.bias, -1)) {
                        st.add     = j;
                        st.add_res = oth;
                        cur        = j;
                    }
                }
            }
            if (cur == i) {
                // more MUL_MATs of the same activations with the same weight shape
                // (the DiT's q / k / v, src/dit.h:197-199) join this launch; their
                // outputs are written here, ahead of their own position
                int nm = 0;
                for (int j = i + 1; j < gi.nn && nm < 2; j++) {
                    const struct ggml_tensor * o = ggml_graph_node(g, j);
                    if (o->op != GGML_OP_MUL_MAT || o->src[1] != n->src[1] || absorbed[(size_t) j] ||
                        o->src[0]->type != n->src[0]->type || o->src[0]->ne[0] != n->src[0]->ne[0] ||
                        o->src[0]->ne[1] != n->src[0]->ne[1] || o->src[0]->nb[1] != n->src[0]->nb[1] ||
                        !ggml_is_contiguous(o) || !ggml_are_same_shape(o, n) || n->src[0]->ne[1] % 256 != 0) {
                        continue;
                    }
                    // o is written early: its memory must hold no other tensor of
                    // the graph (a buffer the allocator shares with anything else,
                    // live before j or not, keeps the launches separate)
                    auto own = [&](const struct ggml_tensor * v) { return v == o || v->view_src == o; };
                    bool clear = !overlaps(o, n->src[0]) && !overlaps(o, o->src[0]);
                    for (int t = 0; t < gi.nn && clear; t++) {
                        const struct ggml_tensor * u = ggml_graph_node(g, t);
                        clear = own(u) || !overlaps(o, u);
                        for (int q = 0; q < GGML_MAX_SRC && clear; q++) {
                            clear = !u->src[q] || own(u->src[q]) || !overlaps(o, u->src[q]);
                        }
                    }
                    if (!clear) {
                        continue;
                    }
                    st.multi[nm++] = j;
                }
                for (int k = 0; k < nm; k++) {
                    absorbed[(size_t) st.multi[k]] = 1;
                }
            }
            if (cur != i || st.slot_in >= 0 || st.multi[0] >= 0) {
                st.node = cur;
                absorbed[(size_t) i] = 1;
                if (st.bias >= 0) {
                    absorbed[(size_t) st.bias] = 1;
                }
                if (st.add >= 0) {
                    absorbed[(size_t) st.add] = 1;
                }
                add_pending(st);
                continue;
            }
        }
        if (n->op == GGML_OP_MUL_MAT && mm_is_gemv(n)) {
            plan_step st;
            st.kind = ST_MM;
            st.node = i;
            const int p = node_index(gi, n->src[1]);
            if (p >= 0 && slot_of[(size_t) p] >= 0) {
                st.slot_in   = slot_of[(size_t) p];
                st.vec_wtype = slot_wtype[(size_t) p];
            }
            if (p >= 0 && norm_of[(size_t) p] >= 0) {
                st.norm     = norm_of[(size_t) p];
                st.norm_mul = p;
            }
            if (p >= 0 && glu_mm[(size_t) p]) {
                st.glu = p;
            }
            // residual ADD in the store
            if (gi.uses[(size_t) i] == 1 && !is_output(n)) {
                const int                  j   = gi.cons[(size_t) i];
                const struct ggml_tensor * ad  = ggml_graph_node(g, j);
                const int                  oth = ad->op == GGML_OP_ADD ? (ad->src[0] == n ? 1 : ad->src[1] == n ? 0 : -1) : -1;
                if (oth >= 0 && ad->src[oth] != n) {
                    const struct ggml_tensor * r = ad->src[oth];
                    // rows over dims 1-3 collapse to M = ne1 ne2 ne3 rows of one
                    // stride (the depth decoder's [DIM, S, B] residual stream)
                    if (r->type == GGML_TYPE_F32 && ggml_are_same_shape(r, n) && ggml_are_same_shape(ad, n) &&
                        rows_contiguous_f32(ad) && mm_collapsible(r) && ggml_is_contiguous(n) &&
                        node_index(gi, r) < j) {
                        st.add     = j;
                        st.add_res = oth;
                        st.node    = j;
                        absorbed[(size_t) j] = 1;
                    }
                }
            }
            if (st.slot_in < 0 && st.norm < 0 && st.glu < 0 && st.add >= 0 && n->src[0]->type != GGML_TYPE_BF16) {
                // quantise the activations into a slot of their own
                st.vec_wtype = n->src[0]->type;
                st.slot_in   = new_slot(st.vec_wtype, n->src[0]->ne[0], n->src[1]->ne[1]);
                st.src       = -2;  // marks "quantise first"
                if (!mm_collapsible(n->src[1])) {
                    st.add = -1, st.node = i, st.slot_in = -1, st.src = -1;
                    absorbed[(size_t) gi.cons[(size_t) i]] = 0;
                }
            }
            if (st.src == -2) {
                // activations straight from an attention output (through a
                // reshape): the attention's split combine quantises them
                const struct ggml_tensor * x  = n->src[1];
                const struct ggml_tensor * fa = x->op == GGML_OP_RESHAPE ? x->src[0] : x;
                const int                  fi = node_index(gi, fa);
                if (fa->op == GGML_OP_FLASH_ATTN_EXT && fi >= 0 && fi < i && step_at[(size_t) fi] < 0 &&
                    !absorbed[(size_t) fi] && ggml_is_contiguous(fa) && ggml_is_contiguous(x) &&
                    fa->ne[0] * fa->ne[1] == x->ne[0] && fa->ne[2] * fa->ne[3] == x->ne[1] * x->ne[2] * x->ne[3] &&
                    supports_fa(fa)) {
                    plan_step fs;
                    fs.kind      = ST_FA_Q;
                    fs.node      = fi;
                    fs.slot_out  = st.slot_in;
                    fs.vec_wtype = st.vec_wtype;
                    add_pending(fs);
                    st.src = -1;
                } else if (fi >= 0 && fi < i && step_at[(size_t) fi] >= 0 &&
                           pending[(size_t) step_at[(size_t) fi]].kind == ST_SATTN && st.vec_wtype == GGML_TYPE_Q8_0 &&
                           fa->ne[0] % 32 == 0 && ggml_is_contiguous(x) && fa->ne[0] * fa->ne[1] == x->ne[0] &&
                           fa->ne[2] * fa->ne[3] == x->ne[1] * x->ne[2] * x->ne[3]) {
                    // the one-launch manual attention quantises its output
                    // rows the same way
                    plan_step & as = pending[(size_t) step_at[(size_t) fi]];
                    as.slot_out    = st.slot_in;
                    as.vec_wtype   = st.vec_wtype;
                    st.src         = -1;
                }
            }
            // (a BF16 GEMV without a fusion too: the persistent decode kernel
            // streams the rows faster than the node's plain BF16 GEMV, e.g.
            // the lm_head behind the final norm, whose rows are a graph output)
            if (st.slot_in >= 0 || st.add >= 0 || st.norm >= 0 || st.glu >= 0 || mm_is_bf16_dec(n)) {
                absorbed[(size_t) i] = 1;
                add_pending(st);
                continue;
            }
        }
    }
    for (int i = 0; i < gi.nn; i++) {
        if (step_at[(size_t) i] >= 0) {
            plan.steps.push_back(pending[(size_t) step_at[(size_t) i]]);
        } else if (!absorbed[(size_t) i]) {
            plan_step st;
            st.node = i;
            plan.steps.push_back(st);
        }
    }
    // HEAD steps separated only by no-op nodes (views) run as one launch, at
    // the later step's position: nothing in between reads their outputs
    std::vector<plan_step> merged;
    merged.reserve(plan.steps.size());
    int last_head = -1;  // index in `merged` of the open HEAD step
    for (const plan_step & st : plan.steps) {
        const bool noop = st.kind == ST_NODE && is_noop(ggml_graph_node(g, st.node)->op);
        if (st.kind == ST_HEAD && last_head >= 0 && merged[(size_t) last_head].n_head + st.n_head <= 4 &&
            merged[(size_t) last_head].head[0].D == st.head[0].D) {
            plan_step m = merged[(size_t) last_head];
            for (int k = 0; k < st.n_head; k++) {
                m.head_end[m.n_head] = st.head_end[k];
                m.head_in[m.n_head]  = st.head_in[k];
                m.head[m.n_head++]   = st.head[k];
            }
            m.node = st.node;
            merged.erase(merged.begin() + last_head);
            merged.push_back(m);
            last_head = (int) merged.size() - 1;
            continue;
        }
        if (last_head >= 0 && st.kind == ST_MM && mm_commutes_with_head(g, merged[(size_t) last_head], st)) {
            // a GEMV that neither reads nor writes the open HEAD step's rows
            // (a separately typed V projection between the K and the V / Q
            // chains) runs before it, so the chains stay one step
            merged.insert(merged.begin() + last_head, st);
            last_head++;
            continue;
        }
        merged.push_back(st);
        if (st.kind == ST_HEAD) {
            last_head = (int) merged.size() - 1;
        } else if (!noop) {
            last_head = -1;
        }
    }
    plan.steps.swap(merged);
    // a HEAD step of Q, K and V chains followed (past views only) by the
    // decode attention they feed: one launch, the chains in its prologue
    if (getenv("GGML_MI355X_DISABLE_FA_HEAD") == nullptr && !no_fuse) {
        std::vector<plan_step> fused;
        fused.reserve(plan.steps.size());
        for (size_t x = 0; x < plan.steps.size(); x++) {
            const plan_step & st = plan.steps[x];
            size_t            y  = x + 1;
            while (y < plan.steps.size() && plan.steps[y].kind == ST_NODE &&
                   is_noop(ggml_graph_node(g, plan.steps[y].node)->op)) {
                y++;
            }
            plan_step f;
            if (st.kind == ST_HEAD && st.n_head == 3 && y < plan.steps.size() && fa_head_fuse(g, gi, st, plan.steps[y], f)) {
                for (size_t z = x + 1; z < y; z++) {
                    fused.push_back(plan.steps[z]);
                }
                fused.push_back(f);
                x = y;
                continue;
            }
            fused.push_back(st);
        }
        plan.steps.swap(fused);
    }
    return plan;
}

// Activation slots: device memory of the plan's quantised activations, kept
// by the backend (separate from the per-op workspace).
void * slots(mi_backend * c, size_t need) {
    if (need <= c->slot_size) {
        return c->slot;
    }
    if (c->capturing) {
        return nullptr;
    }
    HIP_OK(hipStreamSynchronize(c->stream));
    if (c->slot) {
        (void) hipFree(c->slot);
        drop_captured(c);
    }
    c->slot      = nullptr;
    c->slot_size = 0;
    if (!HIP_OK(hipMalloc(&c->slot, need))) {
        return nullptr;
    }
    c->slot_size = need;
    return c->slot;
}

int run_step(mi_backend * c, struct ggml_cgraph * g, const plan_step & st, char * slot) {
    hipStream_t          s = c->stream;
    struct ggml_tensor * n = ggml_graph_node(g, st.node);
    int                  rc;
    switch (st.kind) {
        case ST_NODE:
            return run_node(c, n);
        case ST_NORM: {
            const struct ggml_tensor * rn = ggml_graph_node(g, st.src);
            float                      eps;
            memcpy(&eps, &rn->op_params[0], sizeof(float));
            mmhip_view x = view_of(rn->src[0]), w = view_of(n->src[1]);
            if (st.slot_out >= 0) {
                rc = mmhip_rms_norm_quant(&x, &w, eps, st.write_f32 ? (float *) n->data : nullptr, st.vec_wtype,
                                          slot + st.slot_out, s);
            } else {
                rc = mmhip_rms_norm(&x, &w, eps, (float *) n->data, s);
            }
            break;
        }
        case ST_SWIGLU_Q: {
            mmhip_view a = view_of(n->src[0]);
            mmhip_view b;
            if (n->src[1]) {
                b = view_of(n->src[1]);
            }
            rc = mmhip_swiglu_quant(&a, n->src[1] ? &b : nullptr, n->op_params[1],
                                    st.write_f32 ? (float *) n->data : nullptr, st.vec_wtype, slot + st.slot_out, s);
            break;
        }
        case ST_HEAD:
            rc = mmhip_head_rows_n(st.head, st.n_head, s);
            break;
        case ST_SATTN: {
            const struct ggml_tensor * m1 = ggml_graph_node(g, st.mm);
            const struct ggml_tensor * sc = ggml_graph_node(g, st.mul);
            const struct ggml_tensor * dm = ggml_graph_node(g, st.bias);
            const struct ggml_tensor * vt = ggml_graph_node(g, st.src);
            float                      scale, bias;
            memcpy(&scale, &sc->op_params[0], sizeof(float));
            memcpy(&bias, &sc->op_params[1], sizeof(float));
            mmhip_view q = view_of(m1->src[1]), k = view_of(m1->src[0]), v = view_of(vt->src[0]->src[0]);
            rc = mmhip_small_attn_q(&q, &k, &v, scale, bias, dm->op_params[0], (float *) n->data,
                                    st.slot_out >= 0 ? st.vec_wtype : 0, st.slot_out >= 0 ? slot + st.slot_out : nullptr,
                                    s);
            break;
        }
        case ST_ROPE_H: {
            const struct ggml_tensor * r      = ggml_graph_node(g, st.src);
            const int                  n_dims = r->op_params[1];
            float                      base;
            memcpy(&base, &r->op_params[5], sizeof(float));
            mmhip_view x = view_of(r->src[0]), d = rope_h_dst(n);
            rc = mmhip_rope_neox_f16(&x, (const int32_t *) r->src[1]->data, n_dims, powf(base, -2.0f / (float) n_dims),
                                     &d, s);
            break;
        }
        case ST_GLU_V: {
            const struct ggml_tensor * ga = st.src >= 0 ? ggml_graph_node(g, st.src)->src[0] : n->src[0];
            const struct ggml_tensor * gb = st.mul >= 0 ? ggml_graph_node(g, st.mul)->src[0] : n->src[1];
            mmhip_view                 a = view_of(ga), b = view_of(gb);
            rc = mmhip_swiglu(&a, &b, n->op_params[1], (float *) n->data, s);
            break;
        }
        case ST_LN: {
            const struct ggml_tensor * nn = ggml_graph_node(g, st.src);
            const struct ggml_tensor * mu = ggml_graph_node(g, st.mul);
            float                      eps;
            memcpy(&eps, &nn->op_params[0], sizeof(float));
            mmhip_view x = view_of(nn->src[0]);
            rc = mmhip_norm_affine_h(&x, eps, (const float *) mu->src[st.add_res]->data,
                                     (const float *) n->src[st.bias_src]->data,
                                     st.write_f32 ? (float *) n->data : nullptr,
                                     st.slot_out >= 0 ? (void *) (slot + st.slot_out) : nullptr, s);
            break;
        }
        case ST_GEMM: {
            const struct ggml_tensor * mm = ggml_graph_node(g, st.mm);
            const struct ggml_tensor * w  = mm->src[0];
            const struct ggml_tensor * x  = mm->src[1];
            const int64_t              N = w->ne[1], K = w->ne[0], M = x->ne[1] * x->ne[2] * x->ne[3];
            const float *              bias = st.bias >= 0 ? (const float *) ggml_graph_node(g, st.bias)->src[st.bias_src]->data
                                                           : nullptr;
            const struct ggml_tensor * r  = st.add >= 0 ? ggml_graph_node(g, st.add)->src[st.add_res] : nullptr;
            if (st.multi[0] >= 0) {
                // this MUL_MAT and up to two more of the same activations in one launch
                const void * wm[3];
                float *      ym[3];
                int64_t      lm[3];
                int          nmat = 0;
                for (int k = -1; k < 2; k++) {
                    const int                  ni = k < 0 ? st.mm : st.multi[k];
                    const struct ggml_tensor * o  = ni >= 0 ? ggml_graph_node(g, ni) : nullptr;
                    if (!o) {
                        continue;
                    }
                    wm[nmat] = o->src[0]->data;
                    ym[nmat] = (float *) o->data;
                    lm[nmat] = (int64_t) (o->nb[1] / sizeof(float));
                    nmat++;
                }
                if (st.slot_in >= 0) {
                    rc = mmhip_mul_mat_multi_h(w->type, nmat, wm, N, K, (int64_t) w->nb[1], slot + st.slot_in, M,
                                               nullptr, ym, lm, s);
                    break;
                }
                const size_t ws = mmhip_mul_mat_workspace(w->type, N, K, M);
                void *       wp = ws ? workspace(c, ws) : nullptr;
                if (ws && !wp) {
                    return -1;
                }
                rc = mmhip_mul_mat_multi(w->type, nmat, wm, N, K, (int64_t) w->nb[1], (const float *) x->data,
                                         (int64_t) (x->nb[1] / sizeof(float)), M, nullptr, ym, lm, wp, ws, s);
                break;
            }
            if (st.glu_epi >= 0) {
                // the SwiGLU of the two output halves in the epilogue
                float * h  = st.write_f32 ? (float *) ggml_graph_node(g, st.glu_epi)->data : nullptr;
                void *  hh = st.slot_out >= 0 ? (void *) (slot + st.slot_out) : nullptr;
                if (st.slot_in >= 0) {
                    rc = mmhip_mul_mat_bias_swiglu_h(w->type, w->data, N, K, (int64_t) w->nb[1], slot + st.slot_in, M,
                                                     bias, st.glu_swapped, h, hh, s);
                    break;
                }
                const size_t ws = mmhip_mul_mat_workspace(w->type, N, K, M);
                void *       wp = ws ? workspace(c, ws) : nullptr;
                if (ws && !wp) {
                    return -1;
                }
                rc = mmhip_mul_mat_bias_swiglu(w->type, w->data, N, K, (int64_t) w->nb[1], (const float *) x->data,
                                               (int64_t) (x->nb[1] / sizeof(float)), M, bias, st.glu_swapped, h, hh,
                                               wp, ws, s);
                break;
            }
            if (st.slot_in >= 0) {
                const size_t hws = mmhip_mul_mat_h_workspace(w->type, N, K, M);  // split-K partial sums
                void *       hwp = hws ? workspace(c, hws) : nullptr;
                if (hws && !hwp) {
                    return -1;
                }
                rc = mmhip_mul_mat_bias_add_hw(w->type, w->data, N, K, (int64_t) w->nb[1], slot + st.slot_in, M, bias,
                                               r ? (const float *) r->data : nullptr,
                                               r ? (int64_t) (r->nb[1] / sizeof(float)) : 0, (float *) n->data, N, hwp,
                                               hws, s);
                break;
            }
            const size_t               ws = mmhip_mul_mat_workspace(w->type, N, K, M);
            void *                     wp = ws ? workspace(c, ws) : nullptr;
            if (ws && !wp) {
                return -1;
            }
            rc = mmhip_mul_mat_bias_add(w->type, w->data, N, K, (int64_t) w->nb[1], (const float *) x->data,
                                        (int64_t) (x->nb[1] / sizeof(float)), M, bias,
                                        r ? (const float *) r->data : nullptr, r ? (int64_t) (r->nb[1] / sizeof(float)) : 0,
                                        (float *) n->data, N, wp, ws, s);
            break;
        }
        case ST_FA_Q: {
            mmhip_view q = view_of(n->src[0]), k = view_of(n->src[1]), v = view_of(n->src[2]);
            mmhip_view m;
            const bool has_m = n->src[3] != nullptr;
            if (has_m) {
                m = view_of(n->src[3]);
            }
            float scale;
            memcpy(&scale, &n->op_params[0], sizeof(float));
            const size_t ws = mmhip_flash_attn_workspace(&q, &k, &v);
            void *       wp = ws ? workspace(c, ws) : nullptr;
            if (ws && !wp) {
                return -1;
            }
            if (st.n_head == 3) {
                rc = mmhip_flash_attn_ext_head(&q, &k, &v, has_m ? &m : nullptr, scale, (float *) n->data, wp, ws,
                                               st.slot_out >= 0 ? st.vec_wtype : 0,
                                               st.slot_out >= 0 ? slot + st.slot_out : nullptr, st.head, s);
            } else {
                rc = mmhip_flash_attn_ext_q(&q, &k, &v, has_m ? &m : nullptr, scale, (float *) n->data, wp, ws,
                                            st.vec_wtype, slot + st.slot_out, s);
            }
            break;
        }
        case ST_MM: {
            const struct ggml_tensor * mm = st.add >= 0 ? ggml_graph_node(g, st.add)->src[1 - st.add_res] : n;
            const struct ggml_tensor * w  = mm->src[0];
            const struct ggml_tensor * x  = mm->src[1];
            const int64_t              N = w->ne[1], K = w->ne[0], M = x->ne[1] * x->ne[2] * x->ne[3];
            if (w->type == GGML_TYPE_BF16) {
                // the BF16 decode GEMV: norm prologue, residual or SwiGLU epilogue
                const float * xp  = (const float *) x->data;
                int64_t       ldx = (int64_t) (x->nb[1] / 4);
                const float * nwp = nullptr;
                float         eps = 0.0f;
                if (st.norm >= 0) {
                    const struct ggml_tensor * rn = ggml_graph_node(g, st.norm);
                    xp                            = (const float *) rn->src[0]->data;
                    ldx                           = (int64_t) (rn->src[0]->nb[1] / 4);
                    nwp = (const float *) ggml_graph_node(g, st.norm_mul)->src[1]->data;
                    memcpy(&eps, &rn->op_params[0], sizeof(float));
                }
                const struct ggml_tensor * r   = st.add >= 0 ? ggml_graph_node(g, st.add)->src[st.add_res] : nullptr;
                const struct ggml_tensor * gn  = st.glu_epi >= 0 ? ggml_graph_node(g, st.glu_epi) : nullptr;
                float *                    yp  = gn ? (float *) gn->data : (float *) n->data;
                const int64_t              ldy = gn ? N / 2 : N;
                rc = mmhip_mul_mat_bf16_dec(w->data, N, K, (int64_t) (w->nb[1] / 2), xp, ldx, M, nwp, eps,
                                            r ? (const float *) r->data : nullptr, r ? (int64_t) (r->nb[1] / 4) : 0,
                                            gn ? 1 : 0, yp, ldy, s);
                break;
            }
            if (st.norm >= 0) {
                const struct ggml_tensor * rn  = ggml_graph_node(g, st.norm);
                const struct ggml_tensor * xr  = rn->src[0];
                const struct ggml_tensor * nwt = ggml_graph_node(g, st.norm_mul)->src[1];
                const struct ggml_tensor * r   = st.add >= 0 ? ggml_graph_node(g, st.add)->src[st.add_res] : nullptr;
                float                      eps;
                memcpy(&eps, &rn->op_params[0], sizeof(float));
                if (st.glu_epi >= 0) {
                    const struct ggml_tensor * gn = ggml_graph_node(g, st.glu_epi);
                    rc = mmhip_rms_norm_mul_mat_glu(w->type, w->data, N, K, (int64_t) w->nb[1], (const float *) xr->data,
                                                    (int64_t) (xr->nb[1] / 4), M, (const float *) nwt->data, eps,
                                                    gn->op_params[1] != 0, slot + st.slot_out,
                                                    st.write_f32 ? (float *) gn->data : nullptr, s);
                    break;
                }
                rc = mmhip_rms_norm_mul_mat(w->type, w->data, N, K, (int64_t) w->nb[1], (const float *) xr->data,
                                            (int64_t) (xr->nb[1] / 4), M, (const float *) nwt->data, eps, nullptr,
                                            r ? (const float *) r->data : nullptr, r ? (int64_t) (r->nb[1] / 4) : 0,
                                            (float *) n->data, N, s);
                break;
            }
            if (st.glu >= 0) {
                const struct ggml_tensor * gn = ggml_graph_node(g, st.glu);
                const struct ggml_tensor * r  = st.add >= 0 ? ggml_graph_node(g, st.add)->src[st.add_res] : nullptr;
                const float *              gp = nullptr;
                const float *              up = nullptr;
                int64_t                    ldg = 0, ldu = 0;
                if (!glu_rows(gn, gp, ldg, up, ldu)) {
                    rc = MMHIP_ERR_INVALID;
                    break;
                }
                rc = mmhip_swiglu_mul_mat(w->type, w->data, N, K, (int64_t) w->nb[1], gp, ldg, up, ldu, M, nullptr,
                                          r ? (const float *) r->data : nullptr, r ? (int64_t) (r->nb[1] / 4) : 0,
                                          (float *) n->data, N, s);
                break;
            }
            if (st.src == -2) {
                rc = mmhip_quantize_act(w->type, (const float *) x->data, (int64_t) (x->nb[1] / 4), K, M,
                                        slot + st.slot_in, s);
                if (rc != MMHIP_OK) {
                    break;
                }
            }
            if (st.add >= 0) {
                const struct ggml_tensor * r = ggml_graph_node(g, st.add)->src[st.add_res];
                rc = mmhip_mul_mat_q_add(w->type, w->data, N, K, (int64_t) w->nb[1], slot + st.slot_in, M,
                                         (const float *) r->data, (int64_t) (r->nb[1] / 4), (float *) n->data, N, s);
            } else {
                rc = mmhip_mul_mat_q(w->type, w->data, N, K, (int64_t) w->nb[1], slot + st.slot_in, M,
                                     (float *) n->data, N, s);
            }
            break;
        }
        default:
            return -1;
    }
    return rc == MMHIP_OK ? MMHIP_OK : (fail(n, rc), -1);
}

bool run_plan(mi_backend * c, struct ggml_cgraph * g, const graph_plan & plan) {
    char * slot = nullptr;
    if (plan.slot_bytes) {
        slot = (char *) slots(c, plan.slot_bytes);
        if (!slot) {
            return false;
        }
    }
    for (const plan_step & st : plan.steps) {
        if (run_step(c, g, st, slot) != MMHIP_OK) {
            return false;
        }
    }
    return true;
}

// Everything a graph's launches depend on, node by node: the node's address,
// op and type, data address, shape, strides and op_params (scales, top-k,
// eps, RoPE parameters are taken by value), and for each source its address
// and data address, plus shape and strides for sources that are not graph
// nodes (weights, inputs).  A graph rebuilt at the same addresses with other
// op_params (the depth decoder's cfg, src/depth-decoder.h:439-447) or other
// views therefore gets a new signature.
void signature(struct ggml_cgraph * g, std::vector<uint64_t> & sig) {
    sig.clear();
    const int nn = ggml_graph_n_nodes(g);
    sig.reserve((size_t) nn * 40);
    static_assert(sizeof(((struct ggml_tensor *) nullptr)->op_params) % sizeof(uint64_t) == 0, "op_params words");
    for (int i = 0; i < nn; i++) {
        const struct ggml_tensor * n = ggml_graph_node(g, i);
        sig.push_back((uint64_t) (uintptr_t) n);
        sig.push_back((uint64_t) n->op | ((uint64_t) n->type << 16) | ((uint64_t) (uint32_t) n->flags << 32));
        sig.push_back((uint64_t) (uintptr_t) n->data);
        for (int d = 0; d < 4; d++) {
            sig.push_back((uint64_t) n->ne[d]);
            sig.push_back((uint64_t) n->nb[d]);
        }
        uint64_t op_words[sizeof(n->op_params) / sizeof(uint64_t)];
        memcpy(op_words, n->op_params, sizeof(n->op_params));
        sig.insert(sig.end(), op_words, op_words + sizeof(n->op_params) / sizeof(uint64_t));
        for (int s = 0; s < GGML_MAX_SRC; s++) {
            const struct ggml_tensor * t = n->src[s];
            if (!t) {
                continue;
            }
            sig.push_back((uint64_t) s << 56 | (uint64_t) t->type << 48);
            sig.push_back((uint64_t) (uintptr_t) t);
            sig.push_back((uint64_t) (uintptr_t) t->data);
            if (t->op == GGML_OP_NONE) {
                for (int d = 0; d < 4; d++) {
                    sig.push_back((uint64_t) t->ne[d]);
                    sig.push_back((uint64_t) t->nb[d]);
                }
            }
        }
    }
}

mi_graph_entry * find_graph(mi_backend * c, struct ggml_cgraph * g, const std::vector<uint64_t> & sig) {
    const int    nn    = ggml_graph_n_nodes(g);
    const void * first = nn ? ggml_graph_node(g, 0) : nullptr;
    const void * last  = nn ? ggml_graph_node(g, nn - 1) : nullptr;
    for (mi_graph_entry & e : c->graphs) {
        if (e.graph == g && e.n_nodes == nn && e.first == first && e.last == last && e.sig == sig) {
            return &e;
        }
    }
    return nullptr;
}

// A new entry for graph g (the least recently used one is replaced when the
// cache is full); its plan is built here, once.
mi_graph_entry * add_graph(mi_backend * c, struct ggml_cgraph * g, std::vector<uint64_t> & sig) {
    mi_graph_entry * e = nullptr;
    if ((int) c->graphs.size() < mi_backend::GRAPH_ENTRIES) {
        c->graphs.emplace_back();
        e = &c->graphs.back();
    } else {
        e = &c->graphs[0];
        for (mi_graph_entry & x : c->graphs) {
            if (x.stamp < e->stamp) {
                e = &x;
            }
        }
        if (e->exec) {
            HIP_OK(hipStreamSynchronize(c->stream));  // a launch of it may still be queued
            (void) hipGraphExecDestroy(e->exec);
        }
        *e = mi_graph_entry();
    }
    const int nn = ggml_graph_n_nodes(g);
    e->graph     = g;
    e->n_nodes   = nn;
    e->first     = nn ? ggml_graph_node(g, 0) : nullptr;
    e->last      = nn ? ggml_graph_node(g, nn - 1) : nullptr;
    e->sig.swap(sig);
    e->plan = std::make_shared<graph_plan>(build_plan(g));
    return e;
}

// Capture the entry's launches into a HIP graph; false (nothing launched)
// when the capture or the instantiation fails.
bool capture_graph(mi_backend * c, struct ggml_cgraph * g, mi_graph_entry * e) {
    hipGraph_t graph = nullptr;
    if (!HIP_OK(hipStreamBeginCapture(c->stream, hipStreamCaptureModeRelaxed))) {
        (void) hipGetLastError();
        return false;
    }
    c->capturing     = true;
    const bool ok    = run_plan(c, g, *e->plan);
    c->capturing     = false;
    const bool ended = HIP_OK(hipStreamEndCapture(c->stream, &graph));
    if (!ok || !ended) {
        if (graph) {
            (void) hipGraphDestroy(graph);
        }
        (void) hipGetLastError();
        return false;
    }
    const bool inst = HIP_OK(hipGraphInstantiate(&e->exec, graph, nullptr, nullptr, 0));
    (void) hipGraphDestroy(graph);
    if (!inst) {
        e->exec = nullptr;
        (void) hipGetLastError();
        return false;
    }
    c->n_captures++;
    return true;
}

// f16 copies (within the budget) of the quantised weights that the graph
// multiplies at more than 16 tokens and that have none yet; the conversions
// run on the backend's stream ahead of the graph's own work.
// Copies are a cache and must not crowd out the caller's own allocations (the
// reference sizes residency by its weight buffers, src/model-store.h:81-84, :115):
// besides the process-wide budget, a copy is made only while at least half
// of the device's memory stays free after it.  The copies are device
// allocations, so the device's get_memory (hipMemGetInfo) reports them as
// used; ggml_backend_mi355x_f16_weight_bytes gives their total.
void make_f16_copies(mi_backend * c, struct ggml_cgraph * g) {
    const size_t lim  = f16_limit();
    bool         made = false;
    size_t       dev_free = 0, dev_total = 0;
    if (lim > 0 && !HIP_OK(hipMemGetInfo(&dev_free, &dev_total))) {
        return;
    }
    for (int i = 0; i < ggml_graph_n_nodes(g) && lim > 0; i++) {
        const struct ggml_tensor * n = ggml_graph_node(g, i);
        if (n->op != GGML_OP_MUL_MAT || !is_repacked(n->src[0]->type) || mm_is_gemv(n) || !supports_mul_mat(n)) {
            continue;
        }
        const struct ggml_tensor * w    = n->src[0];
        const struct ggml_tensor * base = w->view_src ? w->view_src : w;
        ggml_backend_buffer_t      wb   = base->buffer;
        if (!wb || wb->iface.free_buffer != buf_free) {
            continue;
        }
        mi_buffer * bc   = (mi_buffer *) wb->context;
        bool        have = false;
        for (const mi_f16_copy & f : bc->f16) {
            have = have || f.w == w->data;
        }
        const int64_t N = w->ne[1], K = w->ne[0];
        const size_t  bytes = mmhip_weights_f16_bytes(N, K);
        if (have || bc->device != c->dev->id || g_f16_bytes.load() + bytes > lim) {
            continue;
        }
        if (dev_free < bytes || dev_free - bytes < dev_total / 2) {
            break;
        }
        void * p = nullptr;
        if (hipMalloc(&p, bytes) != hipSuccess) {
            (void) hipGetLastError();
            break;  // out of memory: the GEMMs convert per call as before
        }
        mi_f16_copy f{ w->data, p, bytes, ggml_nbytes(w), (int) w->type, N, K, (int64_t) w->nb[1] };
        if (mmhip_weights_to_f16(f.type, f.w, N, K, f.rs, p, c->stream) != MMHIP_OK ||
            mmhip_register_weights_f16(f.w, N, K, p) != MMHIP_OK) {
            MI_LOG("f16 weight copy of %s not made: %s\n", w->name, mmhip_last_error());
            HIP_OK(hipStreamSynchronize(c->stream));
            (void) hipFree(p);
            continue;
        }
        bc->f16.push_back(f);
        g_f16_bytes.fetch_add(bytes);
        dev_free -= bytes;
        made = true;
    }
    if (made) {
        g_f16_gen.fetch_add(1);
    }
}

enum ggml_status graph_compute_inner(ggml_backend_t b, struct ggml_cgraph * g) {
    mi_backend * c = (mi_backend *) b->context;
    hipSetDevice(c->dev->id);
    if (g_poisoned_buffers.load() > 0 && graph_poisoned(g)) {
        MI_LOG("graph_compute: the graph reads or writes a buffer whose transfer failed\n");
        return GGML_STATUS_FAILED;
    }
    signature(g, c->sig_buf);
    mi_graph_entry * e = find_graph(c, g, c->sig_buf);
    if (!e) {
        // first sight: check every node, build the plan and run eagerly (this
        // sizes the workspace and opts kernels in to their LDS limits)
        for (int i = 0; i < ggml_graph_n_nodes(g); i++) {
            if (!supports(ggml_graph_node(g, i))) {
                MI_LOG("graph_compute: node %d %s (%s) is not supported\n", i, ggml_graph_node(g, i)->name,
                       ggml_op_name(ggml_graph_node(g, i)->op));
                return GGML_STATUS_FAILED;
            }
        }
        e = add_graph(c, g, c->sig_buf);
    }
    e->stamp = ++c->clock;
    e->sights++;
    if (e->sights == 3) {
        // a graph that repeats (the DiT's, once per diffusion step): f16
        // copies of the weights its token-count GEMMs multiply
        make_f16_copies(c, g);
    }
    if (e->exec && e->f16_gen != g_f16_gen.load()) {
        // weight copies appeared or went since the capture: capture again
        HIP_OK(hipStreamSynchronize(c->stream));
        (void) hipGraphExecDestroy(e->exec);
        e->exec = nullptr;
    }
    if (e->exec) {
        c->n_replays++;
        return HIP_OK(hipGraphLaunch(e->exec, c->stream)) ? GGML_STATUS_SUCCESS : GGML_STATUS_FAILED;
    }
    if (c->use_graphs && !e->no_capture && e->sights >= 2) {
        // second sight of the same graph: capture it, then launch the capture
        const uint64_t gen = g_f16_gen.load();
        if (capture_graph(c, g, e)) {
            e->f16_gen = gen;
            c->n_replays++;
            return HIP_OK(hipGraphLaunch(e->exec, c->stream)) ? GGML_STATUS_SUCCESS : GGML_STATUS_FAILED;
        }
        e->no_capture = true;
    }
    c->n_eager++;
    return run_plan(c, g, *e->plan) ? GGML_STATUS_SUCCESS : GGML_STATUS_FAILED;
}

enum ggml_status be_graph_compute(ggml_backend_t b, struct ggml_cgraph * g) {
    mi_backend * c = (mi_backend *) b->context;
    hipSetDevice(c->dev->id);
    collect_time(c);
    if (!c->ev0 && !(HIP_OK(hipEventCreate(&c->ev0)) && HIP_OK(hipEventCreate(&c->ev1)))) {
        return GGML_STATUS_FAILED;
    }
    if (!HIP_OK(hipEventRecord(c->ev0, c->stream))) {
        return GGML_STATUS_FAILED;
    }
    const enum ggml_status st = graph_compute_inner(b, g);
    if (st == GGML_STATUS_SUCCESS && HIP_OK(hipEventRecord(c->ev1, c->stream))) {
        c->ev_pending = true;
    }
    return st;
}

void be_set_async(ggml_backend_t b, struct ggml_tensor * t, const void * data, size_t off, size_t size) {
    mi_backend * c = (mi_backend *) b->context;
    if (is_repacked(t->type)) {
        HIP_OK(hipStreamSynchronize(c->stream));
        ggml_backend_tensor_set(t, data, off, size);
        return;
    }
    HIP_OK(hipMemcpyAsync((char *) t->data + off, data, size, hipMemcpyHostToDevice, c->stream));
}

void be_get_async(ggml_backend_t b, const struct ggml_tensor * t, void * data, size_t off, size_t size) {
    mi_backend * c = (mi_backend *) b->context;
    if (is_repacked(t->type)) {
        HIP_OK(hipStreamSynchronize(c->stream));
        ggml_backend_tensor_get(t, data, off, size);
        return;
    }
    HIP_OK(hipMemcpyAsync(data, (const char *) t->data + off, size, hipMemcpyDeviceToHost, c->stream));
}

ggml_guid k_guid = { { 0x6d, 0x69, 0x33, 0x35, 0x35, 0x78, 0x2d, 0x67, 0x66, 0x78, 0x39, 0x35, 0x30, 0x00, 0x01,
                       0x02 } };

const struct ggml_backend_i k_be_iface = {
    /* get_name           */ be_name,
    /* free               */ be_free,
    /* set_tensor_async   */ be_set_async,
    /* get_tensor_async   */ be_get_async,
    /* cpy_tensor_async   */ nullptr,
    /* synchronize        */ be_sync,
    /* graph_plan_create  */ nullptr,
    /* graph_plan_free    */ nullptr,
    /* graph_plan_update  */ nullptr,
    /* graph_plan_compute */ nullptr,
    /* graph_compute      */ be_graph_compute,
    /* event_record       */ nullptr,
    /* event_wait         */ nullptr,
    /* graph_optimize     */ nullptr,
};

// ---- device iface ----

mi_device * device_by_id(int id) {
    if (!g_reg) {
        return nullptr;
    }
    for (mi_device * d : g_reg->devs) {
        if (d->id == id) {
            return d;
        }
    }
    return nullptr;
}

mi_device * devctx(ggml_backend_dev_t d) {
    return (mi_device *) d->context;
}

const char * dev_name(ggml_backend_dev_t d) {
    return devctx(d)->name.c_str();
}

const char * dev_desc(ggml_backend_dev_t d) {
    return devctx(d)->desc.c_str();
}

void dev_memory(ggml_backend_dev_t d, size_t * free, size_t * total) {
    hipSetDevice(devctx(d)->id);
    if (!HIP_OK(hipMemGetInfo(free, total))) {
        *free  = 0;
        *total = 0;
    }
}

enum ggml_backend_dev_type dev_type(ggml_backend_dev_t) {
    return GGML_BACKEND_DEVICE_TYPE_GPU;
}

void dev_props(ggml_backend_dev_t d, struct ggml_backend_dev_props * p) {
    p->name        = dev_name(d);
    p->description = dev_desc(d);
    p->type        = GGML_BACKEND_DEVICE_TYPE_GPU;
    p->device_id   = nullptr;
    dev_memory(d, &p->memory_free, &p->memory_total);
    p->caps = { true, true, false, false };
}

ggml_backend_t dev_init(ggml_backend_dev_t d, const char * params) {
    (void) params;
    mi_device * dv = devctx(d);
    hipSetDevice(dv->id);
    mi_backend * c = new mi_backend();
    c->dev         = dv;
    c->graphs.reserve(mi_backend::GRAPH_ENTRIES);  // entries stay at fixed addresses
    {
        std::lock_guard<std::mutex> lk(dv->stream_mu);
        if (!dv->idle_streams.empty()) {
            c->stream = dv->idle_streams.back();
            dv->idle_streams.pop_back();
        }
    }
    if (!c->stream && !HIP_OK(hipStreamCreate(&c->stream))) {  // default priority, blocking
        delete c;
        return nullptr;
    }
    const char * e = getenv("GGML_MI355X_DISABLE_GRAPHS");
    c->use_graphs  = !(e && atoi(e) != 0);
    return new ggml_backend{ &k_guid, k_be_iface, d, c };
}

ggml_backend_buffer_type_t dev_buft(ggml_backend_dev_t d) {
    return &devctx(d)->buft;
}

ggml_backend_buffer_type_t dev_host_buft(ggml_backend_dev_t) {
    return ggml_backend_mi355x_host_buffer_type();
}

bool dev_supports_op(ggml_backend_dev_t, const struct ggml_tensor * op) {
    return supports(op);
}

bool dev_supports_buft(ggml_backend_dev_t d, ggml_backend_buffer_type_t buft) {
    return buft == &devctx(d)->buft;
}

bool dev_offload_op(ggml_backend_dev_t, const struct ggml_tensor * op) {
    // large-batch matmuls are worth moving weights for (ggml-cuda does the same)
    return op->op == GGML_OP_MUL_MAT && op->src[1] && op->src[1]->ne[1] >= 32;
}

const struct ggml_backend_device_i k_dev_iface = {
    dev_name,  dev_desc,        dev_memory,        dev_type,       dev_props, dev_init, dev_buft, dev_host_buft,
    nullptr,   dev_supports_op, dev_supports_buft, dev_offload_op, nullptr,   nullptr,  nullptr,
};

// ---- registry iface ----

const char * reg_name(ggml_backend_reg_t) {
    return GGML_MI355X_NAME;
}

size_t reg_count(ggml_backend_reg_t) {
    return g_reg ? g_reg->devs.size() : 0;
}

ggml_backend_dev_t reg_dev(ggml_backend_reg_t, size_t i) {
    return i < g_reg->gdevs.size() ? &g_reg->gdevs[i] : nullptr;
}

void * reg_proc(ggml_backend_reg_t, const char * name) {
    if (strcmp(name, "ggml_backend_mi355x_graph_stats") == 0) {
        return (void *) ggml_backend_mi355x_graph_stats;
    }
    if (strcmp(name, "ggml_backend_mi355x_gpu_time") == 0) {
        return (void *) ggml_backend_mi355x_gpu_time;
    }
    if (strcmp(name, "ggml_backend_mi355x_graph_cache_info") == 0) {
        return (void *) ggml_backend_mi355x_graph_cache_info;
    }
    if (strcmp(name, "ggml_backend_mi355x_f16_weight_bytes") == 0) {
        return (void *) ggml_backend_mi355x_f16_weight_bytes;
    }
    return nullptr;
}

const struct ggml_backend_reg_i k_reg_iface = { reg_name, reg_count, reg_dev, reg_proc };

}  // namespace

// ---------------------------------------------------------------------------
// public API

extern "C" ggml_backend_reg_t ggml_backend_mi355x_reg(void) {
    std::lock_guard<std::mutex> lock(g_reg_mu);
    if (g_reg) {
        return &g_reg->reg;
    }
    g_reg = new mi_registry();
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void) hipGetLastError();
        n = 0;
    }
    for (int i = 0; i < n; i++) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, i) != hipSuccess) {
            continue;
        }
        mi_device * d = new mi_device();
        d->id         = i;
        d->name       = std::string(GGML_MI355X_NAME) + std::to_string(i);
        d->desc       = std::string(prop.name) + " (" + prop.gcnArchName + ")";
        d->buft       = { { buft_name, buft_alloc, buft_alignment, buft_max_size, buft_alloc_size, buft_is_host },
                          nullptr,
                          d };
        g_reg->devs.push_back(d);
    }
    g_reg->reg       = { GGML_BACKEND_API_VERSION, k_reg_iface, nullptr };
    g_reg->host_buft = { { hbuft_name, hbuft_alloc, hbuft_alignment, nullptr, nullptr, hbuft_is_host },
                         nullptr,
                         nullptr };
    g_reg->gdevs.resize(g_reg->devs.size());
    for (size_t i = 0; i < g_reg->devs.size(); i++) {
        g_reg->gdevs[i]             = { k_dev_iface, &g_reg->reg, g_reg->devs[i] };
        g_reg->devs[i]->buft.device = &g_reg->gdevs[i];
    }
    return &g_reg->reg;
}

extern "C" int ggml_backend_mi355x_get_device_count(void) {
    return (int) reg_count(ggml_backend_mi355x_reg());
}

extern "C" ggml_backend_t ggml_backend_mi355x_init(int device) {
    ggml_backend_reg_t r = ggml_backend_mi355x_reg();
    if (device < 0 || (size_t) device >= reg_count(r)) {
        MI_LOG("no device %d\n", device);
        return nullptr;
    }
    return dev_init(&g_reg->gdevs[device], nullptr);
}

extern "C" bool ggml_backend_is_mi355x(ggml_backend_t backend) {
    return backend && backend->guid == &k_guid;
}

extern "C" ggml_backend_buffer_type_t ggml_backend_mi355x_buffer_type(int device) {
    ggml_backend_reg_t r = ggml_backend_mi355x_reg();
    if (device < 0 || (size_t) device >= reg_count(r)) {
        return nullptr;
    }
    return &g_reg->devs[device]->buft;
}

extern "C" ggml_backend_buffer_type_t ggml_backend_mi355x_host_buffer_type(void) {
    ggml_backend_mi355x_reg();
    return &g_reg->host_buft;
}

extern "C" void ggml_backend_mi355x_graph_stats(ggml_backend_t backend, int64_t * replays, int64_t * eager) {
    mi_backend * c = (mi_backend *) backend->context;
    *replays       = c->n_replays;
    *eager         = c->n_eager;
}

extern "C" void ggml_backend_mi355x_graph_cache_info(ggml_backend_t backend, int64_t * n_entries, int64_t * n_captured,
                                                     int64_t * n_captures) {
    mi_backend * c = (mi_backend *) backend->context;
    int64_t      k = 0;
    for (const mi_graph_entry & e : c->graphs) {
        k += e.exec != nullptr;
    }
    *n_entries  = (int64_t) c->graphs.size();
    *n_captured = k;
    *n_captures = c->n_captures;
}

extern "C" void ggml_backend_mi355x_gpu_time(ggml_backend_t backend, double * total_ms, int64_t * n_calls, int reset) {
    mi_backend * c = (mi_backend *) backend->context;
    hipSetDevice(c->dev->id);
    collect_time(c);
    *total_ms = c->gpu_ms;
    *n_calls  = c->gpu_n;
    if (reset) {
        c->gpu_ms = 0.0;
        c->gpu_n  = 0;
    }
}

extern "C" size_t ggml_backend_mi355x_f16_weight_bytes(void) {
    return g_f16_bytes.load();
}

// dynamic-loading entry points
extern "C" GGML_API ggml_backend_reg_t ggml_backend_init(void) {
    return ggml_backend_mi355x_reg();
}

extern "C" GGML_API int ggml_backend_score(void) {
    return ggml_backend_mi355x_get_device_count() > 0 ? 100 : 0;
}
