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

struct mi_device {
    int                             id;
    std::string                     name;
    std::string                     desc;
    struct ggml_backend_buffer_type buft;
};

struct mi_registry {
    std::vector<mi_device *>                 devs;
    std::vector<struct ggml_backend_device> gdevs;
    struct ggml_backend_reg                  reg;
    struct ggml_backend_buffer_type          host_buft;
};

mi_registry * g_reg = nullptr;
std::mutex    g_reg_mu;

bool is_repacked(enum ggml_type t) {
    return t == GGML_TYPE_Q8_0 || t == GGML_TYPE_Q4_K || t == GGML_TYPE_Q6_K;
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

struct mi_buffer {
    int    device;
    void * ptr;
};

void buf_free(ggml_backend_buffer_t b) {
    mi_buffer * c = (mi_buffer *) b->context;
    hipSetDevice(c->device);
    (void) hipFree(c->ptr);
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

void buf_memset(ggml_backend_buffer_t b, struct ggml_tensor * t, uint8_t value, size_t offset, size_t size) {
    mi_buffer * c = (mi_buffer *) b->context;
    hipSetDevice(c->device);
    HIP_OK(hipMemset((char *) t->data + offset, value, size));
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

void buf_set_tensor(ggml_backend_buffer_t b, struct ggml_tensor * t, const void * data, size_t offset, size_t size) {
    mi_buffer * c = (mi_buffer *) b->context;
    hipSetDevice(c->device);
    if (is_repacked(t->type)) {
        if (!quant_rows_io(t, offset, size, data, nullptr)) {
            abort();
        }
        return;
    }
    HIP_OK(hipMemcpy((char *) t->data + offset, data, size, hipMemcpyHostToDevice));
}

void buf_get_tensor(ggml_backend_buffer_t b, const struct ggml_tensor * t, void * data, size_t offset, size_t size) {
    mi_buffer * c = (mi_buffer *) b->context;
    hipSetDevice(c->device);
    if (is_repacked(t->type)) {
        if (!quant_rows_io(t, offset, size, nullptr, data)) {
            abort();
        }
        return;
    }
    HIP_OK(hipMemcpy(data, (const char *) t->data + offset, size, hipMemcpyDeviceToHost));
}

bool buf_cpy_tensor(ggml_backend_buffer_t b, const struct ggml_tensor * src, struct ggml_tensor * dst) {
    // same layout on both sides: device-to-device copy of the bytes
    ggml_backend_buffer_t sb = src->view_src ? src->view_src->buffer : src->buffer;
    if (!sb || sb->iface.free_buffer != buf_free || src->type != dst->type) {
        return false;
    }
    mi_buffer * c = (mi_buffer *) b->context;
    hipSetDevice(c->device);
    return HIP_OK(hipMemcpy(dst->data, src->data, ggml_nbytes(src), hipMemcpyDeviceToDevice));
}

void buf_clear(ggml_backend_buffer_t b, uint8_t value) {
    mi_buffer * c = (mi_buffer *) b->context;
    hipSetDevice(c->device);
    HIP_OK(hipMemset(c->ptr, value, b->size));
    HIP_OK(hipDeviceSynchronize());
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

struct mi_graph_cache {
    std::vector<uint64_t> sig;        // signature of the captured graph
    std::vector<uint64_t> seen_sig;   // signature of the last eager run
    hipGraphExec_t        exec = nullptr;
};

struct mi_backend {
    mi_device *    dev;
    hipStream_t    stream = nullptr;
    void *         ws     = nullptr;
    size_t         ws_size = 0;
    bool           capturing = false;
    bool           use_graphs = true;
    mi_graph_cache cache;
    int64_t        n_replays = 0;
    int64_t        n_eager   = 0;
};

const char * be_name(ggml_backend_t b) {
    return ((mi_backend *) b->context)->dev->name.c_str();
}

void be_free(ggml_backend_t b) {
    mi_backend * c = (mi_backend *) b->context;
    hipSetDevice(c->dev->id);
    if (c->cache.exec) {
        (void) hipGraphExecDestroy(c->cache.exec);
    }
    if (c->ws) {
        (void) hipFree(c->ws);
    }
    (void) hipStreamDestroy(c->stream);
    delete c;
    delete b;
}

void be_sync(ggml_backend_t b) {
    mi_backend * c = (mi_backend *) b->context;
    HIP_OK(hipStreamSynchronize(c->stream));
}

// Workspace large enough for `need` bytes; returns nullptr when it would have
// to grow during a capture (the caller then abandons the capture).
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
           op->src[1]->type == GGML_TYPE_I32 && ggml_is_contiguous(op->src[1]) && op->src[0]->ne[3] == 1;
}

bool is_f32_or_f16(enum ggml_type t) {
    return t == GGML_TYPE_F32 || t == GGML_TYPE_F16;
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
            return supports_mul_mat(op);
        case GGML_OP_FLASH_ATTN_EXT:
            return supports_fa(op);
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
            return is_f32_or_f16(op->src[0]->type) && is_f32_or_f16(op->type);
        case GGML_OP_GET_ROWS:
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

int run_node(mi_backend * c, struct ggml_cgraph * g, int i, const std::vector<int> & uses) {
    struct ggml_tensor * n = ggml_graph_node(g, i);
    hipStream_t          s = c->stream;
    int                  rc = MMHIP_OK;
    switch (n->op) {
        case GGML_OP_NONE:
        case GGML_OP_RESHAPE:
        case GGML_OP_VIEW:
        case GGML_OP_PERMUTE:
        case GGML_OP_TRANSPOSE:
            return 1;
        case GGML_OP_MUL_MAT:
            return run_mul_mat(c, n) ? 1 : -1;
        case GGML_OP_FLASH_ATTN_EXT:
            return run_fa(c, n) ? 1 : -1;
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
            // fuse with the next node when it multiplies this result (only use)
            if (i + 1 < ggml_graph_n_nodes(g)) {
                struct ggml_tensor * nx = ggml_graph_node(g, i + 1);
                if (nx->op == GGML_OP_MUL && nx->src[0] == n && uses[i] == 1 &&
                    !(n->flags & GGML_TENSOR_FLAG_OUTPUT) && nx->src[1]->type == GGML_TYPE_F32 &&
                    ggml_are_same_shape(nx, n)) {
                    mmhip_view w = view_of(nx->src[1]);
                    rc           = mmhip_rms_norm(&x, &w, eps, (float *) nx->data, s);
                    return rc == MMHIP_OK ? 2 : (fail(n, rc), -1);
                }
            }
            rc = mmhip_rms_norm(&x, nullptr, eps, (float *) n->data, s);
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
        default:
            MI_LOG("unsupported node %s (%s)\n", n->name, ggml_op_name(n->op));
            return -1;
    }
    return rc == MMHIP_OK ? 1 : (fail(n, rc), -1);
}

bool run_graph(mi_backend * c, struct ggml_cgraph * g) {
    const int                                     nn = ggml_graph_n_nodes(g);
    std::vector<int>                              uses(nn, 0);
    std::unordered_map<const ggml_tensor *, int> index;
    index.reserve((size_t) nn * 2);
    for (int i = 0; i < nn; i++) {
        struct ggml_tensor * n = ggml_graph_node(g, i);
        for (int s = 0; s < GGML_MAX_SRC; s++) {
            if (n->src[s]) {
                auto it = index.find(n->src[s]);
                if (it != index.end()) {
                    uses[it->second]++;
                }
            }
        }
        index[n] = i;
    }
    for (int i = 0; i < nn;) {
        const int step = run_node(c, g, i, uses);
        if (step < 0) {
            return false;
        }
        i += step;
    }
    return true;
}

std::vector<uint64_t> signature(struct ggml_cgraph * g) {
    std::vector<uint64_t> sig;
    const int             nn = ggml_graph_n_nodes(g);
    sig.reserve((size_t) nn * 8);
    for (int i = 0; i < nn; i++) {
        const struct ggml_tensor * n = ggml_graph_node(g, i);
        sig.push_back((uint64_t) (uintptr_t) n);
        sig.push_back((uint64_t) n->op);
        sig.push_back((uint64_t) (uintptr_t) n->data);
        for (int d = 0; d < 4; d++) {
            sig.push_back((uint64_t) n->ne[d]);
        }
        for (int s = 0; s < GGML_MAX_SRC; s++) {
            if (n->src[s]) {
                sig.push_back((uint64_t) (uintptr_t) n->src[s]->data);
            }
        }
    }
    return sig;
}

enum ggml_status be_graph_compute(ggml_backend_t b, struct ggml_cgraph * g) {
    mi_backend * c = (mi_backend *) b->context;
    hipSetDevice(c->dev->id);
    for (int i = 0; i < ggml_graph_n_nodes(g); i++) {
        if (!supports(ggml_graph_node(g, i))) {
            MI_LOG("graph_compute: node %d %s (%s) is not supported\n", i, ggml_graph_node(g, i)->name,
                   ggml_op_name(ggml_graph_node(g, i)->op));
            return GGML_STATUS_FAILED;
        }
    }
    if (!c->use_graphs) {
        c->n_eager++;
        return run_graph(c, g) ? GGML_STATUS_SUCCESS : GGML_STATUS_FAILED;
    }
    std::vector<uint64_t> sig = signature(g);
    if (c->cache.exec && sig == c->cache.sig) {
        c->n_replays++;
        return HIP_OK(hipGraphLaunch(c->cache.exec, c->stream)) ? GGML_STATUS_SUCCESS : GGML_STATUS_FAILED;
    }
    if (sig != c->cache.seen_sig) {
        // first sight: run eagerly (sizes the workspace, opts kernels in to
        // their LDS limits) and remember the graph
        c->cache.seen_sig = std::move(sig);
        c->n_eager++;
        return run_graph(c, g) ? GGML_STATUS_SUCCESS : GGML_STATUS_FAILED;
    }
    // second sight of the same graph: capture it
    hipGraph_t graph = nullptr;
    if (!HIP_OK(hipStreamBeginCapture(c->stream, hipStreamCaptureModeRelaxed))) {
        return GGML_STATUS_FAILED;
    }
    c->capturing  = true;
    const bool ok = run_graph(c, g);
    c->capturing  = false;
    const bool ended = HIP_OK(hipStreamEndCapture(c->stream, &graph));
    if (!ok || !ended) {
        if (graph) {
            (void) hipGraphDestroy(graph);
        }
        (void) hipGetLastError();
        c->n_eager++;
        return run_graph(c, g) ? GGML_STATUS_SUCCESS : GGML_STATUS_FAILED;
    }
    if (c->cache.exec) {
        (void) hipGraphExecDestroy(c->cache.exec);
        c->cache.exec = nullptr;
    }
    const bool inst = HIP_OK(hipGraphInstantiate(&c->cache.exec, graph, nullptr, nullptr, 0));
    (void) hipGraphDestroy(graph);
    if (!inst) {
        c->cache.exec = nullptr;
        c->n_eager++;
        return run_graph(c, g) ? GGML_STATUS_SUCCESS : GGML_STATUS_FAILED;
    }
    c->cache.sig = c->cache.seen_sig;
    c->n_replays++;
    return HIP_OK(hipGraphLaunch(c->cache.exec, c->stream)) ? GGML_STATUS_SUCCESS : GGML_STATUS_FAILED;
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
    if (!HIP_OK(hipStreamCreate(&c->stream))) {  // default priority, blocking
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

// dynamic-loading entry points
extern "C" GGML_API ggml_backend_reg_t ggml_backend_init(void) {
    return ggml_backend_mi355x_reg();
}

extern "C" GGML_API int ggml_backend_score(void) {
    return ggml_backend_mi355x_get_device_count() > 0 ? 100 : 0;
}
