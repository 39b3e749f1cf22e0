// ggml_core.cpp - a restated subset of ggml-base (context, tensors, views, the
// graph-builder ops used on minimaxmusic.cpp's hot path, graphs, the backend
// registry / buffer / tensor API and a graph allocator).
//
// ggml is not present in the reference tree (un-vendored submodule,
// .gitmodules:1-3), so this library stands in for libggml-base in this build:
// it lets the MI355X backend be built, tested and benchmarked behind the same
// C interface the reference calls (src/backend.h, src/static-graph.h,
// src/qwen3-lm.h:645-934).  Semantics follow upstream ggml by name; the graph
// allocator is simpler (no memory reuse between intermediate tensors).
#include <dlfcn.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <vector>

#include "ggml-backend-impl.h"
#include "ggml-backend.h"
#include "ggml.h"

// ---------------------------------------------------------------------------
// logging

static ggml_log_callback g_log_cb   = nullptr;
static void *            g_log_user = nullptr;

extern "C" void ggml_log_set(ggml_log_callback cb, void * user) {
    g_log_cb   = cb;
    g_log_user = user;
}

static void core_log(enum ggml_log_level level, const char * fmt, ...) {
    char    buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    if (g_log_cb) {
        g_log_cb(level, buf, g_log_user);
    } else {
        fputs(buf, stderr);
    }
}

#define CORE_ABORT(...)                                    \
    do {                                                   \
        core_log(GGML_LOG_LEVEL_ERROR, __VA_ARGS__);       \
        abort();                                           \
    } while (0)
#define CORE_ASSERT(x)                                                                  \
    do {                                                                                \
        if (!(x)) {                                                                     \
            CORE_ABORT("ggml core: %s:%d: assertion failed: %s\n", __FILE__, __LINE__, #x); \
        }                                                                               \
    } while (0)

extern "C" void ggml_abort(const char * file, int line, const char * fmt, ...) {
    char    buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    core_log(GGML_LOG_LEVEL_ERROR, "%s:%d: %s\n", file, line, buf);
    abort();
}

// ---------------------------------------------------------------------------
// scalars

extern "C" float ggml_fp16_to_fp32(ggml_fp16_t h) {
    _Float16 v;
    memcpy(&v, &h, 2);
    return (float) v;
}

extern "C" ggml_fp16_t ggml_fp32_to_fp16(float f) {
    const _Float16 v = (_Float16) f;  // round to nearest even
    ggml_fp16_t    h;
    memcpy(&h, &v, 2);
    return h;
}

extern "C" void ggml_fp16_to_fp32_row(const ggml_fp16_t * x, float * y, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        y[i] = ggml_fp16_to_fp32(x[i]);
    }
}

extern "C" void ggml_fp32_to_fp16_row(const float * x, ggml_fp16_t * y, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        y[i] = ggml_fp32_to_fp16(x[i]);
    }
}

extern "C" void ggml_bf16_to_fp32_row(const ggml_bf16_t * x, float * y, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        const uint32_t u = (uint32_t) x[i].bits << 16;
        memcpy(&y[i], &u, 4);
    }
}

// ---------------------------------------------------------------------------
// types

struct type_info {
    const char * name;
    int64_t      blck;
    size_t       size;
    bool         quantized;
};

static type_info tinfo(enum ggml_type t) {
    switch (t) {
        case GGML_TYPE_F32: return { "f32", 1, 4, false };
        case GGML_TYPE_F16: return { "f16", 1, 2, false };
        case GGML_TYPE_BF16: return { "bf16", 1, 2, false };
        case GGML_TYPE_Q4_0: return { "q4_0", 32, 18, true };
        case GGML_TYPE_Q4_1: return { "q4_1", 32, 20, true };
        case GGML_TYPE_Q5_0: return { "q5_0", 32, 22, true };
        case GGML_TYPE_Q5_1: return { "q5_1", 32, 24, true };
        case GGML_TYPE_Q8_0: return { "q8_0", 32, 34, true };
        case GGML_TYPE_Q8_1: return { "q8_1", 32, 36, true };
        case GGML_TYPE_Q2_K: return { "q2_K", 256, 84, true };
        case GGML_TYPE_Q3_K: return { "q3_K", 256, 110, true };
        case GGML_TYPE_Q4_K: return { "q4_K", 256, 144, true };
        case GGML_TYPE_Q5_K: return { "q5_K", 256, 176, true };
        case GGML_TYPE_Q6_K: return { "q6_K", 256, 210, true };
        case GGML_TYPE_Q8_K: return { "q8_K", 256, 292, true };
        case GGML_TYPE_I8: return { "i8", 1, 1, false };
        case GGML_TYPE_I16: return { "i16", 1, 2, false };
        case GGML_TYPE_I32: return { "i32", 1, 4, false };
        case GGML_TYPE_I64: return { "i64", 1, 8, false };
        case GGML_TYPE_F64: return { "f64", 1, 8, false };
        default: return { "unknown", 1, 0, false };
    }
}

extern "C" int64_t ggml_blck_size(enum ggml_type t) {
    return tinfo(t).blck;
}

extern "C" size_t ggml_type_size(enum ggml_type t) {
    return tinfo(t).size;
}

extern "C" size_t ggml_row_size(enum ggml_type t, int64_t ne) {
    CORE_ASSERT(ne % ggml_blck_size(t) == 0);
    return ggml_type_size(t) * (size_t) (ne / ggml_blck_size(t));
}

extern "C" const char * ggml_type_name(enum ggml_type t) {
    return tinfo(t).name;
}

extern "C" bool ggml_is_quantized(enum ggml_type t) {
    return tinfo(t).quantized;
}

extern "C" const char * ggml_op_name(enum ggml_op op) {
    switch (op) {
        case GGML_OP_NONE: return "NONE";
        case GGML_OP_ADD: return "ADD";
        case GGML_OP_SUB: return "SUB";
        case GGML_OP_MUL: return "MUL";
        case GGML_OP_SCALE: return "SCALE";
        case GGML_OP_CLAMP: return "CLAMP";
        case GGML_OP_SOFT_MAX: return "SOFT_MAX";
        case GGML_OP_ARGSORT: return "ARGSORT";
        case GGML_OP_CUMSUM: return "CUMSUM";
        case GGML_OP_SUM: return "SUM";
        case GGML_OP_UNARY: return "UNARY";
        case GGML_OP_DIAG_MASK_INF: return "DIAG_MASK_INF";
        case GGML_OP_NORM: return "NORM";
        case GGML_OP_CONCAT: return "CONCAT";
        case GGML_OP_RMS_NORM: return "RMS_NORM";
        case GGML_OP_MUL_MAT: return "MUL_MAT";
        case GGML_OP_CPY: return "CPY";
        case GGML_OP_CONT: return "CONT";
        case GGML_OP_RESHAPE: return "RESHAPE";
        case GGML_OP_VIEW: return "VIEW";
        case GGML_OP_PERMUTE: return "PERMUTE";
        case GGML_OP_TRANSPOSE: return "TRANSPOSE";
        case GGML_OP_GET_ROWS: return "GET_ROWS";
        case GGML_OP_SET_ROWS: return "SET_ROWS";
        case GGML_OP_ROPE: return "ROPE";
        case GGML_OP_FLASH_ATTN_EXT: return "FLASH_ATTN_EXT";
        case GGML_OP_GLU: return "GLU";
        default: return "OP";
    }
}

extern "C" const char * ggml_op_desc(const struct ggml_tensor * t) {
    return ggml_op_name(t->op);
}

// ---------------------------------------------------------------------------
// tensor queries

extern "C" int64_t ggml_nelements(const struct ggml_tensor * t) {
    return t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3];
}

extern "C" int64_t ggml_nrows(const struct ggml_tensor * t) {
    return t->ne[1] * t->ne[2] * t->ne[3];
}

extern "C" size_t ggml_nbytes(const struct ggml_tensor * t) {
    for (int i = 0; i < GGML_MAX_DIMS; i++) {
        if (t->ne[i] <= 0) {
            return 0;
        }
    }
    size_t       nbytes;
    const size_t blck = (size_t) ggml_blck_size(t->type);
    if (blck == 1) {
        nbytes = ggml_type_size(t->type);
        for (int i = 0; i < GGML_MAX_DIMS; i++) {
            nbytes += (size_t) (t->ne[i] - 1) * t->nb[i];
        }
    } else {
        nbytes = (size_t) t->ne[0] * t->nb[0] / blck;
        for (int i = 1; i < GGML_MAX_DIMS; i++) {
            nbytes += (size_t) (t->ne[i] - 1) * t->nb[i];
        }
    }
    return nbytes;
}

extern "C" size_t ggml_element_size(const struct ggml_tensor * t) {
    return ggml_type_size(t->type);
}

extern "C" int ggml_n_dims(const struct ggml_tensor * t) {
    for (int i = GGML_MAX_DIMS - 1; i >= 1; --i) {
        if (t->ne[i] > 1) {
            return i + 1;
        }
    }
    return 1;
}

static bool is_contiguous_n(const struct ggml_tensor * t, int n) {
    size_t next_nb = ggml_type_size(t->type);
    if (t->ne[0] != ggml_blck_size(t->type) && t->nb[0] != next_nb) {
        return false;
    }
    next_nb *= (size_t) (t->ne[0] / ggml_blck_size(t->type));
    for (int i = 1; i < GGML_MAX_DIMS; i++) {
        if (t->ne[i] != 1) {
            if (i > n) {
                if (t->nb[i] != next_nb) {
                    return false;
                }
                next_nb *= (size_t) t->ne[i];
            } else {
                next_nb = (size_t) t->ne[i] * t->nb[i];
            }
        }
    }
    return true;
}

extern "C" bool ggml_is_contiguous(const struct ggml_tensor * t) {
    return is_contiguous_n(t, 0);
}

extern "C" bool ggml_is_contiguous_rows(const struct ggml_tensor * t) {
    return t->ne[0] == ggml_blck_size(t->type) || t->nb[0] == ggml_type_size(t->type);
}

extern "C" bool ggml_is_transposed(const struct ggml_tensor * t) {
    return t->nb[0] > t->nb[1];
}

extern "C" bool ggml_is_permuted(const struct ggml_tensor * t) {
    return t->nb[0] > t->nb[1] || t->nb[1] > t->nb[2] || t->nb[2] > t->nb[3];
}

extern "C" bool ggml_is_empty(const struct ggml_tensor * t) {
    for (int i = 0; i < GGML_MAX_DIMS; i++) {
        if (t->ne[i] == 0) {
            return true;
        }
    }
    return false;
}

extern "C" bool ggml_are_same_shape(const struct ggml_tensor * a, const struct ggml_tensor * b) {
    return a->ne[0] == b->ne[0] && a->ne[1] == b->ne[1] && a->ne[2] == b->ne[2] && a->ne[3] == b->ne[3];
}

// t0 can be broadcast (repeated) to the shape of t1
extern "C" bool ggml_can_repeat(const struct ggml_tensor * t0, const struct ggml_tensor * t1) {
    return ggml_is_empty(t0) ? ggml_is_empty(t1)
                             : (t1->ne[0] % t0->ne[0] == 0) && (t1->ne[1] % t0->ne[1] == 0) &&
                                   (t1->ne[2] % t0->ne[2] == 0) && (t1->ne[3] % t0->ne[3] == 0);
}

// ---------------------------------------------------------------------------
// context: objects laid out back to back in one memory block

struct ggml_object {
    size_t               offs;
    size_t               size;
    struct ggml_object * next;
    int                  kind;  // 0 tensor, 1 graph
    char                 padding[4];
};

static const size_t OBJ_SIZE = sizeof(struct ggml_object);

struct ggml_context {
    size_t               mem_size;
    void *               mem_buffer;
    bool                 mem_buffer_owned;
    bool                 no_alloc;
    int                  n_objects;
    struct ggml_object * objects_begin;
    struct ggml_object * objects_end;
};

extern "C" size_t ggml_tensor_overhead(void) {
    return OBJ_SIZE + GGML_TENSOR_SIZE;
}

extern "C" struct ggml_context * ggml_init(struct ggml_init_params params) {
    ggml_context * ctx = (ggml_context *) calloc(1, sizeof(ggml_context));
    if (!ctx) {
        return nullptr;
    }
    ctx->mem_size = params.mem_size ? GGML_PAD(params.mem_size, GGML_MEM_ALIGN) : GGML_MEM_ALIGN;
    if (params.mem_buffer) {
        ctx->mem_buffer = params.mem_buffer;
    } else {
        ctx->mem_buffer = aligned_alloc(64, GGML_PAD(ctx->mem_size, 64));
        if (!ctx->mem_buffer) {
            free(ctx);
            return nullptr;
        }
        ctx->mem_buffer_owned = true;
    }
    ctx->no_alloc = params.no_alloc;
    return ctx;
}

extern "C" void ggml_reset(struct ggml_context * ctx) {
    if (!ctx) {
        return;
    }
    ctx->n_objects     = 0;
    ctx->objects_begin = nullptr;
    ctx->objects_end   = nullptr;
}

extern "C" void ggml_free(struct ggml_context * ctx) {
    if (!ctx) {
        return;
    }
    if (ctx->mem_buffer_owned) {
        free(ctx->mem_buffer);
    }
    free(ctx);
}

extern "C" size_t ggml_used_mem(const struct ggml_context * ctx) {
    return ctx->objects_end ? ctx->objects_end->offs + ctx->objects_end->size : 0;
}

extern "C" bool ggml_get_no_alloc(struct ggml_context * ctx) {
    return ctx->no_alloc;
}

extern "C" void ggml_set_no_alloc(struct ggml_context * ctx, bool no_alloc) {
    ctx->no_alloc = no_alloc;
}

static struct ggml_object * new_object(struct ggml_context * ctx, int kind, size_t size) {
    const size_t cur_end   = ctx->objects_end ? ctx->objects_end->offs + ctx->objects_end->size : 0;
    const size_t size_need = GGML_PAD(size, GGML_MEM_ALIGN);
    if (cur_end + size_need + OBJ_SIZE > ctx->mem_size) {
        CORE_ABORT("ggml core: context out of memory (need %zu, have %zu)\n", cur_end + size_need + OBJ_SIZE,
                   ctx->mem_size);
    }
    struct ggml_object * obj = (struct ggml_object *) ((char *) ctx->mem_buffer + cur_end);
    obj->offs                = cur_end + OBJ_SIZE;
    obj->size                = size_need;
    obj->next                = nullptr;
    obj->kind                = kind;
    if (ctx->objects_end) {
        ctx->objects_end->next = obj;
    } else {
        ctx->objects_begin = obj;
    }
    ctx->objects_end = obj;
    ctx->n_objects++;
    return obj;
}

static struct ggml_tensor * new_tensor_impl(struct ggml_context * ctx, enum ggml_type type, int n_dims,
                                            const int64_t * ne, struct ggml_tensor * view_src, size_t view_offs) {
    CORE_ASSERT(type >= 0 && type < GGML_TYPE_COUNT && ggml_type_size(type) > 0);
    CORE_ASSERT(n_dims >= 1 && n_dims <= GGML_MAX_DIMS);
    if (view_src && view_src->view_src) {
        view_offs += view_src->view_offs;
        view_src = view_src->view_src;
    }
    size_t data_size = ggml_row_size(type, ne[0]);
    for (int i = 1; i < n_dims; i++) {
        data_size *= (size_t) ne[i];
    }
    void * data = view_src ? view_src->data : nullptr;
    if (data) {
        data = (char *) data + view_offs;
    }
    size_t obj_alloc = 0;
    if (!view_src && !ctx->no_alloc) {
        obj_alloc = data_size;
    }
    struct ggml_object * obj = new_object(ctx, 0, GGML_TENSOR_SIZE + obj_alloc);
    struct ggml_tensor * t   = (struct ggml_tensor *) ((char *) ctx->mem_buffer + obj->offs);
    memset(t, 0, sizeof(*t));
    t->type      = type;
    t->buffer    = view_src ? view_src->buffer : nullptr;
    t->view_src  = view_src;
    t->view_offs = view_offs;
    t->data      = (!view_src && obj_alloc) ? (void *) (t + 1) : data;
    for (int i = 0; i < n_dims; i++) {
        t->ne[i] = ne[i];
    }
    for (int i = n_dims; i < GGML_MAX_DIMS; i++) {
        t->ne[i] = 1;
    }
    t->nb[0] = ggml_type_size(type);
    t->nb[1] = t->nb[0] * (size_t) (t->ne[0] / ggml_blck_size(type));
    for (int i = 2; i < GGML_MAX_DIMS; i++) {
        t->nb[i] = t->nb[i - 1] * (size_t) t->ne[i - 1];
    }
    return t;
}

extern "C" struct ggml_tensor * ggml_new_tensor(struct ggml_context * ctx, enum ggml_type type, int n_dims,
                                                const int64_t * ne) {
    return new_tensor_impl(ctx, type, n_dims, ne, nullptr, 0);
}

extern "C" struct ggml_tensor * ggml_new_tensor_1d(struct ggml_context * ctx, enum ggml_type type, int64_t ne0) {
    return ggml_new_tensor(ctx, type, 1, &ne0);
}

extern "C" struct ggml_tensor * ggml_new_tensor_2d(struct ggml_context * ctx, enum ggml_type type, int64_t ne0,
                                                   int64_t ne1) {
    const int64_t ne[2] = { ne0, ne1 };
    return ggml_new_tensor(ctx, type, 2, ne);
}

extern "C" struct ggml_tensor * ggml_new_tensor_3d(struct ggml_context * ctx, enum ggml_type type, int64_t ne0,
                                                   int64_t ne1, int64_t ne2) {
    const int64_t ne[3] = { ne0, ne1, ne2 };
    return ggml_new_tensor(ctx, type, 3, ne);
}

extern "C" struct ggml_tensor * ggml_new_tensor_4d(struct ggml_context * ctx, enum ggml_type type, int64_t ne0,
                                                   int64_t ne1, int64_t ne2, int64_t ne3) {
    const int64_t ne[4] = { ne0, ne1, ne2, ne3 };
    return ggml_new_tensor(ctx, type, 4, ne);
}

extern "C" struct ggml_tensor * ggml_dup_tensor(struct ggml_context * ctx, const struct ggml_tensor * src) {
    return ggml_new_tensor(ctx, src->type, GGML_MAX_DIMS, src->ne);
}

extern "C" struct ggml_tensor * ggml_view_tensor(struct ggml_context * ctx, struct ggml_tensor * src) {
    struct ggml_tensor * r = new_tensor_impl(ctx, src->type, GGML_MAX_DIMS, src->ne, src, 0);
    for (int i = 0; i < GGML_MAX_DIMS; i++) {
        r->nb[i] = src->nb[i];
    }
    snprintf(r->name, sizeof(r->name), "%s (view)", src->name);
    return r;
}

extern "C" struct ggml_tensor * ggml_get_first_tensor(const struct ggml_context * ctx) {
    for (struct ggml_object * o = ctx->objects_begin; o; o = o->next) {
        if (o->kind == 0) {
            return (struct ggml_tensor *) ((char *) ctx->mem_buffer + o->offs);
        }
    }
    return nullptr;
}

extern "C" struct ggml_tensor * ggml_get_next_tensor(const struct ggml_context * ctx, struct ggml_tensor * tensor) {
    struct ggml_object * o = (struct ggml_object *) ((char *) tensor - OBJ_SIZE);
    for (o = o->next; o; o = o->next) {
        if (o->kind == 0) {
            return (struct ggml_tensor *) ((char *) ctx->mem_buffer + o->offs);
        }
    }
    return nullptr;
}

extern "C" struct ggml_tensor * ggml_get_tensor(struct ggml_context * ctx, const char * name) {
    for (struct ggml_tensor * t = ggml_get_first_tensor(ctx); t; t = ggml_get_next_tensor(ctx, t)) {
        if (strcmp(t->name, name) == 0) {
            return t;
        }
    }
    return nullptr;
}

extern "C" const char * ggml_get_name(const struct ggml_tensor * t) {
    return t->name;
}

extern "C" struct ggml_tensor * ggml_set_name(struct ggml_tensor * t, const char * name) {
    size_t i;
    for (i = 0; i < sizeof(t->name) - 1 && name[i] != '\0'; i++) {
        t->name[i] = name[i];
    }
    t->name[i] = '\0';
    return t;
}

extern "C" struct ggml_tensor * ggml_format_name(struct ggml_tensor * t, const char * fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t->name, sizeof(t->name), fmt, ap);
    va_end(ap);
    return t;
}

extern "C" void ggml_set_input(struct ggml_tensor * t) {
    t->flags |= GGML_TENSOR_FLAG_INPUT;
}

extern "C" void ggml_set_output(struct ggml_tensor * t) {
    t->flags |= GGML_TENSOR_FLAG_OUTPUT;
}

extern "C" void * ggml_get_data(const struct ggml_tensor * t) {
    return t->data;
}

// ---------------------------------------------------------------------------
// ops

static void set_op_params(struct ggml_tensor * t, const void * params, size_t size) {
    CORE_ASSERT(size <= GGML_MAX_OP_PARAMS);
    memcpy(t->op_params, params, size);
}

static struct ggml_tensor * binary(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b,
                                   enum ggml_op op) {
    CORE_ASSERT(ggml_can_repeat(b, a));
    struct ggml_tensor * r = ggml_dup_tensor(ctx, a);
    r->op                  = op;
    r->src[0]              = a;
    r->src[1]              = b;
    return r;
}

extern "C" struct ggml_tensor * ggml_add(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b) {
    return binary(ctx, a, b, GGML_OP_ADD);
}

extern "C" struct ggml_tensor * ggml_sub(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b) {
    return binary(ctx, a, b, GGML_OP_SUB);
}

extern "C" struct ggml_tensor * ggml_mul(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b) {
    return binary(ctx, a, b, GGML_OP_MUL);
}

extern "C" struct ggml_tensor * ggml_scale(struct ggml_context * ctx, struct ggml_tensor * a, float s) {
    struct ggml_tensor * r         = ggml_dup_tensor(ctx, a);
    const float          params[2] = { s, 0.0f };
    set_op_params(r, params, sizeof(params));
    r->op     = GGML_OP_SCALE;
    r->src[0] = a;
    return r;
}

extern "C" struct ggml_tensor * ggml_clamp(struct ggml_context * ctx, struct ggml_tensor * a, float min, float max) {
    struct ggml_tensor * r         = ggml_view_tensor(ctx, a);
    const float          params[2] = { min, max };
    set_op_params(r, params, sizeof(params));
    r->op     = GGML_OP_CLAMP;
    r->src[0] = a;
    return r;
}

// softmax over rows (no mask, scale 1, no ALiBi): op_params = {scale, max_bias}
extern "C" struct ggml_tensor * ggml_soft_max(struct ggml_context * ctx, struct ggml_tensor * a) {
    struct ggml_tensor * r         = ggml_dup_tensor(ctx, a);
    const float          params[2] = { 1.0f, 0.0f };
    set_op_params(r, params, sizeof(params));
    r->op     = GGML_OP_SOFT_MAX;
    r->src[0] = a;
    return r;
}

extern "C" struct ggml_tensor * ggml_soft_max_ext(struct ggml_context * ctx, struct ggml_tensor * a,
                                                  struct ggml_tensor * mask, float scale, float max_bias) {
    CORE_ASSERT(mask == nullptr || (mask->ne[0] == a->ne[0] && mask->ne[1] >= a->ne[1] &&
                                    a->ne[2] % mask->ne[2] == 0 && a->ne[3] % mask->ne[3] == 0));
    struct ggml_tensor * r         = ggml_dup_tensor(ctx, a);
    const float          params[2] = { scale, max_bias };
    set_op_params(r, params, sizeof(params));
    r->op     = GGML_OP_SOFT_MAX;
    r->src[0] = a;
    r->src[1] = mask;
    return r;
}

// a * s + b; op_params = {s, b} (GGML_OP_SCALE)
extern "C" struct ggml_tensor * ggml_scale_bias(struct ggml_context * ctx, struct ggml_tensor * a, float s, float b) {
    struct ggml_tensor * r         = ggml_dup_tensor(ctx, a);
    const float          params[2] = { s, b };
    set_op_params(r, params, sizeof(params));
    r->op     = GGML_OP_SCALE;
    r->src[0] = a;
    return r;
}

// indices (I32) that sort each row; op_params[0] = order
extern "C" struct ggml_tensor * ggml_argsort(struct ggml_context * ctx, struct ggml_tensor * a,
                                             enum ggml_sort_order order) {
    struct ggml_tensor * r         = ggml_new_tensor(ctx, GGML_TYPE_I32, GGML_MAX_DIMS, a->ne);
    const int32_t        params[1] = { (int32_t) order };
    set_op_params(r, params, sizeof(params));
    r->op     = GGML_OP_ARGSORT;
    r->src[0] = a;
    return r;
}

// the first k indices of the descending argsort of each row (a view)
extern "C" struct ggml_tensor * ggml_argsort_top_k(struct ggml_context * ctx, struct ggml_tensor * a, int k) {
    CORE_ASSERT(k >= 1 && k <= a->ne[0]);
    struct ggml_tensor * s = ggml_argsort(ctx, a, GGML_SORT_ORDER_DESC);
    return ggml_view_4d(ctx, s, k, s->ne[1], s->ne[2], s->ne[3], s->nb[1], s->nb[2], s->nb[3], 0);
}

// running sum along dim 0
extern "C" struct ggml_tensor * ggml_cumsum(struct ggml_context * ctx, struct ggml_tensor * a) {
    struct ggml_tensor * r = ggml_dup_tensor(ctx, a);
    r->op                  = GGML_OP_CUMSUM;
    r->src[0]              = a;
    return r;
}

// the sum of all elements, a one-element tensor
extern "C" struct ggml_tensor * ggml_sum(struct ggml_context * ctx, struct ggml_tensor * a) {
    struct ggml_tensor * r = ggml_new_tensor_1d(ctx, a->type, 1);
    r->op                  = GGML_OP_SUM;
    r->src[0]              = a;
    return r;
}

// x > 0 ? 1 : 0 (GGML_OP_UNARY, op_params[0] = GGML_UNARY_OP_STEP)
extern "C" struct ggml_tensor * ggml_step(struct ggml_context * ctx, struct ggml_tensor * a) {
    struct ggml_tensor * r         = ggml_dup_tensor(ctx, a);
    const int32_t        params[1] = { (int32_t) GGML_UNARY_OP_STEP };
    set_op_params(r, params, sizeof(params));
    r->op     = GGML_OP_UNARY;
    r->src[0] = a;
    return r;
}

// elements (i0, i1) with i0 > n_past + i1 set to -inf; op_params[0] = n_past
extern "C" struct ggml_tensor * ggml_diag_mask_inf(struct ggml_context * ctx, struct ggml_tensor * a, int n_past) {
    struct ggml_tensor * r        = ggml_dup_tensor(ctx, a);
    const int32_t        params[1] = { n_past };
    set_op_params(r, params, sizeof(params));
    r->op     = GGML_OP_DIAG_MASK_INF;
    r->src[0] = a;
    return r;
}

// a and b joined along dim (equal extents elsewhere); op_params[0] = dim
extern "C" struct ggml_tensor * ggml_concat(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b,
                                            int dim) {
    CORE_ASSERT(dim >= 0 && dim < 4 && a->type == b->type);
    int64_t ne[4];
    for (int i = 0; i < 4; i++) {
        CORE_ASSERT(i == dim || a->ne[i] == b->ne[i]);
        ne[i] = a->ne[i] + (i == dim ? b->ne[i] : 0);
    }
    struct ggml_tensor * r = ggml_new_tensor(ctx, a->type, 4, ne);
    const int32_t        d = dim;
    set_op_params(r, &d, sizeof(d));
    r->op     = GGML_OP_CONCAT;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

static struct ggml_tensor * norm_impl(struct ggml_context * ctx, struct ggml_tensor * a, float eps, enum ggml_op op) {
    struct ggml_tensor * r = ggml_dup_tensor(ctx, a);
    set_op_params(r, &eps, sizeof(eps));
    r->op     = op;
    r->src[0] = a;
    return r;
}

extern "C" struct ggml_tensor * ggml_rms_norm(struct ggml_context * ctx, struct ggml_tensor * a, float eps) {
    return norm_impl(ctx, a, eps, GGML_OP_RMS_NORM);
}

extern "C" struct ggml_tensor * ggml_norm(struct ggml_context * ctx, struct ggml_tensor * a, float eps) {
    return norm_impl(ctx, a, eps, GGML_OP_NORM);
}

extern "C" struct ggml_tensor * ggml_mul_mat(struct ggml_context * ctx, struct ggml_tensor * a,
                                             struct ggml_tensor * b) {
    CORE_ASSERT(a->ne[0] == b->ne[0] && b->ne[2] % a->ne[2] == 0 && b->ne[3] % a->ne[3] == 0);
    CORE_ASSERT(!ggml_is_transposed(a));
    const int64_t        ne[4] = { a->ne[1], b->ne[1], b->ne[2], b->ne[3] };
    struct ggml_tensor * r     = ggml_new_tensor(ctx, GGML_TYPE_F32, 4, ne);
    r->op                      = GGML_OP_MUL_MAT;
    r->src[0]                  = a;
    r->src[1]                  = b;
    return r;
}

extern "C" struct ggml_tensor * ggml_cpy(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b) {
    CORE_ASSERT(ggml_nelements(a) == ggml_nelements(b));
    struct ggml_tensor * r = ggml_view_tensor(ctx, b);
    if (strlen(b->name) > 0) {
        ggml_format_name(r, "%s (copy of %s)", b->name, a->name);
    } else {
        ggml_format_name(r, "%s (copy)", a->name);
    }
    r->op     = GGML_OP_CPY;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

extern "C" struct ggml_tensor * ggml_cast(struct ggml_context * ctx, struct ggml_tensor * a, enum ggml_type type) {
    struct ggml_tensor * r = ggml_new_tensor(ctx, type, GGML_MAX_DIMS, a->ne);
    ggml_format_name(r, "%s (copy)", a->name);
    r->op     = GGML_OP_CPY;
    r->src[0] = a;
    r->src[1] = r;
    return r;
}

extern "C" struct ggml_tensor * ggml_cont(struct ggml_context * ctx, struct ggml_tensor * a) {
    struct ggml_tensor * r = ggml_new_tensor(ctx, a->type, GGML_MAX_DIMS, a->ne);
    ggml_format_name(r, "%s (cont)", a->name);
    r->op     = GGML_OP_CONT;
    r->src[0] = a;
    return r;
}

static struct ggml_tensor * reshape_impl(struct ggml_context * ctx, struct ggml_tensor * a, int n_dims,
                                         const int64_t * ne) {
    CORE_ASSERT(ggml_is_contiguous(a));
    int64_t n = 1;
    for (int i = 0; i < n_dims; i++) {
        n *= ne[i];
    }
    CORE_ASSERT(n == ggml_nelements(a));
    struct ggml_tensor * r = new_tensor_impl(ctx, a->type, n_dims, ne, a, 0);
    ggml_format_name(r, "%s (reshaped)", a->name);
    r->op     = GGML_OP_RESHAPE;
    r->src[0] = a;
    return r;
}

extern "C" struct ggml_tensor * ggml_reshape(struct ggml_context * ctx, struct ggml_tensor * a,
                                             struct ggml_tensor * b) {
    return reshape_impl(ctx, a, GGML_MAX_DIMS, b->ne);
}

extern "C" struct ggml_tensor * ggml_reshape_1d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0) {
    return reshape_impl(ctx, a, 1, &ne0);
}

extern "C" struct ggml_tensor * ggml_reshape_2d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0,
                                                int64_t ne1) {
    const int64_t ne[2] = { ne0, ne1 };
    return reshape_impl(ctx, a, 2, ne);
}

extern "C" struct ggml_tensor * ggml_reshape_3d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0,
                                                int64_t ne1, int64_t ne2) {
    const int64_t ne[3] = { ne0, ne1, ne2 };
    return reshape_impl(ctx, a, 3, ne);
}

extern "C" struct ggml_tensor * ggml_reshape_4d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0,
                                                int64_t ne1, int64_t ne2, int64_t ne3) {
    const int64_t ne[4] = { ne0, ne1, ne2, ne3 };
    return reshape_impl(ctx, a, 4, ne);
}

static struct ggml_tensor * view_impl(struct ggml_context * ctx, struct ggml_tensor * a, int n_dims,
                                      const int64_t * ne, size_t offset) {
    struct ggml_tensor * r = new_tensor_impl(ctx, a->type, n_dims, ne, a, offset);
    ggml_format_name(r, "%s (view)", a->name);
    set_op_params(r, &offset, sizeof(offset));
    r->op     = GGML_OP_VIEW;
    r->src[0] = a;
    return r;
}

extern "C" struct ggml_tensor * ggml_view_1d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0,
                                             size_t offset) {
    return view_impl(ctx, a, 1, &ne0, offset);
}

extern "C" struct ggml_tensor * ggml_view_2d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0,
                                             int64_t ne1, size_t nb1, size_t offset) {
    const int64_t        ne[2] = { ne0, ne1 };
    struct ggml_tensor * r     = view_impl(ctx, a, 2, ne, offset);
    r->nb[1]                   = nb1;
    r->nb[2]                   = r->nb[1] * (size_t) ne1;
    r->nb[3]                   = r->nb[2];
    return r;
}

extern "C" struct ggml_tensor * ggml_view_3d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0,
                                             int64_t ne1, int64_t ne2, size_t nb1, size_t nb2, size_t offset) {
    const int64_t        ne[3] = { ne0, ne1, ne2 };
    struct ggml_tensor * r     = view_impl(ctx, a, 3, ne, offset);
    r->nb[1]                   = nb1;
    r->nb[2]                   = nb2;
    r->nb[3]                   = r->nb[2] * (size_t) ne2;
    return r;
}

extern "C" struct ggml_tensor * ggml_view_4d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0,
                                             int64_t ne1, int64_t ne2, int64_t ne3, size_t nb1, size_t nb2,
                                             size_t nb3, size_t offset) {
    const int64_t        ne[4] = { ne0, ne1, ne2, ne3 };
    struct ggml_tensor * r     = view_impl(ctx, a, 4, ne, offset);
    r->nb[1]                   = nb1;
    r->nb[2]                   = nb2;
    r->nb[3]                   = nb3;
    return r;
}

extern "C" struct ggml_tensor * ggml_permute(struct ggml_context * ctx, struct ggml_tensor * a, int axis0, int axis1,
                                             int axis2, int axis3) {
    CORE_ASSERT(axis0 != axis1 && axis0 != axis2 && axis0 != axis3 && axis1 != axis2 && axis1 != axis3 &&
                axis2 != axis3);
    struct ggml_tensor * r = ggml_view_tensor(ctx, a);
    ggml_format_name(r, "%s (permuted)", a->name);
    int64_t ne[4];
    size_t  nb[4];
    const int ax[4] = { axis0, axis1, axis2, axis3 };
    for (int i = 0; i < 4; i++) {
        ne[ax[i]] = a->ne[i];
        nb[ax[i]] = a->nb[i];
    }
    for (int i = 0; i < 4; i++) {
        r->ne[i] = ne[i];
        r->nb[i] = nb[i];
    }
    r->op                = GGML_OP_PERMUTE;
    r->src[0]            = a;
    const int32_t p[4]   = { axis0, axis1, axis2, axis3 };
    set_op_params(r, p, sizeof(p));
    return r;
}

extern "C" struct ggml_tensor * ggml_transpose(struct ggml_context * ctx, struct ggml_tensor * a) {
    struct ggml_tensor * r = ggml_view_tensor(ctx, a);
    ggml_format_name(r, "%s (transposed)", a->name);
    r->ne[0]  = a->ne[1];
    r->ne[1]  = a->ne[0];
    r->nb[0]  = a->nb[1];
    r->nb[1]  = a->nb[0];
    r->op     = GGML_OP_TRANSPOSE;
    r->src[0] = a;
    return r;
}

extern "C" struct ggml_tensor * ggml_get_rows(struct ggml_context * ctx, struct ggml_tensor * a,
                                              struct ggml_tensor * b) {
    CORE_ASSERT(a->ne[2] == b->ne[1] && b->ne[3] == 1 && b->type == GGML_TYPE_I32);
    const enum ggml_type type = a->type == GGML_TYPE_I32 ? GGML_TYPE_I32 : GGML_TYPE_F32;
    struct ggml_tensor * r    = ggml_new_tensor_4d(ctx, type, a->ne[0], b->ne[0], b->ne[1], b->ne[2]);
    r->op                     = GGML_OP_GET_ROWS;
    r->src[0]                 = a;
    r->src[1]                 = b;
    return r;
}

extern "C" struct ggml_tensor * ggml_set_rows(struct ggml_context * ctx, struct ggml_tensor * a,
                                              struct ggml_tensor * b, struct ggml_tensor * c) {
    CORE_ASSERT(a->ne[0] == b->ne[0] && a->ne[2] == b->ne[2] && a->ne[3] == b->ne[3]);
    CORE_ASSERT(b->ne[1] == c->ne[0] && b->ne[2] % c->ne[1] == 0 && b->ne[3] % c->ne[2] == 0 && c->ne[3] == 1);
    CORE_ASSERT(b->type == GGML_TYPE_F32 && (c->type == GGML_TYPE_I64 || c->type == GGML_TYPE_I32));
    struct ggml_tensor * r = ggml_view_tensor(ctx, a);
    r->op                  = GGML_OP_SET_ROWS;
    r->src[0]              = b;
    r->src[1]              = c;
    return r;
}

extern "C" struct ggml_tensor * ggml_rope_ext(struct ggml_context * ctx, struct ggml_tensor * a,
                                              struct ggml_tensor * b, struct ggml_tensor * c, int n_dims, int mode,
                                              int n_ctx_orig, float freq_base, float freq_scale, float ext_factor,
                                              float attn_factor, float beta_fast, float beta_slow) {
    CORE_ASSERT(b->type == GGML_TYPE_I32 && a->ne[2] == b->ne[0]);
    struct ggml_tensor * r          = ggml_dup_tensor(ctx, a);
    int32_t              params[15] = { 0, n_dims, mode, 0, n_ctx_orig };
    memcpy(params + 5, &freq_base, sizeof(float));
    memcpy(params + 6, &freq_scale, sizeof(float));
    memcpy(params + 7, &ext_factor, sizeof(float));
    memcpy(params + 8, &attn_factor, sizeof(float));
    memcpy(params + 9, &beta_fast, sizeof(float));
    memcpy(params + 10, &beta_slow, sizeof(float));
    set_op_params(r, params, sizeof(params));
    r->op     = GGML_OP_ROPE;
    r->src[0] = a;
    r->src[1] = b;
    r->src[2] = c;
    return r;
}

extern "C" struct ggml_tensor * ggml_flash_attn_ext(struct ggml_context * ctx, struct ggml_tensor * q,
                                                    struct ggml_tensor * k, struct ggml_tensor * v,
                                                    struct ggml_tensor * mask, float scale, float max_bias,
                                                    float logit_softcap) {
    CORE_ASSERT(q->ne[0] == k->ne[0] && k->ne[1] == v->ne[1]);
    CORE_ASSERT(q->ne[2] % k->ne[2] == 0 && q->ne[3] % k->ne[3] == 0);
    if (mask) {
        CORE_ASSERT(mask->ne[0] >= k->ne[1] && mask->ne[1] >= q->ne[1]);
        CORE_ASSERT(q->ne[2] % mask->ne[2] == 0 && q->ne[3] % mask->ne[3] == 0);
    }
    // result is permuted: [D_v, n_head, n_queries, ne3]
    const int64_t        ne[4] = { v->ne[0], q->ne[2], q->ne[1], q->ne[3] };
    struct ggml_tensor * r     = ggml_new_tensor(ctx, GGML_TYPE_F32, 4, ne);
    const float          params[3] = { scale, max_bias, logit_softcap };
    set_op_params(r, params, sizeof(params));
    r->op     = GGML_OP_FLASH_ATTN_EXT;
    r->src[0] = q;
    r->src[1] = k;
    r->src[2] = v;
    r->src[3] = mask;
    return r;
}

extern "C" void ggml_flash_attn_ext_set_prec(struct ggml_tensor * a, enum ggml_prec prec) {
    CORE_ASSERT(a->op == GGML_OP_FLASH_ATTN_EXT);
    a->op_params[3] = (int32_t) prec;
}

extern "C" enum ggml_prec ggml_flash_attn_ext_get_prec(const struct ggml_tensor * a) {
    return (enum ggml_prec) a->op_params[3];
}

extern "C" struct ggml_tensor * ggml_glu(struct ggml_context * ctx, struct ggml_tensor * a, enum ggml_glu_op op,
                                         bool swapped) {
    CORE_ASSERT(a->ne[0] % 2 == 0);
    int64_t ne[4] = { a->ne[0] / 2, a->ne[1], a->ne[2], a->ne[3] };
    struct ggml_tensor * r         = ggml_new_tensor(ctx, a->type, 4, ne);
    const int32_t        params[2] = { (int32_t) op, (int32_t) swapped };
    set_op_params(r, params, sizeof(params));
    r->op     = GGML_OP_GLU;
    r->src[0] = a;
    return r;
}

extern "C" struct ggml_tensor * ggml_glu_split(struct ggml_context * ctx, struct ggml_tensor * a,
                                               struct ggml_tensor * b, enum ggml_glu_op op) {
    CORE_ASSERT(ggml_are_same_shape(a, b) && a->type == b->type);
    struct ggml_tensor * r         = ggml_dup_tensor(ctx, a);
    const int32_t        params[2] = { (int32_t) op, 0 };
    set_op_params(r, params, sizeof(params));
    r->op     = GGML_OP_GLU;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

extern "C" struct ggml_tensor * ggml_swiglu(struct ggml_context * ctx, struct ggml_tensor * a) {
    return ggml_glu(ctx, a, GGML_GLU_OP_SWIGLU, false);
}

extern "C" struct ggml_tensor * ggml_swiglu_split(struct ggml_context * ctx, struct ggml_tensor * a,
                                                  struct ggml_tensor * b) {
    return ggml_glu_split(ctx, a, b, GGML_GLU_OP_SWIGLU);
}

extern "C" enum ggml_glu_op ggml_get_glu_op(const struct ggml_tensor * t) {
    return (enum ggml_glu_op) t->op_params[0];
}

// ---------------------------------------------------------------------------
// graphs

struct ggml_cgraph {
    int                   size;
    int                   n_nodes;
    int                   n_leafs;
    struct ggml_tensor ** nodes;
    struct ggml_tensor ** leafs;
    struct ggml_tensor ** visited;  // open-addressing set
    size_t                visited_size;
};

static size_t visited_size_for(size_t size) {
    size_t n = 1;
    while (n < 2 * size + 1) {
        n <<= 1;
    }
    return n;
}

static size_t graph_nbytes(size_t size) {
    return sizeof(struct ggml_cgraph) + 2 * size * sizeof(struct ggml_tensor *) +
           visited_size_for(size) * sizeof(struct ggml_tensor *);
}

extern "C" size_t ggml_graph_overhead_custom(size_t size, bool grads) {
    (void) grads;
    return OBJ_SIZE + GGML_PAD(graph_nbytes(size), GGML_MEM_ALIGN);
}

extern "C" size_t ggml_graph_overhead(void) {
    return ggml_graph_overhead_custom(GGML_DEFAULT_GRAPH_SIZE, false);
}

extern "C" struct ggml_cgraph * ggml_new_graph_custom(struct ggml_context * ctx, size_t size, bool grads) {
    (void) grads;
    struct ggml_object * obj = new_object(ctx, 1, graph_nbytes(size));
    struct ggml_cgraph * g   = (struct ggml_cgraph *) ((char *) ctx->mem_buffer + obj->offs);
    struct ggml_tensor ** p  = (struct ggml_tensor **) (g + 1);
    g->size                  = (int) size;
    g->n_nodes               = 0;
    g->n_leafs               = 0;
    g->nodes                 = p;
    g->leafs                 = p + size;
    g->visited               = p + 2 * size;
    g->visited_size          = visited_size_for(size);
    memset(g->visited, 0, g->visited_size * sizeof(struct ggml_tensor *));
    return g;
}

extern "C" struct ggml_cgraph * ggml_new_graph(struct ggml_context * ctx) {
    return ggml_new_graph_custom(ctx, GGML_DEFAULT_GRAPH_SIZE, false);
}

static bool visit_insert(struct ggml_cgraph * g, struct ggml_tensor * t) {
    size_t h = ((uintptr_t) t >> 4) & (g->visited_size - 1);
    while (g->visited[h]) {
        if (g->visited[h] == t) {
            return false;
        }
        h = (h + 1) & (g->visited_size - 1);
    }
    g->visited[h] = t;
    return true;
}

static void visit(struct ggml_cgraph * g, struct ggml_tensor * t) {
    if (!visit_insert(g, t)) {
        return;
    }
    for (int i = 0; i < GGML_MAX_SRC; i++) {
        if (t->src[i]) {
            visit(g, t->src[i]);
        }
    }
    if (t->op == GGML_OP_NONE && !(t->flags & GGML_TENSOR_FLAG_PARAM)) {
        CORE_ASSERT(g->n_leafs < g->size);
        if (strlen(t->name) == 0) {
            ggml_format_name(t, "leaf_%d", g->n_leafs);
        }
        g->leafs[g->n_leafs++] = t;
    } else {
        CORE_ASSERT(g->n_nodes < g->size);
        if (strlen(t->name) == 0) {
            ggml_format_name(t, "node_%d", g->n_nodes);
        }
        g->nodes[g->n_nodes++] = t;
    }
}

extern "C" void ggml_build_forward_expand(struct ggml_cgraph * g, struct ggml_tensor * t) {
    visit(g, t);
}

extern "C" int ggml_graph_size(struct ggml_cgraph * g) {
    return g->size;
}

extern "C" int ggml_graph_n_nodes(struct ggml_cgraph * g) {
    return g->n_nodes;
}

extern "C" struct ggml_tensor * ggml_graph_node(struct ggml_cgraph * g, int i) {
    if (i < 0) {
        CORE_ASSERT(g->n_nodes + i >= 0);
        return g->nodes[g->n_nodes + i];
    }
    CORE_ASSERT(i < g->n_nodes);
    return g->nodes[i];
}

extern "C" int ggml_graph_n_leafs(struct ggml_cgraph * g) {
    return g->n_leafs;
}

extern "C" struct ggml_tensor * ggml_graph_leaf(struct ggml_cgraph * g, int i) {
    CORE_ASSERT(i >= 0 && i < g->n_leafs);
    return g->leafs[i];
}

extern "C" struct ggml_tensor * ggml_graph_get_tensor(const struct ggml_cgraph * g, const char * name) {
    for (int i = 0; i < g->n_leafs; i++) {
        if (strcmp(g->leafs[i]->name, name) == 0) {
            return g->leafs[i];
        }
    }
    for (int i = 0; i < g->n_nodes; i++) {
        if (strcmp(g->nodes[i]->name, name) == 0) {
            return g->nodes[i];
        }
    }
    return nullptr;
}

extern "C" void ggml_graph_clear(struct ggml_cgraph * g) {
    g->n_nodes = 0;
    g->n_leafs = 0;
    memset(g->visited, 0, g->visited_size * sizeof(struct ggml_tensor *));
}

// ---------------------------------------------------------------------------
// backend buffer types / buffers

extern "C" const char * ggml_backend_buft_name(ggml_backend_buffer_type_t buft) {
    return buft->iface.get_name(buft);
}

extern "C" ggml_backend_buffer_t ggml_backend_buft_alloc_buffer(ggml_backend_buffer_type_t buft, size_t size) {
    return buft->iface.alloc_buffer(buft, size);
}

extern "C" size_t ggml_backend_buft_get_alignment(ggml_backend_buffer_type_t buft) {
    return buft->iface.get_alignment(buft);
}

extern "C" size_t ggml_backend_buft_get_max_size(ggml_backend_buffer_type_t buft) {
    return buft->iface.get_max_size ? buft->iface.get_max_size(buft) : SIZE_MAX;
}

extern "C" size_t ggml_backend_buft_get_alloc_size(ggml_backend_buffer_type_t buft, const struct ggml_tensor * t) {
    return buft->iface.get_alloc_size ? buft->iface.get_alloc_size(buft, t) : ggml_nbytes(t);
}

extern "C" bool ggml_backend_buft_is_host(ggml_backend_buffer_type_t buft) {
    return buft->iface.is_host ? buft->iface.is_host(buft) : false;
}

extern "C" ggml_backend_dev_t ggml_backend_buft_get_device(ggml_backend_buffer_type_t buft) {
    return buft->device;
}

extern "C" ggml_backend_buffer_t ggml_backend_buffer_init(ggml_backend_buffer_type_t buft,
                                                          struct ggml_backend_buffer_i iface, void * context,
                                                          size_t size) {
    ggml_backend_buffer_t b = new ggml_backend_buffer{ iface, buft, context, size, GGML_BACKEND_BUFFER_USAGE_ANY };
    return b;
}

extern "C" const char * ggml_backend_buffer_name(ggml_backend_buffer_t buffer) {
    return ggml_backend_buft_name(buffer->buft);
}

extern "C" void ggml_backend_buffer_free(ggml_backend_buffer_t buffer) {
    if (!buffer) {
        return;
    }
    if (buffer->iface.free_buffer) {
        buffer->iface.free_buffer(buffer);
    }
    delete buffer;
}

extern "C" void * ggml_backend_buffer_get_base(ggml_backend_buffer_t buffer) {
    return buffer->size ? buffer->iface.get_base(buffer) : nullptr;
}

extern "C" size_t ggml_backend_buffer_get_size(ggml_backend_buffer_t buffer) {
    return buffer->size;
}

extern "C" enum ggml_status ggml_backend_buffer_init_tensor(ggml_backend_buffer_t buffer, struct ggml_tensor * t) {
    return buffer->iface.init_tensor ? buffer->iface.init_tensor(buffer, t) : GGML_STATUS_SUCCESS;
}

extern "C" size_t ggml_backend_buffer_get_alignment(ggml_backend_buffer_t buffer) {
    return ggml_backend_buft_get_alignment(buffer->buft);
}

extern "C" size_t ggml_backend_buffer_get_alloc_size(ggml_backend_buffer_t buffer, const struct ggml_tensor * t) {
    return ggml_backend_buft_get_alloc_size(buffer->buft, t);
}

extern "C" void ggml_backend_buffer_clear(ggml_backend_buffer_t buffer, uint8_t value) {
    if (buffer->size) {
        buffer->iface.clear(buffer, value);
    }
}

extern "C" bool ggml_backend_buffer_is_host(ggml_backend_buffer_t buffer) {
    return ggml_backend_buft_is_host(buffer->buft);
}

extern "C" void ggml_backend_buffer_set_usage(ggml_backend_buffer_t buffer, enum ggml_backend_buffer_usage usage) {
    buffer->usage = usage;
}

extern "C" enum ggml_backend_buffer_usage ggml_backend_buffer_get_usage(ggml_backend_buffer_t buffer) {
    return buffer->usage;
}

extern "C" ggml_backend_buffer_type_t ggml_backend_buffer_get_type(ggml_backend_buffer_t buffer) {
    return buffer->buft;
}

// ---------------------------------------------------------------------------
// backend

extern "C" const char * ggml_backend_name(ggml_backend_t backend) {
    return backend ? backend->iface.get_name(backend) : "NULL";
}

extern "C" void ggml_backend_free(ggml_backend_t backend) {
    if (backend) {
        backend->iface.free(backend);
    }
}

extern "C" ggml_backend_buffer_type_t ggml_backend_get_default_buffer_type(ggml_backend_t backend) {
    return ggml_backend_dev_buffer_type(backend->device);
}

extern "C" ggml_backend_buffer_t ggml_backend_alloc_buffer(ggml_backend_t backend, size_t size) {
    return ggml_backend_buft_alloc_buffer(ggml_backend_get_default_buffer_type(backend), size);
}

extern "C" size_t ggml_backend_get_alignment(ggml_backend_t backend) {
    return ggml_backend_buft_get_alignment(ggml_backend_get_default_buffer_type(backend));
}

static void check_tensor_range(const struct ggml_tensor * t, size_t offset, size_t size) {
    ggml_backend_buffer_t buf = t->view_src ? t->view_src->buffer : t->buffer;
    CORE_ASSERT(buf != nullptr && "tensor buffer not set");
    CORE_ASSERT(t->data != nullptr && "tensor not allocated");
    CORE_ASSERT(offset + size <= ggml_nbytes(t) && "tensor read/write out of bounds");
}

extern "C" void ggml_backend_tensor_set_async(ggml_backend_t backend, struct ggml_tensor * t, const void * data,
                                              size_t offset, size_t size) {
    check_tensor_range(t, offset, size);
    if (backend->iface.set_tensor_async) {
        backend->iface.set_tensor_async(backend, t, data, offset, size);
    } else {
        ggml_backend_tensor_set(t, data, offset, size);
    }
}

extern "C" void ggml_backend_tensor_get_async(ggml_backend_t backend, const struct ggml_tensor * t, void * data,
                                              size_t offset, size_t size) {
    check_tensor_range(t, offset, size);
    if (backend->iface.get_tensor_async) {
        backend->iface.get_tensor_async(backend, t, data, offset, size);
    } else {
        ggml_backend_tensor_get(t, data, offset, size);
    }
}

extern "C" void ggml_backend_tensor_set(struct ggml_tensor * t, const void * data, size_t offset, size_t size) {
    if (size == 0) {
        return;
    }
    check_tensor_range(t, offset, size);
    ggml_backend_buffer_t buf = t->view_src ? t->view_src->buffer : t->buffer;
    buf->iface.set_tensor(buf, t, data, offset, size);
}

extern "C" void ggml_backend_tensor_get(const struct ggml_tensor * t, void * data, size_t offset, size_t size) {
    if (size == 0) {
        return;
    }
    check_tensor_range(t, offset, size);
    ggml_backend_buffer_t buf = t->view_src ? t->view_src->buffer : t->buffer;
    buf->iface.get_tensor(buf, t, data, offset, size);
}

extern "C" void ggml_backend_tensor_memset(struct ggml_tensor * t, uint8_t value, size_t offset, size_t size) {
    if (size == 0) {
        return;
    }
    check_tensor_range(t, offset, size);
    ggml_backend_buffer_t buf = t->view_src ? t->view_src->buffer : t->buffer;
    CORE_ASSERT(buf->iface.memset_tensor != nullptr);
    buf->iface.memset_tensor(buf, t, value, offset, size);
}

extern "C" void ggml_backend_tensor_copy(struct ggml_tensor * src, struct ggml_tensor * dst) {
    CORE_ASSERT(ggml_nbytes(src) == ggml_nbytes(dst));
    if (src == dst) {
        return;
    }
    ggml_backend_buffer_t sb = src->view_src ? src->view_src->buffer : src->buffer;
    ggml_backend_buffer_t db = dst->view_src ? dst->view_src->buffer : dst->buffer;
    if (ggml_backend_buffer_is_host(sb)) {
        ggml_backend_tensor_set(dst, src->data, 0, ggml_nbytes(src));
    } else if (ggml_backend_buffer_is_host(db)) {
        ggml_backend_tensor_get(src, dst->data, 0, ggml_nbytes(src));
    } else if (!(db->iface.cpy_tensor && db->iface.cpy_tensor(db, src, dst))) {
        std::vector<uint8_t> tmp(ggml_nbytes(src));
        ggml_backend_tensor_get(src, tmp.data(), 0, tmp.size());
        ggml_backend_tensor_set(dst, tmp.data(), 0, tmp.size());
    }
}

extern "C" void ggml_backend_synchronize(ggml_backend_t backend) {
    if (backend->iface.synchronize) {
        backend->iface.synchronize(backend);
    }
}

extern "C" enum ggml_status ggml_backend_graph_compute_async(ggml_backend_t backend, struct ggml_cgraph * cgraph) {
    return backend->iface.graph_compute(backend, cgraph);
}

extern "C" enum ggml_status ggml_backend_graph_compute(ggml_backend_t backend, struct ggml_cgraph * cgraph) {
    enum ggml_status st = ggml_backend_graph_compute_async(backend, cgraph);
    ggml_backend_synchronize(backend);
    return st;
}

extern "C" bool ggml_backend_supports_op(ggml_backend_t backend, const struct ggml_tensor * op) {
    return ggml_backend_dev_supports_op(backend->device, op);
}

extern "C" bool ggml_backend_supports_buft(ggml_backend_t backend, ggml_backend_buffer_type_t buft) {
    return ggml_backend_dev_supports_buft(backend->device, buft);
}

extern "C" bool ggml_backend_offload_op(ggml_backend_t backend, const struct ggml_tensor * op) {
    return ggml_backend_dev_offload_op(backend->device, op);
}

extern "C" ggml_backend_dev_t ggml_backend_get_device(ggml_backend_t backend) {
    return backend->device;
}

// ---------------------------------------------------------------------------
// devices / registry

extern "C" const char * ggml_backend_dev_name(ggml_backend_dev_t d) {
    return d->iface.get_name(d);
}

extern "C" const char * ggml_backend_dev_description(ggml_backend_dev_t d) {
    return d->iface.get_description(d);
}

extern "C" void ggml_backend_dev_memory(ggml_backend_dev_t d, size_t * free, size_t * total) {
    d->iface.get_memory(d, free, total);
}

extern "C" enum ggml_backend_dev_type ggml_backend_dev_type(ggml_backend_dev_t d) {
    return d->iface.get_type(d);
}

extern "C" void ggml_backend_dev_get_props(ggml_backend_dev_t d, struct ggml_backend_dev_props * props) {
    memset(props, 0, sizeof(*props));
    d->iface.get_props(d, props);
}

extern "C" ggml_backend_reg_t ggml_backend_dev_backend_reg(ggml_backend_dev_t d) {
    return d->reg;
}

extern "C" ggml_backend_t ggml_backend_dev_init(ggml_backend_dev_t d, const char * params) {
    return d->iface.init_backend(d, params);
}

extern "C" ggml_backend_buffer_type_t ggml_backend_dev_buffer_type(ggml_backend_dev_t d) {
    return d->iface.get_buffer_type(d);
}

extern "C" ggml_backend_buffer_type_t ggml_backend_dev_host_buffer_type(ggml_backend_dev_t d) {
    return d->iface.get_host_buffer_type ? d->iface.get_host_buffer_type(d) : nullptr;
}

extern "C" bool ggml_backend_dev_supports_op(ggml_backend_dev_t d, const struct ggml_tensor * op) {
    return d->iface.supports_op(d, op);
}

extern "C" bool ggml_backend_dev_supports_buft(ggml_backend_dev_t d, ggml_backend_buffer_type_t buft) {
    return d->iface.supports_buft(d, buft);
}

extern "C" bool ggml_backend_dev_offload_op(ggml_backend_dev_t d, const struct ggml_tensor * op) {
    return d->iface.offload_op ? d->iface.offload_op(d, op) : false;
}

extern "C" const char * ggml_backend_reg_name(ggml_backend_reg_t reg) {
    return reg->iface.get_name(reg);
}

extern "C" size_t ggml_backend_reg_dev_count(ggml_backend_reg_t reg) {
    return reg->iface.get_device_count(reg);
}

extern "C" ggml_backend_dev_t ggml_backend_reg_dev_get(ggml_backend_reg_t reg, size_t index) {
    return reg->iface.get_device(reg, index);
}

extern "C" void * ggml_backend_reg_get_proc_address(ggml_backend_reg_t reg, const char * name) {
    return reg->iface.get_proc_address ? reg->iface.get_proc_address(reg, name) : nullptr;
}

struct registry {
    std::vector<ggml_backend_reg_t> regs;
    std::vector<ggml_backend_dev_t> devs;
    std::vector<void *>             handles;
};

static registry & get_reg() {
    static registry r;
    return r;
}

extern "C" void ggml_backend_register(ggml_backend_reg_t reg) {
    if (!reg) {
        return;
    }
    registry & r = get_reg();
    for (auto * x : r.regs) {
        if (x == reg) {
            return;
        }
    }
    r.regs.push_back(reg);
    for (size_t i = 0; i < ggml_backend_reg_dev_count(reg); i++) {
        r.devs.push_back(ggml_backend_reg_dev_get(reg, i));
    }
}

extern "C" size_t ggml_backend_reg_count(void) {
    return get_reg().regs.size();
}

extern "C" ggml_backend_reg_t ggml_backend_reg_get(size_t index) {
    return index < get_reg().regs.size() ? get_reg().regs[index] : nullptr;
}

extern "C" ggml_backend_reg_t ggml_backend_reg_by_name(const char * name) {
    for (auto * r : get_reg().regs) {
        if (strcasecmp(ggml_backend_reg_name(r), name) == 0) {
            return r;
        }
    }
    return nullptr;
}

extern "C" size_t ggml_backend_dev_count(void) {
    return get_reg().devs.size();
}

extern "C" ggml_backend_dev_t ggml_backend_dev_get(size_t index) {
    return index < get_reg().devs.size() ? get_reg().devs[index] : nullptr;
}

extern "C" ggml_backend_dev_t ggml_backend_dev_by_name(const char * name) {
    for (auto * d : get_reg().devs) {
        if (strcasecmp(ggml_backend_dev_name(d), name) == 0) {
            return d;
        }
    }
    return nullptr;
}

extern "C" ggml_backend_dev_t ggml_backend_dev_by_type(enum ggml_backend_dev_type type) {
    for (auto * d : get_reg().devs) {
        if (ggml_backend_dev_type(d) == type) {
            return d;
        }
    }
    return nullptr;
}

extern "C" ggml_backend_t ggml_backend_init_by_name(const char * name, const char * params) {
    ggml_backend_dev_t d = ggml_backend_dev_by_name(name);
    return d ? ggml_backend_dev_init(d, params) : nullptr;
}

extern "C" ggml_backend_t ggml_backend_init_by_type(enum ggml_backend_dev_type type, const char * params) {
    ggml_backend_dev_t d = ggml_backend_dev_by_type(type);
    return d ? ggml_backend_dev_init(d, params) : nullptr;
}

extern "C" ggml_backend_t ggml_backend_init_best(void) {
    ggml_backend_dev_t d = ggml_backend_dev_by_type(GGML_BACKEND_DEVICE_TYPE_GPU);
    if (!d) {
        d = ggml_backend_dev_by_type(GGML_BACKEND_DEVICE_TYPE_CPU);
    }
    return d ? ggml_backend_dev_init(d, nullptr) : nullptr;
}

// Dynamic backends: libggml-*.so next to this library (or in
// GGML_BACKEND_PATH) exporting ggml_backend_init() are loaded and registered.
extern "C" void ggml_backend_load_all(void) {
    static bool done = false;
    if (done) {
        return;
    }
    done = true;
    std::vector<std::string> dirs;
    if (const char * p = getenv("GGML_BACKEND_PATH")) {
        dirs.emplace_back(p);
    }
    Dl_info info;
    if (dladdr((void *) &ggml_backend_load_all, &info) && info.dli_fname) {
        std::string f = info.dli_fname;
        size_t      s = f.find_last_of('/');
        dirs.push_back(s == std::string::npos ? "." : f.substr(0, s));
    }
    for (const auto & dir : dirs) {
        const std::string path = dir + "/libggml-mi355x.so";
        void *            h    = dlopen(path.c_str(), RTLD_NOW | RTLD_LOCAL);
        if (!h) {
            continue;
        }
        auto init = (ggml_backend_init_t) dlsym(h, "ggml_backend_init");
        if (!init) {
            dlclose(h);
            continue;
        }
        get_reg().handles.push_back(h);
        ggml_backend_register(init());
        break;
    }
}

// ---------------------------------------------------------------------------
// allocation of context tensors and graphs

extern "C" enum ggml_status ggml_backend_tensor_alloc(ggml_backend_buffer_t buffer, struct ggml_tensor * t,
                                                      void * addr) {
    CORE_ASSERT(t->buffer == nullptr && t->data == nullptr && t->view_src == nullptr);
    t->buffer = buffer;
    t->data   = addr;
    return ggml_backend_buffer_init_tensor(buffer, t);
}

extern "C" enum ggml_status ggml_backend_view_init(struct ggml_tensor * t) {
    CORE_ASSERT(t->view_src != nullptr && t->view_src->data != nullptr);
    t->buffer = t->view_src->buffer;
    t->data   = (char *) t->view_src->data + t->view_offs;
    return ggml_backend_buffer_init_tensor(t->buffer, t);
}

static ggml_backend_buffer_t alloc_tensors(const std::vector<struct ggml_tensor *> & ts, ggml_backend_buffer_type_t buft,
                                           ggml_backend_buffer_t reuse) {
    const size_t        align = ggml_backend_buft_get_alignment(buft);
    std::vector<size_t> offs(ts.size());
    size_t              total = 0;
    for (size_t i = 0; i < ts.size(); i++) {
        offs[i] = total;
        total += GGML_PAD(ggml_backend_buft_get_alloc_size(buft, ts[i]), align);
    }
    ggml_backend_buffer_t buf = reuse;
    if (!buf || buf->size < total) {
        if (buf) {
            ggml_backend_buffer_free(buf);
        }
        buf = ggml_backend_buft_alloc_buffer(buft, total ? total : align);
        if (!buf) {
            return nullptr;
        }
    }
    char * base = (char *) ggml_backend_buffer_get_base(buf);
    for (size_t i = 0; i < ts.size(); i++) {
        ts[i]->buffer = nullptr;
        ts[i]->data   = nullptr;
        ggml_backend_tensor_alloc(buf, ts[i], base + offs[i]);
    }
    return buf;
}

extern "C" struct ggml_backend_buffer * ggml_backend_alloc_ctx_tensors_from_buft(struct ggml_context *      ctx,
                                                                                ggml_backend_buffer_type_t buft) {
    std::vector<struct ggml_tensor *> ts, views;
    for (struct ggml_tensor * t = ggml_get_first_tensor(ctx); t; t = ggml_get_next_tensor(ctx, t)) {
        if (t->data == nullptr) {
            (t->view_src ? views : ts).push_back(t);
        }
    }
    if (ts.empty()) {
        return nullptr;
    }
    ggml_backend_buffer_t buf = alloc_tensors(ts, buft, nullptr);
    for (auto * v : views) {
        if (v->view_src->data) {
            ggml_backend_view_init(v);
        }
    }
    return buf;
}

extern "C" struct ggml_backend_buffer * ggml_backend_alloc_ctx_tensors(struct ggml_context * ctx,
                                                                      ggml_backend_t        backend) {
    return ggml_backend_alloc_ctx_tensors_from_buft(ctx, ggml_backend_get_default_buffer_type(backend));
}

struct ggml_gallocr {
    ggml_backend_buffer_type_t buft;
    ggml_backend_buffer_t      buffer;
};

extern "C" ggml_gallocr_t ggml_gallocr_new(ggml_backend_buffer_type_t buft) {
    return new ggml_gallocr{ buft, nullptr };
}

extern "C" void ggml_gallocr_free(ggml_gallocr_t g) {
    if (!g) {
        return;
    }
    ggml_backend_buffer_free(g->buffer);
    delete g;
}

static void collect_graph(struct ggml_cgraph * graph, std::vector<struct ggml_tensor *> & own,
                          std::vector<struct ggml_tensor *> & views) {
    auto add = [&](struct ggml_tensor * t) {
        if (t->data != nullptr && t->buffer != nullptr) {
            return;  // pre-allocated (weights, caches)
        }
        if (t->view_src) {
            views.push_back(t);
        } else {
            own.push_back(t);
        }
    };
    for (int i = 0; i < graph->n_leafs; i++) {
        add(graph->leafs[i]);
    }
    for (int i = 0; i < graph->n_nodes; i++) {
        add(graph->nodes[i]);
    }
}

extern "C" bool ggml_gallocr_reserve(ggml_gallocr_t g, struct ggml_cgraph * graph) {
    return ggml_gallocr_alloc_graph(g, graph);
}

// Every non-view tensor without memory gets its own slot (no reuse); views are
// resolved after their base tensors.
extern "C" bool ggml_gallocr_alloc_graph(ggml_gallocr_t g, struct ggml_cgraph * graph) {
    std::vector<struct ggml_tensor *> own, views;
    // tensors allocated by a previous call of this allocator are re-laid out
    for (int i = 0; i < graph->n_leafs + graph->n_nodes; i++) {
        struct ggml_tensor * t = i < graph->n_leafs ? graph->leafs[i] : graph->nodes[i - graph->n_leafs];
        if (g->buffer && t->buffer == g->buffer) {
            t->buffer = nullptr;
            t->data   = nullptr;
        }
    }
    collect_graph(graph, own, views);
    if (!own.empty()) {
        ggml_backend_buffer_t b = alloc_tensors(own, g->buft, g->buffer);
        if (!b) {
            return false;
        }
        g->buffer = b;
        ggml_backend_buffer_set_usage(b, GGML_BACKEND_BUFFER_USAGE_COMPUTE);
    }
    for (auto * v : views) {
        if (!v->view_src->data) {
            return false;
        }
        ggml_backend_view_init(v);
    }
    return true;
}

extern "C" size_t ggml_gallocr_get_buffer_size(ggml_gallocr_t g, int buffer_id) {
    (void) buffer_id;
    return g->buffer ? g->buffer->size : 0;
}

// ---------------------------------------------------------------------------
// type traits: host decoders of the GGUF block layouts (to_float)
//
// Q8_0: 32 elements per 34-byte block {f16 d; i8 qs[32]}, y = d * q.
// Q4_K: 256 per 144 bytes {f16 d; f16 dmin; u8 scales[12]; u8 qs[128]}: eight
//   6-bit (scale, min) pairs packed in scales[] (pairs 0..3 in the low six bits
//   of bytes 0..3 / 4..7; pairs 4..7 from the nibbles of bytes 8..11 with their
//   top two bits in the high bits of bytes 0..3 / 4..7); each 64-element chunk
//   j takes its low nibbles with pair 2j and its high nibbles with pair 2j+1,
//   y = (d * sc) * q - (dmin * m).
// Q5_K: 256 per 176 bytes {f16 d; f16 dmin; u8 scales[12]; u8 qh[32];
//   u8 qs[128]}: Q4_K's scales and nibbles, plus a fifth quant bit per
//   element (bit j of qh[l] for element 32j + l), q in [0, 31].
// Q6_K: 256 per 210 bytes {u8 ql[128]; u8 qh[64]; i8 scales[16]; f16 d}: each
//   128-element half takes 64 bytes of ql (low nibbles then high nibbles of
//   two 32-byte rows) and 32 bytes of qh (two bits per element), q in
//   [0, 63], y = (d * scale[16-element group]) * (q - 32).

namespace {

float h2f(const uint8_t * p) {
    ggml_fp16_t h;
    memcpy(&h, p, 2);
    return ggml_fp16_to_fp32(h);
}

void to_float_f16(const void * x, float * y, int64_t k) {
    ggml_fp16_to_fp32_row((const ggml_fp16_t *) x, y, k);
}

void to_float_bf16(const void * x, float * y, int64_t k) {
    ggml_bf16_to_fp32_row((const ggml_bf16_t *) x, y, k);
}

void to_float_q8_0(const void * x, float * y, int64_t k) {
    const uint8_t * b = (const uint8_t *) x;
    for (int64_t i = 0; i < k / 32; i++, b += 34) {
        const float d = h2f(b);
        for (int j = 0; j < 32; j++) {
            y[i * 32 + j] = d * (float) (int8_t) b[2 + j];
        }
    }
}

void q4_k_pair(int j, const uint8_t * sc, uint8_t & s, uint8_t & m) {
    if (j < 4) {
        s = sc[j] & 63;
        m = sc[j + 4] & 63;
    } else {
        s = (uint8_t) ((sc[j + 4] & 0x0F) | ((sc[j - 4] >> 6) << 4));
        m = (uint8_t) ((sc[j + 4] >> 4) | ((sc[j] >> 6) << 4));
    }
}

void to_float_q4_k(const void * x, float * y, int64_t k) {
    const uint8_t * b = (const uint8_t *) x;
    for (int64_t i = 0; i < k / 256; i++, b += 144) {
        const float     d    = h2f(b);
        const float     dmin = h2f(b + 2);
        const uint8_t * sc   = b + 4;
        const uint8_t * q    = b + 16;
        float *         out  = y + i * 256;
        for (int c = 0; c < 4; c++) {
            uint8_t s0, m0, s1, m1;
            q4_k_pair(2 * c, sc, s0, m0);
            q4_k_pair(2 * c + 1, sc, s1, m1);
            const float d0 = d * s0, n0 = dmin * m0, d1 = d * s1, n1 = dmin * m1;
            for (int l = 0; l < 32; l++) {
                out[64 * c + l]      = d0 * (float) (q[32 * c + l] & 0x0F) - n0;
                out[64 * c + 32 + l] = d1 * (float) (q[32 * c + l] >> 4) - n1;
            }
        }
    }
}

void to_float_q5_k(const void * x, float * y, int64_t k) {
    const uint8_t * b = (const uint8_t *) x;
    for (int64_t i = 0; i < k / 256; i++, b += 176) {
        const float     d    = h2f(b);
        const float     dmin = h2f(b + 2);
        const uint8_t * sc   = b + 4;
        const uint8_t * qh   = b + 16;
        const uint8_t * q    = b + 48;
        float *         out  = y + i * 256;
        for (int c = 0; c < 4; c++) {
            uint8_t s0, m0, s1, m1;
            q4_k_pair(2 * c, sc, s0, m0);
            q4_k_pair(2 * c + 1, sc, s1, m1);
            const float d0 = d * s0, n0 = dmin * m0, d1 = d * s1, n1 = dmin * m1;
            for (int l = 0; l < 32; l++) {
                const int lo = (q[32 * c + l] & 0x0F) | (((qh[l] >> (2 * c)) & 1) << 4);
                const int hi = (q[32 * c + l] >> 4) | (((qh[l] >> (2 * c + 1)) & 1) << 4);
                out[64 * c + l]      = d0 * (float) lo - n0;
                out[64 * c + 32 + l] = d1 * (float) hi - n1;
            }
        }
    }
}

void to_float_q6_k(const void * x, float * y, int64_t k) {
    const uint8_t * b = (const uint8_t *) x;
    for (int64_t i = 0; i < k / 256; i++, b += 210) {
        const float d = h2f(b + 208);
        for (int h = 0; h < 2; h++) {
            const uint8_t * ql  = b + 64 * h;
            const uint8_t * qh  = b + 128 + 32 * h;
            const int8_t *  sc  = (const int8_t *) (b + 192 + 8 * h);
            float *         out = y + i * 256 + 128 * h;
            for (int l = 0; l < 32; l++) {
                const int g  = l / 16;
                const int q1 = (int) ((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int q2 = (int) ((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int q3 = (int) ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int q4 = (int) ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                out[l]      = (d * (float) sc[g]) * (float) q1;
                out[l + 32] = (d * (float) sc[g + 2]) * (float) q2;
                out[l + 64] = (d * (float) sc[g + 4]) * (float) q3;
                out[l + 96] = (d * (float) sc[g + 6]) * (float) q4;
            }
        }
    }
}

}  // namespace

extern "C" const struct ggml_type_traits * ggml_get_type_traits(enum ggml_type type) {
    static ggml_type_traits table[GGML_TYPE_COUNT];
    static bool             init = false;
    if (!init) {
        for (int t = 0; t < GGML_TYPE_COUNT; t++) {
            const type_info ti = tinfo((enum ggml_type) t);
            table[t]           = { ti.name, ti.blck, 0, ti.size, ti.quantized, nullptr, nullptr };
        }
        table[GGML_TYPE_F16].to_float  = to_float_f16;
        table[GGML_TYPE_BF16].to_float = to_float_bf16;
        table[GGML_TYPE_Q8_0].to_float = to_float_q8_0;
        table[GGML_TYPE_Q4_K].to_float = to_float_q4_k;
        table[GGML_TYPE_Q5_K].to_float = to_float_q5_k;
        table[GGML_TYPE_Q6_K].to_float = to_float_q6_k;
        init                           = true;
    }
    CORE_ASSERT(type >= 0 && type < GGML_TYPE_COUNT);
    return &table[type];
}

// ---------------------------------------------------------------------------
// scheduler: the whole graph on the first listed backend that runs every node

struct ggml_backend_sched {
    std::vector<ggml_backend_t>             backends;
    std::vector<ggml_backend_buffer_type_t> bufts;
    std::vector<ggml_gallocr_t>             galloc;  // one per backend, made on first use
    int                                     chosen = -1;  // backend of the allocated graph
};

extern "C" ggml_backend_sched_t ggml_backend_sched_new(ggml_backend_t * backends, ggml_backend_buffer_type_t * bufts,
                                                       int n_backends, size_t graph_size, bool parallel,
                                                       bool op_offload) {
    (void) graph_size;
    (void) parallel;
    (void) op_offload;
    if (!backends || n_backends < 1) {
        return nullptr;
    }
    auto * s = new ggml_backend_sched();
    for (int i = 0; i < n_backends; i++) {
        if (!backends[i]) {
            delete s;
            return nullptr;
        }
        s->backends.push_back(backends[i]);
        s->bufts.push_back(bufts && bufts[i] ? bufts[i] : ggml_backend_get_default_buffer_type(backends[i]));
    }
    s->galloc.assign(s->backends.size(), nullptr);
    return s;
}

extern "C" void ggml_backend_sched_free(ggml_backend_sched_t s) {
    if (!s) {
        return;
    }
    for (auto * g : s->galloc) {
        if (g) {
            ggml_gallocr_free(g);
        }
    }
    delete s;
}

extern "C" void ggml_backend_sched_reset(ggml_backend_sched_t s) {
    s->chosen = -1;
}

extern "C" int ggml_backend_sched_get_n_backends(ggml_backend_sched_t s) {
    return (int) s->backends.size();
}

extern "C" ggml_backend_t ggml_backend_sched_get_backend(ggml_backend_sched_t s, int i) {
    return i >= 0 && (size_t) i < s->backends.size() ? s->backends[(size_t) i] : nullptr;
}

extern "C" int ggml_backend_sched_get_n_splits(ggml_backend_sched_t s) {
    return s->chosen >= 0 ? 1 : 0;
}

extern "C" int ggml_backend_sched_get_n_copies(ggml_backend_sched_t s) {
    (void) s;
    return 1;
}

extern "C" void ggml_backend_sched_set_tensor_backend(ggml_backend_sched_t s, struct ggml_tensor * node,
                                                      ggml_backend_t backend) {
    (void) s;
    (void) node;
    (void) backend;  // placement is per graph in this scheduler
}

extern "C" ggml_backend_t ggml_backend_sched_get_tensor_backend(ggml_backend_sched_t s, struct ggml_tensor * node) {
    (void) node;
    return s->chosen >= 0 ? s->backends[(size_t) s->chosen] : nullptr;
}

// Can backend i run the whole graph: every node supported, and every tensor
// already placed in a buffer (weights, caches) usable by that backend.
static bool sched_fits(ggml_backend_sched_t s, size_t i, struct ggml_cgraph * g, const struct ggml_tensor ** bad) {
    ggml_backend_t b = s->backends[i];
    for (int n = 0; n < g->n_nodes; n++) {
        const struct ggml_tensor * t = g->nodes[n];
        if (!ggml_backend_supports_op(b, t)) {
            *bad = t;
            return false;
        }
        for (int k = 0; k < GGML_MAX_SRC; k++) {
            const struct ggml_tensor * src = t->src[k];
            if (!src) {
                continue;
            }
            const struct ggml_tensor * base = src->view_src ? src->view_src : src;
            if (base->buffer && !ggml_backend_supports_buft(b, ggml_backend_buffer_get_type(base->buffer))) {
                *bad = t;
                return false;
            }
        }
    }
    return true;
}

extern "C" bool ggml_backend_sched_reserve(ggml_backend_sched_t s, struct ggml_cgraph * g) {
    const struct ggml_tensor * bad = nullptr;
    for (size_t i = 0; i < s->backends.size(); i++) {
        if (sched_fits(s, i, g, &bad)) {
            if (!s->galloc[i]) {
                s->galloc[i] = ggml_gallocr_new(s->bufts[i]);
            }
            return s->galloc[i] && ggml_gallocr_reserve(s->galloc[i], g);
        }
    }
    return false;
}

extern "C" bool ggml_backend_sched_alloc_graph(ggml_backend_sched_t s, struct ggml_cgraph * g) {
    const struct ggml_tensor * bad = nullptr;
    for (size_t i = 0; i < s->backends.size(); i++) {
        if (!sched_fits(s, i, g, &bad)) {
            continue;
        }
        if (!s->galloc[i]) {
            s->galloc[i] = ggml_gallocr_new(s->bufts[i]);
        }
        if (!s->galloc[i] || !ggml_gallocr_alloc_graph(s->galloc[i], g)) {
            core_log(GGML_LOG_LEVEL_ERROR, "ggml_backend_sched_alloc_graph: allocation on %s failed\n",
                     ggml_backend_name(s->backends[i]));
            return false;
        }
        s->chosen = (int) i;
        return true;
    }
    core_log(GGML_LOG_LEVEL_ERROR,
             "ggml_backend_sched_alloc_graph: no backend runs the whole graph (first refusal: node %s, %s); this "
             "build has no CPU compute backend to split to\n",
             bad ? bad->name : "?", bad ? ggml_op_name(bad->op) : "?");
    return false;
}

extern "C" enum ggml_status ggml_backend_sched_graph_compute_async(ggml_backend_sched_t s, struct ggml_cgraph * g) {
    if (s->chosen < 0 && !ggml_backend_sched_alloc_graph(s, g)) {
        return GGML_STATUS_ALLOC_FAILED;
    }
    return ggml_backend_graph_compute_async(s->backends[(size_t) s->chosen], g);
}

extern "C" void ggml_backend_sched_synchronize(ggml_backend_sched_t s) {
    for (auto * b : s->backends) {
        ggml_backend_synchronize(b);
    }
}

extern "C" enum ggml_status ggml_backend_sched_graph_compute(ggml_backend_sched_t s, struct ggml_cgraph * g) {
    const enum ggml_status st = ggml_backend_sched_graph_compute_async(s, g);
    ggml_backend_sched_synchronize(s);
    return st;
}
