// mm_lm.cpp - Qwen3-shape LM batched CFG decode step on the MI355X ggml
// backend (include/mm_lm.h).  The graph construction follows
// qw3lm_forward_batch (src/qwen3-lm.h:645-934) with its helpers
// qwen3_rms_norm / qwen3_linear / qwen3_build_mlp (src/qwen3-enc.h:67-115):
// same ops, same order, same views, so the backend sees the node sequence
// the reference hands to ggml_backend_graph_compute.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <vector>

#include "ggml-alloc.h"
#include "ggml-backend.h"
#include "ggml-mi355x.h"
#include "ggml.h"
#include "mm_lm.h"
#include "mmhip.h"
#include "mmhip_synth.h"

namespace {

thread_local char g_err[512];

int err(const char * fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return -1;
}

constexpr int GRAPH_NODES = 16384;  // QW3LM_GRAPH_NODES, src/qwen3-lm.h:35

struct Layer {
    ggml_tensor * input_layernorm;
    ggml_tensor * qkv;  // [H, q_dim + 2 kv_dim]: q | k | v rows (one type)
    ggml_tensor * qk;   // [H, q_dim + kv_dim]: q | k rows, when v's type differs
    ggml_tensor * v;    // [H, kv_dim]
    ggml_tensor * q_norm;
    ggml_tensor * k_norm;
    ggml_tensor * o_proj;
    ggml_tensor * post_attn_layernorm;
    ggml_tensor * gate_up;  // [H, 2 ffn]: gate | up rows
    ggml_tensor * down;
};

struct Lm {
    mm_lm_config          c;
    ggml_backend_t        backend = nullptr;
    bool                  owns_backend = true;
    ggml_context *        wctx    = nullptr;
    ggml_backend_buffer_t wbuf    = nullptr;
    std::vector<Layer>    layers;
    ggml_tensor *         final_norm = nullptr;
    ggml_tensor *         lm_head    = nullptr;

    ggml_context *             kv_ctx = nullptr;
    ggml_backend_buffer_t      kv_buf = nullptr;
    std::vector<ggml_tensor *> kv_k4, kv_v4;
    std::vector<int>           kv_pos;

    // persistent arena + static graph (src/graph-arena.h, src/static-graph.h)
    ggml_context * arena   = nullptr;
    ggml_gallocr_t galloc  = nullptr;
    bool           built   = false;
    int            key_pad = 0, key_N = 0, key_s0 = 0;
    ggml_cgraph *  gf         = nullptr;
    ggml_tensor *  embeds_t   = nullptr;
    ggml_tensor *  positions  = nullptr;
    ggml_tensor *  kv_rows    = nullptr;
    ggml_tensor *  attn_mask  = nullptr;
    ggml_tensor *  lgt        = nullptr;
    ggml_tensor *  hidden_out = nullptr;

    std::vector<int32_t>  pos_data;
    std::vector<int64_t>  rows_data;
    std::vector<uint16_t> mask_data;
};

ggml_tensor * rms_norm_mul(ggml_context * ctx, ggml_tensor * x, ggml_tensor * w, float eps) {
    return ggml_mul(ctx, ggml_rms_norm(ctx, x, eps), w);  // qwen3_rms_norm
}

// Fill a quantized weight with synthetic GGUF blocks (staged on the device,
// then converted to the row-grouped layout).
bool fill_quant(ggml_tensor * t, uint64_t seed) {
    const int64_t rows   = ggml_nrows(t);
    const int64_t bsize  = ggml_blck_size(t->type);
    const int64_t blocks = ggml_nelements(t) / bsize;
    void *        stage  = nullptr;
    if (hipMalloc(&stage, ggml_nbytes(t)) != hipSuccess) {
        return false;
    }
    bool ok = mmhip_synth_gguf(t->type, stage, blocks, seed, nullptr) == MMHIP_OK &&
              mmhip_repack_rows(t->type, stage, t->data, rows, t->ne[0], nullptr) == MMHIP_OK &&
              hipDeviceSynchronize() == hipSuccess;
    (void) hipFree(stage);
    return ok;
}

bool fill_normal(ggml_tensor * t, uint64_t seed, float mean, float stdv) {
    const int ty = t->type == GGML_TYPE_F16 ? 1 : t->type == GGML_TYPE_BF16 ? 30 : 0;
    if (!(t->type == GGML_TYPE_F16 || t->type == GGML_TYPE_BF16 || t->type == GGML_TYPE_F32)) {
        return false;
    }
    return mmhip_synth_normal(ty, t->data, ggml_nelements(t), seed, mean, stdv, nullptr) == MMHIP_OK &&
           hipDeviceSynchronize() == hipSuccess;
}

// Weights and caches by name, then the current decode graph's tensors (the
// graph allocator gives each its own memory, so a node's rows stay readable
// until the next step).
// The "_M" variants' choice of layers whose V and down projections take the
// larger type (tools/quantize.cpp:127-150, bump_mode 2): the first n/9, the
// last n/7 and every third layer.
bool lm_layer_bumped(const mm_lm_config & c, int l) {
    const int n = c.n_layers;
    return c.bump_type != 0 && c.bump_type != c.wtype && (l < n / 9 || l >= n - n / 7 || l % 3 == 0);
}

ggml_tensor * find_tensor(Lm * m, const char * name) {
    ggml_tensor * t = ggml_get_tensor(m->wctx, name);
    t               = t ? t : ggml_get_tensor(m->kv_ctx, name);
    return t || !m->gf ? t : ggml_graph_get_tensor(m->gf, name);
}

// Build the batched decode graph: src/qwen3-lm.h:695-856.
void build_graph(Lm * m, int N, int n_kv_pad, int s0) {
    const mm_lm_config & c   = m->c;
    const int            H   = c.hidden;
    const int            D   = c.head_dim;
    const int            Nh  = c.n_heads;
    const int            Nkv = c.n_kv_heads;

    ggml_reset(m->arena);  // graph_arena_begin
    ggml_context * ctx = m->arena;
    m->gf              = ggml_new_graph_custom(ctx, GRAPH_NODES, false);
    ggml_cgraph * gf   = m->gf;

    m->embeds_t = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, H, N);
    ggml_set_name(m->embeds_t, "input_embeds");
    ggml_set_input(m->embeds_t);
    m->positions = ggml_new_tensor_1d(ctx, GGML_TYPE_I32, N);
    ggml_set_name(m->positions, "positions");
    ggml_set_input(m->positions);
    m->attn_mask = ggml_new_tensor_4d(ctx, GGML_TYPE_F16, n_kv_pad, 1, 1, N);
    ggml_set_name(m->attn_mask, "attn_mask");
    ggml_set_input(m->attn_mask);
    m->kv_rows = ggml_new_tensor_3d(ctx, GGML_TYPE_I64, 1, 1, N);
    ggml_set_name(m->kv_rows, "kv_rows");
    ggml_set_input(m->kv_rows);

    ggml_tensor * hidden = m->embeds_t;
    const int     q_dim  = Nh * D;
    const int     kv_dim = Nkv * D;
    const float   scale  = 1.0f / sqrtf((float) D);

    for (int l = 0; l < c.n_layers; l++) {
        Layer * ly = &m->layers[(size_t) l];

        ggml_tensor * norm = rms_norm_mul(ctx, hidden, ly->input_layernorm, c.rms_eps);

        // fused Q | K | V, or fused Q | K and a separate V (src/qwen3-lm.h:742-757)
        ggml_tensor *q, *k, *v;
        if (ly->qkv) {
            ggml_tensor * qkv = ggml_mul_mat(ctx, ly->qkv, norm);
            q = ggml_cont(ctx, ggml_view_2d(ctx, qkv, q_dim, N, qkv->nb[1], 0));
            k = ggml_cont(ctx, ggml_view_2d(ctx, qkv, kv_dim, N, qkv->nb[1], (size_t) q_dim * qkv->nb[0]));
            v = ggml_cont(ctx, ggml_view_2d(ctx, qkv, kv_dim, N, qkv->nb[1], (size_t) (q_dim + kv_dim) * qkv->nb[0]));
        } else {
            ggml_tensor * qk = ggml_mul_mat(ctx, ly->qk, norm);
            q = ggml_cont(ctx, ggml_view_2d(ctx, qk, q_dim, N, qk->nb[1], 0));
            k = ggml_cont(ctx, ggml_view_2d(ctx, qk, kv_dim, N, qk->nb[1], (size_t) q_dim * qk->nb[0]));
            v = ggml_mul_mat(ctx, ly->v, norm);
        }

        q = ggml_reshape_3d(ctx, q, D, Nh, N);
        k = ggml_reshape_3d(ctx, k, D, Nkv, N);
        v = ggml_reshape_3d(ctx, v, D, Nkv, N);

        q = rms_norm_mul(ctx, q, ly->q_norm, c.rms_eps);
        k = rms_norm_mul(ctx, k, ly->k_norm, c.rms_eps);

        q = ggml_rope_ext(ctx, q, m->positions, NULL, D, GGML_ROPE_TYPE_NEOX, 0, c.rope_theta, 1.0f, 0.0f, 1.0f, 0.0f,
                          0.0f);
        k = ggml_rope_ext(ctx, k, m->positions, NULL, D, GGML_ROPE_TYPE_NEOX, 0, c.rope_theta, 1.0f, 0.0f, 1.0f, 0.0f,
                          0.0f);

        q = ggml_cont(ctx, q);
        k = ggml_cont(ctx, k);
        v = ggml_cont(ctx, v);

        ggml_tensor * kk    = m->kv_k4[(size_t) l];
        ggml_tensor * vv    = m->kv_v4[(size_t) l];
        const size_t  off   = (size_t) s0 * kk->nb[3];
        ggml_tensor * k_set = ggml_view_4d(ctx, kk, D, c.max_seq, Nkv, N, kk->nb[1], kk->nb[2], kk->nb[3], off);
        ggml_tensor * v_set = ggml_view_4d(ctx, vv, D, c.max_seq, Nkv, N, vv->nb[1], vv->nb[2], vv->nb[3], off);
        ggml_tensor * k_new = ggml_reshape_4d(ctx, k, D, 1, Nkv, N);
        ggml_tensor * v_new = ggml_reshape_4d(ctx, v, D, 1, Nkv, N);
        ggml_build_forward_expand(gf, ggml_set_rows(ctx, k_set, k_new, m->kv_rows));
        ggml_build_forward_expand(gf, ggml_set_rows(ctx, v_set, v_new, m->kv_rows));

        ggml_tensor * q4      = ggml_reshape_4d(ctx, q, D, 1, Nh, N);
        ggml_tensor * k_batch = ggml_view_4d(ctx, kk, D, n_kv_pad, Nkv, N, kk->nb[1], kk->nb[2], kk->nb[3], off);
        ggml_tensor * v_batch = ggml_view_4d(ctx, vv, D, n_kv_pad, Nkv, N, vv->nb[1], vv->nb[2], vv->nb[3], off);

        ggml_tensor * attn = ggml_flash_attn_ext(ctx, q4, k_batch, v_batch, m->attn_mask, scale, 0.0f, 0.0f);
        ggml_flash_attn_ext_set_prec(attn, GGML_PREC_F32);
        ggml_tensor * attn_cat = ggml_reshape_2d(ctx, attn, Nh * D, N);

        ggml_tensor * attn_out = ggml_mul_mat(ctx, ly->o_proj, attn_cat);
        hidden                 = ggml_add(ctx, hidden, attn_out);

        norm             = rms_norm_mul(ctx, hidden, ly->post_attn_layernorm, c.rms_eps);
        ggml_tensor * gu = ggml_mul_mat(ctx, ly->gate_up, norm);
        ggml_tensor * ff = ggml_swiglu(ctx, gu);
        ggml_tensor * mlp = ggml_mul_mat(ctx, ly->down, ff);
        hidden            = ggml_add(ctx, hidden, mlp);
        ggml_format_name(hidden, "layer_out-%d", l);  // readable after the step (mm_lm_get_tensor)
    }

    hidden = rms_norm_mul(ctx, hidden, m->final_norm, c.rms_eps);
    ggml_set_name(hidden, "hidden_out");
    ggml_set_output(hidden);
    ggml_build_forward_expand(gf, hidden);
    m->hidden_out = hidden;
    m->lgt        = ggml_mul_mat(ctx, m->lm_head, hidden);
    ggml_set_name(m->lgt, "logits");
    ggml_set_output(m->lgt);
    ggml_build_forward_expand(gf, m->lgt);
}

int prepare(Lm * m, const float * embeds, const int * kv_sets, int N) {
    const mm_lm_config & c = m->c;
    if (N <= 0 || N > c.n_sets) {
        return err("decode: N=%d out of range", N);
    }
    const int s0 = kv_sets[0];
    for (int i = 0; i < N; i++) {
        if (kv_sets[i] != s0 + i || kv_sets[i] < 0 || kv_sets[i] >= c.n_sets) {
            return err("decode: kv sets must be consecutive and in range");
        }
    }
    int max_kv_len = 0;
    for (int i = 0; i < N; i++) {
        const int kl = m->kv_pos[(size_t) kv_sets[i]] + 1;
        if (kl > c.max_seq) {
            return err("decode: kv_len %d > max_seq %d (set %d)", kl, c.max_seq, kv_sets[i]);
        }
        max_kv_len = kl > max_kv_len ? kl : max_kv_len;
    }
    const int pad_raw  = (int) GGML_PAD(max_kv_len, 256);
    const int n_kv_pad = pad_raw < c.max_seq ? pad_raw : c.max_seq;
    if (!m->built || m->key_pad != n_kv_pad || m->key_N != N || m->key_s0 != s0) {
        if (m->galloc) {
            ggml_gallocr_free(m->galloc);
            m->galloc = nullptr;
        }
        m->built = false;
        build_graph(m, N, n_kv_pad, s0);
        for (int i = 0; i < ggml_graph_n_nodes(m->gf); i++) {
            if (!ggml_backend_supports_op(m->backend, ggml_graph_node(m->gf, i))) {
                return err("decode: node %s (%s) not supported", ggml_graph_node(m->gf, i)->name,
                           ggml_op_name(ggml_graph_node(m->gf, i)->op));
            }
        }
        m->galloc = ggml_gallocr_new(ggml_backend_get_default_buffer_type(m->backend));
        if (!ggml_gallocr_alloc_graph(m->galloc, m->gf)) {
            return err("decode: graph allocation failed");
        }
        m->key_pad = n_kv_pad;
        m->key_N   = N;
        m->key_s0  = s0;
        m->pos_data.resize((size_t) N);
        m->rows_data.resize((size_t) N);
        m->mask_data.resize((size_t) n_kv_pad * N);
        m->built = true;
    }
    ggml_backend_tensor_set(m->embeds_t, embeds, 0, (size_t) N * c.hidden * sizeof(float));
    for (int i = 0; i < N; i++) {
        m->pos_data[(size_t) i]  = m->kv_pos[(size_t) kv_sets[i]];
        m->rows_data[(size_t) i] = (int64_t) m->kv_pos[(size_t) kv_sets[i]];
    }
    ggml_backend_tensor_set(m->positions, m->pos_data.data(), 0, (size_t) N * sizeof(int32_t));
    ggml_backend_tensor_set(m->kv_rows, m->rows_data.data(), 0, (size_t) N * sizeof(int64_t));
    const uint16_t zero = ggml_fp32_to_fp16(0.0f), ninf = ggml_fp32_to_fp16(-INFINITY);
    for (int i = 0; i < N; i++) {
        const int kvl = m->kv_pos[(size_t) kv_sets[i]] + 1;
        for (int j = 0; j < n_kv_pad; j++) {
            m->mask_data[(size_t) i * n_kv_pad + j] = j < kvl ? zero : ninf;
        }
    }
    ggml_backend_tensor_set(m->attn_mask, m->mask_data.data(), 0, m->mask_data.size() * sizeof(uint16_t));
    return 0;
}

}  // namespace

extern "C" const char * mm_lm_error(void) {
    return g_err;
}

namespace {

// backend: an MI355X backend shared with other modules (not owned), or NULL
// to create one on `device` (owned)
void * lm_create(const mm_lm_config * cfg, int device, ggml_backend_t backend, uint64_t seed) {
    g_err[0] = 0;
    if (!cfg || cfg->n_layers <= 0 || cfg->n_heads % cfg->n_kv_heads != 0 || cfg->n_sets <= 0 ||
        cfg->hidden % 256 != 0 || cfg->ffn % 256 != 0 || (cfg->n_heads * cfg->head_dim) % 256 != 0) {
        err("create: bad config");
        return nullptr;
    }
    if (cfg->bump_type != 0 && !(cfg->bump_type == GGML_TYPE_Q8_0 || cfg->bump_type == GGML_TYPE_Q4_K ||
                                 cfg->bump_type == GGML_TYPE_Q5_K || cfg->bump_type == GGML_TYPE_Q6_K)) {
        err("create: bad bump_type %d", cfg->bump_type);
        return nullptr;
    }
    if (backend && !ggml_backend_is_mi355x(backend)) {
        err("create: the backend is not an MI355X backend");
        return nullptr;
    }
    Lm * m = new Lm();
    m->c   = *cfg;
    const mm_lm_config & c = m->c;
    m->owns_backend        = backend == nullptr;
    m->backend             = backend ? backend : ggml_backend_mi355x_init(device);
    if (!m->backend) {
        err("create: no MI355X device %d", device);
        delete m;
        return nullptr;
    }
    const enum ggml_type wt     = (enum ggml_type) c.wtype;
    const int            q_dim  = c.n_heads * c.head_dim;
    const int            kv_dim = c.n_kv_heads * c.head_dim;

    // weights (src/qwen3-enc.h:119-160 layout: ne0 = input dim)
    const size_t n_w = (size_t) c.n_layers * 9 + 4;
    m->wctx          = ggml_init({ n_w * ggml_tensor_overhead() + 1024, nullptr, true });
    m->layers.resize((size_t) c.n_layers);
    char name[96];
    for (int l = 0; l < c.n_layers; l++) {
        Layer & ly              = m->layers[(size_t) l];
        const bool bump         = lm_layer_bumped(c, l);
        const enum ggml_type bt = bump ? (enum ggml_type) c.bump_type : wt;
        ly.input_layernorm      = ggml_new_tensor_1d(m->wctx, GGML_TYPE_F32, c.hidden);
        ly.qkv                  = bt == wt ? ggml_new_tensor_2d(m->wctx, wt, c.hidden, q_dim + 2 * kv_dim) : nullptr;
        ly.qk                   = bt == wt ? nullptr : ggml_new_tensor_2d(m->wctx, wt, c.hidden, q_dim + kv_dim);
        ly.v                    = bt == wt ? nullptr : ggml_new_tensor_2d(m->wctx, bt, c.hidden, kv_dim);
        ly.q_norm               = ggml_new_tensor_1d(m->wctx, GGML_TYPE_F32, c.head_dim);
        ly.k_norm               = ggml_new_tensor_1d(m->wctx, GGML_TYPE_F32, c.head_dim);
        ly.o_proj               = ggml_new_tensor_2d(m->wctx, wt, q_dim, c.hidden);
        ly.post_attn_layernorm  = ggml_new_tensor_1d(m->wctx, GGML_TYPE_F32, c.hidden);
        ly.gate_up              = ggml_new_tensor_2d(m->wctx, wt, c.hidden, 2 * c.ffn);
        ly.down                 = ggml_new_tensor_2d(m->wctx, bt, c.ffn, c.hidden);
        const char * names[10]  = { "attn_norm", "qkv", "qk", "v", "q_norm", "k_norm", "o_proj", "ffn_norm",
                                    "gate_up", "down" };
        ggml_tensor * ts[10] = { ly.input_layernorm, ly.qkv, ly.qk, ly.v, ly.q_norm, ly.k_norm,
                                 ly.o_proj, ly.post_attn_layernorm, ly.gate_up, ly.down };
        for (int i = 0; i < 10; i++) {
            if (ts[i]) {
                snprintf(name, sizeof(name), "blk.%d.%s", l, names[i]);
                ggml_set_name(ts[i], name);
            }
        }
    }
    m->final_norm = ggml_new_tensor_1d(m->wctx, GGML_TYPE_F32, c.hidden);
    ggml_set_name(m->final_norm, "output_norm");
    m->lm_head = ggml_new_tensor_2d(m->wctx, wt, c.hidden, c.vocab);
    ggml_set_name(m->lm_head, "lm_head");
    m->wbuf = ggml_backend_alloc_ctx_tensors(m->wctx, m->backend);
    if (!m->wbuf) {
        err("create: weight allocation failed");
        mm_lm_free(m);
        return nullptr;
    }
    ggml_backend_buffer_set_usage(m->wbuf, GGML_BACKEND_BUFFER_USAGE_WEIGHTS);
    uint64_t s = seed * 1000003ull;
    for (ggml_tensor * t = ggml_get_first_tensor(m->wctx); t; t = ggml_get_next_tensor(m->wctx, t)) {
        const bool ok = ggml_is_quantized(t->type) ? fill_quant(t, ++s) : fill_normal(t, ++s, 1.0f, 0.02f);
        if (!ok) {
            err("create: weight init failed for %s", t->name);
            mm_lm_free(m);
            return nullptr;
        }
    }

    // KV cache (src/qwen3-lm.h:235-274)
    m->kv_ctx = ggml_init({ (size_t) c.n_layers * 2 * ggml_tensor_overhead() + 1024, nullptr, true });
    for (int l = 0; l < c.n_layers; l++) {
        ggml_tensor * k = ggml_new_tensor_4d(m->kv_ctx, GGML_TYPE_F16, c.head_dim, c.max_seq, c.n_kv_heads, c.n_sets);
        ggml_tensor * v = ggml_new_tensor_4d(m->kv_ctx, GGML_TYPE_F16, c.head_dim, c.max_seq, c.n_kv_heads, c.n_sets);
        snprintf(name, sizeof(name), "kv_k4_%d", l);
        ggml_set_name(k, name);
        snprintf(name, sizeof(name), "kv_v4_%d", l);
        ggml_set_name(v, name);
        m->kv_k4.push_back(k);
        m->kv_v4.push_back(v);
    }
    m->kv_buf = ggml_backend_alloc_ctx_tensors(m->kv_ctx, m->backend);
    if (!m->kv_buf) {
        err("create: KV cache allocation failed");
        mm_lm_free(m);
        return nullptr;
    }
    ggml_backend_buffer_clear(m->kv_buf, 0);
    m->kv_pos.assign((size_t) c.n_sets, 0);

    m->arena = ggml_init({ ggml_tensor_overhead() * GRAPH_NODES + ggml_graph_overhead_custom(GRAPH_NODES, false),
                           nullptr, true });
    return m;
}

}  // namespace

extern "C" void * mm_lm_create(const mm_lm_config * cfg, int device, uint64_t seed) {
    return lm_create(cfg, device, nullptr, seed);
}

extern "C" void * mm_lm_create_on_backend(const mm_lm_config * cfg, void * backend, uint64_t seed) {
    if (!backend) {
        err("create: no backend");
        return nullptr;
    }
    return lm_create(cfg, -1, (ggml_backend_t) backend, seed);
}

extern "C" void mm_lm_free(void * h) {
    Lm * m = (Lm *) h;
    if (!m) {
        return;
    }
    if (m->backend) {
        ggml_backend_synchronize(m->backend);  // no replay still reading the buffers freed below
    }
    if (m->galloc) {
        ggml_gallocr_free(m->galloc);
    }
    ggml_free(m->arena);
    ggml_backend_buffer_free(m->kv_buf);
    ggml_free(m->kv_ctx);
    ggml_backend_buffer_free(m->wbuf);
    ggml_free(m->wctx);
    if (m->owns_backend) {
        ggml_backend_free(m->backend);
    }
    delete m;
}

extern "C" int mm_lm_fill_kv(void * h, int set, int n_pos, uint64_t seed) {
    Lm * m = (Lm *) h;
    if (!m || set < 0 || set >= m->c.n_sets || n_pos < 0 || n_pos >= m->c.max_seq) {
        return err("fill_kv: bad arguments");
    }
    const int64_t per_set = (int64_t) m->c.head_dim * m->c.max_seq * m->c.n_kv_heads;
    for (int l = 0; l < m->c.n_layers; l++) {
        for (int kv = 0; kv < 2; kv++) {
            ggml_tensor * t = kv ? m->kv_v4[(size_t) l] : m->kv_k4[(size_t) l];
            char *        p = (char *) t->data + (size_t) set * t->nb[3];
            if (mmhip_synth_normal(1, p, per_set, seed * 7919ull + (uint64_t) (l * 2 + kv), 0.0f, 1.0f, nullptr) !=
                MMHIP_OK) {
                return err("fill_kv: %s", mmhip_last_error());
            }
        }
    }
    if (hipDeviceSynchronize() != hipSuccess) {
        return err("fill_kv: device error");
    }
    m->kv_pos[(size_t) set] = n_pos;
    return 0;
}

extern "C" int mm_lm_set_pos(void * h, int set, int pos) {
    Lm * m = (Lm *) h;
    if (!m || set < 0 || set >= m->c.n_sets || pos < 0 || pos >= m->c.max_seq) {
        return err("set_pos: bad arguments");
    }
    m->kv_pos[(size_t) set] = pos;
    return 0;
}

extern "C" int mm_lm_get_pos(void * h, int set) {
    Lm * m = (Lm *) h;
    return (m && set >= 0 && set < m->c.n_sets) ? m->kv_pos[(size_t) set] : -1;
}

extern "C" int mm_lm_decode_device(void * h, const float * embeds, const int * kv_sets, int N) {
    Lm * m = (Lm *) h;
    if (!m || !embeds || !kv_sets) {
        return err("decode: bad arguments");
    }
    if (prepare(m, embeds, kv_sets, N) != 0) {
        return -1;
    }
    if (ggml_backend_graph_compute(m->backend, m->gf) != GGML_STATUS_SUCCESS) {
        return err("decode: graph_compute failed");
    }
    for (int i = 0; i < N; i++) {
        m->kv_pos[(size_t) kv_sets[i]]++;
    }
    return 0;
}

extern "C" int mm_lm_decode(void * h, const float * embeds, const int * kv_sets, int N, float * logits,
                            float * hidden) {
    Lm * m = (Lm *) h;
    if (mm_lm_decode_device(h, embeds, kv_sets, N) != 0) {
        return -1;
    }
    if (logits) {
        ggml_backend_tensor_get(m->lgt, logits, 0, (size_t) m->c.vocab * N * sizeof(float));
    }
    if (hidden) {
        ggml_backend_tensor_get(m->hidden_out, hidden, 0, (size_t) m->c.hidden * N * sizeof(float));
    }
    return 0;
}

extern "C" int64_t mm_lm_tensor_nbytes(void * h, const char * name) {
    Lm *          m = (Lm *) h;
    ggml_tensor * t = m ? find_tensor(m, name) : nullptr;
    return t ? (int64_t) ggml_nbytes(t) : -1;
}

extern "C" int mm_lm_tensor_type(void * h, const char * name) {
    Lm *          m = (Lm *) h;
    ggml_tensor * t = m ? find_tensor(m, name) : nullptr;
    return t ? (int) t->type : -1;
}

extern "C" int mm_lm_get_tensor(void * h, const char * name, void * dst, size_t size) {
    Lm *          m = (Lm *) h;
    ggml_tensor * t = m ? find_tensor(m, name) : nullptr;
    if (!t || size != ggml_nbytes(t)) {
        return err("get_tensor: no tensor %s of %zu bytes", name, size);
    }
    ggml_backend_tensor_get(t, dst, 0, size);
    return 0;
}

extern "C" int mm_lm_set_tensor(void * h, const char * name, const void * src, size_t size) {
    Lm *          m = (Lm *) h;
    ggml_tensor * t = m ? find_tensor(m, name) : nullptr;
    if (!t || size != ggml_nbytes(t)) {
        return err("set_tensor: no tensor %s of %zu bytes", name, size);
    }
    ggml_backend_tensor_set(t, src, 0, size);
    return 0;
}

extern "C" int mm_lm_graph_nodes(void * h) {
    Lm * m = (Lm *) h;
    return (m && m->gf) ? ggml_graph_n_nodes(m->gf) : 0;
}

extern "C" double mm_lm_gpu_ms(void * h, int reset) {
    Lm *    m     = (Lm *) h;
    double  total = 0.0;
    int64_t n     = 0;
    if (!m) {
        return -1.0;
    }
    ggml_backend_mi355x_gpu_time(m->backend, &total, &n, reset);
    return n ? total / (double) n : 0.0;
}

extern "C" void mm_lm_graph_stats(void * h, int64_t * replays, int64_t * eager) {
    Lm * m = (Lm *) h;
    ggml_backend_mi355x_graph_stats(m->backend, replays, eager);
}
