/*
 * mm_lm.h - Qwen3-shape LM with the batched CFG decode step of
 * minimaxmusic.cpp, run on the MI355X ggml backend with random-init weights.
 *
 * The decode step builds the same ggml graph, node for node, as
 * qw3lm_forward_batch (src/qwen3-lm.h:645-934, input_embeds path) and runs it
 * with ggml_backend_graph_compute; the weights follow the reference's fused
 * layout (QKV rows q|k|v and gate|up, src/gguf-weights.h:289-362) and the
 * KV cache is the reference's 4-D f16 [D, max_seq, Nkv, n_sets] tensor per
 * layer (src/qwen3-lm.h:232-233).  No checkpoint is available offline, so
 * weights are seeded synthetic GGUF blocks (include/mmhip_synth.h) and norm
 * weights 1 + N(0, 0.02).
 */
#ifndef MM_LM_H
#define MM_LM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int   n_layers;     /* 36 */
    int   hidden;       /* 4096 */
    int   n_heads;      /* 32 */
    int   n_kv_heads;   /* 8 */
    int   head_dim;     /* 128 */
    int   ffn;          /* 12288 */
    int   vocab;        /* 151936 (config) / 200000 (real model) */
    int   max_seq;      /* KV cache capacity */
    int   n_sets;       /* KV sets (2 = CFG cond + uncond) */
    int   wtype;        /* GGML type of the linear weights and lm_head: 8 Q8_0, 14 Q6_K, 13 Q5_K,
                           12 Q4_K, 30 BF16 */
    float rms_eps;      /* 1e-6 */
    float rope_theta;   /* 1e6 */
    int   bump_type;    /* 0, or the "_M" files' type of v_proj and down_proj in the first
                           n_layers/9, the last n_layers/7 and every third layer
                           (tools/quantize.cpp:47-48, :127-150; Q5_K_M: wtype 13,
                           bump_type 14); q_proj | k_proj are then one weight "blk.<l>.qk"
                           and v_proj is "blk.<l>.v" (src/qwen3-lm.h:749-753) */
} mm_lm_config;

/* Create on MI355X device `device`; NULL on failure (see mm_lm_error). */
void *       mm_lm_create(const mm_lm_config * cfg, int device, uint64_t seed);
/* The same on an existing MI355X ggml backend (a ggml_backend_t), shared with
 * other modules as the reference shares one backend between the LM, the DiT
 * and the depth decoder (src/backend.h:21-23, :150-165); the LM does not free
 * it. */
void *       mm_lm_create_on_backend(const mm_lm_config * cfg, void * backend, uint64_t seed);
const char * mm_lm_error(void);
void         mm_lm_free(void * lm);

/* Fill every layer's K/V of set `set` with N(0, 1) f16 and set its position
 * to n_pos (a synthetic prompt of n_pos tokens). */
int mm_lm_fill_kv(void * lm, int set, int n_pos, uint64_t seed);
int mm_lm_set_pos(void * lm, int set, int pos);
int mm_lm_get_pos(void * lm, int set);

/* One batched decode step for N consecutive sets kv_sets[0] .. +N-1:
 * embeds f32 [N][hidden] (the feedback path's input embeddings,
 * src/pipeline.cpp:545-547); writes logits f32 [N][vocab] and the final-norm
 * hidden states f32 [N][hidden] when non-NULL, then advances the positions. */
int mm_lm_decode(void * lm, const float * embeds, const int * kv_sets, int N, float * logits, float * hidden);

/* Same step without host transfers of the outputs (benchmark loop): inputs
 * are uploaded, the graph runs, the call returns once the GPU has finished. */
int mm_lm_decode_device(void * lm, const float * embeds, const int * kv_sets, int N);

/* Host copy of a weight or cache tensor by name ("blk.3.qkv", "lm_head",
 * "output_norm", "kv_k4_3", ...): quantized weights come back as GGUF bytes.
 * Tensors of the last decode step's graph are found by name too: each
 * layer's output rows "layer_out-<l>" f32 [N][hidden], "hidden_out",
 * "logits". */
int64_t mm_lm_tensor_nbytes(void * lm, const char * name);
/* GGML type of the tensor of that name, -1 if there is none ("blk.<l>.qkv"
 * exists in the layers of one weight type, "blk.<l>.qk" / "blk.<l>.v" in the
 * others). */
int     mm_lm_tensor_type(void * lm, const char * name);
int     mm_lm_get_tensor(void * lm, const char * name, void * dst, size_t size);
/* Overwrite a tensor from host bytes (GGUF bytes for quantized weights). */
int     mm_lm_set_tensor(void * lm, const char * name, const void * src, size_t size);

/* Number of nodes of the current decode graph; HIP-graph replays and eager
 * runs of the backend so far. */
int  mm_lm_graph_nodes(void * lm);
void mm_lm_graph_stats(void * lm, int64_t * replays, int64_t * eager);
/* Mean GPU time (ms) of the decode graph executions since the last reset,
 * from HIP events on the backend stream; reset != 0 starts a new window. */
double mm_lm_gpu_ms(void * lm, int reset);

#ifdef __cplusplus
}
#endif
#endif
