/*
 * oracle.h - CPU restatement of the ggml-CPU arithmetic on minimaxmusic.cpp's
 * attention + quantized-matmul hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product path (the HIP library and the ggml backend) never links or calls it.
 *
 * What it restates (ggml is an un-vendored submodule of the reference, see
 * .gitmodules:1-3 of the reference; its pinned commit is unknown, so every
 * ggml-internal statement below is a restatement of public upstream ggml
 * behaviour, marked [ext]):
 *   - GGUF block formats Q8_0 / Q4_K / Q5_K / Q6_K / Q8_K and their dequantisation
 *     (the weights the reference's quantizer writes, tools/quantize.cpp:40-51,
 *     :375-383, and uploads raw, src/gguf-weights.h:161-203);
 *   - ggml-CPU mul_mat semantics: activations quantized to Q8_0 (for Q8_0
 *     weights) or Q8_K (for K-quants), integer block dots, float combine
 *     [ext]; called from src/qwen3-enc.h:67-69, src/dit.h:197-199;
 *   - ggml-CPU flash_attn_ext semantics: Q rounded to f16, f16 K dot, online
 *     softmax with the V accumulator held in f16 [ext]; called from
 *     src/qwen3-lm.h:816-821 (decode), :432-436 (prefill), src/dit.h:221-222;
 *   - fp64 "textbook" versions of both, used to bound the error of the
 *     ggml-semantics versions and of the GPU path.
 *
 * Pinning status of each function is listed in the header comment of
 * oracle.c.
 */
#ifndef MM_ORACLE_H
#define MM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF-stable type ids (on-disk format, identical in every ggml revision). */
enum {
    ORC_TYPE_F32  = 0,
    ORC_TYPE_F16  = 1,
    ORC_TYPE_Q8_0 = 8,
    ORC_TYPE_Q4_K = 12,
    ORC_TYPE_Q5_K = 13,
    ORC_TYPE_Q6_K = 14,
    ORC_TYPE_Q8_K = 15,
    ORC_TYPE_I32  = 26,
    ORC_TYPE_I64  = 27,
    ORC_TYPE_BF16 = 30,
};

#define ORC_QK8_0 32
#define ORC_QK_K  256

/* Block layouts (byte-exact GGUF layouts). */
typedef struct { uint16_t d; int8_t qs[32]; } orc_block_q8_0;                               /* 34 B  */
typedef struct { uint16_t d; uint16_t dmin; uint8_t scales[12]; uint8_t qs[128]; } orc_block_q4_K; /* 144 B */
typedef struct { uint16_t d; uint16_t dmin; uint8_t scales[12]; uint8_t qh[32]; uint8_t qs[128]; } orc_block_q5_K; /* 176 B */
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } orc_block_q6_K;  /* 210 B */
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } orc_block_q8_K;               /* 292 B */

/* Strided tensor view with ggml's ne/nb convention (ne[0] fastest). */
typedef struct {
    const void * data;
    int          type;
    int64_t      ne[4];
    size_t       nb[4];
} orc_tensor;

/* ---- scalar conversions ---- */
uint16_t orc_fp32_to_fp16(float f);     /* round to nearest even, IEEE binary16 */
float    orc_fp16_to_fp32(uint16_t h);
uint16_t orc_fp32_to_bf16(float f);     /* round to nearest even; NaN stays quiet NaN */
float    orc_bf16_to_fp32(uint16_t h);
void     orc_fp32_to_fp16_row(const float * x, uint16_t * y, int64_t n);
void     orc_fp16_to_fp32_row(const uint16_t * x, float * y, int64_t n);

/* ---- block formats ---- */
size_t orc_type_size(int type);         /* bytes per block */
int    orc_blck_size(int type);         /* elements per block */
size_t orc_row_size(int type, int64_t ne0);

/* Dequantize k elements (k a multiple of the block size). */
void orc_dequantize_row(int type, const void * src, float * dst, int64_t k);

/* Activation quantizers of ggml-CPU [ext]. */
void orc_quantize_row_q8_0(const float * x, void * y, int64_t k);
void orc_quantize_row_q8_K(const float * x, void * y, int64_t k);

/* Block dot products with ggml's generic (scalar) accumulation [ext]:
 * weight row of `type` against the activation row already quantized to the
 * matching vec_dot type (Q8_0 for Q8_0, Q8_K for Q4_K / Q5_K / Q6_K). */
float orc_vec_dot(int type, int64_t k, const void * wrow, const void * xq);

/* mul_mat on a 2-D weight W (N rows of K elements, row stride = row_size)
 * against M activation rows x (f32, row stride x_stride floats):
 *   y[m*N + n] = sum_k deq(W)[n,k] * x[m,k]
 * _ggml: ggml-CPU semantics (activation quantisation + integer dots).
 * _f64 : exact dequantised weights, x as given, double accumulation.
 * nthreads <= 0 means 1. */
void orc_mul_mat_ggml(int type, const void * W, int64_t N, int64_t K,
                      const float * x, int64_t x_stride, int64_t M, float * y, int nthreads);
void orc_mul_mat_f64(int type, const void * W, int64_t N, int64_t K,
                     const float * x, int64_t x_stride, int64_t M, double * y, int nthreads);

/* flash_attn_ext, ggml layouts:
 *   q    f32 [D,  n_q,  Hq,  B ]  (any nb)
 *   k,v  f16 [D,  n_kv, Hkv, Bk]  (any nb; Hq % Hkv == 0, B % Bk == 0)
 *   mask f16 [n_kv', n_q', M2, M3] or data == NULL; broadcast over dims 2,3
 *        (n_kv' >= n_kv, n_q' >= n_q)
 *   out  f32 [D, Hq, n_q, B] contiguous (ggml's permuted result layout).
 * _ggml: Q rounded to f16, f16 V accumulator, expf online softmax [ext].
 * _f64 : textbook softmax in double; fully masked rows give 0. */
void orc_flash_attn_ext_ggml(const orc_tensor * q, const orc_tensor * k, const orc_tensor * v,
                             const orc_tensor * mask, float scale, float * out, int nthreads);
void orc_flash_attn_ext_f64(const orc_tensor * q, const orc_tensor * k, const orc_tensor * v,
                            const orc_tensor * mask, float scale, double * out, int nthreads);

/* ---- decode-step glue, closed-form definitions (qwen3-lm.h:730-859) ---- */
/* y = x / sqrt(mean(x^2) + eps) * w, rows of n (w may be NULL). */
void orc_rms_norm_mul(const float * x, const float * w, float * y, int64_t n, int64_t rows, float eps);
/* LayerNorm without affine part (GGML_OP_NORM, src/dit.h:161-167): mean from
 * a double sum, y = x - mean, variance from the double sum of y^2,
 * y *= 1 / sqrtf(variance + eps) -- ggml-CPU's norm_f32 steps [ext]. */
void orc_layer_norm(const float * x, float * y, int64_t n, int64_t rows, float eps);
/* NeoX RoPE (mode 2) on rows of head_dim, rotating the first n_dims, with
 * positions[row / heads]; freq_base as ggml's theta, freq_scale 1. */
void orc_rope_neox(const float * x, float * y, int64_t head_dim, int64_t n_dims, int64_t heads,
                   int64_t tokens, const int32_t * positions, float freq_base);
/* swiglu over rows of 2n: y = silu(x[:n]) * x[n:] */
void orc_swiglu(const float * x, float * y, int64_t n, int64_t rows);

#ifdef __cplusplus
}
#endif
#endif
