/*
 * mmhip.h - C-ABI of the MI355X (gfx950) kernels behind the ggml backend.
 *
 * Plain pointers, sizes and byte strides; every pointer argument named
 * data / W / x / y / out / ws is DEVICE memory; `stream` is a hipStream_t (or
 * NULL for the null stream).  Every entry point returns MMHIP_OK (0) or a
 * negative MMHIP_ERR_* code and never aborts; mmhip_last_error() gives the
 * message of the last failure on the calling thread.
 *
 * Each entry point names the reference interface it replaces.  In the
 * reference those operations are ggml ops executed by a ggml backend's
 * graph_compute; the ggml backend in ggml-mi355x.h dispatches them here.
 */
#ifndef MMHIP_H
#define MMHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MMHIP_OK               0
#define MMHIP_ERR_INVALID     -1  /* bad argument or shape */
#define MMHIP_ERR_UNSUPPORTED -2  /* valid ggml op this library does not run */
#define MMHIP_ERR_HIP         -3  /* HIP runtime error */
#define MMHIP_ERR_WORKSPACE   -4  /* workspace smaller than required */

/* GGUF-stable type ids used below. */
#define MMHIP_TYPE_F32  0
#define MMHIP_TYPE_F16  1
#define MMHIP_TYPE_BF16 30
#define MMHIP_TYPE_Q8_0 8
#define MMHIP_TYPE_Q4_K 12
#define MMHIP_TYPE_Q5_K 13
#define MMHIP_TYPE_Q6_K 14
#define MMHIP_TYPE_Q8_K 15

/* A device tensor view in ggml's convention: ne[0] fastest, nb[] in bytes
 * (same meaning as ggml_tensor::ne / ::nb). */
typedef struct {
    const void * data;
    int64_t      ne[4];
    int64_t      nb[4];
} mmhip_view;

const char * mmhip_last_error(void);
int          mmhip_version(void);

/* ---------------------------------------------------------------------
 * Weight layout.  Quantized weights live on the device in a row-grouped
 * layout of the same byte size as GGUF rows (ggml_row_size), so tensor sizes,
 * row strides and row views are unchanged.  Replaces the raw upload of GGUF
 * blocks: src/gguf-weights.h:161-203 (ggml_backend_tensor_set of the mmapped
 * bytes) reaches the ggml backend's set_tensor, which calls repack; its
 * get_tensor calls unpack, so host reads see GGUF bytes.
 * ------------------------------------------------------------------- */
int mmhip_repack_rows(int type, const void * src_gguf, void * dst, int64_t nrows, int64_t ne0, void * stream);
int mmhip_unpack_rows(int type, const void * src, void * dst_gguf, int64_t nrows, int64_t ne0, void * stream);

/* Dequantise nrows rows (row-grouped layout, or F16/F32) to f32, bit-exact
 * with the GGUF to_float definitions.  Replaces
 * ggml_get_type_traits(t)->to_float as used at src/gguf-weights.h:230-235 and
 * src/pipeline.cpp:114-126.  dst is [nrows][ne0] contiguous. */
int mmhip_dequantize_rows(int type, const void * w, int64_t nrows, int64_t ne0, int64_t row_stride, float * dst,
                          void * stream);

/* ---------------------------------------------------------------------
 * Quantized matrix products: GGML_OP_MUL_MAT with src0 in {Q8_0, Q4_K,
 * Q5_K, Q6_K} (row-grouped layout), src1 f32, as emitted by qwen3_linear
 * (src/qwen3-enc.h:67-69), the DiT projections (src/dit.h:197-199, :228,
 * :237, :243) and the depth decoder (src/depth-decoder.h:206-230).
 *   y[m*ldy + n] = sum_k deq(W)[n,k] * x[m*ldx + k],  n < N, m < M
 * W has N rows of K elements, row stride w_row_stride bytes.
 * M <= 16: activation-quantised GEMV (ggml-CPU arithmetic: Q8_0 / Q8_K
 * activations, integer block dots).  M > 16: MFMA GEMM on f16-rounded
 * dequantised weights and f16-rounded activations, f32 accumulation.
 * type MMHIP_TYPE_BF16 (BF16 weight rows as stored, w_row_stride bytes apart,
 * 16-byte aligned; the native-BF16 model files): ggml's BF16 arithmetic
 * (activations rounded to bf16, exact products, f32 sums) -- at M <= 16
 * mmhip_mul_mat_bf16 with no workspace (K % 8 == 0), above it the bf16 MFMA
 * GEMM on a bf16 copy of the activations in the workspace (K % 32 == 0).
 * ------------------------------------------------------------------- */
size_t mmhip_mul_mat_workspace(int type, int64_t N, int64_t K, int64_t M);
int    mmhip_mul_mat(int type, const void * W, int64_t N, int64_t K, int64_t w_row_stride, const float * x, int64_t ldx,
                     int64_t M, float * y, int64_t ldy, void * ws, size_t ws_bytes, void * stream);
/* f16 copies of quantised weights for the token-count GEMMs.  No counterpart
 * in the reference: ggml's MUL_MAT on quantised weights (src/dit.h:197-199,
 * :228, :237, :243) is what they speed up.  A weight multiplied at M > 16 many
 * times (the DiT's, once per diffusion step) can be converted once to f16 rows
 * [N][K] (mmhip_weights_f16_bytes bytes, 16-byte aligned; the GEMM's own exact
 * dequantisation) and registered under the quantised weight's address; every
 * GEMM form above 16 tokens on that weight (plain, bias / residual, SwiGLU,
 * multi-matrix, f32 or f16 activations) then reads the copy with no per-call
 * conversion and returns the same bits.  The caller keeps the copy current
 * (convert again after rewriting the weight) and unregisters it before
 * freeing either.  Registration is process-wide and thread-safe. */
size_t mmhip_weights_f16_bytes(int64_t N, int64_t K);
int    mmhip_weights_to_f16(int type, const void * W, int64_t N, int64_t K, int64_t w_row_stride, void * wh,
                            void * stream);
int    mmhip_register_weights_f16(const void * W, int64_t N, int64_t K, const void * wh);
int    mmhip_unregister_weights_f16(const void * W);
/* MUL_MAT at token counts (M > 16) with the ADDs that follow it fused into the
 * store: y = (x W^T + bias[n]) + r[m*ldr + n], each ADD rounded as its op;
 * bias and r may be NULL (r may alias y).  The DiT's projection biases and
 * residuals (src/dit.h:228-229, :237-245).  Workspace as mmhip_mul_mat. */
/* MUL_MAT over BF16 weight rows (ldw elements apart) at 1..16 activation
 * rows: ggml's BF16 dot (activations rounded to bf16, f32 products summed in
 * f32); the BF16 files of the depth decoder and LM (src/depth-decoder.h:206-257,
 * src/qwen3-lm.h:743-856).  K % 8 == 0, 16-byte aligned rows. */
int    mmhip_mul_mat_bf16(const void * W, int64_t N, int64_t K, int64_t ldw, const float * x, int64_t ldx, int64_t M,
                          float * y, int64_t ldy, void * stream);
/* BF16 weights at decode, 1-2 activation columns, as one persistent launch:
 * the LM's projections from a BF16 model file (qwen3_linear,
 * src/qwen3-enc.h:67-69, in qw3lm_forward_batch, src/qwen3-lm.h:742-856).
 * norm_w != NULL: x is the block's input and its RMS norm times norm_w
 * (src/qwen3-enc.h:87-93, eps) is computed first, with k_rms_norm_row's
 * arithmetic; the activations are then rounded to bf16 as ggml rounds the
 * src1 of a BF16 MUL_MAT.  r != NULL: y = r + W x (the residual ADD,
 * src/qwen3-lm.h:827, :836).  glu != 0: the rows are a fused gate|up pair
 * (src/qwen3-enc.h:106-108) and y[j] = silu(W_j x) * W_{N/2 + j} x, N / 2
 * outputs per column.  W rows ldw elements apart, 16-byte aligned;
 * K % 4096 == 0 and M K <= 32768. */
int    mmhip_mul_mat_bf16_dec_supported(int64_t N, int64_t K, int64_t M, int glu);
int    mmhip_mul_mat_bf16_dec(const void * W, int64_t N, int64_t K, int64_t ldw, const float * x, int64_t ldx,
                              int64_t M, const float * norm_w, float eps, const float * r, int64_t ldr, int glu,
                              float * y, int64_t ldy, void * stream);
int    mmhip_mul_mat_bias_add(int type, const void * W, int64_t N, int64_t K, int64_t w_row_stride, const float * x,
                              int64_t ldx, int64_t M, const float * bias, const float * r, int64_t ldr, float * y,
                              int64_t ldy, void * ws, size_t ws_bytes, void * stream);
/* The same on activations already rounded to f16 (xh: M rows of K halves,
 * contiguous, 16-byte aligned; as mmhip_norm_affine_h writes them): no
 * workspace.  Used when a LayerNorm feeds only GEMMs (src/dit.h:193-199, :236). */
int    mmhip_mul_mat_bias_add_h(int type, const void * W, int64_t N, int64_t K, int64_t w_row_stride, const void * xh,
                                int64_t M, const float * bias, const float * r, int64_t ldr, float * y, int64_t ldy,
                                void * stream);
/* The same with a workspace (mmhip_mul_mat_h_workspace bytes, 16-byte
 * aligned; 0 for shapes that do not need one): a product with few output
 * tiles and a long K (the DiT's ff_out, src/dit.h:243-246: 2048 rows, K =
 * 8192) then splits K into parts whose partial sums are added in order before
 * the ADDs (each ADD rounded as its op). */
size_t mmhip_mul_mat_h_workspace(int type, int64_t N, int64_t K, int64_t M);
int    mmhip_mul_mat_bias_add_hw(int type, const void * W, int64_t N, int64_t K, int64_t w_row_stride, const void * xh,
                                 int64_t M, const float * bias, const float * r, int64_t ldr, float * y, int64_t ldy,
                                 void * ws, size_t ws_bytes, void * stream);
/* The DiT feed-forward input (src/dit.h:236-242): ff = MUL_MAT(W, x) + bias
 * over N = 2F weight rows, value = ff rows [0, F), gate = ff rows [F, 2F)
 * (swapped: the other way round), act = swiglu_split(gate, value) =
 * silu(gate) * value, with the GGML_OP_ADD, the two CONTs and the GGML_OP_GLU
 * in the GEMM's epilogue: ff is never written.  act [M, F] goes to h (f32)
 * and / or hh (f16, rounded as mmhip_mul_mat_bias_add_h's activation copy);
 * bias may be NULL.  Values equal those of the separate ops bit for bit.
 * mmhip_mul_mat_bias_swiglu takes f32 activations and a workspace
 * (mmhip_mul_mat_workspace of the N x K x M product); the _h form takes
 * them in f16. */
int    mmhip_mul_mat_bias_swiglu(int type, const void * W, int64_t N, int64_t K, int64_t w_row_stride, const float * x,
                                 int64_t ldx, int64_t M, const float * bias, int swapped, float * h, void * hh,
                                 void * ws, size_t ws_bytes, void * stream);
int    mmhip_mul_mat_bias_swiglu_h(int type, const void * W, int64_t N, int64_t K, int64_t w_row_stride, const void * xh,
                                   int64_t M, const float * bias, int swapped, float * h, void * hh, void * stream);
/* Several MUL_MATs of one activation tensor in one launch: the DiT's
 * q / k / v projections of the same LayerNorm output (src/dit.h:197-199).
 * n (1..3) weight matrices W[i] of N rows x K (same type and row stride),
 * y[i][m*ldy[i] + r] = MUL_MAT(W[i], x)[m, r] (+ bias[i][r] when bias and
 * bias[i] are given), each equal bit for bit to mmhip_mul_mat_bias_add on
 * W[i].  N a multiple of 256.  mmhip_mul_mat_multi takes f32 activations and
 * a workspace (mmhip_mul_mat_workspace of one N x K x M product); the _h form
 * takes them in f16 (as mmhip_mul_mat_bias_add_h). */
int    mmhip_mul_mat_multi(int type, int n, const void * const * W, int64_t N, int64_t K, int64_t w_row_stride,
                           const float * x, int64_t ldx, int64_t M, const float * const * bias, float * const * y,
                           const int64_t * ldy, void * ws, size_t ws_bytes, void * stream);
int    mmhip_mul_mat_multi_h(int type, int n, const void * const * W, int64_t N, int64_t K, int64_t w_row_stride,
                             const void * xh, int64_t M, const float * const * bias, float * const * y,
                             const int64_t * ldy, void * stream);

/* The two halves of the GEMV path, exposed for fusion and for testing:
 * quantise M activation rows into the layout mmhip_mul_mat_q consumes
 * (size from mmhip_act_bytes), then run the GEMV on them (any M, in groups
 * of 8 activation rows). */
size_t mmhip_act_bytes(int type, int64_t K, int64_t M);
int    mmhip_quantize_act(int type, const float * x, int64_t ldx, int64_t K, int64_t M, void * xq, void * stream);
int    mmhip_mul_mat_q(int type, const void * W, int64_t N, int64_t K, int64_t w_row_stride, const void * xq, int64_t M,
                       float * y, int64_t ldy, void * stream);
/* The GEMV with the residual GGML_OP_ADD that follows the output projections
 * fused into its store: y[m*ldy + n] = mul_mat + r[m*ldr + n] (attention out
 * src/qwen3-lm.h:826-828, MLP down src/qwen3-lm.h:835-836); r may alias y. */
int    mmhip_mul_mat_q_add(int type, const void * W, int64_t N, int64_t K, int64_t w_row_stride, const void * xq,
                           int64_t M, const float * r, int64_t ldr, float * y, int64_t ldy, void * stream);
/* The GEMV that follows an RMS norm, with the norm in its prologue: the
 * GGML_OP_RMS_NORM + GGML_OP_MUL by the norm weight of qwen3_rms_norm
 * (src/qwen3-lm.h:736, :834, :843) feeding the Q/K/V, gate/up and lm_head
 * GGML_OP_MUL_MATs (src/qwen3-lm.h:742-757, :835, :856).  x holds the M raw
 * rows (row stride ldx floats); each workgroup recomputes the norm and the
 * activation quantisation of mmhip_rms_norm_quant in LDS, with identical
 * arithmetic, so y equals rms_norm_quant + mul_mat_q(_add) bit for bit.
 * xn_out (optional) receives the f32 normalised rows [M, K]; r (optional) is
 * the residual of mmhip_mul_mat_q_add.  Q8_0 weights, M <= 2, K a multiple of
 * 256 up to 4096: mmhip_rms_norm_mul_mat_supported says whether a shape is
 * taken.  y must not overlap x. */
int mmhip_rms_norm_mul_mat_supported(int type, int64_t N, int64_t K, int64_t M);
int mmhip_rms_norm_mul_mat(int type, const void * W, int64_t N, int64_t K, int64_t w_row_stride, const float * x,
                           int64_t ldx, int64_t M, const float * norm_w, float eps, float * xn_out, const float * r,
                           int64_t ldr, float * y, int64_t ldy, void * stream);
/* The GEMV that follows a SwiGLU, with the SwiGLU in its prologue: the
 * GGML_OP_GLU (swiglu / swiglu_split, src/qwen3-enc.h:106-113) feeding the
 * MLP down GGML_OP_MUL_MAT (src/qwen3-enc.h:114) whose residual GGML_OP_ADD
 * follows (src/qwen3-lm.h:835-836).  g and u hold the M gate and up rows
 * (row strides ldg / ldu floats); each workgroup recomputes silu(g) * u and
 * its activation quantisation with the arithmetic of mmhip_swiglu_quant, so
 * y equals swiglu_quant + mul_mat_q(_add) bit for bit.  h_out (optional)
 * receives the f32 SwiGLU rows [M, K]; r (optional) is the residual.  Q8_0
 * weights, M <= 2, K a multiple of 256 up to 12288.  y must not overlap g/u. */
int mmhip_swiglu_mul_mat_supported(int type, int64_t N, int64_t K, int64_t M);
int mmhip_swiglu_mul_mat(int type, const void * W, int64_t N, int64_t K, int64_t w_row_stride, const float * g,
                         int64_t ldg, const float * u, int64_t ldu, int64_t M, float * h_out, const float * r,
                         int64_t ldr, float * y, int64_t ldy, void * stream);
/* The MLP's gate_up GEMV with the RMS norm in its prologue and the SwiGLU
 * that follows it in its epilogue: GGML_OP_RMS_NORM + GGML_OP_MUL
 * (src/qwen3-lm.h:834) -> gate_up GGML_OP_MUL_MAT over the fused [gate | up]
 * rows (src/qwen3-enc.h:106-108, src/gguf-weights.h:289-362) -> GGML_OP_GLU
 * swiglu (src/qwen3-enc.h:108), whose output feeds the down projection
 * (src/qwen3-enc.h:114).  W holds N = 2F rows (gate rows first, or up rows
 * first when swapped); the result is the down GEMV's Q8_0 activation buffer
 * xq (mmhip_act_bytes(8, F, M) bytes, as mmhip_swiglu_quant writes it) and,
 * if h_out is given, the f32 SwiGLU rows [M, F].  Identical arithmetic:
 * xq and h_out equal rms_norm_mul_mat followed by swiglu_quant bit for bit.
 * Q8_0 weights, M <= 2, K a multiple of 256 up to 4096, N a multiple of 512. */
int mmhip_rms_norm_mul_mat_glu_supported(int type, int64_t N, int64_t K, int64_t M);
int mmhip_rms_norm_mul_mat_glu(int type, const void * W, int64_t N, int64_t K, int64_t w_row_stride, const float * x,
                               int64_t ldx, int64_t M, const float * norm_w, float eps, int swapped, void * xq,
                               float * h_out, void * stream);

/* ---------------------------------------------------------------------
 * GGML_OP_FLASH_ATTN_EXT, replacing the ggml backend kernel behind
 *   src/qwen3-lm.h:816-821 (batched CFG decode over the f16 4-D KV cache),
 *   src/qwen3-lm.h:432-436 (causal prefill),
 *   src/dit.h:221-222      (DiT bidirectional, mask NULL).
 * q    f32 [D, n_q, Hq, B]      any strides (permuted views allowed)
 * k, v f16 [D, n_kv, Hkv, Bk]   any row/head/batch strides, rows contiguous
 * mask f16 [>=n_kv, >=n_q, M2, M3] or NULL (broadcast over heads / batch)
 * out  f32 [D, Hq, n_q, B] contiguous
 * Requires D in {64, 128, 256}, Hq % Hkv == 0, B % Bk == 0.  scale is
 * op_params[0]; max_bias and softcap must be 0 (as in every call of the
 * reference).  Accumulation is f32 (GGML_PREC_F32).
 * ------------------------------------------------------------------- */
size_t mmhip_flash_attn_workspace(const mmhip_view * q, const mmhip_view * k, const mmhip_view * v);
int    mmhip_flash_attn_ext(const mmhip_view * q, const mmhip_view * k, const mmhip_view * v, const mmhip_view * mask,
                            float scale, float * out, void * ws, size_t ws_bytes, void * stream);
/* The same attention with its output rows (b, iq) of Hq * D f32 also
 * quantised into the activation layout of mmhip_mul_mat_q for weights of
 * `type`: the input of the attention output projection (src/qwen3-lm.h:
 * 823-826), quantised by the split combine instead of a separate pass. */
int    mmhip_flash_attn_ext_q(const mmhip_view * q, const mmhip_view * k, const mmhip_view * v,
                              const mmhip_view * mask, float scale, float * out, void * ws, size_t ws_bytes, int type,
                              void * xq, void * stream);

/* The attention of mmhip_flash_attn_ext with no workspace argument and no
 * allocation: no counterpart in the reference.  For callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The workspace lives in a file-scope
 * device array of mmhip_flash_attn_noalloc_max_workspace() bytes (8 MiB),
 * one copy per GPU, held until the process ends; shapes whose
 * mmhip_flash_attn_workspace exceeds it are rejected with
 * MMHIP_ERR_WORKSPACE.  Calls on one GPU share the array: calls that overlap
 * on one GPU (different streams, or host threads) race.  Results equal
 * mmhip_flash_attn_ext's bit for bit. */
size_t mmhip_flash_attn_noalloc_max_workspace(void);
int    mmhip_flash_attn_ext_noalloc(const mmhip_view * q, const mmhip_view * k, const mmhip_view * v,
                                    const mmhip_view * mask, float scale, float * out, void * stream);

/* ---------------------------------------------------------------------
 * Decode-step glue ops (the nodes between the hot-path ops in the LM
 * batched decode graph, src/qwen3-lm.h:730-859).  Operands are ggml views;
 * `dst` outputs are contiguous f32 unless a view is given.  A view passed as
 * destination is written through its (non-const) data pointer.
 * ------------------------------------------------------------------- */
/* GGML_OP_ADD / SUB / MUL (op 0 / 1 / 2), b broadcast over a:
 * residual adds src/qwen3-lm.h:827, :836; norm-weight MUL src/qwen3-enc.h:92. */
int mmhip_binary(int op, const mmhip_view * a, const mmhip_view * b, float * dst, void * stream);
/* GGML_OP_RMS_NORM over dim 0, optionally fused with the following MUL by w:
 * qwen3_rms_norm src/qwen3-enc.h:87-93, qk-norm src/qwen3-lm.h:765-768. */
int mmhip_rms_norm(const mmhip_view * x, const mmhip_view * w, float eps, float * dst, void * stream);
/* The same RMS_NORM (+ MUL by w) with the normalised rows also quantised into
 * the activation layout of mmhip_mul_mat_q for weights of `type` (the
 * GEMV consuming the norm: QKV src/qwen3-lm.h:742-747, gate_up
 * src/qwen3-enc.h:106-108, lm_head src/qwen3-lm.h:856), saving the separate
 * quantisation pass.  dst may be NULL when the f32 rows are not needed.
 * Rows must be contiguous with ne0 % 256 == 0. */
int mmhip_rms_norm_quant(const mmhip_view * x, const mmhip_view * w, float eps, float * dst, int type, void * xq,
                         void * stream);
/* Per-head post-processing of the fused QKV projection in one launch: the
 * node chain CONT(view of qkv) -> RESHAPE [D, H, T] -> [RMS_NORM -> MUL(w)]
 * -> [ROPE NeoX] -> [CONT] -> [RESHAPE [D, 1, H, T] -> SET_ROWS] of the
 * attention block (src/qwen3-lm.h:744-804 batched decode, src/qwen3-lm.h:
 * 371-421 prefill).  Row (h, t) of D f32 elements is read at
 * src + h*src_nb_h + t*src_nb_t.  norm != 0: RMS_NORM over D with eps, then
 * times norm_w[D] when non-NULL.  pos != NULL: NeoX RoPE over all D dims at
 * position pos[t], theta_i = pos * theta_scale^i.  ids == NULL: written as
 * contiguous f32 dst[T][H][D]; else written as SET_ROWS into the dst view:
 * row r = ids[(h % ids_ne1)*ids_nb1 + (t % ids_ne2)*ids_nb2] (i32 type 26 or
 * i64 type 27) at dst + r*dst_nb1 + h*dst_nb2 + t*dst_nb3, as f32 or f16. */
typedef struct {
    const void *    src;
    int64_t         src_nb_h, src_nb_t;
    int             D, H, T;
    int             norm;
    const float *   norm_w;
    float           eps;
    const int32_t * pos;
    float           theta_scale;
    void *          dst;
    int             dst_type;
    const void *    ids;
    int             ids_type;
    int64_t         ids_nb1, ids_nb2, ids_ne1, ids_ne2;
    int64_t         dst_nb1, dst_nb2, dst_nb3;
} mmhip_head_rows_args;
int mmhip_head_rows(const mmhip_head_rows_args * args, void * stream);
/* n (1..4) such chains with a common D in one launch (the Q, K and V chains
 * of one attention block). */
int mmhip_head_rows_n(const mmhip_head_rows_args * args, int n, void * stream);
/* Batched decode attention with the head chains of its block in the prologue
 * (src/qwen3-lm.h:764-821: the QKV views' RMS_NORM + MUL q/k norm, NeoX
 * ROPE, SET_ROWS of the new key / value rows into the f16 caches, then
 * GGML_OP_FLASH_ATTN_EXT).  heads[0] is the query chain (ids NULL; q is a
 * view of its dst, which is not written), heads[1] / heads[2] the key and
 * value chains whose dst are the caches k / v view (same base and strides,
 * same ids); all three as mmhip_head_rows_n would run them.  The new rows are
 * written to the caches and used by the attention of this call; results equal
 * mmhip_head_rows_n + mmhip_flash_attn_ext(_q) (xq NULL: no quantised
 * output).  Decode shapes only: (Hq / Hkv) * nq + 2 <= 8, one cache set per
 * batch: mmhip_flash_attn_ext_head_supported says whether q, k, v qualify. */
int mmhip_flash_attn_ext_head_supported(const mmhip_view * q, const mmhip_view * k, const mmhip_view * v);
int mmhip_flash_attn_ext_head(const mmhip_view * q, const mmhip_view * k, const mmhip_view * v,
                              const mmhip_view * mask, float scale, float * out, void * ws, size_t ws_bytes, int type,
                              void * xq, const mmhip_head_rows_args * heads, void * stream);
/* GGML_OP_GLU SwiGLU (as mmhip_swiglu) with the result also quantised into
 * the activation layout of mmhip_mul_mat_q for weights of `type` (the down
 * projection, src/qwen3-enc.h:108-110).  dst may be NULL.  Rows contiguous,
 * output width % 256 == 0. */
int mmhip_swiglu_quant(const mmhip_view * a, const mmhip_view * b, int swapped, float * dst, int type, void * xq,
                       void * stream);
/* GGML_OP_ROPE, NeoX mode (2), freq_scale 1, ext_factor 0, attn_factor 1:
 * src/qwen3-lm.h:771-772, src/dit.h:206-209 (partial, n_dims < head_dim).
 * x [head_dim, heads, tokens, B], pos int32 [tokens]; theta_scale =
 * powf(freq_base, -2/n_dims) computed by the caller. */
int mmhip_rope_neox(const mmhip_view * x, const int32_t * pos, int n_dims, float theta_scale, float * dst,
                    void * stream);
/* mmhip_rope_neox whose result is rounded to f16 (as GGML_OP_CPY rounds) and
 * stored through the strided f16 view dst (same ne as x; nb[0] == 2): the
 * DiT's ggml_cast(ggml_permute(ggml_rope_ext(k))) to F16 (src/dit.h:207-220)
 * as one launch, dst being the cast's rows seen in the rope's dim order.
 * Takes n_dims <= 256 with n_dims / 2 % 4 == 0, ne0 % 4 == 0, 16-byte
 * aligned x rows and 8-byte aligned dst rows (else MMHIP_ERR_UNSUPPORTED). */
int mmhip_rope_neox_f16(const mmhip_view * x, const int32_t * pos, int n_dims, float theta_scale,
                        const mmhip_view * dst, void * stream);
/* GGML_OP_CPY / GGML_OP_CONT between f32 and f16 views of equal element count:
 * src/qwen3-lm.h:775-777, src/dit.h:219-220 (f32 -> f16 cast). */
int mmhip_cpy(const mmhip_view * src, int src_type, const mmhip_view * dst, int dst_type, void * stream);
/* GGML_OP_GET_ROWS (ids int32 [n, ne1, ne2]) from f32, f16 or quantized
 * (row-grouped) rows: embedding lookup src/qwen3-lm.h:730. */
int mmhip_get_rows(int src_type, const mmhip_view * src, const mmhip_view * ids, float * dst, void * stream);
/* GGML_OP_SET_ROWS: f32 rows into an f16 / f32 destination at int32 / int64
 * row ids (ids_type 26 / 27), broadcast over dims 2-3: KV-cache write
 * src/qwen3-lm.h:803-804, :420-421. */
int mmhip_set_rows(const mmhip_view * src, const mmhip_view * ids, int ids_type, const mmhip_view * dst,
                   int dst_type, void * stream);
/* GGML_OP_GLU SwiGLU: fused halves (b NULL; src/qwen3-enc.h:108) or split
 * (src/dit.h:242). */
int mmhip_swiglu(const mmhip_view * a, const mmhip_view * b, int swapped, float * dst, void * stream);
/* GGML_OP_SCALE: dst = a * s + bias (src/depth-decoder.h:355). */
int mmhip_scale(const mmhip_view * a, float s, float bias, float * dst, void * stream);
/* GGML_OP_NORM: per-row LayerNorm without the affine part, eps as given
 * (dit_layer_norm, src/dit.h:161-167, eps 1e-5); dst contiguous f32 rows.
 * ggml-CPU's steps: mean and variance from double sums. */
int mmhip_norm(const mmhip_view * x, float eps, float * dst, void * stream);
/* GGML_OP_NORM followed by the MUL by w[ne0] and the ADD of b[ne0] of
 * dit_layer_norm (src/dit.h:161-167), fused: dst = (norm(x) * w) + b, each
 * step rounded as in the three ops; w or b may be NULL. */
int mmhip_norm_affine(const mmhip_view * x, float eps, const float * w, const float * b, float * dst, void * stream);
/* The same writing the rows also (or only: dst NULL) rounded to f16 into dsth,
 * contiguous, the activation copy mmhip_mul_mat_bias_add_h consumes. */
int mmhip_norm_affine_h(const mmhip_view * x, float eps, const float * w, const float * b, float * dst, void * dsth,
                        void * stream);
/* GGML_OP_MUL_MAT of two f32 tensors (activation x activation: the depth
 * decoder's manual attention scores and P.V, src/depth-decoder.h:214-219):
 * dst[i, j, i2, i3] = sum_k a[k, i, i2/r2, i3/r3] * b[k, j, i2, i3], any
 * strides with contiguous dim 0, a broadcast over dims 2/3; dst contiguous
 * [a->ne[1], b->ne[1], b->ne[2], b->ne[3]]. */
int mmhip_mul_mat_f32(const mmhip_view * a, const mmhip_view * b, float * dst, void * stream);
/* GGML_OP_DIAG_MASK_INF (src/depth-decoder.h:216): elements with i0 > n_past
 * + i1 become -inf; dst contiguous. */
int mmhip_diag_mask_inf(const mmhip_view * a, int n_past, float * dst, void * stream);
/* GGML_OP_SOFT_MAX without mask, scale 1 (src/depth-decoder.h:217, :348):
 * row softmax with ggml-CPU's steps (f32 exp, double sum); dst contiguous. */
int mmhip_soft_max(const mmhip_view * a, float * dst, void * stream);
/* The depth decoder's manual causal attention in one launch
 * (src/depth-decoder.h:214-221): SOFT_MAX(DIAG_MASK_INF(SCALE(MUL_MAT(k, q)),
 * n_past)) times the keys' V rows, written as CONT(PERMUTE(.., 0, 2, 1, 3)):
 * q, k, v are [D, S, H, B] f32 views with contiguous dim 0 (k / v heads and
 * batches may broadcast); SCALE is x * scale + bias; S_q, S_kv <= 16 and
 * D <= 256 (else MMHIP_ERR_UNSUPPORTED); dst
 * contiguous [D, H, S_q, B].  The same bits as the seven separate ops. */
int mmhip_small_attn(const mmhip_view * q, const mmhip_view * k, const mmhip_view * v, float scale, float bias,
                     int n_past, float * dst, void * stream);
/* mmhip_small_attn that also quantises its output rows (D x H values, S_q x B
 * rows) for the following projection (src/depth-decoder.h:222-223,
 * MUL_MAT(wo, attn)) into xq, laid out as mmhip_quantize_act writes
 * (mmhip_act_bytes(qtype, D * H, S_q * B) bytes), with the same bits;
 * qtype 0 = no quantisation, else GGML_TYPE_Q8_0 (8) with D % 32 == 0. */
int mmhip_small_attn_q(const mmhip_view * q, const mmhip_view * k, const mmhip_view * v, float scale, float bias,
                       int n_past, float * dst, int qtype, void * xq, void * stream);
/* The depth decoder's in-graph CFG sampler (src/depth-decoder.h:345-361):
 * GGML_OP_ARGSORT descending (I32 indices, rows of <= 4096; equal values in
 * ascending index order), GGML_OP_CUMSUM along dim 0 (running f32 sum),
 * GGML_OP_SUM of all elements (double accumulation, dst[0]), the STEP unary
 * (x > 0 ? 1 : 0) and the casts to I32 (truncation) and back; dst contiguous. */
int mmhip_argsort_desc(const mmhip_view * a, int32_t * dst, void * stream);
int mmhip_cumsum(const mmhip_view * a, float * dst, void * stream);
int mmhip_sum(const mmhip_view * a, float * dst, void * stream);
int mmhip_step(const mmhip_view * a, float * dst, void * stream);
int mmhip_cast_i32(const mmhip_view * a, int32_t * dst, void * stream);
int mmhip_cast_f32_of_i32(const mmhip_view * a, float * dst, void * stream);
/* GGML_OP_CONCAT of f32 a and b along dim 0..3 (the DiT input channel concat
 * and the timestep token, src/dit.h:262-264, :273); dst contiguous. */
int mmhip_concat(const mmhip_view * a, const mmhip_view * b, int dim, float * dst, void * stream);
/* GGML_OP_CLAMP: dst = MAX(MIN(a, hi), lo) (the DiT's f16-range clamp,
 * src/dit.h:276-278); dst may alias a contiguous a (ggml_clamp is in place). */
int mmhip_clamp(const mmhip_view * a, float lo, float hi, float * dst, void * stream);

#ifdef __cplusplus
}
#endif
#endif
