// mmhip_internal.h - host-side helpers shared by the C-ABI translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include <algorithm>

#include "mmhip.h"

namespace mmhip {

int  set_error(int code, const char * fmt, ...) __attribute__((format(printf, 2, 3)));

// Opt a kernel in to `bytes` of dynamic LDS (above the 64 KiB default) once
// per process; thread-safe.  Returns false if the runtime refuses.
bool ensure_lds_limit(const void * kernel, size_t bytes);
int  check_launch(const char * what);
void clear_error();

inline bool is_repacked_type(int type) {
    return type == 8 /*Q8_0*/ || type == 12 /*Q4_K*/ || type == 13 /*Q5_K*/ || type == 14 /*Q6_K*/;
}

// Quantised-activation buffer layout for M rows of K elements:
//   qs [M][K] int8 | d [M][K/blk] f32 | bsums [M][K/16] int16 (Q8_K only)
// with every field 256-byte aligned.
struct ActLayout {
    int    vec_type;  // 8 = Q8_0, 15 = Q8_K, 0 = unsupported
    int    blk;
    size_t qs_off, d_off, bs_off, total;
};

inline size_t align_up(size_t v, size_t a) {
    return (v + a - 1) / a * a;
}

inline ActLayout act_layout(int wtype, int64_t K, int64_t M) {
    ActLayout L{};
    if (wtype == 8 && K % 32 == 0) {
        L.vec_type = 8;
        L.blk      = 32;
    } else if ((wtype == 12 || wtype == 13 || wtype == 14) && K % 256 == 0) {
        L.vec_type = 15;
        L.blk      = 256;
    } else {
        return L;
    }
    L.qs_off = 0;
    L.d_off  = align_up((size_t) (M * K), 256);
    L.bs_off = align_up(L.d_off + sizeof(float) * (size_t) (M * (K / L.blk)), 256);
    L.total  = L.vec_type == 15 ? align_up(L.bs_off + 2 * (size_t) (M * (K / 16)), 256) : L.bs_off;
    return L;
}

int quantize_act(int wtype, const float * x, int64_t ldx, int64_t K, int64_t M, void * xq, hipStream_t stream);

// Field pointers of a quantised-activation buffer.
struct ActPtrs {
    const int8_t *  qs;
    const float *   d;
    const int16_t * bs;
    int             blk;

    static ActPtrs from(const ActLayout & L, const void * base) {
        const char * b = (const char *) base;
        return { (const int8_t *) (b + L.qs_off), (const float *) (b + L.d_off),
                 L.vec_type == 15 ? (const int16_t *) (b + L.bs_off) : nullptr, L.blk };
    }
    ActPtrs slice(int64_t c0, int64_t K) const {
        return { qs + c0 * K, d + c0 * (K / blk), bs ? bs + c0 * (K / 16) : nullptr, blk };
    }
};

// Quantized GEMV on pre-quantised activations (any M; column groups of <= 8).
bool gemv_supported(int wtype, int64_t N, int64_t K, int64_t row_stride, const void * W);
int  gemv_q(int wtype, const void * W, int64_t N, int64_t K, int64_t row_stride, const ActPtrs & x, int64_t M, float * y,
            int64_t ldy, hipStream_t stream, const float * r = nullptr, int64_t ldr = 0);

// MFMA GEMM with in-LDS dequantisation (any M); the workspace holds the f16
// copy of the activations (gemm_workspace bytes, 16-byte aligned).
size_t gemm_workspace(int64_t K, int64_t M);
// SwiGLU epilogue: the N = 2 F weight rows are the value (first half, second
// if swapped) and gate halves; the GEMM then writes silu(gate + bias) *
// (value + bias) rows [M, F] to h (f32) and / or hh (f16) instead of y.
struct GemmGlu {
    int64_t    F       = 0;  // 0: the plain epilogue
    int        swapped = 0;
    float *    h       = nullptr;
    _Float16 * hh      = nullptr;
};
// Up to 3 weight matrices of Nper rows each (same type, K and activations)
// in one launch: weight rows [i Nper, (i + 1) Nper) come from W[i], their
// outputs go to y[i] (row stride ldy[i]) with bias[i]; Nper is a multiple of
// the tile height, so no tile straddles two matrices.
struct GemmMulti {
    int             n    = 0;  // 0: the single matrix of the call
    int64_t         Nper = 0;
    const uint8_t * W[3]{};
    float *         y[3]{};
    int64_t         ldy[3]{};
    const float *   bias[3]{};
};
// Split-K: the K range is cut into n parts, each tile-and-part writes its
// f32 partial sums to part[(i M + m) N + n], and a reduce kernel sums the
// parts in order, then adds the bias and the residual as the epilogue would.
struct GemmSplit {
    int     n    = 1;
    float * part = nullptr;
};
// Parts the GEMM would split K into for this shape (1: no split), and the
// bytes of partial sums that takes.
int    gemm_split(int64_t N, int64_t K, int64_t M);
size_t gemm_split_bytes(int64_t N, int64_t K, int64_t M);
// the f16 weight copy gemm_q makes first at large token counts (0: none), and
// gemm_q's whole workspace: f16 activations, f16 weights, split-K partials
bool   gemm_use_wh(int64_t N, int64_t K, int64_t M);
size_t gemm_wh_bytes(int64_t N, int64_t K, int64_t M);
size_t gemm_q_workspace(int64_t N, int64_t K, int64_t M);
// Registered f16 copies of quantised weights (k_w_to_f16's rows [N][K]),
// which the token-count GEMMs use in place of converting per call.
int register_f16_weights(const void * W, int64_t N, int64_t K, const void * wh);
int unregister_f16_weights(const void * W);
int weights_to_f16_checked(int wtype, const void * W, int64_t N, int64_t K, int64_t rs, void * wh, hipStream_t stream);
// BF16 weights: the GEMV takes up to this many activation rows, the GEMM more.
constexpr int BF16_GEMV_MAXM = 16;
// BF16 weights at token counts (rows rs bytes apart, read in place): the
// bf16 activation copy the workspace holds, the shape / alignment check, and
// the call (y = x W^T, ggml's BF16 arithmetic: bf16 activations, f32 sums).
// F32 weight rows (ldw floats apart) x f32 activation rows at token counts
// (K % 32 == 0, 16-byte aligned rows), f32 MFMA.
bool   gemm_f32_supported(int64_t N, int64_t K, int64_t ldw, const void * W, const float * x, int64_t ldx);
int    gemm_f32(const float * W, int64_t ldw, const float * x, int64_t ldx, int64_t N, int64_t K, int64_t M, float * y,
                int64_t ldy, hipStream_t stream);
size_t gemm_bf16_workspace(int64_t K, int64_t M);
bool   gemm_bf16_supported(int64_t N, int64_t K, int64_t rs, const void * W, const float * x, int64_t ldx);
int    gemm_bf16(const void * W, int64_t N, int64_t K, int64_t rs, const float * x, int64_t ldx, int64_t M, float * y,
                 int64_t ldy, void * ws, size_t ws_bytes, hipStream_t stream);
// The epilogue adds bias[n] (if given), then res[m * ldr + n] (if given).
int    gemm_q(int wtype, const void * W, int64_t N, int64_t K, int64_t row_stride, const float * x, int64_t ldx,
              int64_t M, float * y, int64_t ldy, void * ws, size_t ws_bytes, hipStream_t stream,
              const float * bias = nullptr, const float * res = nullptr, int64_t ldr = 0,
              const GemmGlu * glu = nullptr);
// Shape / alignment the GEMM takes (16-byte weight rows and activations).
bool   gemm_supported(int wtype, int64_t N, int64_t K, int64_t rs, const void * W, const float * x, int64_t ldx);
// f32 activation rows -> the packed f16 copy the GEMM reads (K % 8 == 0).
int    convert_act_f16(const float * x, int64_t ldx, int64_t K, int64_t M, void * xh, hipStream_t stream);
// The same on activations already rounded to f16 (rows of K halves, 16-byte aligned).
// With a workspace of gemm_split_bytes (else none) the plain form may split K.
int    gemm_q_h(int wtype, const void * W, int64_t N, int64_t K, int64_t row_stride, const void * xh, int64_t M,
                float * y, int64_t ldy, hipStream_t stream, const float * bias, const float * res, int64_t ldr,
                const GemmGlu * glu = nullptr, const GemmMulti * mul = nullptr, void * split_ws = nullptr,
                size_t split_ws_bytes = 0);

}  // namespace mmhip

#define MMHIP_API_BEGIN() ::mmhip::clear_error()
