// mmhip_api.hip - C-ABI entry points: argument validation, error reporting,
// workspace sizing and kernel selection for MUL_MAT and FLASH_ATTN_EXT.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <unordered_map>

#include "k_fa_common.h"
#include "mmhip_device.h"
#include "mmhip_internal.h"

namespace mmhip {

static thread_local char g_err[512];

void clear_error() {
    g_err[0] = 0;
}

int set_error(int code, const char * fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

bool ensure_lds_limit(const void * kernel, size_t bytes) {
    static std::mutex                               mu;
    static std::unordered_map<const void *, size_t> raised;
    std::lock_guard<std::mutex>                     lock(mu);
    auto                                            it = raised.find(kernel);
    if (it != raised.end() && it->second >= bytes) {
        return true;
    }
    if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int) bytes) != hipSuccess) {
        (void) hipGetLastError();
        return false;
    }
    raised[kernel] = bytes;
    return true;
}

int check_launch(const char * what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        return set_error(MMHIP_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    }
    return MMHIP_OK;
}

// MUL_MAT dispatch: GEMV for small M (column groups of 8, each streaming the
// weights; the second group's rows come back from the Infinity Cache), MFMA
// GEMM beyond: at 9..16 tokens a GEMM has too few tiles to cover the CUs.
constexpr int64_t GEMV_MAX_M = 16;

static bool use_gemm(int type, int64_t M) {
    (void) type;
    return M > GEMV_MAX_M;
}

}  // namespace mmhip

using namespace mmhip;

extern "C" const char * mmhip_last_error(void) {
    return g_err;
}

extern "C" int mmhip_version(void) {
    return 1;
}

extern "C" size_t mmhip_mul_mat_workspace(int type, int64_t N, int64_t K, int64_t M) {
    if (type == TYPE_BF16) {
        // the GEMV reads f32 activations; the GEMM their bf16 copy
        return M > BF16_GEMV_MAXM ? gemm_bf16_workspace(K, M) : 0;
    }
    if (use_gemm(type, M)) {
        return gemm_q_workspace(N, K, M);
    }
    return act_layout(type, K, M).total;
}

extern "C" size_t mmhip_weights_f16_bytes(int64_t N, int64_t K) {
    return N > 0 && K > 0 ? (size_t) N * (size_t) K * 2 : 0;
}

extern "C" int mmhip_weights_to_f16(int type, const void * W, int64_t N, int64_t K, int64_t w_row_stride, void * wh,
                                    void * stream) {
    MMHIP_API_BEGIN();
    return weights_to_f16_checked(type, W, N, K, w_row_stride, wh, (hipStream_t) stream);
}

extern "C" int mmhip_register_weights_f16(const void * W, int64_t N, int64_t K, const void * wh) {
    MMHIP_API_BEGIN();
    return register_f16_weights(W, N, K, wh);
}

extern "C" int mmhip_unregister_weights_f16(const void * W) {
    MMHIP_API_BEGIN();
    return unregister_f16_weights(W);
}

extern "C" size_t mmhip_mul_mat_h_workspace(int type, int64_t N, int64_t K, int64_t M) {
    return is_repacked_type(type) && use_gemm(type, M) ? gemm_split_bytes(N, K, M) : 0;
}

extern "C" int mmhip_mul_mat(int type, const void * W, int64_t N, int64_t K, int64_t w_row_stride, const float * x,
                             int64_t ldx, int64_t M, float * y, int64_t ldy, void * ws, size_t ws_bytes,
                             void * stream) {
    MMHIP_API_BEGIN();
    if (!W || !x || !y || N <= 0 || K <= 0 || M <= 0 || ldx < K || ldy < N) {
        return set_error(MMHIP_ERR_INVALID, "mul_mat: bad arguments N=%lld K=%lld M=%lld", (long long) N,
                         (long long) K, (long long) M);
    }
    hipStream_t st = (hipStream_t) stream;
    if (type == TYPE_BF16) {
        if (M <= BF16_GEMV_MAXM) {
            if (w_row_stride % 2 != 0) {
                return set_error(MMHIP_ERR_UNSUPPORTED, "mul_mat bf16: row stride %lld bytes", (long long) w_row_stride);
            }
            return mmhip_mul_mat_bf16(W, N, K, w_row_stride / 2, x, ldx, M, y, ldy, stream);
        }
        return gemm_bf16(W, N, K, w_row_stride, x, ldx, M, y, ldy, ws, ws_bytes, st);
    }
    if (!is_repacked_type(type)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "mul_mat: weight type %d", type);
    }
    if (use_gemm(type, M)) {
        return gemm_q(type, W, N, K, w_row_stride, x, ldx, M, y, ldy, ws, ws_bytes, st);
    }
    const ActLayout L = act_layout(type, K, M);
    if (L.total == 0 || !gemv_supported(type, N, K, w_row_stride, W)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "mul_mat: type %d N=%lld K=%lld rs=%lld", type, (long long) N,
                         (long long) K, (long long) w_row_stride);
    }
    if (!ws || ws_bytes < L.total) {
        return set_error(MMHIP_ERR_WORKSPACE, "mul_mat: workspace %zu < %zu", ws_bytes, L.total);
    }
    int rc = quantize_act(type, x, ldx, K, M, ws, st);
    if (rc != MMHIP_OK) {
        return rc;
    }
    return gemv_q(type, W, N, K, w_row_stride, ActPtrs::from(L, ws), M, y, ldy, st);
}

extern "C" int mmhip_mul_mat_bias_add(int type, const void * W, int64_t N, int64_t K, int64_t w_row_stride,
                                      const float * x, int64_t ldx, int64_t M, const float * bias, const float * r,
                                      int64_t ldr, float * y, int64_t ldy, void * ws, size_t ws_bytes, void * stream) {
    MMHIP_API_BEGIN();
    if (!W || !x || !y || N <= 0 || K <= 0 || M <= 0 || ldx < K || ldy < N || (r && ldr < N)) {
        return set_error(MMHIP_ERR_INVALID, "mul_mat_bias_add: bad arguments N=%lld K=%lld M=%lld", (long long) N,
                         (long long) K, (long long) M);
    }
    if (!is_repacked_type(type)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "mul_mat_bias_add: weight type %d", type);
    }
    if (!use_gemm(type, M)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "mul_mat_bias_add: token count %lld takes the GEMV path",
                         (long long) M);
    }
    return gemm_q(type, W, N, K, w_row_stride, x, ldx, M, y, ldy, ws, ws_bytes, (hipStream_t) stream, bias, r, ldr);
}

extern "C" int mmhip_mul_mat_bias_add_h(int type, const void * W, int64_t N, int64_t K, int64_t w_row_stride,
                                        const void * xh, int64_t M, const float * bias, const float * r, int64_t ldr,
                                        float * y, int64_t ldy, void * stream) {
    MMHIP_API_BEGIN();
    if (!W || !xh || !y || N <= 0 || K <= 0 || M <= 0 || ldy < N || (r && ldr < N)) {
        return set_error(MMHIP_ERR_INVALID, "mul_mat_bias_add_h: bad arguments N=%lld K=%lld M=%lld", (long long) N,
                         (long long) K, (long long) M);
    }
    if (!is_repacked_type(type) || !use_gemm(type, M)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "mul_mat_bias_add_h: weight type %d at %lld tokens", type,
                         (long long) M);
    }
    return gemm_q_h(type, W, N, K, w_row_stride, xh, M, y, ldy, (hipStream_t) stream, bias, r, ldr);
}

extern "C" int mmhip_mul_mat_bias_add_hw(int type, const void * W, int64_t N, int64_t K, int64_t w_row_stride,
                                         const void * xh, int64_t M, const float * bias, const float * r, int64_t ldr,
                                         float * y, int64_t ldy, void * ws, size_t ws_bytes, void * stream) {
    MMHIP_API_BEGIN();
    if (!W || !xh || !y || N <= 0 || K <= 0 || M <= 0 || ldy < N || (r && ldr < N)) {
        return set_error(MMHIP_ERR_INVALID, "mul_mat_bias_add_hw: bad arguments N=%lld K=%lld M=%lld", (long long) N,
                         (long long) K, (long long) M);
    }
    if (!is_repacked_type(type) || !use_gemm(type, M)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "mul_mat_bias_add_hw: weight type %d at %lld tokens", type,
                         (long long) M);
    }
    return gemm_q_h(type, W, N, K, w_row_stride, xh, M, y, ldy, (hipStream_t) stream, bias, r, ldr, nullptr, nullptr,
                    ws, ws_bytes);
}

static int swiglu_gemm_args(const char * who, int type, const void * W, int64_t N, int64_t K, int64_t M,
                            const float * h, const void * hh) {
    if (!W || (!h && !hh) || N <= 0 || (N & 1) || K <= 0 || M <= 0 || ((uintptr_t) hh) % 2 != 0) {
        return set_error(MMHIP_ERR_INVALID, "%s: bad arguments N=%lld K=%lld M=%lld", who, (long long) N,
                         (long long) K, (long long) M);
    }
    if (!is_repacked_type(type) || !use_gemm(type, M)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "%s: weight type %d at %lld tokens", who, type, (long long) M);
    }
    return MMHIP_OK;
}

extern "C" int mmhip_mul_mat_bias_swiglu(int type, const void * W, int64_t N, int64_t K, int64_t w_row_stride,
                                         const float * x, int64_t ldx, int64_t M, const float * bias, int swapped,
                                         float * h, void * hh, void * ws, size_t ws_bytes, void * stream) {
    MMHIP_API_BEGIN();
    int rc = swiglu_gemm_args("mul_mat_bias_swiglu", type, W, N, K, M, h, hh);
    if (rc != MMHIP_OK) {
        return rc;
    }
    if (!x || ldx < K) {
        return set_error(MMHIP_ERR_INVALID, "mul_mat_bias_swiglu: bad activations");
    }
    GemmGlu glu;
    glu.F       = N / 2;
    glu.swapped = swapped ? 1 : 0;
    glu.h       = h;
    glu.hh      = (_Float16 *) hh;
    return gemm_q(type, W, N, K, w_row_stride, x, ldx, M, nullptr, N, ws, ws_bytes, (hipStream_t) stream, bias,
                  nullptr, 0, &glu);
}

extern "C" int mmhip_mul_mat_bias_swiglu_h(int type, const void * W, int64_t N, int64_t K, int64_t w_row_stride,
                                           const void * xh, int64_t M, const float * bias, int swapped, float * h,
                                           void * hh, void * stream) {
    MMHIP_API_BEGIN();
    int rc = swiglu_gemm_args("mul_mat_bias_swiglu_h", type, W, N, K, M, h, hh);
    if (rc != MMHIP_OK) {
        return rc;
    }
    if (!xh) {
        return set_error(MMHIP_ERR_INVALID, "mul_mat_bias_swiglu_h: null activations");
    }
    GemmGlu glu;
    glu.F       = N / 2;
    glu.swapped = swapped ? 1 : 0;
    glu.h       = h;
    glu.hh      = (_Float16 *) hh;
    return gemm_q_h(type, W, N, K, w_row_stride, xh, M, nullptr, N, (hipStream_t) stream, bias, nullptr, 0, &glu);
}

static int multi_args(const char * who, int type, int n, const void * const * W, int64_t N, int64_t K,
                      int64_t w_row_stride, int64_t M, const float * const * bias, float * const * y,
                      const int64_t * ldy, GemmMulti & mul) {
    if (n < 1 || n > 3 || !W || !y || !ldy || N <= 0 || N % 256 != 0 || K <= 0 || M <= 0) {
        return set_error(MMHIP_ERR_INVALID, "%s: bad arguments n=%d N=%lld K=%lld M=%lld", who, n, (long long) N,
                         (long long) K, (long long) M);
    }
    if (!is_repacked_type(type) || !use_gemm(type, M)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "%s: weight type %d at %lld tokens", who, type, (long long) M);
    }
    mul.n    = n;
    mul.Nper = N;
    for (int i = 0; i < n; i++) {
        if (!W[i] || !y[i] || ldy[i] < N || ((uintptr_t) W[i]) % 16 != 0) {
            return set_error(MMHIP_ERR_INVALID, "%s: matrix %d: null or unaligned operand", who, i);
        }
        mul.W[i]    = (const uint8_t *) W[i];
        mul.y[i]    = y[i];
        mul.ldy[i]  = ldy[i];
        mul.bias[i] = bias ? bias[i] : nullptr;
    }
    return MMHIP_OK;
}

extern "C" int mmhip_mul_mat_multi(int type, int n, const void * const * W, int64_t N, int64_t K, int64_t w_row_stride,
                                   const float * x, int64_t ldx, int64_t M, const float * const * bias,
                                   float * const * y, const int64_t * ldy, void * ws, size_t ws_bytes, void * stream) {
    MMHIP_API_BEGIN();
    GemmMulti mul;
    int       rc = multi_args("mul_mat_multi", type, n, W, N, K, w_row_stride, M, bias, y, ldy, mul);
    if (rc != MMHIP_OK) {
        return rc;
    }
    if (!x || ldx < K || !gemm_supported(type, N, K, w_row_stride, W[0], x, ldx)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "mul_mat_multi: activations or weights not supported");
    }
    const size_t need = gemm_workspace(K, M);
    if (!ws || ws_bytes < need || ((uintptr_t) ws) % 16 != 0) {
        return set_error(MMHIP_ERR_WORKSPACE, "mul_mat_multi: workspace %zu < %zu (16-byte aligned)", ws_bytes, need);
    }
    rc = convert_act_f16(x, ldx, K, M, ws, (hipStream_t) stream);
    if (rc != MMHIP_OK) {
        return rc;
    }
    return gemm_q_h(type, W[0], (int64_t) n * N, K, w_row_stride, ws, M, y[0], ldy[0], (hipStream_t) stream, nullptr,
                    nullptr, 0, nullptr, &mul);
}

extern "C" int mmhip_mul_mat_multi_h(int type, int n, const void * const * W, int64_t N, int64_t K,
                                     int64_t w_row_stride, const void * xh, int64_t M, const float * const * bias,
                                     float * const * y, const int64_t * ldy, void * stream) {
    MMHIP_API_BEGIN();
    GemmMulti mul;
    int       rc = multi_args("mul_mat_multi_h", type, n, W, N, K, w_row_stride, M, bias, y, ldy, mul);
    if (rc != MMHIP_OK) {
        return rc;
    }
    if (!xh) {
        return set_error(MMHIP_ERR_INVALID, "mul_mat_multi_h: null activations");
    }
    return gemm_q_h(type, W[0], (int64_t) n * N, K, w_row_stride, xh, M, y[0], ldy[0], (hipStream_t) stream, nullptr,
                    nullptr, 0, nullptr, &mul);
}

// ---------------------------------------------------------------------
// FLASH_ATTN_EXT

static int fa_validate(const mmhip_view * q, const mmhip_view * k, const mmhip_view * v, const mmhip_view * mask,
                       FaArgs & a, int & D) {
    if (!q || !k || !v || !q->data || !k->data || !v->data) {
        return set_error(MMHIP_ERR_INVALID, "flash_attn: null operand");
    }
    D = (int) q->ne[0];
    if (!(D == 64 || D == 128 || D == 256) || k->ne[0] != D || v->ne[0] != D) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "flash_attn: head dims q=%lld k=%lld v=%lld", (long long) q->ne[0],
                         (long long) k->ne[0], (long long) v->ne[0]);
    }
    if (q->nb[0] != 4 || k->nb[0] != 2 || v->nb[0] != 2) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "flash_attn: dim 0 must be contiguous (q f32, k/v f16)");
    }
    if (k->ne[1] != v->ne[1] || k->ne[2] != v->ne[2] || k->ne[3] != v->ne[3]) {
        return set_error(MMHIP_ERR_INVALID, "flash_attn: k/v shape mismatch");
    }
    if (k->ne[1] <= 0 || q->ne[1] <= 0 || k->ne[2] <= 0 || q->ne[2] % k->ne[2] != 0 || q->ne[3] % k->ne[3] != 0) {
        return set_error(MMHIP_ERR_INVALID, "flash_attn: head/batch broadcast mismatch");
    }
    const int64_t lim = (int64_t) 1 << 30;
    if (q->ne[1] > lim || k->ne[1] > lim || q->ne[2] > 65535 || q->ne[3] > 65535) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "flash_attn: sizes out of range");
    }
    // 16-byte K/V row loads
    const uintptr_t kv_align = (uintptr_t) k->data | (uintptr_t) v->data | (uintptr_t) k->nb[1] |
                               (uintptr_t) k->nb[2] | (uintptr_t) k->nb[3] | (uintptr_t) v->nb[1] |
                               (uintptr_t) v->nb[2] | (uintptr_t) v->nb[3];
    if (kv_align % 16 != 0 || ((uintptr_t) q->data | (uintptr_t) q->nb[1] | (uintptr_t) q->nb[2] |
                               (uintptr_t) q->nb[3]) % 4 != 0) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "flash_attn: misaligned operands");
    }
    memset(&a, 0, sizeof(a));
    a.q    = (const char *) q->data;
    a.qnb1 = q->nb[1];
    a.qnb2 = q->nb[2];
    a.qnb3 = q->nb[3];
    a.k    = (const char *) k->data;
    a.knb1 = k->nb[1];
    a.knb2 = k->nb[2];
    a.knb3 = k->nb[3];
    a.v    = (const char *) v->data;
    a.vnb1 = v->nb[1];
    a.vnb2 = v->nb[2];
    a.vnb3 = v->nb[3];
    a.nq   = (int) q->ne[1];
    a.Hq   = (int) q->ne[2];
    a.B    = (int) q->ne[3];
    a.nkv  = (int) k->ne[1];
    a.Hkv  = (int) k->ne[2];
    a.Bk   = (int) k->ne[3];
    if (mask && mask->data) {
        if (mask->nb[0] != 2 || mask->ne[0] < k->ne[1] || mask->ne[1] < q->ne[1] || mask->ne[2] <= 0 ||
            mask->ne[3] <= 0 || q->ne[2] % mask->ne[2] != 0 || q->ne[3] % mask->ne[3] != 0) {
            return set_error(MMHIP_ERR_INVALID, "flash_attn: mask shape [%lld,%lld,%lld,%lld] does not cover q/k",
                             (long long) mask->ne[0], (long long) mask->ne[1], (long long) mask->ne[2],
                             (long long) mask->ne[3]);
        }
        a.mask = (const char *) mask->data;
        a.mnb1 = mask->nb[1];
        a.mnb2 = mask->nb[2];
        a.mnb3 = mask->nb[3];
        a.mne2 = (int) mask->ne[2];
        a.mne3 = (int) mask->ne[3];
    } else {
        a.mne2 = 1;
        a.mne3 = 1;
    }
    return MMHIP_OK;
}

extern "C" size_t mmhip_flash_attn_workspace(const mmhip_view * q, const mmhip_view * k, const mmhip_view * v) {
    FaArgs a;
    int    D;
    if (fa_validate(q, k, v, nullptr, a, D) != MMHIP_OK) {
        return 0;
    }
    return fa_use_mfma(a, D) ? fa_mfma_workspace(a) : fa_decode_workspace(a, D);
}

extern "C" int mmhip_flash_attn_ext(const mmhip_view * q, const mmhip_view * k, const mmhip_view * v,
                                    const mmhip_view * mask, float scale, float * out, void * ws, size_t ws_bytes,
                                    void * stream) {
    MMHIP_API_BEGIN();
    FaArgs a;
    int    D;
    int    rc = fa_validate(q, k, v, mask, a, D);
    if (rc != MMHIP_OK) {
        return rc;
    }
    if (!out) {
        return set_error(MMHIP_ERR_INVALID, "flash_attn: null output");
    }
    a.scale = scale;
    if (fa_use_mfma(a, D)) {
        return fa_mfma(a, D, out, ws, ws_bytes, (hipStream_t) stream);
    }
    return fa_decode(a, D, out, ws, ws_bytes, (hipStream_t) stream);
}

// The Q / K / V head chains (mmhip_head_rows_args) folded into the decode
// attention: checks that they feed this attention exactly and builds FaHead.
static int fa_head_args(const mmhip_view * q, const mmhip_view * k, const mmhip_view * v, const FaArgs & a, int D,
                        const mmhip_head_rows_args * hr, FaHead & h) {
    const mmhip_head_rows_args & hq = hr[0];
    const mmhip_head_rows_args & hk = hr[1];
    const mmhip_head_rows_args & hv = hr[2];
    const int64_t                rb = (int64_t) D * 4;  // bytes of one processed query row
    const int64_t                qoff = (const char *) q->data - (const char *) hq.dst;
    const bool q_ok = hq.D == D && !hq.ids && hq.dst && hq.src && hq.H > 0 && hq.T > 0 && qoff >= 0 && qoff % rb == 0 &&
                      q->nb[1] % rb == 0 && q->nb[2] % rb == 0 && q->nb[3] % rb == 0 &&
                      qoff + (q->ne[1] - 1) * q->nb[1] + (q->ne[2] - 1) * q->nb[2] + (q->ne[3] - 1) * q->nb[3] + rb <=
                          (int64_t) hq.H * hq.T * rb;
    auto cache_ok = [&](const mmhip_head_rows_args & c, const mmhip_view * kv) {
        return c.D == D && c.src && c.ids && c.dst == kv->data && c.dst_type == 1 && c.dst_nb1 == kv->nb[1] &&
               c.dst_nb2 == kv->nb[2] && c.dst_nb3 == kv->nb[3] && c.H == a.Hkv && c.T == a.B &&
               (c.ids_type == 26 || c.ids_type == 27) && c.ids_ne1 > 0 && c.ids_ne2 > 0;
    };
    const bool same_ids = hk.ids == hv.ids && hk.ids_type == hv.ids_type && hk.ids_nb1 == hv.ids_nb1 &&
                          hk.ids_nb2 == hv.ids_nb2 && hk.ids_ne1 == hv.ids_ne1 && hk.ids_ne2 == hv.ids_ne2;
    if (!q_ok || !cache_ok(hk, k) || !cache_ok(hv, v) || !same_ids || hv.norm || hv.pos) {
        return set_error(MMHIP_ERR_INVALID, "flash_attn_head: the head chains do not feed this attention");
    }
    memset(&h, 0, sizeof(h));
    h.q_src    = (const char *) hq.src;
    h.q_nbh    = hq.src_nb_h;
    h.q_nbt    = hq.src_nb_t;
    h.q_H      = hq.H;
    h.q_w      = hq.norm ? hq.norm_w : nullptr;
    h.q_eps    = hq.eps;
    h.q_norm   = hq.norm;
    h.q_pos    = hq.pos;
    h.q_ts     = hq.theta_scale;
    h.qr0      = qoff / rb;
    h.qr1      = q->nb[1] / rb;
    h.qr2      = q->nb[2] / rb;
    h.qr3      = q->nb[3] / rb;
    h.k_src    = (const char *) hk.src;
    h.k_nbh    = hk.src_nb_h;
    h.k_nbt    = hk.src_nb_t;
    h.k_w      = hk.norm ? hk.norm_w : nullptr;
    h.k_eps    = hk.eps;
    h.k_norm   = hk.norm;
    h.k_pos    = hk.pos;
    h.k_ts     = hk.theta_scale;
    h.v_src    = (const char *) hv.src;
    h.v_nbh    = hv.src_nb_h;
    h.v_nbt    = hv.src_nb_t;
    h.ids      = (const char *) hk.ids;
    h.ids_type = hk.ids_type;
    h.ids_nb1  = hk.ids_nb1;
    h.ids_nb2  = hk.ids_nb2;
    h.ids_ne1  = hk.ids_ne1;
    h.ids_ne2  = hk.ids_ne2;
    return MMHIP_OK;
}

extern "C" int mmhip_flash_attn_ext_head_supported(const mmhip_view * q, const mmhip_view * k, const mmhip_view * v) {
    FaArgs a;
    int    D;
    if (fa_validate(q, k, v, nullptr, a, D) != MMHIP_OK) {
        clear_error();
        return 0;
    }
    return !fa_use_mfma(a, D) && fa_decode_head_supported(a, D);
}

extern "C" int mmhip_flash_attn_ext_head(const mmhip_view * q, const mmhip_view * k, const mmhip_view * v,
                                         const mmhip_view * mask, float scale, float * out, void * ws, size_t ws_bytes,
                                         int type, void * xq, const mmhip_head_rows_args * heads, void * stream) {
    MMHIP_API_BEGIN();
    FaArgs a;
    int    D;
    int    rc = fa_validate(q, k, v, mask, a, D);
    if (rc != MMHIP_OK) {
        return rc;
    }
    if (!out || !heads || fa_use_mfma(a, D) || !fa_decode_head_supported(a, D)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "flash_attn_head: not a decode shape the fused prologue takes");
    }
    const int64_t K = (int64_t) a.Hq * D, M = (int64_t) a.B * a.nq;
    if (xq && act_layout(type, K, M).total == 0) {
        return set_error(MMHIP_ERR_INVALID, "flash_attn_head: activation type %d for K=%lld", type, (long long) K);
    }
    FaHead h;
    rc = fa_head_args(q, k, v, a, D, heads, h);
    if (rc != MMHIP_OK) {
        return rc;
    }
    a.scale        = scale;
    bool quantised = false;
    rc = fa_decode(a, D, out, ws, ws_bytes, (hipStream_t) stream, xq ? type : 0, xq, &quantised, &h);
    if (rc != MMHIP_OK || !xq || quantised) {
        return rc;
    }
    return quantize_act(type, out, K, K, M, xq, (hipStream_t) stream);
}

extern "C" int mmhip_flash_attn_ext_q(const mmhip_view * q, const mmhip_view * k, const mmhip_view * v,
                                      const mmhip_view * mask, float scale, float * out, void * ws, size_t ws_bytes,
                                      int type, void * xq, void * stream) {
    MMHIP_API_BEGIN();
    FaArgs a;
    int    D;
    int    rc = fa_validate(q, k, v, mask, a, D);
    if (rc != MMHIP_OK) {
        return rc;
    }
    const int64_t K = (int64_t) a.Hq * D, M = (int64_t) a.B * a.nq;
    if (!out || !xq || act_layout(type, K, M).total == 0) {
        return set_error(MMHIP_ERR_INVALID, "flash_attn_q: bad output / activation type %d for K=%lld", type,
                         (long long) K);
    }
    a.scale        = scale;
    bool quantised = false;
    if (fa_use_mfma(a, D)) {
        rc = fa_mfma(a, D, out, ws, ws_bytes, (hipStream_t) stream);
    } else {
        rc = fa_decode(a, D, out, ws, ws_bytes, (hipStream_t) stream, type, xq, &quantised);
    }
    if (rc != MMHIP_OK || quantised) {
        return rc;
    }
    // output rows (b, iq) of Hq * D contiguous f32: quantise them separately
    return quantize_act(type, out, K, K, M, xq, (hipStream_t) stream);
}

// ---------------------------------------------------------------------------
// Attention without allocation: the workspace of mmhip_flash_attn_ext (the
// split-KV partials of the decode kernels, the mask prepass rows of the MFMA
// kernel) lives in a file-scope device array, one copy per GPU, held until the
// process ends.  Its device address is looked up once per device with that
// device current; kernels receive that address, never the array's name.
// Every call on one GPU shares the array (calls that overlap on one GPU race);
// nothing in it has to start at zero: each launch writes every partial /
// row entry it later reads.

namespace {

constexpr size_t   NOALLOC_SCRATCH_BYTES = 8u << 20;  // 8 MiB per GPU
constexpr int      NOALLOC_MAX_DEVICES   = 64;
std::mutex         g_scratch_mu;
void *             g_scratch_ptr[NOALLOC_MAX_DEVICES] = {};

}  // namespace

static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

// The device address of `scratch` on the current device (looked up on the
// first call per device); nullptr with the error set on failure.
static void * scratch_on_current_device() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= NOALLOC_MAX_DEVICES) {
        (void) hipGetLastError();
        set_error(MMHIP_ERR_HIP, "flash_attn_noalloc: no current device");
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *           p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            (void) hipGetLastError();
            set_error(MMHIP_ERR_HIP, "flash_attn_noalloc: scratch address on device %d: %s", dev,
                      hipGetErrorString(e));
            return nullptr;
        }
        g_scratch_ptr[dev] = p;
    }
    return g_scratch_ptr[dev];
}

extern "C" size_t mmhip_flash_attn_noalloc_max_workspace(void) {
    return NOALLOC_SCRATCH_BYTES;
}

extern "C" int mmhip_flash_attn_ext_noalloc(const mmhip_view * q, const mmhip_view * k, const mmhip_view * v,
                                            const mmhip_view * mask, float scale, float * out, void * stream) {
    MMHIP_API_BEGIN();
    FaArgs a;
    int    D;
    int    rc = fa_validate(q, k, v, mask, a, D);
    if (rc != MMHIP_OK) {
        return rc;
    }
    if (!out) {
        return set_error(MMHIP_ERR_INVALID, "flash_attn_noalloc: null output");
    }
    const size_t need = fa_use_mfma(a, D) ? fa_mfma_workspace(a) : fa_decode_workspace(a, D);
    if (need > NOALLOC_SCRATCH_BYTES) {
        return set_error(MMHIP_ERR_WORKSPACE, "flash_attn_noalloc: needs %zu bytes of scratch, the maximum is %zu",
                         need, NOALLOC_SCRATCH_BYTES);
    }
    void * ws = scratch_on_current_device();
    if (!ws) {
        return MMHIP_ERR_HIP;
    }
    a.scale = scale;
    if (fa_use_mfma(a, D)) {
        return fa_mfma(a, D, out, ws, NOALLOC_SCRATCH_BYTES, (hipStream_t) stream);
    }
    return fa_decode(a, D, out, ws, NOALLOC_SCRATCH_BYTES, (hipStream_t) stream);
}
