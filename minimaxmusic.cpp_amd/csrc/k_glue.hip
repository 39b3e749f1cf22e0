// k_glue.hip - the element-wise / row ops around the hot path of the LM
// batched decode step (src/qwen3-lm.h:730-859, src/qwen3-enc.h:87-115):
// ADD / SUB / MUL with ggml broadcasting, RMS_NORM optionally fused with the
// following MUL by the norm weight, NeoX RoPE, CPY / CONT (f32 / f16),
// GET_ROWS (f32, f16 and quantized rows), SET_ROWS (f32 -> f16 / f32), GLU
// SwiGLU and SCALE.  All operands are ggml views (ne, byte strides nb); outputs
// of ADD/MUL/RMS_NORM/ROPE/GLU/SCALE/GET_ROWS are contiguous, as ggml creates
// them.  These are launch-bound at decode sizes; they are written for
// correctness on any strides, with float math matching ggml-CPU's definitions
// (no contraction where ggml rounds twice).
#include "mmhip_device.h"
#include "mmhip_internal.h"

namespace mmhip {

struct TV {
    char *  data;
    int64_t ne[4];
    int64_t nb[4];
};

static TV tv(const mmhip_view * v) {
    TV t;
    t.data = (char *) v->data;
    for (int i = 0; i < 4; i++) {
        t.ne[i] = v->ne[i];
        t.nb[i] = v->nb[i];
    }
    return t;
}

// Element index -> (i0, i1, i2, i3).  Glue tensors are far below 2^31
// elements (the API checks), so the divisions are 32-bit.
__device__ __forceinline__ void unravel(int64_t i64, const int64_t * ne, int64_t & i0, int64_t & i1, int64_t & i2,
                                        int64_t & i3) {
    uint32_t       i  = (uint32_t) i64;
    const uint32_t n0 = (uint32_t) ne[0], n1 = (uint32_t) ne[1], n2 = (uint32_t) ne[2];
    i0                = i % n0;
    i /= n0;
    i1 = i % n1;
    i /= n1;
    i2 = i % n2;
    i3 = i / n2;
}

__device__ __forceinline__ char * at(const TV & t, int64_t i0, int64_t i1, int64_t i2, int64_t i3) {
    return t.data + i0 * t.nb[0] + i1 * t.nb[1] + i2 * t.nb[2] + i3 * t.nb[3];
}

static int64_t nel(const mmhip_view * v) {
    return v->ne[0] * v->ne[1] * v->ne[2] * v->ne[3];
}

static unsigned grid_for(int64_t n, int block) {
    return (unsigned) std::min<int64_t>((n + block - 1) / block, 1 << 20);
}

// ---------------------------------------------------------------------------
// binary ops, b broadcast over a (ggml_can_repeat(b, a))

// contiguous a and b with b broadcast over whole rows of ne0 elements
template <int OP>
__global__ void k_binary_rows(const float * __restrict__ a, const float * __restrict__ b, float * __restrict__ dst,
                              uint32_t n, uint32_t ne0, uint32_t b_rows) {
#pragma clang fp contract(off)
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const float x = a[i];
        const float y = b[(i / ne0) % b_rows * ne0 + i % ne0];
        dst[i]        = OP == 0 ? x + y : OP == 1 ? x - y : x * y;
    }
}

template <int OP>
__global__ void k_binary(TV a, TV b, float * __restrict__ dst, int64_t n) {
#pragma clang fp contract(off)
    for (int64_t i = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; i < n; i += (int64_t) gridDim.x * blockDim.x) {
        int64_t i0, i1, i2, i3;
        unravel(i, a.ne, i0, i1, i2, i3);
        const float x = *(const float *) at(a, i0, i1, i2, i3);
        const float y = *(const float *) at(b, i0 % b.ne[0], i1 % b.ne[1], i2 % b.ne[2], i3 % b.ne[3]);
        dst[i]        = OP == 0 ? x + y : OP == 1 ? x - y : x * y;
    }
}

// Pointers of one quantised activation row (layout of act_layout()).
struct QRow {
    int8_t *  qs;
    float *   d;
    int16_t * bs;
    int       qtype;
    int       spb;  // scales per 256-element chunk: 8 (Q8_0) or 1 (Q8_K)

    __device__ void chunk(const float (&v)[4], int lane, int c) const {
        quant_chunk256(v, lane, qtype, qs + 256 * c, d + spb * c, bs ? bs + 16 * c : nullptr);
    }
};

__device__ __forceinline__ QRow qrow(int qtype, int8_t * qs, float * d, int16_t * bs, int64_t row, int n) {
    QRow r;
    r.qtype = qtype;
    r.spb   = qtype == TYPE_Q8_0 ? 8 : 1;
    r.qs    = qs + row * n;
    r.d     = d + row * (n / (qtype == TYPE_Q8_0 ? 32 : 256));
    r.bs    = bs ? bs + row * (n / 16) : nullptr;
    return r;
}

// ---------------------------------------------------------------------------
// rms_norm (+ mul) (+ activation quantisation): one workgroup (4 waves) per
// row of n f32 elements, n % 256 == 0, n <= 1024 * CPW.  The row splits into
// 256-element chunks; wave w owns chunks w, w + 4, ..., lane l elements
// 4l .. 4l+3 of each, so a chunk is exactly the quantisation unit of
// quant_chunk256.  Every load of x and of the norm weight w (contiguous
// vector of n) is issued before the reduction.  Squares are summed in double
// and mean = sum / n rounded to f32, as ggml-CPU's RMS_NORM does.  With
// xq_qs != nullptr the normalised row is also quantised for the GEMV that
// consumes it.

template <int CPW>  // chunks per wave
__global__ __launch_bounds__(256) void k_rms_norm_row(const char * __restrict__ x, int64_t xs1, int64_t xs2,
                                                      int64_t xs3, int ne1, int ne2, int n,
                                                      const float * __restrict__ w, float eps,
                                                      float * __restrict__ dst, int qtype, int8_t * __restrict__ xq_qs,
                                                      float * __restrict__ xq_d, int16_t * __restrict__ xq_bs) {
#pragma clang fp contract(off)
    __shared__ double s_part[4];
    const int     row  = (int) blockIdx.x;
    const int     lane = threadIdx.x & 63;
    const int     wv   = threadIdx.x >> 6;
    const int     nch  = n / 256;
    const int     i1 = row % ne1, i2 = (row / ne1) % ne2, i3 = row / (ne1 * ne2);
    const float * xr = (const float *) (x + i1 * xs1 + i2 * xs2 + i3 * xs3);
    float4_t      v[CPW], wq[CPW];
#pragma unroll
    for (int j = 0; j < CPW; j++) {
        // chunks past the row end re-read the last chunk and are masked below
        const int c = min(4 * j + wv, nch - 1);
        v[j]        = *(const float4_t *) (xr + 256 * c + 4 * lane);
        wq[j]       = w ? *(const float4_t *) (w + 256 * c + 4 * lane) : float4_t{ 1.0f, 1.0f, 1.0f, 1.0f };
    }
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < CPW; j++) {
        if (4 * j + wv < nch) {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                ss += (double) (v[j][k] * v[j][k]);
            }
        }
    }
    ss = wave_sum_d(ss);
    if (lane == 0) {
        s_part[wv] = ss;
    }
    __syncthreads();
    ss               = s_part[0] + s_part[1] + s_part[2] + s_part[3];
    const float mean = (float) (ss / (double) n);
    const float sc   = 1.0f / sqrtf(mean + eps);
    const QRow  q    = xq_qs ? qrow(qtype, xq_qs, xq_d, xq_bs, row, n) : QRow{};
#pragma unroll
    for (int j = 0; j < CPW; j++) {
        const int c = 4 * j + wv;
        if (c < nch) {
            float o[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float t = v[j][k] * sc;
                o[k]          = w ? t * wq[j][k] : t;
            }
            if (dst) {
                *(float4_t *) (dst + (int64_t) row * n + 256 * c + 4 * lane) = float4_t{ o[0], o[1], o[2], o[3] };
            }
            if (xq_qs) {
                q.chunk(o, lane, c);
            }
        }
    }
}

// generic fallback: any strides and any broadcast of w (one workgroup per row)
__global__ __launch_bounds__(256) void k_rms_norm(TV x, TV w, int has_w, float eps, float * __restrict__ dst) {
#pragma clang fp contract(off)
    __shared__ double s_part[4];
    const int64_t     row = blockIdx.x;
    const int64_t     i1 = row % x.ne[1], i2 = (row / x.ne[1]) % x.ne[2], i3 = row / (x.ne[1] * x.ne[2]);
    const int64_t     n  = x.ne[0];
    const char *      xr = at(x, 0, i1, i2, i3);
    double            ss = 0.0;
    for (int64_t i = threadIdx.x; i < n; i += 256) {
        const float v = *(const float *) (xr + i * x.nb[0]);
        ss += (double) (v * v);
    }
    ss = wave_sum_d(ss);
    if ((threadIdx.x & 63) == 0) {
        s_part[threadIdx.x >> 6] = ss;
    }
    __syncthreads();
    ss               = s_part[0] + s_part[1] + s_part[2] + s_part[3];
    const float mean = (float) (ss / (double) n);
    const float sc   = 1.0f / sqrtf(mean + eps);
    float *     dr   = dst + row * n;
    for (int64_t i = threadIdx.x; i < n; i += 256) {
        const float t = *(const float *) (xr + i * x.nb[0]) * sc;
        if (has_w) {
            const float wv = *(const float *) at(w, i % w.ne[0], i1 % w.ne[1], i2 % w.ne[2], i3 % w.ne[3]);
            dr[i]          = t * wv;
        } else {
            dr[i] = t;
        }
    }
}

// GGML_OP_NORM (LayerNorm without affine part, src/dit.h:161-167): one
// workgroup per row, ggml-CPU's steps -- mean from a double sum, y = x - mean,
// variance from the double sum of y^2, y *= 1 / sqrtf(variance + eps).  With
// w / b it also applies the MUL and ADD that follow it (dit_layer_norm),
// each rounded as its own op: (y * w[i]) + b[i].
__global__ __launch_bounds__(256) void k_layer_norm(TV x, float eps, const float * __restrict__ w,
                                                     const float * __restrict__ b, float * dst,
                                                     _Float16 * __restrict__ dsth) {
#pragma clang fp contract(off)
    __shared__ double s_part[4];
    const int64_t     row = blockIdx.x;
    const int64_t     i1 = row % x.ne[1], i2 = (row / x.ne[1]) % x.ne[2], i3 = row / (x.ne[1] * x.ne[2]);
    const int64_t     n  = x.ne[0];
    const char *      xr = at(x, 0, i1, i2, i3);
    double            sm = 0.0;
    for (int64_t i = threadIdx.x; i < n; i += 256) {
        sm += (double) *(const float *) (xr + i * x.nb[0]);
    }
    sm = wave_sum_d(sm);
    if ((threadIdx.x & 63) == 0) {
        s_part[threadIdx.x >> 6] = sm;
    }
    __syncthreads();
    const float mean = (float) ((s_part[0] + s_part[1] + s_part[2] + s_part[3]) / (double) n);
    __syncthreads();
    double ss = 0.0;
    for (int64_t i = threadIdx.x; i < n; i += 256) {
        const float v = *(const float *) (xr + i * x.nb[0]) - mean;
        ss += (double) (v * v);
    }
    ss = wave_sum_d(ss);
    if ((threadIdx.x & 63) == 0) {
        s_part[threadIdx.x >> 6] = ss;
    }
    __syncthreads();
    const float var = (float) ((s_part[0] + s_part[1] + s_part[2] + s_part[3]) / (double) n);
    const float sc  = 1.0f / sqrtf(var + eps);
    for (int64_t i = threadIdx.x; i < n; i += 256) {
        // x - mean again (the same f32 value), then the scale and the affine part
        float t = (*(const float *) (xr + i * x.nb[0]) - mean) * sc;
        if (w) {
            t = t * w[i];
        }
        if (b) {
            t = t + b[i];
        }
        if (dst) {
            dst[row * n + i] = t;
        }
        if (dsth) {
            dsth[row * n + i] = (_Float16) t;
        }
    }
}

// The same on rows held in registers: 16-byte aligned rows of n % 4 == 0
// floats, n <= 1024 C, read once as float4 (the three passes above read each
// row three times).  The same f32 steps; the double sums add each thread's
// four consecutive values first, then across threads.
template <int C>
__global__ __launch_bounds__(256) void k_layer_norm_v(TV x, float eps, const float * __restrict__ w,
                                                       const float * __restrict__ b, float * dst,
                                                       _Float16 * __restrict__ dsth) {
#pragma clang fp contract(off)
    __shared__ double s_part[4];
    const int64_t     row = blockIdx.x;
    const int64_t     i1 = row % x.ne[1], i2 = (row / x.ne[1]) % x.ne[2], i3 = row / (x.ne[1] * x.ne[2]);
    const int         n  = (int) x.ne[0], n4 = n / 4;
    const float4_t *  xr = (const float4_t *) at(x, 0, i1, i2, i3);
    float4_t          v[C];
    double            sm = 0.0;
#pragma unroll
    for (int c = 0; c < C; c++) {
        const int j = threadIdx.x + 256 * c;
        v[c]        = j < n4 ? xr[j] : float4_t{ 0.0f, 0.0f, 0.0f, 0.0f };
        sm += (double) v[c][0] + (double) v[c][1] + (double) v[c][2] + (double) v[c][3];
    }
    sm = wave_sum_d(sm);
    if ((threadIdx.x & 63) == 0) {
        s_part[threadIdx.x >> 6] = sm;
    }
    __syncthreads();
    const float mean = (float) ((s_part[0] + s_part[1] + s_part[2] + s_part[3]) / (double) n);
    __syncthreads();
    double ss = 0.0;
#pragma unroll
    for (int c = 0; c < C; c++) {
        if (threadIdx.x + 256 * c < n4) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float d = v[c][e] - mean;
                ss += (double) (d * d);
            }
        }
    }
    ss = wave_sum_d(ss);
    if ((threadIdx.x & 63) == 0) {
        s_part[threadIdx.x >> 6] = ss;
    }
    __syncthreads();
    const float var = (float) ((s_part[0] + s_part[1] + s_part[2] + s_part[3]) / (double) n);
    const float sc  = 1.0f / sqrtf(var + eps);
#pragma unroll
    for (int c = 0; c < C; c++) {
        const int j = threadIdx.x + 256 * c;
        if (j >= n4) {
            continue;
        }
        float4_t t;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            t[e] = (v[c][e] - mean) * sc;
        }
        if (w) {
            const float4_t wv = ((const float4_t *) w)[j];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                t[e] = t[e] * wv[e];
            }
        }
        if (b) {
            const float4_t bv = ((const float4_t *) b)[j];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                t[e] = t[e] + bv[e];
            }
        }
        if (dst) {
            ((float4_t *) (dst + row * n))[j] = t;
        }
        if (dsth) {
            half4_t h;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                h[e] = (_Float16) t[e];
            }
            ((half4_t *) (dsth + row * n))[j] = h;
        }
    }
}

// GGML_OP_CONCAT of two f32 tensors along dim (src/dit.h:262-273): dst is
// contiguous; an index below a's extent along dim reads a, the rest b.
__global__ void k_concat(TV a, TV b, int dim, int64_t n, float * __restrict__ dst) {
    int64_t ne[4];
    for (int i = 0; i < 4; i++) {
        ne[i] = a.ne[i] + (i == dim ? b.ne[i] : 0);
    }
    for (int64_t i = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; i < n; i += (int64_t) gridDim.x * blockDim.x) {
        int64_t j[4];
        unravel(i, ne, j[0], j[1], j[2], j[3]);
        const int64_t na = a.ne[dim];
        if (j[dim] < na) {
            dst[i] = *(const float *) at(a, j[0], j[1], j[2], j[3]);
        } else {
            j[dim] -= na;
            dst[i] = *(const float *) at(b, j[0], j[1], j[2], j[3]);
        }
    }
}

// GGML_OP_CLAMP (src/dit.h:276-278): ggml-CPU's MAX(MIN(x, hi), lo).
__global__ void k_clamp(TV a, float lo, float hi, int64_t n, float * __restrict__ dst) {
    for (int64_t i = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; i < n; i += (int64_t) gridDim.x * blockDim.x) {
        int64_t i0, i1, i2, i3;
        unravel(i, a.ne, i0, i1, i2, i3);
        const float x = *(const float *) at(a, i0, i1, i2, i3);
        const float t = x < hi ? x : hi;
        dst[i]        = t > lo ? t : lo;
    }
}

// GGML_OP_MUL_MAT of two f32 tensors (activation x activation: the depth
// decoder's manual attention, src/depth-decoder.h:214-219): dst[i, j, i2, i3]
// = sum_k a[k, i, i2 / r2, i3 / r3] * b[k, j, i2, i3] over any strides, f32
// products summed in double.  One thread per output element.
__global__ void k_mul_mat_f32(TV a, TV b, float * __restrict__ dst, int64_t ne0, int64_t ne1, int64_t ne2,
                              int64_t K, int64_t r2, int64_t r3, int64_t n) {
    for (int64_t t = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; t < n; t += (int64_t) gridDim.x * blockDim.x) {
        const int64_t i = t % ne0, j = (t / ne0) % ne1, i2 = (t / (ne0 * ne1)) % ne2, i3 = t / (ne0 * ne1 * ne2);
        const char *  pa = at(a, 0, i, i2 / r2, i3 / r3);
        const char *  pb = at(b, 0, j, i2, i3);
        double        acc = 0.0;
        for (int64_t k = 0; k < K; k++) {
            acc += (double) (*(const float *) (pa + k * a.nb[0]) * *(const float *) (pb + k * b.nb[0]));
        }
        dst[t] = (float) acc;
    }
}

// The same with one wave per output (long K: the attention scores, K = head
// dim 256): lanes stride over K (coalesced), double partial sums reduced
// symmetrically across the wave.
__global__ __launch_bounds__(256) void k_mul_mat_f32_wave(TV a, TV b, float * __restrict__ dst, int64_t ne0,
                                                          int64_t ne1, int64_t ne2, int64_t K, int64_t r2, int64_t r3,
                                                          int64_t n) {
    const int64_t t = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int     l = threadIdx.x & 63;
    if (t >= n) {
        return;
    }
    const int64_t i = t % ne0, j = (t / ne0) % ne1, i2 = (t / (ne0 * ne1)) % ne2, i3 = t / (ne0 * ne1 * ne2);
    const char *  pa = at(a, 0, i, i2 / r2, i3 / r3);
    const char *  pb = at(b, 0, j, i2, i3);
    double        acc = 0.0;
    for (int64_t k = l; k < K; k += 64) {
        acc += (double) (*(const float *) (pa + k * a.nb[0]) * *(const float *) (pb + k * b.nb[0]));
    }
    acc = wave_sum_d(acc);
    if (l == 0) {
        dst[t] = (float) acc;
    }
}

// GGML_OP_DIAG_MASK_INF (src/depth-decoder.h:216): element (i0, i1, ..) of a
// with i0 > n_past + i1 becomes -inf; dst contiguous.
__global__ void k_diag_mask_inf(TV a, int n_past, int64_t n, float * __restrict__ dst) {
    for (int64_t t = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; t < n; t += (int64_t) gridDim.x * blockDim.x) {
        int64_t i0, i1, i2, i3;
        unravel(t, a.ne, i0, i1, i2, i3);
        const float v = *(const float *) at(a, i0, i1, i2, i3);
        dst[t]        = i0 > n_past + i1 ? -INFINITY : v;
    }
}

// GGML_OP_SOFT_MAX without mask, scale 1 (src/depth-decoder.h:217, the
// sampler's softmax :348): one wave per row, ggml-CPU's steps -- the row max,
// e = expf(x - max), the sum of e in double, y = e * (float) (1 / sum).
__global__ __launch_bounds__(256) void k_soft_max_rows(TV a, int64_t rows, float * __restrict__ dst) {
#pragma clang fp contract(off)
    const int64_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int     l   = threadIdx.x & 63;
    if (row >= rows) {
        return;
    }
    const int64_t n  = a.ne[0];
    const int64_t i1 = row % a.ne[1], i2 = (row / a.ne[1]) % a.ne[2], i3 = row / (a.ne[1] * a.ne[2]);
    const char *  xr = at(a, 0, i1, i2, i3);
    float *       dr = dst + row * n;
    float         mx = -INFINITY;
    for (int64_t i = l; i < n; i += 64) {
        const float v = *(const float *) (xr + i * a.nb[0]);
        mx            = v > mx ? v : mx;
    }
    mx         = wave_max(mx);
    double sum = 0.0;
    for (int64_t i = l; i < n; i += 64) {
        const float e = expf(*(const float *) (xr + i * a.nb[0]) - mx);
        dr[i]         = e;
        sum += (double) e;
    }
    sum            = wave_sum_d(sum);
    const float is = (float) (1.0 / sum);
    for (int64_t i = l; i < n; i += 64) {
        dr[i] = dr[i] * is;  // each lane rescales the elements it wrote
    }
}

// The depth decoder's manual causal attention as one launch
// (src/depth-decoder.h:214-221): scores = MUL_MAT(k, q), SCALE (x s + b),
// DIAG_MASK_INF(n_past), SOFT_MAX, MUL_MAT(CONT(TRANSPOSE(v)), P) and the
// CONT of its (0, 2, 1, 3) permutation.  One workgroup per (head, batch):
// the head's q, k and v rows are copied into LDS first (every load in flight
// at once), then each step repeats the separate kernels' arithmetic in their
// order, so the output equals the seven-kernel chain's bit for bit:
//   scores as k_mul_mat_f32_wave (lanes stride over d, f32 products summed in
//   double, wave_sum_d), SCALE with two roundings, the mask, the softmax as
//   k_soft_max_rows (one key per lane), P.V as k_mul_mat_f32 (a sequential
//   double sum over the keys).
// q, k, v: [D, S, H, B] views (d contiguous); dst contiguous [D, H, S_q, B].
constexpr int SATT_MAXS = 16;   // queries and keys
constexpr int SATT_MAXD = 256;  // head dim

__global__ __launch_bounds__(1024) void k_small_attn(TV q, TV k, TV v, float s, float bias, int n_past,
                                                     float * __restrict__ dst, int8_t * __restrict__ xq_qs,
                                                     float * __restrict__ xq_d) {
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(16))) float sq[SATT_MAXS][SATT_MAXD], sk[SATT_MAXS][SATT_MAXD],
        sv[SATT_MAXS][SATT_MAXD];
    __shared__ float sp[SATT_MAXS][SATT_MAXS];  // scores, then P: [query][key]
    const int     D = (int) q.ne[0], Sq = (int) q.ne[1], Sk = (int) k.ne[1];
    const int64_t H = q.ne[2];
    const int64_t h = blockIdx.x % H, b = blockIdx.x / H;
    const int64_t hk = h / (H / k.ne[2]), bk = b / (q.ne[3] / k.ne[3]);
    const int64_t hv = h / (H / v.ne[2]), bv = b / (q.ne[3] / v.ne[3]);
    const int     wv = threadIdx.x >> 6, l = threadIdx.x & 63;
    constexpr int NWV = 16;  // waves
    // 0. the head's rows into LDS, 16 bytes per load when the rows allow it;
    // every thread's loads issued before its stores
    {
        const char * bq = at(q, 0, 0, h, b);
        const char * bkp = at(k, 0, 0, hk, bk);
        const char * bvp = at(v, 0, 0, hv, bv);
        const bool   vec = D % 4 == 0 && ((((uintptr_t) bq | (uintptr_t) bkp | (uintptr_t) bvp) & 15) == 0) &&
                         q.nb[1] % 16 == 0 && k.nb[1] % 16 == 0 && v.nb[1] % 16 == 0;
        if (vec) {
            constexpr int PER = 3 * SATT_MAXS * SATT_MAXD / 4 / 1024;  // float4 per thread
            const int     D4  = D / 4;
            float4_t      val[PER];
#pragma unroll
            for (int u = 0; u < PER; u++) {
                const int e = (int) threadIdx.x + 1024 * u;  // float4 index over [3][S][D / 4]
                // slot e: tensor `which`, row rr (rows past the tensor's are not loaded), float4 c
                const int which = e / (SATT_MAXS * SATT_MAXD / 4), c = e % D4;
                const int rr = (e % (SATT_MAXS * SATT_MAXD / 4)) / D4;
                val[u]       = float4_t{ 0.0f, 0.0f, 0.0f, 0.0f };
                if (rr < (which == 0 ? Sq : Sk)) {
                    const char * base = which == 0 ? bq + rr * q.nb[1] : which == 1 ? bkp + rr * k.nb[1]
                                                                                    : bvp + rr * v.nb[1];
                    val[u] = *(const float4_t *) (base + 16 * c);
                }
            }
#pragma unroll
            for (int u = 0; u < PER; u++) {
                const int e = (int) threadIdx.x + 1024 * u;
                const int which = e / (SATT_MAXS * SATT_MAXD / 4), c = e % D4;
                const int rr = (e % (SATT_MAXS * SATT_MAXD / 4)) / D4;
                if (rr < SATT_MAXS) {
                    *(float4_t *) &(which == 0 ? sq : which == 1 ? sk : sv)[rr][4 * c] = val[u];
                }
            }
        } else {
            for (int e = threadIdx.x; e < 3 * SATT_MAXS * D; e += 1024) {
                const int which = e / (SATT_MAXS * D), r = (e / D) % SATT_MAXS, d = e % D;
                if (r < (which == 0 ? Sq : Sk)) {
                    (which == 0 ? sq : which == 1 ? sk : sv)[r][d] =
                        *(const float *) (which == 0 ? at(q, d, r, h, b) : which == 1 ? at(k, d, r, hk, bk)
                                                                                      : at(v, d, r, hv, bv));
                }
            }
        }
    }
    __syncthreads();
    // 1. scores, one wave per (query, key), then SCALE and DIAG_MASK_INF
    for (int t = wv; t < Sq * Sk; t += NWV) {
        const int i = t / Sk, j = t % Sk;
        double    acc = 0.0;
        for (int d = l; d < D; d += 64) {
            acc += (double) (sk[j][d] * sq[i][d]);
        }
        acc = wave_sum_d(acc);
        if (l == 0) {
            const float x = (float) acc * s + bias;
            sp[i][j]      = j > n_past + i ? -INFINITY : x;
        }
    }
    __syncthreads();
    // 2. the softmax of each query row over its keys, one wave per row
    for (int i = wv; i < Sq; i += NWV) {
        const float  x   = l < Sk ? sp[i][l] : -INFINITY;
        const float  mx  = wave_max(x);
        const float  e   = l < Sk ? expf(x - mx) : 0.0f;
        const double sum = wave_sum_d(l < Sk ? (double) e : 0.0);
        const float  is  = (float) (1.0 / sum);
        if (l < Sk) {
            sp[i][l] = e * is;
        }
    }
    __syncthreads();
    // 3. out[d, h, i, b] = sum_j v[d, j] p[i, j], keys in order
    for (int t = threadIdx.x; t < D * Sq; t += 1024) {
        const int d = t % D, i = t / D;
        double    acc = 0.0;
        for (int j = 0; j < Sk; j++) {
            acc += (double) (sv[j][d] * sp[i][j]);
        }
        const float   o   = (float) acc;
        const int64_t row = i + (int64_t) Sq * b, e = d + (int64_t) D * h, K = D * H;
        dst[e + K * row] = o;
        if (xq_qs) {
            // the output row's Q8_0 activation blocks (32 consecutive d of one
            // query, D % 32 == 0) with k_quant_q8_0's arithmetic
            const float a  = group32_max(fabsf(o));
            const float dd = a / 127.0f;
            const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
            xq_qs[row * K + e] = (int8_t) roundf(o * id);
            if ((d & 31) == 0) {
                xq_d[row * (K / 32) + e / 32] = h2f(f2h(dd));
            }
        }
    }
}

// The depth decoder's in-graph sampler (src/depth-decoder.h:345-361).
// GGML_OP_ARGSORT, descending: one workgroup per row of n <= 4096 f32 values,
// a bitonic sort of (value, index) pairs in LDS padded with -inf; equal values
// keep ascending index order.  dst: contiguous I32 rows.
constexpr int SORT_MAX = 4096;

__global__ __launch_bounds__(256) void k_argsort_desc(TV a, int32_t * __restrict__ dst) {
    __shared__ float   sv[SORT_MAX];
    __shared__ int32_t si[SORT_MAX];
    const int64_t      row = blockIdx.x;
    const int64_t      n   = a.ne[0];
    const int64_t      i1 = row % a.ne[1], i2 = (row / a.ne[1]) % a.ne[2], i3 = row / (a.ne[1] * a.ne[2]);
    const char *       xr  = at(a, 0, i1, i2, i3);
    int                p2  = 1;
    while (p2 < n) {
        p2 <<= 1;
    }
    for (int i = threadIdx.x; i < p2; i += 256) {
        sv[i] = i < n ? *(const float *) (xr + (int64_t) i * a.nb[0]) : -INFINITY;
        si[i] = i;
    }
    __syncthreads();
    // "before": greater value first, then the lower index
    auto before = [](float va, int ia, float vb, int ib) { return va > vb || (va == vb && ia < ib); };
    for (int size = 2; size <= p2; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < p2; i += 256) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool desc = (i & size) == 0;  // this run sorts in "before" order
                    const bool swap = desc ? before(sv[j], si[j], sv[i], si[i]) : before(sv[i], si[i], sv[j], si[j]);
                    if (swap) {
                        const float tv = sv[i];
                        sv[i]          = sv[j];
                        sv[j]          = tv;
                        const int ti   = si[i];
                        si[i]          = si[j];
                        si[j]          = ti;
                    }
                }
            }
            __syncthreads();
        }
    }
    for (int i = threadIdx.x; i < n; i += 256) {
        dst[row * n + i] = si[i];
    }
}

// GGML_OP_CUMSUM along dim 0: one thread per row, the running f32 sum.
__global__ void k_cumsum_rows(TV a, int64_t rows, float * __restrict__ dst) {
#pragma clang fp contract(off)
    for (int64_t r = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; r < rows; r += (int64_t) gridDim.x * blockDim.x) {
        const int64_t i1 = r % a.ne[1], i2 = (r / a.ne[1]) % a.ne[2], i3 = r / (a.ne[1] * a.ne[2]);
        const char *  xr = at(a, 0, i1, i2, i3);
        float         acc = 0.0f;
        for (int64_t i = 0; i < a.ne[0]; i++) {
            acc = acc + *(const float *) (xr + i * a.nb[0]);
            dst[r * a.ne[0] + i] = acc;
        }
    }
}

// GGML_OP_SUM: all elements summed in double, one workgroup.
__global__ __launch_bounds__(256) void k_sum_all(TV a, int64_t n, float * __restrict__ dst) {
    __shared__ double part[4];
    double            acc = 0.0;
    for (int64_t t = threadIdx.x; t < n; t += 256) {
        int64_t i0, i1, i2, i3;
        unravel(t, a.ne, i0, i1, i2, i3);
        acc += (double) *(const float *) at(a, i0, i1, i2, i3);
    }
    acc = wave_sum_d(acc);
    if ((threadIdx.x & 63) == 0) {
        part[threadIdx.x >> 6] = acc;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        dst[0] = (float) (((part[0] + part[1]) + part[2]) + part[3]);
    }
}

// GGML_UNARY_OP_STEP: x > 0 ? 1 : 0; dst contiguous.
__global__ void k_step(TV a, int64_t n, float * __restrict__ dst) {
    for (int64_t t = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; t < n; t += (int64_t) gridDim.x * blockDim.x) {
        int64_t i0, i1, i2, i3;
        unravel(t, a.ne, i0, i1, i2, i3);
        dst[t] = *(const float *) at(a, i0, i1, i2, i3) > 0.0f ? 1.0f : 0.0f;
    }
}

// CPY I32 -> f32 (ggml_cast of the top-k indices to F32); dst contiguous.
__global__ void k_cast_f32_of_i32(TV a, int64_t n, float * __restrict__ dst) {
    for (int64_t t = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; t < n; t += (int64_t) gridDim.x * blockDim.x) {
        int64_t i0, i1, i2, i3;
        unravel(t, a.ne, i0, i1, i2, i3);
        dst[t] = (float) *(const int32_t *) at(a, i0, i1, i2, i3);
    }
}

// CPY f32 -> I32 (ggml_cast to I32): truncation toward zero; dst contiguous.
__global__ void k_cast_i32(TV a, int64_t n, int32_t * __restrict__ dst) {
    for (int64_t t = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; t < n; t += (int64_t) gridDim.x * blockDim.x) {
        int64_t i0, i1, i2, i3;
        unravel(t, a.ne, i0, i1, i2, i3);
        dst[t] = (int32_t) *(const float *) at(a, i0, i1, i2, i3);
    }
}

// ---------------------------------------------------------------------------
// Per-head rows of the QKV projection (the CONT / RMS_NORM / MUL / ROPE /
// SET_ROWS chain of the attention block): one wave per row (h, t) of D = 64 *
// EPL f32 elements, lane l owning elements EPL*l .. EPL*l + EPL-1, so the NeoX
// partner of element i < D/2 (i + D/2) sits in lane l ^ 32.

// Up to 4 chains in one launch (the attention block's Q, K and V chains):
// rows of segment i are row indices start[i] .. start[i+1]-1.
constexpr int HEAD_MAX_SEGS = 4;
struct HeadSegs {
    mmhip_head_rows_args seg[HEAD_MAX_SEGS];
    int                  start[HEAD_MAX_SEGS + 1];
    int                  n;
};

template <int EPL>
__device__ __forceinline__ void head_row(const mmhip_head_rows_args & a, int row, int lane) {
#pragma clang fp contract(off)
    constexpr int D  = 64 * EPL;
    const int     h  = row % a.H;
    const int     t  = row / a.H;
    const float * xr = (const float *) ((const char *) a.src + h * a.src_nb_h + t * a.src_nb_t);
    // every load up front (absent operands read a valid stand-in and are unused)
    const float *   wp = a.norm_w ? a.norm_w : xr;
    const int32_t * pp = a.pos ? a.pos + t : (const int32_t *) xr;
    const char *    ip = a.ids ? (const char *) a.ids + (h % a.ids_ne1) * a.ids_nb1 + (t % a.ids_ne2) * a.ids_nb2
                               : (const char *) xr;
    float v[EPL], wv[EPL];
#pragma unroll
    for (int k = 0; k < EPL; k++) {
        v[k]  = xr[EPL * lane + k];
        wv[k] = wp[EPL * lane + k];
    }
    const int32_t p_t    = *pp;
    const int64_t id_raw = a.ids_type == 27 ? *(const int64_t *) ip : (int64_t) *(const int32_t *) ip;
    if (a.norm) {
        double ss = 0.0;
#pragma unroll
        for (int k = 0; k < EPL; k++) {
            ss += (double) (v[k] * v[k]);
        }
        ss               = wave_sum_d(ss);
        const float mean = (float) (ss / (double) D);
        const float sc   = 1.0f / sqrtf(mean + a.eps);
#pragma unroll
        for (int k = 0; k < EPL; k++) {
            const float y = v[k] * sc;
            v[k]          = a.norm_w ? y * wv[k] : y;
        }
    }
    if (a.pos) {
        // theta_i = pos * theta_scale^i, the power taken by repeated f32
        // multiplication as ggml-CPU's rope cache does
        const int   i0    = EPL * (lane & 31);
        float       theta = (float) p_t;
        for (int k = 0; k < i0; k++) {
            theta *= a.theta_scale;
        }
        const bool upper = lane >= 32;
#pragma unroll
        for (int k = 0; k < EPL; k++) {
            const float other = __shfl_xor(v[k], 32, WAVE);
            const float c = cosf(theta), s = sinf(theta);
            // lower lane holds x0 (element i), upper lane x1 (element i + D/2)
            v[k]  = upper ? other * s + v[k] * c : v[k] * c - other * s;
            theta *= a.theta_scale;
        }
    }
    if (!a.ids) {
        float * dr = (float *) a.dst + (int64_t) row * D;
#pragma unroll
        for (int k = 0; k < EPL; k++) {
            dr[EPL * lane + k] = v[k];
        }
        return;
    }
    char * dp = (char *) a.dst + id_raw * a.dst_nb1 + h * a.dst_nb2 + t * a.dst_nb3;
#pragma unroll
    for (int k = 0; k < EPL; k++) {
        if (a.dst_type == TYPE_F32) {
            ((float *) dp)[EPL * lane + k] = v[k];
        } else {
            ((uint16_t *) dp)[EPL * lane + k] = f2h(v[k]);
        }
    }
}

template <int EPL>
__global__ __launch_bounds__(256) void k_head_rows(HeadSegs hs) {
    const int row  = (int) blockIdx.x * 4 + ((int) threadIdx.x >> 6);  // one wave per row
    const int lane = threadIdx.x & 63;
    if (row >= hs.start[hs.n]) {
        return;
    }
    // constant indices keep the kernel-argument struct out of scratch memory
    if (hs.n > 3 && row >= hs.start[3]) {
        head_row<EPL>(hs.seg[3], row - hs.start[3], lane);
    } else if (hs.n > 2 && row >= hs.start[2]) {
        head_row<EPL>(hs.seg[2], row - hs.start[2], lane);
    } else if (hs.n > 1 && row >= hs.start[1]) {
        head_row<EPL>(hs.seg[1], row - hs.start[1], lane);
    } else {
        head_row<EPL>(hs.seg[0], row, lane);
    }
}

// ---------------------------------------------------------------------------
// NeoX RoPE on x [head_dim, heads, tokens, B] with positions[tokens]: pair
// (i, i + n_dims/2) rotates by theta_i = pos * theta_scale^i, theta_scale
// multiplied in f32 step by step (ggml's cache recurrence).

__global__ void k_rope_neox(TV x, const int32_t * __restrict__ pos, int n_dims, float theta_scale,
                            float * dst) {  // dst may be x (in place): each thread owns its pair
#pragma clang fp contract(off)
    const int64_t D     = x.ne[0];
    const int64_t rows  = x.ne[1] * x.ne[2] * x.ne[3];
    const int64_t half  = n_dims / 2;
    const int64_t per   = half + (D - n_dims);  // work items per row
    const int64_t total = rows * per;
    for (int64_t t = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; t < total;
         t += (int64_t) gridDim.x * blockDim.x) {
        const int64_t row = t / per;
        const int64_t j   = t % per;
        const int64_t i1 = row % x.ne[1], i2 = (row / x.ne[1]) % x.ne[2], i3 = row / (x.ne[1] * x.ne[2]);
        const char *  xr = at(x, 0, i1, i2, i3);
        float *       dr = dst + row * D;
        if (j < half) {
            float theta = (float) pos[i2];
            for (int64_t k = 0; k < j; k++) {
                theta *= theta_scale;
            }
            const float c = cosf(theta), s = sinf(theta);
            const float x0 = *(const float *) (xr + j * x.nb[0]);
            const float x1 = *(const float *) (xr + (j + half) * x.nb[0]);
            dr[j]          = x0 * c - x1 * s;
            dr[j + half]   = x0 * s + x1 * c;
        } else {
            const int64_t i = n_dims + (j - half);
            dr[i]           = *(const float *) (xr + i * x.nb[0]);
        }
    }
}

// ---------------------------------------------------------------------------
// copy with conversion between f32 / f16 (any strides on both sides)

__global__ void k_cpy_linear(const char * __restrict__ src, int st, char * __restrict__ dst, int dt, uint32_t n) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const float v = st == TYPE_F32 ? ((const float *) src)[i] : h2f(((const uint16_t *) src)[i]);
        if (dt == TYPE_F32) {
            ((float *) dst)[i] = v;
        } else {
            ((uint16_t *) dst)[i] = f2h(v);
        }
    }
}

// Rows of ne0 contiguous source elements into a contiguous destination:
// thread t converts elements 4j .. 4j+3 of row r = t / (ne0/4), with the row's
// indices taken once per 4 elements and 16- / 8-byte accesses.
__global__ void k_cpy_rows4(TV src, int st, char * __restrict__ dst, int dt, int64_t n4, int64_t q) {
    for (int64_t t = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; t < n4; t += (int64_t) gridDim.x * blockDim.x) {
        const int64_t r = t / q, j = t % q;
        const int64_t i1 = r % src.ne[1], i2 = (r / src.ne[1]) % src.ne[2], i3 = r / (src.ne[1] * src.ne[2]);
        const char *  sp = at(src, 4 * j, i1, i2, i3);
        float4_t      v;
        if (st == TYPE_F32) {
            v = *(const float4_t *) sp;
        } else {
            const uint2 h = *(const uint2 *) sp;
            v = float4_t{ h2f((uint16_t) (h.x & 0xffff)), h2f((uint16_t) (h.x >> 16)), h2f((uint16_t) (h.y & 0xffff)),
                          h2f((uint16_t) (h.y >> 16)) };
        }
        if (dt == TYPE_F32) {
            *(float4_t *) (dst + 16 * t) = v;
        } else {
            uint2 h;
            h.x = (uint32_t) f2h(v[0]) | ((uint32_t) f2h(v[1]) << 16);
            h.y = (uint32_t) f2h(v[2]) | ((uint32_t) f2h(v[3]) << 16);
            *(uint2 *) (dst + 8 * t) = h;
        }
    }
}

__global__ void k_cpy(TV src, int st, TV dst, int dt, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; i < n; i += (int64_t) gridDim.x * blockDim.x) {
        int64_t s0, s1, s2, s3, d0, d1, d2, d3;
        unravel(i, src.ne, s0, s1, s2, s3);
        unravel(i, dst.ne, d0, d1, d2, d3);
        const char * sp = at(src, s0, s1, s2, s3);
        char *       dp = at(dst, d0, d1, d2, d3);
        const float  v  = st == TYPE_F32 ? *(const float *) sp : h2f(*(const uint16_t *) sp);
        if (dt == TYPE_F32) {
            *(float *) dp = v;
        } else {
            *(uint16_t *) dp = f2h(v);
        }
    }
}

// ---------------------------------------------------------------------------
// get_rows: dst[i0, j, i2, i3] = src[i0, ids[j, i2, i3], i2, i3] as f32

__device__ __forceinline__ float deq_elem(int type, const uint8_t * r, int64_t K, int64_t k) {
#pragma clang fp contract(off)
    if (type == TYPE_F32) {
        return ((const float *) r)[k];
    }
    if (type == TYPE_F16) {
        return h2f(((const uint16_t *) r)[k]);
    }
    if (type == TYPE_Q8_0) {
        const float d = h2f(((const uint16_t *) (r + K))[k >> 5]);
        return d * (float) ((const int8_t *) r)[k];
    }
    if (type == TYPE_Q4_K || type == TYPE_Q5_K) {
        // Q5_K: qh[K/8] after qs, fifth bit of element e at bit e / 32 of
        // the super-block's qh byte e % 32
        const int64_t sb    = k >> 8;
        const int     e     = (int) (k & 255);
        const int     j     = e >> 5;
        const int64_t qh_sz = type == TYPE_Q5_K ? K / 8 : 0;
        int           s, m;
        q4k_scale_min(j, r + K / 2 + qh_sz + 12 * sb, s, m);
        const uint16_t * dm = (const uint16_t *) (r + K / 2 + qh_sz + 12 * (K / 256)) + 2 * sb;
        const uint8_t    b  = r[sb * 128 + (e >> 6) * 32 + (e & 31)];
        int              q  = (e & 32) ? (b >> 4) : (b & 15);
        if (type == TYPE_Q5_K) {
            q |= ((r[K / 2 + sb * 32 + (e & 31)] >> j) & 1) << 4;
        }
        const float      d1 = h2f(dm[0]) * (float) s;
        const float      m1 = h2f(dm[1]) * (float) m;
        return d1 * (float) q - m1;
    }
    // Q6_K
    const int64_t sb = k >> 8;
    const int     e  = (int) (k & 255);
    const int     h = e >> 7, rr = e & 127, t = rr >> 5, c = rr & 31;
    const uint8_t lb = r[sb * 128 + 64 * h + c + 32 * (t & 1)];
    const int     lo = (t < 2) ? (lb & 15) : (lb >> 4);
    const int     hi = (r[K / 2 + sb * 64 + 32 * h + c] >> (2 * t)) & 3;
    const float   d  = h2f(((const uint16_t *) (r + K / 2 + K / 4 + K / 16))[sb]);
    const float   ds = d * (float) ((const int8_t *) (r + K / 2 + K / 4))[sb * 16 + (e >> 4)];
    return ds * (float) ((lo | (hi << 4)) - 32);
}

__global__ void k_get_rows(int type, TV src, TV ids, float * __restrict__ dst, int64_t n_out) {
    const int64_t K = src.ne[0];
    for (int64_t i = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; i < n_out;
         i += (int64_t) gridDim.x * blockDim.x) {
        const int64_t i0 = i % K;
        int64_t       r  = i / K;
        const int64_t j  = r % ids.ne[0];
        r /= ids.ne[0];
        const int64_t  i2  = r % ids.ne[1];
        const int64_t  i3  = r / ids.ne[1];
        const int32_t  row = *(const int32_t *) at(ids, j, i2, i3, 0);
        const uint8_t * sr = (const uint8_t *) at(src, 0, row, i2, i3);
        dst[i]             = deq_elem(type, sr, K, i0);
    }
}

// ---------------------------------------------------------------------------
// set_rows: dst[i0, ids[i1, i2 % ids.ne1, i3 % ids.ne2], i2, i3] = src[i0, i1, i2, i3]

__global__ void k_set_rows(TV src, TV ids, int ids64, TV dst, int dt, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; i < n; i += (int64_t) gridDim.x * blockDim.x) {
        int64_t i0, i1, i2, i3;
        unravel(i, src.ne, i0, i1, i2, i3);
        const char *  ip  = at(ids, i1, i2 % ids.ne[1], i3 % ids.ne[2], 0);
        const int64_t row = ids64 ? *(const int64_t *) ip : (int64_t) *(const int32_t *) ip;
        const float   v   = *(const float *) at(src, i0, i1, i2, i3);
        char *        dp  = at(dst, i0, row, i2, i3);
        if (dt == TYPE_F32) {
            *(float *) dp = v;
        } else {
            *(uint16_t *) dp = f2h(v);
        }
    }
}

// ---------------------------------------------------------------------------
// SwiGLU: dst = silu(g) * u with g, u the two halves of a (fused) or a and b
// (split); silu(x) = x / (1 + exp(-x))

__global__ void k_swiglu(TV a, TV b, int split, int swapped, float * __restrict__ dst, int64_t n, int64_t nout0) {
#pragma clang fp contract(off)
    for (int64_t i = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; i < n; i += (int64_t) gridDim.x * blockDim.x) {
        const int64_t i0 = i % nout0;
        int64_t       r  = i / nout0;
        const int64_t i1 = r % a.ne[1];
        r /= a.ne[1];
        const int64_t i2 = r % a.ne[2];
        const int64_t i3 = r / a.ne[2];
        float         g, u;
        if (split) {
            g = *(const float *) at(a, i0, i1, i2, i3);
            u = *(const float *) at(b, i0, i1, i2, i3);
        } else {
            const int64_t gi = swapped ? i0 + nout0 : i0;
            const int64_t ui = swapped ? i0 : i0 + nout0;
            g                = *(const float *) at(a, gi, i1, i2, i3);
            u                = *(const float *) at(a, ui, i1, i2, i3);
        }
        const float silu = g / (1.0f + expf(-g));
        dst[i]           = silu * u;
    }
}

// SwiGLU of contiguous f32 rows with the result also quantised for the down
// projection's GEMV: one wave per 256-element chunk of an output row.
__global__ __launch_bounds__(256) void k_swiglu_quant(const char * __restrict__ a, int64_t a_nb1,
                                                      const char * __restrict__ b, int64_t b_nb1, int F, int T,
                                                      int swapped, float * __restrict__ dst, int qtype,
                                                      int8_t * __restrict__ xq_qs, float * __restrict__ xq_d,
                                                      int16_t * __restrict__ xq_bs) {
#pragma clang fp contract(off)
    const int chunks = F / 256;
    const int wid    = (int) blockIdx.x * 4 + ((int) threadIdx.x >> 6);
    const int lane   = threadIdx.x & 63;
    if (wid >= chunks * T) {
        return;
    }
    const int     row = wid / chunks;
    const int     c   = wid % chunks;
    const int     e   = 256 * c + 4 * lane;
    const float * ar  = (const float *) (a + (int64_t) row * a_nb1);
    float4_t      g, u;
    if (b) {
        g = *(const float4_t *) (ar + e);
        u = *(const float4_t *) ((const float *) (b + (int64_t) row * b_nb1) + e);
    } else {
        g = *(const float4_t *) (ar + (swapped ? e + F : e));
        u = *(const float4_t *) (ar + (swapped ? e : e + F));
    }
    float v[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float silu = g[k] / (1.0f + expf(-g[k]));
        v[k]             = silu * u[k];
    }
    if (dst) {
        *(float4_t *) (dst + (int64_t) row * F + e) = float4_t{ v[0], v[1], v[2], v[3] };
    }
    qrow(qtype, xq_qs, xq_d, xq_bs, row, F).chunk(v, lane, c);
}

__global__ void k_scale(TV a, float s, float bias, float * __restrict__ dst, int64_t n) {
#pragma clang fp contract(off)
    for (int64_t i = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; i < n; i += (int64_t) gridDim.x * blockDim.x) {
        int64_t i0, i1, i2, i3;
        unravel(i, a.ne, i0, i1, i2, i3);
        dst[i] = *(const float *) at(a, i0, i1, i2, i3) * s + bias;
    }
}

// contiguous view of elements of `es` bytes
static bool is_contig(const mmhip_view * v, int64_t es) {
    int64_t expect = es;
    for (int i = 0; i < 4; i++) {
        if (v->ne[i] != 1 && v->nb[i] != expect) {
            return false;
        }
        expect *= v->ne[i];
    }
    return true;
}

static bool broadcasts(const mmhip_view * b, const mmhip_view * a) {
    for (int i = 0; i < 4; i++) {
        if (b->ne[i] <= 0 || a->ne[i] % b->ne[i] != 0) {
            return false;
        }
    }
    return true;
}

}  // namespace mmhip

using namespace mmhip;

extern "C" int mmhip_binary(int op, const mmhip_view * a, const mmhip_view * b, float * dst, void * stream) {
    MMHIP_API_BEGIN();
    if (!a || !b || !dst || op < 0 || op > 2 || !broadcasts(b, a)) {
        return set_error(MMHIP_ERR_INVALID, "binary: bad arguments");
    }
    const int64_t n = nel(a);
    if (n == 0) {
        return MMHIP_OK;
    }
    if (n >= ((int64_t) 1 << 31)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "binary: too many elements");
    }
    const dim3 g(grid_for(n, 256));
    if (is_contig(a, 4) && is_contig(b, 4) && b->ne[0] == a->ne[0]) {
        const uint32_t b_rows = (uint32_t) (nel(b) / b->ne[0]);
        const uint32_t a_rows = (uint32_t) (n / a->ne[0]);
        if (b_rows == 1 || (b->ne[1] == a->ne[1] && b->ne[2] == a->ne[2] && a_rows % b_rows == 0)) {
            const float * ap = (const float *) a->data;
            const float * bp = (const float *) b->data;
            const uint32_t ne0 = (uint32_t) a->ne[0];
            if (op == 0) {
                hipLaunchKernelGGL(k_binary_rows<0>, g, dim3(256), 0, (hipStream_t) stream, ap, bp, dst, (uint32_t) n,
                                   ne0, b_rows);
            } else if (op == 1) {
                hipLaunchKernelGGL(k_binary_rows<1>, g, dim3(256), 0, (hipStream_t) stream, ap, bp, dst, (uint32_t) n,
                                   ne0, b_rows);
            } else {
                hipLaunchKernelGGL(k_binary_rows<2>, g, dim3(256), 0, (hipStream_t) stream, ap, bp, dst, (uint32_t) n,
                                   ne0, b_rows);
            }
            return check_launch("binary");
        }
    }
    if (op == 0) {
        hipLaunchKernelGGL(k_binary<0>, g, dim3(256), 0, (hipStream_t) stream, tv(a), tv(b), dst, n);
    } else if (op == 1) {
        hipLaunchKernelGGL(k_binary<1>, g, dim3(256), 0, (hipStream_t) stream, tv(a), tv(b), dst, n);
    } else {
        hipLaunchKernelGGL(k_binary<2>, g, dim3(256), 0, (hipStream_t) stream, tv(a), tv(b), dst, n);
    }
    return check_launch("binary");
}

namespace mmhip {
// Row kernel when rows are contiguous and w (if any) is a plain vector of the
// row length; launches the quantising variant when xq is given.
static int rms_norm_launch(const mmhip_view * x, const mmhip_view * w, float eps, float * dst, int qtype,
                           void * xq, hipStream_t stream) {
    const int64_t rows = x->ne[1] * x->ne[2] * x->ne[3];
    const int64_t n    = x->ne[0];
    if (rows == 0 || n == 0) {
        return MMHIP_OK;
    }
    const bool w_vec = !w || (is_contig(w, 4) && w->ne[0] == n && w->ne[1] * w->ne[2] * w->ne[3] == 1 &&
                              ((uintptr_t) w->data) % 16 == 0);
    const bool fast  = x->nb[0] == 4 && n % 256 == 0 && n <= 16384 && w_vec && rows < (1 << 30) &&
                      ((uintptr_t) x->data | (uintptr_t) x->nb[1] | (uintptr_t) x->nb[2] | (uintptr_t) x->nb[3]) % 16 == 0 &&
                      (!dst || ((uintptr_t) dst) % 16 == 0);
    if (xq && !fast) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "rms_norm_quant: row layout not supported");
    }
    if (!fast) {
        if (!dst) {
            return set_error(MMHIP_ERR_INVALID, "rms_norm: no destination");
        }
        TV wv = w ? tv(w) : TV{};
        hipLaunchKernelGGL(k_rms_norm, dim3((unsigned) rows), dim3(256), 0, stream, tv(x), wv, w ? 1 : 0, eps, dst);
        return check_launch("rms_norm");
    }
    int8_t *  qs = nullptr;
    float *   qd = nullptr;
    int16_t * qb = nullptr;
    if (xq) {
        const ActLayout L = act_layout(qtype, n, rows);
        if (L.total == 0) {
            return set_error(MMHIP_ERR_UNSUPPORTED, "rms_norm_quant: weight type %d", qtype);
        }
        qs    = (int8_t *) xq + L.qs_off;
        qd    = (float *) ((char *) xq + L.d_off);
        qb    = L.vec_type == TYPE_Q8_K ? (int16_t *) ((char *) xq + L.bs_off) : nullptr;
        qtype = L.vec_type;
    }
    const dim3    grid((unsigned) rows);
    const float * wp = w ? (const float *) w->data : nullptr;
    const int     ne1 = (int) x->ne[1], ne2 = (int) x->ne[2];
#define MM_RMS(CPW)                                                                                              \
    hipLaunchKernelGGL(k_rms_norm_row<CPW>, grid, dim3(256), 0, stream, (const char *) x->data, x->nb[1], x->nb[2], \
                       x->nb[3], ne1, ne2, (int) n, wp, eps, dst, qtype, qs, qd, qb)
    if (n <= 1024) {
        MM_RMS(1);
    } else if (n <= 2048) {
        MM_RMS(2);
    } else if (n <= 4096) {
        MM_RMS(4);
    } else if (n <= 8192) {
        MM_RMS(8);
    } else {
        MM_RMS(16);
    }
#undef MM_RMS
    return check_launch("rms_norm");
}
}  // namespace mmhip

extern "C" int mmhip_rms_norm(const mmhip_view * x, const mmhip_view * w, float eps, float * dst, void * stream) {
    MMHIP_API_BEGIN();
    if (!x || !dst || (w && !broadcasts(w, x))) {
        return set_error(MMHIP_ERR_INVALID, "rms_norm: bad arguments");
    }
    return rms_norm_launch(x, w, eps, dst, 0, nullptr, (hipStream_t) stream);
}

extern "C" int mmhip_rms_norm_quant(const mmhip_view * x, const mmhip_view * w, float eps, float * dst, int type,
                                    void * xq, void * stream) {
    MMHIP_API_BEGIN();
    if (!x || !xq || (w && !broadcasts(w, x))) {
        return set_error(MMHIP_ERR_INVALID, "rms_norm_quant: bad arguments");
    }
    return rms_norm_launch(x, w, eps, dst, type, xq, (hipStream_t) stream);
}

// The same with the angle of pair j at position i2 computed once for a group
// of RH heads (the DiT's 32 heads, the prefill's 32 / 8): thread (j, head
// group, i2, i3) rotates pair j of those heads and copies their tail
// elements j, j + half, .. past n_dims.  Same theta recurrence, same cosf /
// sinf, same products: bit-identical to k_rope_neox.
constexpr int RH = 8;

__global__ void k_rope_neox_heads(TV x, const int32_t * __restrict__ pos, int n_dims, float theta_scale,
                                  float * dst, int64_t n_items) {  // dst may be x, as k_rope_neox
#pragma clang fp contract(off)
    const int64_t D = x.ne[0], half = n_dims / 2, ng = (x.ne[1] + RH - 1) / RH;
    for (int64_t t = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; t < n_items;
         t += (int64_t) gridDim.x * blockDim.x) {
        const int64_t j = t % half, hg = (t / half) % ng, i2 = (t / (half * ng)) % x.ne[2];
        const int64_t i3 = t / (half * ng * x.ne[2]);
        float         theta = (float) pos[i2];
        for (int64_t k = 0; k < j; k++) {
            theta *= theta_scale;
        }
        const float   c = cosf(theta), sn = sinf(theta);
        const int64_t h1 = min((hg + 1) * RH, x.ne[1]);
        for (int64_t i1 = hg * RH; i1 < h1; i1++) {
            const char * xr = at(x, 0, i1, i2, i3);
            float *      dr = dst + ((i3 * x.ne[2] + i2) * x.ne[1] + i1) * D;
            const float  x0 = *(const float *) (xr + j * x.nb[0]);
            const float  x1 = *(const float *) (xr + (j + half) * x.nb[0]);
            dr[j]           = x0 * c - x1 * sn;
            dr[j + half]    = x0 * sn + x1 * c;
            for (int64_t i = n_dims + j; i < D; i += half) {
                dr[i] = *(const float *) (xr + i * x.nb[0]);
            }
        }
    }
}

// NeoX RoPE with one workgroup per position (i2, i3): the n_dims / 2
// angles of the position computed once into LDS (theta = pos, multiplied
// by theta_scale once per pair index, as k_rope_neox_heads does), then the
// position's rows (every head) four elements per thread, consecutive threads
// on consecutive elements, each reading its own 16 bytes and its partner's
// (d +- n_dims / 2).  Rows with contiguous elements, D and n_dims / 2
// multiples of 4.  The arithmetic of k_rope_neox_heads, so the same bits.
// In place (dst == x, contiguous) when a row's D / 4 chunks divide 64: the two
// elements of a pair are then read and written by lanes of one wave in one
// loop iteration, whose loads all issue before its stores.
__global__ __launch_bounds__(256) void k_rope_neox_pos(TV x, const int32_t * __restrict__ pos, int n_dims,
                                                       float theta_scale, float * dst, TV dh) {
#pragma clang fp contract(off)
    __shared__ float s_c[128], s_s[128];  // n_dims / 2 <= 128
    const int64_t i2 = blockIdx.x % x.ne[2], i3 = blockIdx.x / x.ne[2];
    const int     D = (int) x.ne[0], half = n_dims / 2, D4 = D / 4, H = (int) x.ne[1];
    for (int j = threadIdx.x; j < half; j += 256) {
        float theta = (float) pos[i2];
        for (int k = 0; k < j; k++) {
            theta *= theta_scale;
        }
        s_c[j] = cosf(theta);
        s_s[j] = sinf(theta);
    }
    __syncthreads();
    const char * xb = x.data + i2 * x.nb[2] + i3 * x.nb[3];
    float *      dp = dst + (i3 * x.ne[2] + i2) * (int64_t) H * D;
    for (int e4 = threadIdx.x; e4 < H * D4; e4 += 256) {
        const int      i1 = e4 / D4, d = 4 * (e4 - i1 * D4);
        const float *  xr = (const float *) (xb + (int64_t) i1 * x.nb[1]);
        const float4_t a  = *(const float4_t *) (xr + d);
        float4_t       o  = a;
        if (d < half) {
            const float4_t b = *(const float4_t *) (xr + d + half);
#pragma unroll
            for (int u = 0; u < 4; u++) {
                o[u] = a[u] * s_c[d + u] - b[u] * s_s[d + u];
            }
        } else if (d < n_dims) {
            const float4_t b = *(const float4_t *) (xr + d - half);
#pragma unroll
            for (int u = 0; u < 4; u++) {
                o[u] = b[u] * s_s[d - half + u] + a[u] * s_c[d - half + u];
            }
        }
        if (dh.data) {
            // rounded to f16 (as CPY rounds) into the strided f16 view
            uint2 hv;
            hv.x = (uint32_t) f2h(o[0]) | ((uint32_t) f2h(o[1]) << 16);
            hv.y = (uint32_t) f2h(o[2]) | ((uint32_t) f2h(o[3]) << 16);
            *(uint2 *) (dh.data + 2 * (int64_t) d + i1 * dh.nb[1] + i2 * dh.nb[2] + i3 * dh.nb[3]) = hv;
        } else {
            *(float4_t *) (dp + (int64_t) i1 * D + d) = o;
        }
    }
}

extern "C" int mmhip_rope_neox(const mmhip_view * x, const int32_t * pos, int n_dims, float theta_scale, float * dst,
                               void * stream) {
    MMHIP_API_BEGIN();
    if (!x || !pos || !dst || n_dims <= 0 || n_dims % 2 != 0 || n_dims > x->ne[0]) {
        return set_error(MMHIP_ERR_INVALID, "rope: bad arguments");
    }
    const int64_t rows  = x->ne[1] * x->ne[2] * x->ne[3];
    const int64_t total = rows * (n_dims / 2 + (x->ne[0] - n_dims));
    if (total == 0) {
        return MMHIP_OK;
    }
    // dst is contiguous [ne0, ne1, ne2, ne3]; it may be x itself (ggml runs
    // ROPE in place) but not overlap x otherwise
    const char * x_lo = (const char *) x->data, *x_hi = (const char *) x->data;
    for (int a = 0; a < 4; a++) {
        x_hi += (x->ne[a] - 1) * x->nb[a];
    }
    x_hi += 4;
    const char * d_lo = (const char *) dst, *d_hi = d_lo + 4 * (rows * x->ne[0]);
    const bool   in_place = d_lo < x_hi && x_lo < d_hi;
    if (in_place && (d_lo != x_lo || x->nb[0] != 4 || x->nb[1] != 4 * x->ne[0] || x->nb[2] != x->nb[1] * x->ne[1] ||
                     x->nb[3] != x->nb[2] * x->ne[2])) {
        return set_error(MMHIP_ERR_INVALID, "rope: dst overlaps x without being x (contiguous) itself");
    }
    if (n_dims <= 256 && (n_dims / 2) % 4 == 0 && x->ne[0] % 4 == 0 && (!in_place || 64 % (x->ne[0] / 4) == 0) &&
        x->nb[0] == 4 && x->nb[1] % 16 == 0 &&
        x->nb[2] % 16 == 0 && x->nb[3] % 16 == 0 && ((uintptr_t) x->data) % 16 == 0 && ((uintptr_t) dst) % 16 == 0 &&
        x->ne[2] * x->ne[3] <= 0x7fffffff && x->ne[0] * x->ne[1] <= 0x7fffffff) {
        hipLaunchKernelGGL(k_rope_neox_pos, dim3((unsigned) (x->ne[2] * x->ne[3])), dim3(256), 0, (hipStream_t) stream,
                           tv(x), pos, n_dims, theta_scale, dst, TV{});
        return check_launch("rope");
    }
    if (x->ne[1] >= RH && n_dims >= 2) {
        const int64_t items = (n_dims / 2) * ((x->ne[1] + RH - 1) / RH) * x->ne[2] * x->ne[3];
        hipLaunchKernelGGL(k_rope_neox_heads, dim3(grid_for(items, 256)), dim3(256), 0, (hipStream_t) stream, tv(x), pos,
                           n_dims, theta_scale, dst, items);
        return check_launch("rope");
    }
    hipLaunchKernelGGL(k_rope_neox, dim3(grid_for(total, 256)), dim3(256), 0, (hipStream_t) stream, tv(x), pos, n_dims,
                       theta_scale, dst);
    return check_launch("rope");
}

extern "C" int mmhip_rope_neox_f16(const mmhip_view * x, const int32_t * pos, int n_dims, float theta_scale,
                                   const mmhip_view * dst, void * stream) {
    MMHIP_API_BEGIN();
    if (!x || !pos || !dst || !dst->data || n_dims <= 0 || n_dims % 2 != 0 || n_dims > x->ne[0]) {
        return set_error(MMHIP_ERR_INVALID, "rope_f16: bad arguments");
    }
    for (int a = 0; a < 4; a++) {
        if (dst->ne[a] != x->ne[a]) {
            return set_error(MMHIP_ERR_INVALID, "rope_f16: dst shape differs from x");
        }
    }
    if (x->ne[0] * x->ne[1] * x->ne[2] * x->ne[3] == 0) {
        return MMHIP_OK;
    }
    bool ok = n_dims <= 256 && (n_dims / 2) % 4 == 0 && x->ne[0] % 4 == 0 && x->nb[0] == 4 && dst->nb[0] == 2 &&
              ((uintptr_t) x->data) % 16 == 0 && ((uintptr_t) dst->data) % 8 == 0 &&
              x->ne[2] * x->ne[3] <= 0x7fffffff && x->ne[0] * x->ne[1] <= 0x7fffffff;
    for (int a = 1; a < 4; a++) {
        ok = ok && x->nb[a] % 16 == 0 && dst->nb[a] % 8 == 0;
    }
    if (!ok) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "rope_f16: n_dims=%d ne0=%lld or strides / alignment not taken", n_dims,
                         (long long) x->ne[0]);
    }
    hipLaunchKernelGGL(k_rope_neox_pos, dim3((unsigned) (x->ne[2] * x->ne[3])), dim3(256), 0, (hipStream_t) stream,
                       tv(x), pos, n_dims, theta_scale, nullptr, tv(dst));
    return check_launch("rope_f16");
}

extern "C" int mmhip_cpy(const mmhip_view * src, int src_type, const mmhip_view * dst, int dst_type, void * stream) {
    MMHIP_API_BEGIN();
    if (!src || !dst || nel(src) != nel(dst) || !(src_type == TYPE_F32 || src_type == TYPE_F16) ||
        !(dst_type == TYPE_F32 || dst_type == TYPE_F16)) {
        return set_error(MMHIP_ERR_INVALID, "cpy: bad arguments");
    }
    const int64_t n = nel(src);
    if (n == 0) {
        return MMHIP_OK;
    }
    if (n >= ((int64_t) 1 << 31)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "cpy: too many elements");
    }
    const int64_t ss = src_type == TYPE_F32 ? 4 : 2, ds = dst_type == TYPE_F32 ? 4 : 2;
    if (is_contig(src, ss) && is_contig(dst, ds)) {
        hipLaunchKernelGGL(k_cpy_linear, dim3(grid_for(n, 256)), dim3(256), 0, (hipStream_t) stream,
                           (const char *) src->data, src_type, (char *) dst->data, dst_type, (uint32_t) n);
        return check_launch("cpy");
    }
    // inner rows contiguous, destination contiguous (element i of the source's
    // row-major order lands at dst[i] whatever dst's shape), 4-element aligned
    const int64_t sal = 4 * ss;
    if (src->nb[0] == ss && is_contig(dst, ds) && src->ne[0] % 4 == 0 && ((uintptr_t) src->data) % sal == 0 &&
        src->nb[1] % sal == 0 && src->nb[2] % sal == 0 && src->nb[3] % sal == 0 && ((uintptr_t) dst->data) % (4 * ds) == 0) {
        hipLaunchKernelGGL(k_cpy_rows4, dim3(grid_for(n / 4, 256)), dim3(256), 0, (hipStream_t) stream, tv(src), src_type,
                           (char *) dst->data, dst_type, n / 4, src->ne[0] / 4);
        return check_launch("cpy");
    }
    hipLaunchKernelGGL(k_cpy, dim3(grid_for(n, 256)), dim3(256), 0, (hipStream_t) stream, tv(src), src_type, tv(dst),
                       dst_type, n);
    return check_launch("cpy");
}

extern "C" int mmhip_get_rows(int src_type, const mmhip_view * src, const mmhip_view * ids, float * dst,
                              void * stream) {
    MMHIP_API_BEGIN();
    if (src_type == 26) {
        src_type = TYPE_F32;  // I32 rows: moved as 4-byte words, bit for bit
    }
    const bool q = is_repacked_type(src_type);
    if (!src || !ids || !dst || !(q || src_type == TYPE_F32 || src_type == TYPE_F16) ||
        (src_type == TYPE_Q8_0 && src->ne[0] % 32 != 0) || (q && src_type != TYPE_Q8_0 && src->ne[0] % 256 != 0)) {
        return set_error(MMHIP_ERR_INVALID, "get_rows: bad arguments");
    }
    const int64_t n = src->ne[0] * ids->ne[0] * ids->ne[1] * ids->ne[2];
    if (n == 0) {
        return MMHIP_OK;
    }
    hipLaunchKernelGGL(k_get_rows, dim3(grid_for(n, 256)), dim3(256), 0, (hipStream_t) stream, src_type, tv(src),
                       tv(ids), dst, n);
    return check_launch("get_rows");
}

extern "C" int mmhip_set_rows(const mmhip_view * src, const mmhip_view * ids, int ids_type, const mmhip_view * dst,
                              int dst_type, void * stream) {
    MMHIP_API_BEGIN();
    if (!src || !ids || !dst || !(ids_type == 26 || ids_type == 27) || !(dst_type == TYPE_F32 || dst_type == TYPE_F16) ||
        src->ne[1] != ids->ne[0] || src->ne[2] % ids->ne[1] != 0 || src->ne[3] % ids->ne[2] != 0 ||
        dst->ne[0] != src->ne[0]) {
        return set_error(MMHIP_ERR_INVALID, "set_rows: bad arguments");
    }
    const int64_t n = nel(src);
    if (n == 0) {
        return MMHIP_OK;
    }
    hipLaunchKernelGGL(k_set_rows, dim3(grid_for(n, 256)), dim3(256), 0, (hipStream_t) stream, tv(src), tv(ids),
                       ids_type == 27 ? 1 : 0, tv(dst), dst_type, n);
    return check_launch("set_rows");
}

extern "C" int mmhip_swiglu(const mmhip_view * a, const mmhip_view * b, int swapped, float * dst, void * stream) {
    MMHIP_API_BEGIN();
    if (!a || !dst || (!b && a->ne[0] % 2 != 0) ||
        (b && (b->ne[0] != a->ne[0] || b->ne[1] != a->ne[1] || b->ne[2] != a->ne[2] || b->ne[3] != a->ne[3]))) {
        return set_error(MMHIP_ERR_INVALID, "swiglu: bad arguments");
    }
    const int64_t nout0 = b ? a->ne[0] : a->ne[0] / 2;
    const int64_t n     = nout0 * a->ne[1] * a->ne[2] * a->ne[3];
    if (n == 0) {
        return MMHIP_OK;
    }
    TV bv = b ? tv(b) : TV{};
    hipLaunchKernelGGL(k_swiglu, dim3(grid_for(n, 256)), dim3(256), 0, (hipStream_t) stream, tv(a), bv, b ? 1 : 0,
                       swapped, dst, n, nout0);
    return check_launch("swiglu");
}

extern "C" int mmhip_norm(const mmhip_view * x, float eps, float * dst, void * stream) {
    return mmhip_norm_affine(x, eps, nullptr, nullptr, dst, stream);
}

extern "C" int mmhip_norm_affine(const mmhip_view * x, float eps, const float * w, const float * b, float * dst,
                                 void * stream) {
    if (!dst) {
        MMHIP_API_BEGIN();
        return set_error(MMHIP_ERR_INVALID, "norm: bad arguments");
    }
    return mmhip_norm_affine_h(x, eps, w, b, dst, nullptr, stream);
}

extern "C" int mmhip_norm_affine_h(const mmhip_view * x, float eps, const float * w, const float * b, float * dst,
                                   void * dsth, void * stream) {
    MMHIP_API_BEGIN();
    if (!x || (!dst && !dsth) || x->ne[0] <= 0) {
        return set_error(MMHIP_ERR_INVALID, "norm: bad arguments");
    }
    const int64_t rows = x->ne[1] * x->ne[2] * x->ne[3];
    if (rows == 0) {
        return MMHIP_OK;
    }
    if (rows >= ((int64_t) 1 << 31) || nel(x) >= ((int64_t) 1 << 31)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "norm: too many elements");
    }
    // rows read once into registers when they are whole 16-byte aligned float4s
    auto          al = [](uint64_t v, uint64_t a) { return v % a == 0; };
    const int64_t n  = x->ne[0];
    const bool    vec = x->nb[0] == 4 && n % 4 == 0 && n <= 4096 && al((uintptr_t) x->data, 16) && al(x->nb[1], 16) &&
                     al(x->nb[2], 16) && al(x->nb[3], 16) && (!dst || al((uintptr_t) dst, 16)) &&
                     (!dsth || al((uintptr_t) dsth, 8)) && (!w || al((uintptr_t) w, 16)) && (!b || al((uintptr_t) b, 16));
    if (vec) {
        const TV xv = tv(x);
        if (n <= 1024) {
            hipLaunchKernelGGL(k_layer_norm_v<1>, dim3((unsigned) rows), dim3(256), 0, (hipStream_t) stream, xv, eps, w,
                               b, dst, (_Float16 *) dsth);
        } else if (n <= 2048) {
            hipLaunchKernelGGL(k_layer_norm_v<2>, dim3((unsigned) rows), dim3(256), 0, (hipStream_t) stream, xv, eps, w,
                               b, dst, (_Float16 *) dsth);
        } else {
            hipLaunchKernelGGL(k_layer_norm_v<4>, dim3((unsigned) rows), dim3(256), 0, (hipStream_t) stream, xv, eps, w,
                               b, dst, (_Float16 *) dsth);
        }
        return check_launch("norm");
    }
    hipLaunchKernelGGL(k_layer_norm, dim3((unsigned) rows), dim3(256), 0, (hipStream_t) stream, tv(x), eps, w, b, dst,
                       (_Float16 *) dsth);
    return check_launch("norm");
}

extern "C" int mmhip_mul_mat_f32(const mmhip_view * a, const mmhip_view * b, float * dst, void * stream) {
    MMHIP_API_BEGIN();
    if (!a || !b || !dst || a->ne[0] != b->ne[0] || a->ne[2] <= 0 || a->ne[3] <= 0 || b->ne[2] % a->ne[2] != 0 ||
        b->ne[3] % a->ne[3] != 0 || a->nb[0] != 4 || b->nb[0] != 4) {
        return set_error(MMHIP_ERR_INVALID, "mul_mat_f32: bad arguments");
    }
    const int64_t n = a->ne[1] * b->ne[1] * b->ne[2] * b->ne[3];
    if (n == 0) {
        return MMHIP_OK;
    }
    if (n >= ((int64_t) 1 << 31)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "mul_mat_f32: too many outputs");
    }
    // a 2-D weight against >= 32 activation rows that collapse to one stride
    // (the DiT's k = 1 convs): the f32 MFMA GEMM
    const int64_t M = b->ne[1] * b->ne[2] * b->ne[3];
    if (a->ne[2] == 1 && a->ne[3] == 1 && M >= 32 && b->nb[2] == b->ne[1] * b->nb[1] &&
        b->nb[3] == b->ne[2] * b->nb[2] && a->nb[1] % 4 == 0 && b->nb[1] % 4 == 0 &&
        gemm_f32_supported(a->ne[1], a->ne[0], (int64_t) (a->nb[1] / 4), a->data, (const float *) b->data,
                           (int64_t) (b->nb[1] / 4))) {
        return gemm_f32((const float *) a->data, (int64_t) (a->nb[1] / 4), (const float *) b->data,
                        (int64_t) (b->nb[1] / 4), a->ne[1], a->ne[0], M, dst, a->ne[1], (hipStream_t) stream);
    }
    if (a->ne[0] >= 128 && n <= ((int64_t) 1 << 24)) {
        hipLaunchKernelGGL(k_mul_mat_f32_wave, dim3((unsigned) ((n + 3) / 4)), dim3(256), 0, (hipStream_t) stream, tv(a),
                           tv(b), dst, a->ne[1], b->ne[1], b->ne[2], a->ne[0], b->ne[2] / a->ne[2], b->ne[3] / a->ne[3], n);
        return check_launch("mul_mat_f32");
    }
    hipLaunchKernelGGL(k_mul_mat_f32, dim3(grid_for(n, 256)), dim3(256), 0, (hipStream_t) stream, tv(a), tv(b), dst,
                       a->ne[1], b->ne[1], b->ne[2], a->ne[0], b->ne[2] / a->ne[2], b->ne[3] / a->ne[3], n);
    return check_launch("mul_mat_f32");
}

extern "C" int mmhip_diag_mask_inf(const mmhip_view * a, int n_past, float * dst, void * stream) {
    MMHIP_API_BEGIN();
    if (!a || !dst) {
        return set_error(MMHIP_ERR_INVALID, "diag_mask_inf: bad arguments");
    }
    const int64_t n = nel(a);
    if (n == 0) {
        return MMHIP_OK;
    }
    if (n >= ((int64_t) 1 << 31)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "diag_mask_inf: too many elements");
    }
    hipLaunchKernelGGL(k_diag_mask_inf, dim3(grid_for(n, 256)), dim3(256), 0, (hipStream_t) stream, tv(a), n_past, n,
                       dst);
    return check_launch("diag_mask_inf");
}

extern "C" int mmhip_soft_max(const mmhip_view * a, float * dst, void * stream) {
    MMHIP_API_BEGIN();
    if (!a || !dst || a->ne[0] <= 0) {
        return set_error(MMHIP_ERR_INVALID, "soft_max: bad arguments");
    }
    const int64_t rows = a->ne[1] * a->ne[2] * a->ne[3];
    if (rows == 0) {
        return MMHIP_OK;
    }
    if (rows >= ((int64_t) 1 << 31)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "soft_max: too many rows");
    }
    hipLaunchKernelGGL(k_soft_max_rows, dim3((unsigned) ((rows + 3) / 4)), dim3(256), 0, (hipStream_t) stream, tv(a),
                       rows, dst);
    return check_launch("soft_max");
}

extern "C" int mmhip_small_attn(const mmhip_view * q, const mmhip_view * k, const mmhip_view * v, float scale,
                                float bias, int n_past, float * dst, void * stream) {
    return mmhip_small_attn_q(q, k, v, scale, bias, n_past, dst, 0, nullptr, stream);
}

extern "C" int mmhip_small_attn_q(const mmhip_view * q, const mmhip_view * k, const mmhip_view * v, float scale,
                                  float bias, int n_past, float * dst, int qtype, void * xq, void * stream) {
    MMHIP_API_BEGIN();
    if (!q || !k || !v || !dst || q->ne[0] != k->ne[0] || q->ne[0] != v->ne[0] || k->ne[1] != v->ne[1] ||
        q->nb[0] != 4 || k->nb[0] != 4 || v->nb[0] != 4) {
        return set_error(MMHIP_ERR_INVALID, "small_attn: bad arguments");
    }
    for (const mmhip_view * t : { k, v }) {
        if (t->ne[2] <= 0 || t->ne[3] <= 0 || q->ne[2] % t->ne[2] != 0 || q->ne[3] % t->ne[3] != 0) {
            return set_error(MMHIP_ERR_INVALID, "small_attn: k / v heads or batches do not divide q's");
        }
    }
    if (q->ne[1] > SATT_MAXS || k->ne[1] > SATT_MAXS || q->ne[1] <= 0 || k->ne[1] <= 0 || q->ne[0] <= 0 ||
        q->ne[0] > SATT_MAXD) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "small_attn: S_q=%lld S_kv=%lld D=%lld (at most %d keys, D %d)",
                         (long long) q->ne[1], (long long) k->ne[1], (long long) q->ne[0], SATT_MAXS, SATT_MAXD);
    }
    const int64_t wgs = q->ne[2] * q->ne[3];
    if (wgs == 0) {
        return MMHIP_OK;
    }
    if (wgs > 0x7fffffff || q->ne[0] * q->ne[1] > 0x7fffffff) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "small_attn: too large");
    }
    int8_t * xq_qs = nullptr;
    float *  xq_d  = nullptr;
    if (qtype != 0) {
        // the output rows (D x H values each, S_q x B of them) quantised for Q8_0 weights
        const ActLayout L = act_layout(qtype, q->ne[0] * q->ne[2], q->ne[1] * q->ne[3]);
        if (qtype != TYPE_Q8_0 || L.vec_type != TYPE_Q8_0 || q->ne[0] % 32 != 0 || !xq) {
            return set_error(MMHIP_ERR_UNSUPPORTED, "small_attn: quantisation for weight type %d at D=%lld", qtype,
                             (long long) q->ne[0]);
        }
        xq_qs = (int8_t *) ((uint8_t *) xq + L.qs_off);
        xq_d  = (float *) ((uint8_t *) xq + L.d_off);
    }
    hipLaunchKernelGGL(k_small_attn, dim3((unsigned) wgs), dim3(1024), 0, (hipStream_t) stream, tv(q), tv(k), tv(v),
                       scale, bias, n_past, dst, xq_qs, xq_d);
    return check_launch("small_attn");
}

extern "C" int mmhip_argsort_desc(const mmhip_view * a, int32_t * dst, void * stream) {
    MMHIP_API_BEGIN();
    if (!a || !dst || a->ne[0] <= 0) {
        return set_error(MMHIP_ERR_INVALID, "argsort: bad arguments");
    }
    if (a->ne[0] > SORT_MAX) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "argsort: rows of %lld > %d", (long long) a->ne[0], SORT_MAX);
    }
    const int64_t rows = a->ne[1] * a->ne[2] * a->ne[3];
    if (rows == 0) {
        return MMHIP_OK;
    }
    if (rows >= ((int64_t) 1 << 31)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "argsort: too many rows");
    }
    hipLaunchKernelGGL(k_argsort_desc, dim3((unsigned) rows), dim3(256), 0, (hipStream_t) stream, tv(a), dst);
    return check_launch("argsort");
}

extern "C" int mmhip_cumsum(const mmhip_view * a, float * dst, void * stream) {
    MMHIP_API_BEGIN();
    if (!a || !dst) {
        return set_error(MMHIP_ERR_INVALID, "cumsum: bad arguments");
    }
    const int64_t rows = a->ne[1] * a->ne[2] * a->ne[3];
    if (rows == 0 || a->ne[0] == 0) {
        return MMHIP_OK;
    }
    hipLaunchKernelGGL(k_cumsum_rows, dim3(grid_for(rows, 64)), dim3(64), 0, (hipStream_t) stream, tv(a), rows, dst);
    return check_launch("cumsum");
}

extern "C" int mmhip_sum(const mmhip_view * a, float * dst, void * stream) {
    MMHIP_API_BEGIN();
    if (!a || !dst) {
        return set_error(MMHIP_ERR_INVALID, "sum: bad arguments");
    }
    hipLaunchKernelGGL(k_sum_all, dim3(1), dim3(256), 0, (hipStream_t) stream, tv(a), nel(a), dst);
    return check_launch("sum");
}

extern "C" int mmhip_step(const mmhip_view * a, float * dst, void * stream) {
    MMHIP_API_BEGIN();
    if (!a || !dst) {
        return set_error(MMHIP_ERR_INVALID, "step: bad arguments");
    }
    const int64_t n = nel(a);
    if (n == 0) {
        return MMHIP_OK;
    }
    hipLaunchKernelGGL(k_step, dim3(grid_for(n, 256)), dim3(256), 0, (hipStream_t) stream, tv(a), n, dst);
    return check_launch("step");
}

extern "C" int mmhip_cast_i32(const mmhip_view * a, int32_t * dst, void * stream) {
    MMHIP_API_BEGIN();
    if (!a || !dst) {
        return set_error(MMHIP_ERR_INVALID, "cast_i32: bad arguments");
    }
    const int64_t n = nel(a);
    if (n == 0) {
        return MMHIP_OK;
    }
    hipLaunchKernelGGL(k_cast_i32, dim3(grid_for(n, 256)), dim3(256), 0, (hipStream_t) stream, tv(a), n, dst);
    return check_launch("cast_i32");
}

extern "C" int mmhip_cast_f32_of_i32(const mmhip_view * a, float * dst, void * stream) {
    MMHIP_API_BEGIN();
    if (!a || !dst) {
        return set_error(MMHIP_ERR_INVALID, "cast_f32_of_i32: bad arguments");
    }
    const int64_t n = nel(a);
    if (n == 0) {
        return MMHIP_OK;
    }
    hipLaunchKernelGGL(k_cast_f32_of_i32, dim3(grid_for(n, 256)), dim3(256), 0, (hipStream_t) stream, tv(a), n, dst);
    return check_launch("cast_f32_of_i32");
}

extern "C" int mmhip_concat(const mmhip_view * a, const mmhip_view * b, int dim, float * dst, void * stream) {
    MMHIP_API_BEGIN();
    if (!a || !b || !dst || dim < 0 || dim > 3) {
        return set_error(MMHIP_ERR_INVALID, "concat: bad arguments");
    }
    for (int i = 0; i < 4; i++) {
        if (i != dim && a->ne[i] != b->ne[i]) {
            return set_error(MMHIP_ERR_INVALID, "concat: shapes differ outside dim %d", dim);
        }
    }
    const int64_t n = nel(a) + nel(b);
    if (n == 0) {
        return MMHIP_OK;
    }
    if (n >= ((int64_t) 1 << 31)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "concat: too many elements");
    }
    hipLaunchKernelGGL(k_concat, dim3(grid_for(n, 256)), dim3(256), 0, (hipStream_t) stream, tv(a), tv(b), dim, n,
                       dst);
    return check_launch("concat");
}

extern "C" int mmhip_clamp(const mmhip_view * a, float lo, float hi, float * dst, void * stream) {
    MMHIP_API_BEGIN();
    if (!a || !dst) {
        return set_error(MMHIP_ERR_INVALID, "clamp: bad arguments");
    }
    const int64_t n = nel(a);
    if (n == 0) {
        return MMHIP_OK;
    }
    if (n >= ((int64_t) 1 << 31)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "clamp: too many elements");
    }
    hipLaunchKernelGGL(k_clamp, dim3(grid_for(n, 256)), dim3(256), 0, (hipStream_t) stream, tv(a), lo, hi, n, dst);
    return check_launch("clamp");
}

extern "C" int mmhip_scale(const mmhip_view * a, float s, float bias, float * dst, void * stream) {
    MMHIP_API_BEGIN();
    if (!a || !dst) {
        return set_error(MMHIP_ERR_INVALID, "scale: bad arguments");
    }
    const int64_t n = nel(a);
    if (n == 0) {
        return MMHIP_OK;
    }
    hipLaunchKernelGGL(k_scale, dim3(grid_for(n, 256)), dim3(256), 0, (hipStream_t) stream, tv(a), s, bias, dst, n);
    return check_launch("scale");
}

extern "C" int mmhip_swiglu_quant(const mmhip_view * a, const mmhip_view * b, int swapped, float * dst, int type,
                                  void * xq, void * stream) {
    MMHIP_API_BEGIN();
    if (!a || !xq) {
        return set_error(MMHIP_ERR_INVALID, "swiglu_quant: bad arguments");
    }
    const int64_t F = b ? a->ne[0] : a->ne[0] / 2;
    const int64_t T = a->ne[1] * a->ne[2] * a->ne[3];
    const bool rows_ok = a->nb[0] == 4 && a->nb[2] == a->nb[1] * a->ne[1] && a->nb[3] == a->nb[2] * a->ne[2] &&
                         (b ? true : a->ne[0] % 2 == 0) && a->nb[1] % 16 == 0 && ((uintptr_t) a->data) % 16 == 0;
    const bool b_ok = !b || (b->ne[0] == a->ne[0] && b->ne[1] * b->ne[2] * b->ne[3] == T && b->nb[0] == 4 &&
                             b->nb[2] == b->nb[1] * b->ne[1] && b->nb[3] == b->nb[2] * b->ne[2] &&
                             b->nb[1] % 16 == 0 && ((uintptr_t) b->data) % 16 == 0);
    if (!rows_ok || !b_ok || F % 256 != 0 || T * F >= ((int64_t) 1 << 31) || (dst && ((uintptr_t) dst) % 16 != 0)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "swiglu_quant: layout not supported");
    }
    const ActLayout L = act_layout(type, F, T);
    if (L.total == 0) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "swiglu_quant: weight type %d", type);
    }
    if (T == 0) {
        return MMHIP_OK;
    }
    const int64_t waves = T * (F / 256);
    hipLaunchKernelGGL(k_swiglu_quant, dim3((unsigned) ((waves + 3) / 4)), dim3(256), 0, (hipStream_t) stream,
                       (const char *) a->data, a->nb[1], b ? (const char *) b->data : nullptr, b ? b->nb[1] : 0,
                       (int) F, (int) T, swapped, dst, L.vec_type, (int8_t *) xq + L.qs_off,
                       (float *) ((char *) xq + L.d_off),
                       L.vec_type == TYPE_Q8_K ? (int16_t *) ((char *) xq + L.bs_off) : nullptr);
    return check_launch("swiglu_quant");
}

extern "C" int mmhip_head_rows_n(const mmhip_head_rows_args * args, int n, void * stream) {
    MMHIP_API_BEGIN();
    if (!args || n < 1 || n > HEAD_MAX_SEGS) {
        return set_error(MMHIP_ERR_INVALID, "head_rows: %d chains (1..%d)", n, HEAD_MAX_SEGS);
    }
    HeadSegs hs{};
    hs.n     = n;
    int64_t rows = 0;
    for (int i = 0; i < n; i++) {
        const mmhip_head_rows_args * a = &args[i];
        if (!a->src || !a->dst || a->H <= 0 || a->T < 0) {
            return set_error(MMHIP_ERR_INVALID, "head_rows: bad arguments (chain %d)", i);
        }
        if (!(a->D == 64 || a->D == 128 || a->D == 256) || a->D != args[0].D) {
            return set_error(MMHIP_ERR_UNSUPPORTED, "head_rows: D=%d not supported (chains share D)", a->D);
        }
        if (a->ids && (a->ids_ne1 <= 0 || a->ids_ne2 <= 0 || !(a->ids_type == 26 || a->ids_type == 27) ||
                       !(a->dst_type == TYPE_F32 || a->dst_type == TYPE_F16))) {
            return set_error(MMHIP_ERR_INVALID, "head_rows: bad row ids / destination type (chain %d)", i);
        }
        if (!a->ids && a->dst_type != TYPE_F32) {
            return set_error(MMHIP_ERR_INVALID, "head_rows: contiguous output is f32 (chain %d)", i);
        }
        hs.seg[i]   = *a;
        hs.start[i] = (int) rows;
        rows += (int64_t) a->H * a->T;
        if (rows >= ((int64_t) 1 << 30)) {
            return set_error(MMHIP_ERR_UNSUPPORTED, "head_rows: too many rows");
        }
    }
    hs.start[n] = (int) rows;
    if (rows == 0) {
        return MMHIP_OK;
    }
    const dim3 grid((unsigned) ((rows + 3) / 4));
    if (args[0].D == 64) {
        hipLaunchKernelGGL(k_head_rows<1>, grid, dim3(256), 0, (hipStream_t) stream, hs);
    } else if (args[0].D == 128) {
        hipLaunchKernelGGL(k_head_rows<2>, grid, dim3(256), 0, (hipStream_t) stream, hs);
    } else {
        hipLaunchKernelGGL(k_head_rows<4>, grid, dim3(256), 0, (hipStream_t) stream, hs);
    }
    return check_launch("head_rows");
}

extern "C" int mmhip_head_rows(const mmhip_head_rows_args * a, void * stream) {
    return mmhip_head_rows_n(a, 1, stream);
}
