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

__device__ __forceinline__ void unravel(int64_t i, const int64_t * ne, int64_t & i0, int64_t & i1, int64_t & i2,
                                        int64_t & i3) {
    i0 = i % ne[0];
    i /= ne[0];
    i1 = i % ne[1];
    i /= ne[1];
    i2 = i % ne[2];
    i3 = i / ne[2];
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

// ---------------------------------------------------------------------------
// rms_norm (+ mul): one workgroup per row

__global__ __launch_bounds__(256) void k_rms_norm(TV x, TV w, int has_w, float eps, float * __restrict__ dst) {
#pragma clang fp contract(off)
    __shared__ float s_part[4];
    const int64_t    row = blockIdx.x;
    const int64_t    i1 = row % x.ne[1], i2 = (row / x.ne[1]) % x.ne[2], i3 = row / (x.ne[1] * x.ne[2]);
    const int64_t    n  = x.ne[0];
    const char *     xr = at(x, 0, i1, i2, i3);
    float            ss = 0.0f;
    for (int64_t i = threadIdx.x; i < n; i += 256) {
        const float v = *(const float *) (xr + i * x.nb[0]);
        ss += v * v;
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) {
        s_part[threadIdx.x >> 6] = ss;
    }
    __syncthreads();
    ss               = s_part[0] + s_part[1] + s_part[2] + s_part[3];
    const float mean = ss / (float) n;
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

// ---------------------------------------------------------------------------
// NeoX RoPE on x [head_dim, heads, tokens, B] with positions[tokens]: pair
// (i, i + n_dims/2) rotates by theta_i = pos * theta_scale^i, theta_scale
// multiplied in f32 step by step (ggml's cache recurrence).

__global__ void k_rope_neox(TV x, const int32_t * __restrict__ pos, int n_dims, float theta_scale,
                            float * __restrict__ dst) {
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
    if (type == TYPE_Q4_K) {
        const int64_t sb = k >> 8;
        const int     e  = (int) (k & 255);
        const int     j  = e >> 5;
        int           s, m;
        q4k_scale_min(j, r + K / 2 + 12 * sb, s, m);
        const uint16_t * dm = (const uint16_t *) (r + K / 2 + 12 * (K / 256)) + 2 * sb;
        const uint8_t    b  = r[sb * 128 + (e >> 6) * 32 + (e & 31)];
        const int        q  = (e & 32) ? (b >> 4) : (b & 15);
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

__global__ void k_scale(TV a, float s, float bias, float * __restrict__ dst, int64_t n) {
#pragma clang fp contract(off)
    for (int64_t i = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; i < n; i += (int64_t) gridDim.x * blockDim.x) {
        int64_t i0, i1, i2, i3;
        unravel(i, a.ne, i0, i1, i2, i3);
        dst[i] = *(const float *) at(a, i0, i1, i2, i3) * s + bias;
    }
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
    const dim3 g(grid_for(n, 256));
    if (op == 0) {
        hipLaunchKernelGGL(k_binary<0>, g, dim3(256), 0, (hipStream_t) stream, tv(a), tv(b), dst, n);
    } else if (op == 1) {
        hipLaunchKernelGGL(k_binary<1>, g, dim3(256), 0, (hipStream_t) stream, tv(a), tv(b), dst, n);
    } else {
        hipLaunchKernelGGL(k_binary<2>, g, dim3(256), 0, (hipStream_t) stream, tv(a), tv(b), dst, n);
    }
    return check_launch("binary");
}

extern "C" int mmhip_rms_norm(const mmhip_view * x, const mmhip_view * w, float eps, float * dst, void * stream) {
    MMHIP_API_BEGIN();
    if (!x || !dst || (w && !broadcasts(w, x))) {
        return set_error(MMHIP_ERR_INVALID, "rms_norm: bad arguments");
    }
    const int64_t rows = x->ne[1] * x->ne[2] * x->ne[3];
    if (rows == 0 || x->ne[0] == 0) {
        return MMHIP_OK;
    }
    if (rows > 0x7fffffff) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "rms_norm: too many rows");
    }
    TV wv = w ? tv(w) : TV{};
    hipLaunchKernelGGL(k_rms_norm, dim3((unsigned) rows), dim3(256), 0, (hipStream_t) stream, tv(x), wv, w ? 1 : 0, eps,
                       dst);
    return check_launch("rms_norm");
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
    hipLaunchKernelGGL(k_rope_neox, dim3(grid_for(total, 256)), dim3(256), 0, (hipStream_t) stream, tv(x), pos, n_dims,
                       theta_scale, dst);
    return check_launch("rope");
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
    hipLaunchKernelGGL(k_cpy, dim3(grid_for(n, 256)), dim3(256), 0, (hipStream_t) stream, tv(src), src_type, tv(dst),
                       dst_type, n);
    return check_launch("cpy");
}

extern "C" int mmhip_get_rows(int src_type, const mmhip_view * src, const mmhip_view * ids, float * dst,
                              void * stream) {
    MMHIP_API_BEGIN();
    const bool q = src_type == TYPE_Q8_0 || src_type == TYPE_Q4_K || src_type == TYPE_Q6_K;
    if (!src || !ids || !dst || !(q || src_type == TYPE_F32 || src_type == TYPE_F16) ||
        (src_type == TYPE_Q8_0 && src->ne[0] % 32 != 0) || ((src_type == TYPE_Q4_K || src_type == TYPE_Q6_K) &&
                                                            src->ne[0] % 256 != 0)) {
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
