// k_quant.hip - weight-format kernels: GGUF <-> row-grouped layout, bit-exact
// dequantisation, and the ggml activation quantisers (Q8_0, Q8_K) that the
// quantized GEMVs consume.
#include "mmhip_device.h"
#include "mmhip_internal.h"

namespace mmhip {

// Field tables: for each field in device order, its byte offset inside the
// GGUF block and its size per block.
struct FieldTable {
    int n;
    int gguf_off[4];
    int size[4];
    int block_bytes;
    int block_elems;
};

static __host__ __device__ FieldTable field_table(int type) {
    switch (type) {
        case TYPE_Q8_0: return { 2, { 2, 0, 0, 0 }, { 32, 2, 0, 0 }, 34, 32 };
        case TYPE_Q4_K: return { 3, { 16, 4, 0, 0 }, { 128, 12, 4, 0 }, 144, 256 };
        case TYPE_Q5_K: return { 4, { 48, 16, 4, 0 }, { 128, 32, 12, 4 }, 176, 256 };
        case TYPE_Q6_K: return { 4, { 0, 128, 192, 208 }, { 128, 64, 16, 2 }, 210, 256 };
        default:        return { 0, { 0 }, { 0 }, 0, 0 };
    }
}

// One thread per (row, block, field); to_dev selects the direction.
__global__ void k_repack(int type, const uint8_t * __restrict__ src, uint8_t * __restrict__ dst, int64_t nrows,
                         int64_t nb, int64_t row_bytes_, int to_dev) {
    const FieldTable ft    = field_table(type);
    const int64_t    total = nrows * nb * ft.n;
    for (int64_t i = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; i < total; i += (int64_t) gridDim.x * blockDim.x) {
        const int     f   = (int) (i % ft.n);
        const int64_t b   = (i / ft.n) % nb;
        const int64_t row = i / (ft.n * nb);
        int64_t       dev_off = 0;
        for (int j = 0; j < f; j++) {
            dev_off += (int64_t) ft.size[j] * nb;
        }
        dev_off += (int64_t) ft.size[f] * b;
        const int64_t gguf_off = b * ft.block_bytes + ft.gguf_off[f];
        const uint8_t * s = src + row * row_bytes_ + (to_dev ? gguf_off : dev_off);
        uint8_t *       d = dst + row * row_bytes_ + (to_dev ? dev_off : gguf_off);
        for (int j = 0; j < ft.size[f]; j++) {
            d[j] = s[j];
        }
    }
}

// Bit-exact dequantisation from the row-grouped layout; one thread per 32
// output elements.  Contraction is off so d1*q - m1 rounds twice exactly as
// the GGUF reference definition does.
__global__ void k_dequant(int type, const uint8_t * __restrict__ w, int64_t nrows, int64_t K, int64_t row_stride,
                          float * __restrict__ y) {
#pragma clang fp contract(off)
    const int64_t groups = K / 32;
    const int64_t total  = nrows * groups;
    for (int64_t i = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; i < total; i += (int64_t) gridDim.x * blockDim.x) {
        const int64_t   g   = i % groups;
        const int64_t   row = i / groups;
        const uint8_t * r   = w + row * row_stride;
        float *         out = y + row * K + g * 32;
        if (type == TYPE_Q8_0) {
            const int8_t * qs = (const int8_t *) r + g * 32;
            const float    d  = h2f(((const uint16_t *) (r + K))[g]);
            for (int j = 0; j < 32; j++) {
                out[j] = d * (float) qs[j];
            }
        } else if (type == TYPE_Q4_K || type == TYPE_Q5_K) {
            // Q5_K: qh[K/8] follows qs; the fifth bit of element 32j + l of a
            // super-block is bit j of its qh byte l
            const int64_t   nbk   = K / 256;
            const int64_t   sb    = g / 8;
            const int       j     = (int) (g % 8);
            const int64_t   qh_sz = type == TYPE_Q5_K ? K / 8 : 0;
            const uint8_t * qs    = r + sb * 128 + (j / 2) * 32;
            const uint8_t * qh    = r + K / 2 + sb * 32;
            const uint8_t * sc    = r + K / 2 + qh_sz + sb * 12;
            const uint16_t * dm   = (const uint16_t *) (r + K / 2 + qh_sz + nbk * 12) + 2 * sb;
            int             s, m;
            q4k_scale_min(j, sc, s, m);
            const float d1 = h2f(dm[0]) * (float) s;
            const float m1 = h2f(dm[1]) * (float) m;
            for (int l = 0; l < 32; l++) {
                int q = (j & 1) ? (qs[l] >> 4) : (qs[l] & 0x0f);
                if (type == TYPE_Q5_K) {
                    q |= ((qh[l] >> j) & 1) << 4;
                }
                out[l] = d1 * (float) q - m1;
            }
        } else if (type == TYPE_Q6_K) {
            const int64_t   nbk = K / 256;
            const int64_t   sb  = g / 8;
            const int       e0  = (int) (g % 8) * 32;
            const uint8_t * ql  = r + sb * 128;
            const uint8_t * qh  = r + K / 2 + sb * 64;
            const int8_t *  sc  = (const int8_t *) (r + K / 2 + K / 4) + sb * 16;
            const float     d   = h2f(((const uint16_t *) (r + K / 2 + K / 4 + K / 16))[sb]);
            (void) nbk;
            for (int l = 0; l < 32; l++) {
                const int e  = e0 + l;
                const int h  = e >> 7, rr = e & 127, t = rr >> 5, c = rr & 31;
                const int lb = ql[64 * h + c + 32 * (t & 1)];
                const int lo = (t < 2) ? (lb & 0x0f) : (lb >> 4);
                const int hi = (qh[32 * h + c] >> (2 * t)) & 3;
                const float ds = d * (float) sc[e >> 4];
                out[l] = ds * (float) ((lo | (hi << 4)) - 32);
            }
        } else if (type == TYPE_F16) {
            const uint16_t * h = (const uint16_t *) r + g * 32;
            for (int j = 0; j < 32; j++) {
                out[j] = h2f(h[j]);
            }
        } else if (type == TYPE_F32) {
            const float * f = (const float *) r + g * 32;
            for (int j = 0; j < 32; j++) {
                out[j] = f[j];
            }
        }
    }
}

// ggml Q8_0 activation quantiser: one 32-lane half-wave per block.
// Output layout: qs[M][K] int8, then d[M][K/32] f32 (the f16-rounded scale).
__global__ __launch_bounds__(256) void k_quant_q8_0(const float * __restrict__ x, int64_t ldx, int64_t K, int64_t M,
                                                     int8_t * __restrict__ qs, float * __restrict__ dout) {
    const int64_t nblk  = K / 32;
    const int64_t total = M * nblk;
    const int     lane  = threadIdx.x & 31;
    for (int64_t blk = (blockIdx.x * (int64_t) blockDim.x + threadIdx.x) / 32; blk < total;
         blk += ((int64_t) gridDim.x * blockDim.x) / 32) {
        const int64_t m  = blk / nblk;
        const int64_t b  = blk % nblk;
        const float   xv = x[m * ldx + b * 32 + lane];
        const float   a  = group32_max(fabsf(xv));
        const float d  = a / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        qs[m * K + b * 32 + lane] = (int8_t) roundf(xv * id);
        if (lane == 0) {
            dout[m * nblk + b] = h2f(f2h(d));
        }
    }
}

// ggml Q8_K activation quantiser: one 256-thread block per super-block.
// Output layout: qs[M][K] int8, d[M][K/256] f32, bsums[M][K/16] int16.
__global__ __launch_bounds__(256) void k_quant_q8_K(const float * __restrict__ x, int64_t ldx, int64_t K, int64_t M,
                                                     int8_t * __restrict__ qs, float * __restrict__ dout,
                                                     int16_t * __restrict__ bsums) {
    __shared__ float s_amax[4];
    __shared__ int   s_idx[4];
    const int64_t    nsb  = K / 256;
    const int        tid  = threadIdx.x;
    for (int64_t sbi = blockIdx.x; sbi < M * nsb; sbi += gridDim.x) {
        const int64_t m  = sbi / nsb;
        const int64_t sb = sbi % nsb;
        const float * xb = x + m * ldx + sb * 256;
        const float   xv = xb[tid];
        float         a  = fabsf(xv);
        float         vm = xv;
        int           ix = tid;
        wave_argmax_abs(a, vm, ix);
        if ((tid & 63) == 0) {
            s_amax[tid >> 6] = a;
            s_idx[tid >> 6]  = ix;
        }
        __syncthreads();
        a  = s_amax[0];
        ix = s_idx[0];
        for (int w = 1; w < 4; w++) {
            if (s_amax[w] > a || (s_amax[w] == a && s_idx[w] < ix)) {
                a  = s_amax[w];
                ix = s_idx[w];
            }
        }
        __syncthreads();
        int8_t qv = 0;
        float  d  = 0.0f;
        if (a != 0.0f) {
            const float iscale = -127.0f / xb[ix];
            int         v      = (int) rintf(iscale * xv);
            qv                 = (int8_t) (v > 127 ? 127 : v);
            d                  = 1.0f / iscale;
        }
        qs[m * K + sb * 256 + tid] = qv;
        const int s = group16_sum_i(qv);
        if ((tid & 15) == 0) {
            bsums[m * (K / 16) + sb * 16 + tid / 16] = (int16_t) s;
        }
        if (tid == 0) {
            dout[m * nsb + sb] = d;
        }
    }
}

}  // namespace mmhip

using namespace mmhip;

extern "C" int mmhip_repack_rows(int type, const void * src, void * dst, int64_t nrows, int64_t ne0, void * stream) {
    MMHIP_API_BEGIN();
    if (!is_repacked_type(type)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "repack: type %d has no row-grouped layout", type);
    }
    const FieldTable ft = field_table(type);
    if (ne0 <= 0 || ne0 % ft.block_elems != 0 || nrows < 0) {
        return set_error(MMHIP_ERR_INVALID, "repack: ne0=%lld not a multiple of %d", (long long) ne0, ft.block_elems);
    }
    if (nrows == 0) {
        return MMHIP_OK;
    }
    const int64_t nb    = ne0 / ft.block_elems;
    const int64_t total = nrows * nb * ft.n;
    const int     grid  = (int) std::min<int64_t>((total + 255) / 256, 65536);
    hipLaunchKernelGGL(k_repack, dim3(grid), dim3(256), 0, (hipStream_t) stream, type, (const uint8_t *) src,
                       (uint8_t *) dst, nrows, nb, row_bytes(type, ne0), 1);
    return check_launch("repack");
}

extern "C" int mmhip_unpack_rows(int type, const void * src, void * dst, int64_t nrows, int64_t ne0, void * stream) {
    MMHIP_API_BEGIN();
    if (!is_repacked_type(type)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "unpack: type %d has no row-grouped layout", type);
    }
    const FieldTable ft = field_table(type);
    if (ne0 <= 0 || ne0 % ft.block_elems != 0 || nrows < 0) {
        return set_error(MMHIP_ERR_INVALID, "unpack: ne0=%lld not a multiple of %d", (long long) ne0, ft.block_elems);
    }
    if (nrows == 0) {
        return MMHIP_OK;
    }
    const int64_t nb    = ne0 / ft.block_elems;
    const int64_t total = nrows * nb * ft.n;
    const int     grid  = (int) std::min<int64_t>((total + 255) / 256, 65536);
    hipLaunchKernelGGL(k_repack, dim3(grid), dim3(256), 0, (hipStream_t) stream, type, (const uint8_t *) src,
                       (uint8_t *) dst, nrows, nb, row_bytes(type, ne0), 0);
    return check_launch("unpack");
}

extern "C" int mmhip_dequantize_rows(int type, const void * w, int64_t nrows, int64_t ne0, int64_t row_stride,
                                     float * dst, void * stream) {
    MMHIP_API_BEGIN();
    const int blk = (type == TYPE_Q4_K || type == TYPE_Q5_K || type == TYPE_Q6_K) ? 256 : 32;
    if (!(is_repacked_type(type) || type == TYPE_F16 || type == TYPE_F32)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "dequantize: type %d", type);
    }
    if (ne0 <= 0 || ne0 % blk != 0 || nrows < 0 || row_stride < row_bytes(type, ne0)) {
        return set_error(MMHIP_ERR_INVALID, "dequantize: bad shape ne0=%lld stride=%lld", (long long) ne0,
                         (long long) row_stride);
    }
    if (nrows == 0) {
        return MMHIP_OK;
    }
    const int64_t total = nrows * (ne0 / 32);
    const int     grid  = (int) std::min<int64_t>((total + 255) / 256, 65536);
    hipLaunchKernelGGL(k_dequant, dim3(grid), dim3(256), 0, (hipStream_t) stream, type, (const uint8_t *) w, nrows, ne0,
                       row_stride, dst);
    return check_launch("dequantize");
}

extern "C" size_t mmhip_act_bytes(int wtype, int64_t K, int64_t M) {
    return act_layout(wtype, K, M).total;
}

namespace mmhip {
int quantize_act(int wtype, const float * x, int64_t ldx, int64_t K, int64_t M, void * xq, hipStream_t stream) {
    const ActLayout L = act_layout(wtype, K, M);
    if (L.total == 0) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "quantize_act: weight type %d K=%lld", wtype, (long long) K);
    }
    uint8_t * base = (uint8_t *) xq;
    if (L.vec_type == TYPE_Q8_0) {
        const int64_t blocks = M * (K / 32);
        const int     grid   = (int) std::min<int64_t>((blocks * 32 + 255) / 256, 65536);
        hipLaunchKernelGGL(k_quant_q8_0, dim3(grid), dim3(256), 0, stream, x, ldx, K, M, (int8_t *) (base + L.qs_off),
                           (float *) (base + L.d_off));
    } else {
        const int64_t sbs  = M * (K / 256);
        const int     grid = (int) std::min<int64_t>(sbs, 65536);
        hipLaunchKernelGGL(k_quant_q8_K, dim3(grid), dim3(256), 0, stream, x, ldx, K, M, (int8_t *) (base + L.qs_off),
                           (float *) (base + L.d_off), (int16_t *) (base + L.bs_off));
    }
    return check_launch("quantize_act");
}
}  // namespace mmhip

extern "C" int mmhip_quantize_act(int wtype, const float * x, int64_t ldx, int64_t K, int64_t M, void * xq,
                                  void * stream) {
    MMHIP_API_BEGIN();
    if (M <= 0 || K <= 0 || ldx < K || !x || !xq) {
        return set_error(MMHIP_ERR_INVALID, "quantize_act: bad arguments");
    }
    return quantize_act(wtype, x, ldx, K, M, xq, (hipStream_t) stream);
}
