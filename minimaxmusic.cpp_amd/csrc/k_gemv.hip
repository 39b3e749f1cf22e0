// k_gemv.hip - decode GEMV for quantized weights (M <= 8 activation rows).
//
// Arithmetic follows ggml-CPU's mul_mat for these types: activations are
// quantised to Q8_0 (Q8_0 weights) or Q8_K (Q4_K / Q6_K weights) by
// k_quant.hip, integer dot products are exact (v_dot4_i32_i8), and each
// (half-)block's integer sum is scaled by d_w * d_x in f32.  Only the f32
// summation order differs from the CPU backend.
//
// Mapping: 256 threads = 4 waves; each wave owns R weight rows at a time and
// streams them with 16-byte loads, 64 lanes covering 1024 contiguous bytes of
// a field per step (every field of the row-grouped layout is contiguous).
// The quantised activations of all M columns are staged once per workgroup
// in LDS and re-read there, so HBM carries only the weights.
#include "mmhip_device.h"
#include "mmhip_internal.h"

namespace mmhip {

__device__ __forceinline__ int4_t ld16(const void * p) {
    return *(const int4_t *) p;
}

__device__ __forceinline__ int dot16(int4_t a, int4_t b) {
    int s = dot4(a.x, b.x, 0);
    s     = dot4(a.y, b.y, s);
    s     = dot4(a.z, b.z, s);
    return dot4(a.w, b.w, s);
}

// Reduce V per-lane partial sums over the 64 lanes.  Reduce-scatter first
// (V halves per step), then a plain butterfly; returns the total of value
// index idx(lane) = sum_k bit(lane, 5-k) * V/2^(k+1).
template <int V> __device__ __forceinline__ float wave_reduce_scatter(float (&a)[V], int lane) {
    constexpr int LOGV = V == 1 ? 0 : V == 2 ? 1 : V == 4 ? 2 : V == 8 ? 3 : V == 16 ? 4 : 5;
    static_assert((1 << LOGV) == V, "V must be a power of two <= 32");
#pragma unroll
    for (int k = 0; k < LOGV; k++) {
        const int  o     = 32 >> k;
        const int  half  = V >> (k + 1);
        const bool upper = (lane & o) != 0;
#pragma unroll
        for (int i = 0; i < half; i++) {
            const float send = upper ? a[i] : a[i + half];
            const float keep = upper ? a[i + half] : a[i];
            a[i]             = keep + __shfl_xor(send, o, WAVE);
        }
    }
    float v = a[0];
#pragma unroll
    for (int o = 32 >> LOGV; o >= 1; o >>= 1) {
        v += __shfl_xor(v, o, WAVE);
    }
    return v;
}

template <int V> __device__ __forceinline__ int reduce_index(int lane) {
    int idx = 0;
    int w   = V;
#pragma unroll
    for (int k = 0; (1 << k) < V; k++) {
        w >>= 1;
        if (lane & (32 >> k)) {
            idx += w;
        }
    }
    return idx;
}

// Store R x NC reduced sums: value index v = r*NC + c.
template <int NC, int R>
__device__ __forceinline__ void store_rows(float (&acc)[R][NC], int lane, int64_t row0, int64_t N, float * y,
                                           int64_t ldy) {
    constexpr int V  = R * NC;
    constexpr int VP = V <= 1 ? 1 : V <= 2 ? 2 : V <= 4 ? 4 : V <= 8 ? 8 : V <= 16 ? 16 : 32;
    float         a[VP];
#pragma unroll
    for (int i = 0; i < VP; i++) {
        a[i] = i < V ? acc[i / NC][i % NC] : 0.0f;
    }
    const float total = wave_reduce_scatter<VP>(a, lane);
    const int   idx   = reduce_index<VP>(lane);
    // lanes below the reduce-scatter span hold distinct indices
    if ((lane & ((64 / VP) - 1)) == 0 && idx < V) {
        const int     r   = idx / NC;
        const int     c   = idx % NC;
        const int64_t row = row0 + r;
        if (row < N) {
            y[c * ldy + row] = total;
        }
    }
}

template <int NC>
__device__ __forceinline__ void stage_act(uint8_t * lds, const uint8_t * xq, size_t qs_bytes, const float * xd,
                                          int nd, const int16_t * xbs, int nbs) {
    const int tid = threadIdx.x;
    for (size_t i = (size_t) tid * 16; i < qs_bytes; i += 256 * 16) {
        *(int4_t *) (lds + i) = ld16(xq + i);
    }
    float * ld = (float *) (lds + qs_bytes);
    for (int i = tid; i < nd; i += 256) {
        ld[i] = xd[i];
    }
    if (xbs) {
        int16_t * lb = (int16_t *) (lds + qs_bytes + 4 * (size_t) nd);
        for (int i = tid; i < nbs; i += 256) {
            lb[i] = xbs[i];
        }
    }
    __syncthreads();
}

template <int NC, int R>
__global__ __launch_bounds__(256) void k_gemv_q8_0(const uint8_t * __restrict__ W, int64_t N, int64_t K, int64_t rs,
                                                    const uint8_t * __restrict__ xq, const float * __restrict__ xd,
                                                    float * __restrict__ y, int64_t ldy) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int64_t qs_bytes = (int64_t) NC * K;
    const int     nblk     = (int) (K / 32);
    stage_act<NC>(lds, xq, qs_bytes, xd, NC * nblk, nullptr, 0);
    const int8_t * lq = (const int8_t *) lds;
    const float *  ld = (const float *) (lds + qs_bytes);

    const int     wave    = threadIdx.x >> 6;
    const int     lane    = threadIdx.x & 63;
    const int64_t ngroups = (N + R - 1) / R;
    for (int64_t g = (int64_t) blockIdx.x * 4 + wave; g < ngroups; g += (int64_t) gridDim.x * 4) {
        const uint8_t * wr[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int64_t row = g * R + r < N ? g * R + r : N - 1;
            wr[r]             = W + row * rs;
        }
        float acc[R][NC];
#pragma unroll
        for (int r = 0; r < R; r++) {
#pragma unroll
            for (int c = 0; c < NC; c++) {
                acc[r][c] = 0.0f;
            }
        }
        for (int64_t off = (int64_t) lane * 16; off < K; off += 1024) {
            int4_t wv[R];
            float  dw[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                wv[r] = ld16(wr[r] + off);
                dw[r] = h2f(*(const uint16_t *) (wr[r] + K + 2 * (off >> 5)));
            }
            const int b = (int) (off >> 5);
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const int4_t xv = *(const int4_t *) (lq + c * K + off);
                const float  dx = ld[c * nblk + b];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    acc[r][c] += (float) dot16(wv[r], xv) * (dw[r] * dx);
                }
            }
        }
        store_rows<NC, R>(acc, lane, g * R, N, y, ldy);
    }
}

template <int NC, int R>
__global__ __launch_bounds__(256) void k_gemv_q4_K(const uint8_t * __restrict__ W, int64_t N, int64_t K, int64_t rs,
                                                    const uint8_t * __restrict__ xq, const float * __restrict__ xd,
                                                    const int16_t * __restrict__ xbs, float * __restrict__ y,
                                                    int64_t ldy) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int64_t qs_bytes = (int64_t) NC * K;
    const int     nsb      = (int) (K / 256);
    const int     ngrp     = (int) (K / 16);
    stage_act<NC>(lds, xq, qs_bytes, xd, NC * nsb, xbs, NC * ngrp);
    const int8_t *  lq = (const int8_t *) lds;
    const float *   ld = (const float *) (lds + qs_bytes);
    const int16_t * lb = (const int16_t *) (lds + qs_bytes + 4 * (size_t) (NC * nsb));

    const int     wave    = threadIdx.x >> 6;
    const int     lane    = threadIdx.x & 63;
    const int64_t half_k  = K / 2;
    const int64_t ngroups = (N + R - 1) / R;
    for (int64_t g = (int64_t) blockIdx.x * 4 + wave; g < ngroups; g += (int64_t) gridDim.x * 4) {
        const uint8_t * wr[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int64_t row = g * R + r < N ? g * R + r : N - 1;
            wr[r]             = W + row * rs;
        }
        float acc[R][NC];
#pragma unroll
        for (int r = 0; r < R; r++) {
#pragma unroll
            for (int c = 0; c < NC; c++) {
                acc[r][c] = 0.0f;
            }
        }
        for (int64_t off = (int64_t) lane * 16; off < half_k; off += 1024) {
            const int sb   = (int) (off >> 7);
            const int o    = (int) (off & 127);
            const int c64  = o >> 5;
            const int hf   = (o >> 4) & 1;
            const int e_lo = sb * 256 + c64 * 64 + hf * 16;
            const int e_hi = e_lo + 32;
            int4_t    wv[R];
            int       sc_lo[R], sc_hi[R], mn_lo[R], mn_hi[R];
            float     d[R], dmin[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                wv[r]               = ld16(wr[r] + off);
                const uint32_t * sw = (const uint32_t *) (wr[r] + half_k + 12 * sb);
                const uint32_t   w0 = sw[0], w1 = sw[1], w2 = sw[2];
                const uint32_t   dm = *(const uint32_t *) (wr[r] + half_k + 12 * (int64_t) nsb + 4 * sb);
                q4k_scale_min_w(2 * c64, w0, w1, w2, sc_lo[r], mn_lo[r]);
                q4k_scale_min_w(2 * c64 + 1, w0, w1, w2, sc_hi[r], mn_hi[r]);
                d[r]    = h2f((uint16_t) (dm & 0xffff));
                dmin[r] = h2f((uint16_t) (dm >> 16));
            }
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const int4_t xlo   = *(const int4_t *) (lq + c * K + e_lo);
                const int4_t xhi   = *(const int4_t *) (lq + c * K + e_hi);
                const float  dx    = ld[c * nsb + sb];
                const int    bs_lo = lb[c * ngrp + (e_lo >> 4)];
                const int    bs_hi = lb[c * ngrp + (e_hi >> 4)];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const int4_t lo = { wv[r].x & 0x0F0F0F0F, wv[r].y & 0x0F0F0F0F, wv[r].z & 0x0F0F0F0F,
                                        wv[r].w & 0x0F0F0F0F };
                    const int4_t hi = { (wv[r].x >> 4) & 0x0F0F0F0F, (wv[r].y >> 4) & 0x0F0F0F0F,
                                        (wv[r].z >> 4) & 0x0F0F0F0F, (wv[r].w >> 4) & 0x0F0F0F0F };
                    const int isum = sc_lo[r] * dot16(lo, xlo) + sc_hi[r] * dot16(hi, xhi);
                    const int msum = mn_lo[r] * bs_lo + mn_hi[r] * bs_hi;
                    acc[r][c] += (d[r] * dx) * (float) isum - (dmin[r] * dx) * (float) msum;
                }
            }
        }
        store_rows<NC, R>(acc, lane, g * R, N, y, ldy);
    }
}

template <int NC, int R>
__global__ __launch_bounds__(256) void k_gemv_q6_K(const uint8_t * __restrict__ W, int64_t N, int64_t K, int64_t rs,
                                                    const uint8_t * __restrict__ xq, const float * __restrict__ xd,
                                                    const int16_t * __restrict__ xbs, float * __restrict__ y,
                                                    int64_t ldy) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int64_t qs_bytes = (int64_t) NC * K;
    const int     nsb      = (int) (K / 256);
    const int     ngrp     = (int) (K / 16);
    stage_act<NC>(lds, xq, qs_bytes, xd, NC * nsb, xbs, NC * ngrp);
    const int8_t *  lq = (const int8_t *) lds;
    const float *   ld = (const float *) (lds + qs_bytes);
    const int16_t * lb = (const int16_t *) (lds + qs_bytes + 4 * (size_t) (NC * nsb));

    const int     wave    = threadIdx.x >> 6;
    const int     lane    = threadIdx.x & 63;
    const int64_t qh_off  = K / 2;
    const int64_t sc_off  = K / 2 + K / 4;
    const int64_t d_off   = sc_off + K / 16;
    const int     units   = (int) (K / 64);
    const int64_t ngroups = (N + R - 1) / R;
    for (int64_t g = (int64_t) blockIdx.x * 4 + wave; g < ngroups; g += (int64_t) gridDim.x * 4) {
        const uint8_t * wr[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int64_t row = g * R + r < N ? g * R + r : N - 1;
            wr[r]             = W + row * rs;
        }
        float acc[R][NC];
#pragma unroll
        for (int r = 0; r < R; r++) {
#pragma unroll
            for (int c = 0; c < NC; c++) {
                acc[r][c] = 0.0f;
            }
        }
        for (int u = lane; u < units; u += 64) {
            const int sb  = u >> 2;
            const int h   = (u >> 1) & 1;
            const int l0  = (u & 1) * 16;
            const int g0  = sb * 16 + h * 8 + (l0 >> 4);  // 16-element group of t = 0
            const int eb  = sb * 256 + h * 128 + l0;      // element of t = 0, i = 0
            int4_t    qa[R], qb[R], qh[R];
            int       sc[R][4];
            float     d[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                qa[r] = ld16(wr[r] + sb * 128 + h * 64 + l0);
                qb[r] = ld16(wr[r] + sb * 128 + h * 64 + 32 + l0);
                qh[r] = ld16(wr[r] + qh_off + sb * 64 + h * 32 + l0);
                const uint8_t * s8 = wr[r] + sc_off + sb * 16 + h * 8;
                const uint2     sw = *(const uint2 *) s8;
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const int      bi = (l0 >> 4) + 2 * t;
                    const uint32_t wd = bi < 4 ? sw.x : sw.y;
                    sc[r][t]          = (int) (int8_t) ((wd >> (8 * (bi & 3))) & 0xff);
                }
                d[r] = h2f(*(const uint16_t *) (wr[r] + d_off + 2 * sb));
            }
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const float dx = ld[c * nsb + sb];
                int4_t      xv[4];
                int         bs[4];
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    xv[t] = *(const int4_t *) (lq + c * K + eb + 32 * t);
                    bs[t] = lb[c * ngrp + g0 + 2 * t];
                }
#pragma unroll
                for (int r = 0; r < R; r++) {
                    int isum = 0;
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        const int4_t src = (t & 1) ? qb[r] : qa[r];
                        const int    sh  = (t < 2) ? 0 : 4;
                        int4_t       q;
                        q.x = ((src.x >> sh) & 0x0F0F0F0F) | (((qh[r].x >> (2 * t)) & 0x03030303) << 4);
                        q.y = ((src.y >> sh) & 0x0F0F0F0F) | (((qh[r].y >> (2 * t)) & 0x03030303) << 4);
                        q.z = ((src.z >> sh) & 0x0F0F0F0F) | (((qh[r].z >> (2 * t)) & 0x03030303) << 4);
                        q.w = ((src.w >> sh) & 0x0F0F0F0F) | (((qh[r].w >> (2 * t)) & 0x03030303) << 4);
                        isum += sc[r][t] * (dot16(q, xv[t]) - 32 * bs[t]);
                    }
                    acc[r][c] += (d[r] * dx) * (float) isum;
                }
            }
        }
        store_rows<NC, R>(acc, lane, g * R, N, y, ldy);
    }
}

// ---------------------------------------------------------------------
// host dispatch

constexpr int GEMV_R = 2;

static size_t gemv_lds_bytes(int wtype, int64_t K, int M) {
    if (wtype == TYPE_Q8_0) {
        return (size_t) M * K + 4 * (size_t) M * (K / 32);
    }
    return (size_t) M * K + 4 * (size_t) M * (K / 256) + 2 * (size_t) M * (K / 16);
}

template <typename F, typename... Args>
static int launch_gemv(F kern, size_t lds, int64_t N, hipStream_t stream, Args... args) {
    static thread_local const void * raised[64] = {};
    if (lds > 64 * 1024) {
        // opt in to the large-LDS limit once per kernel instance
        bool seen = false;
        for (const void * p : raised) {
            if (p == (const void *) kern) {
                seen = true;
                break;
            }
        }
        if (!seen) {
            if (hipFuncSetAttribute((const void *) kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int) lds) !=
                hipSuccess) {
                return set_error(MMHIP_ERR_HIP, "gemv: cannot raise LDS limit to %zu", lds);
            }
            for (auto & p : raised) {
                if (!p) {
                    p = (const void *) kern;
                    break;
                }
            }
        }
    }
    const int64_t groups = (N + GEMV_R - 1) / GEMV_R;
    const int64_t wgs    = (groups + 3) / 4;
    const int     grid   = (int) std::min<int64_t>(wgs, 1024);
    hipLaunchKernelGGL(kern, dim3(grid), dim3(256), lds, stream, args...);
    return check_launch("gemv");
}

template <int NC>
static int gemv_dispatch(int wtype, const uint8_t * W, int64_t N, int64_t K, int64_t rs, const ActPtrs & x, float * y,
                         int64_t ldy, hipStream_t stream) {
    const size_t    lds = gemv_lds_bytes(wtype, K, NC);
    const uint8_t * xq  = (const uint8_t *) x.qs;
    if (wtype == TYPE_Q8_0) {
        return launch_gemv(k_gemv_q8_0<NC, GEMV_R>, lds, N, stream, W, N, K, rs, xq, x.d, y, ldy);
    }
    if (wtype == TYPE_Q4_K) {
        return launch_gemv(k_gemv_q4_K<NC, GEMV_R>, lds, N, stream, W, N, K, rs, xq, x.d, x.bs, y, ldy);
    }
    return launch_gemv(k_gemv_q6_K<NC, GEMV_R>, lds, N, stream, W, N, K, rs, xq, x.d, x.bs, y, ldy);
}

bool gemv_supported(int wtype, int64_t N, int64_t K, int64_t rs, const void * W) {
    return (wtype == TYPE_Q8_0 || wtype == TYPE_Q4_K || wtype == TYPE_Q6_K) && K % 256 == 0 && N > 0 &&
           rs >= row_bytes(wtype, K) && rs % 16 == 0 && ((uintptr_t) W) % 16 == 0 &&
           gemv_lds_bytes(wtype, K, 1) <= 160 * 1024;
}

int gemv_q(int wtype, const void * W, int64_t N, int64_t K, int64_t rs, const ActPtrs & x, int64_t M, float * y,
           int64_t ldy, hipStream_t stream) {
    if (!gemv_supported(wtype, N, K, rs, W) || M < 1 || ldy < N) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "gemv: type %d N=%lld K=%lld M=%lld rs=%lld not supported", wtype,
                         (long long) N, (long long) K, (long long) M, (long long) rs);
    }
    // column groups of up to 8 that fit the LDS budget
    int mc = 8;
    while (mc > 1 && gemv_lds_bytes(wtype, K, mc) > 160 * 1024) {
        mc--;
    }
    const uint8_t * wb = (const uint8_t *) W;
    for (int64_t c0 = 0; c0 < M; c0 += mc) {
        const int64_t nc = std::min<int64_t>(mc, M - c0);
        ActPtrs       xs = x.slice(c0, K);
        float *       ys = y + c0 * ldy;
        int           rc;
        switch (nc) {
            case 1: rc = gemv_dispatch<1>(wtype, wb, N, K, rs, xs, ys, ldy, stream); break;
            case 2: rc = gemv_dispatch<2>(wtype, wb, N, K, rs, xs, ys, ldy, stream); break;
            case 3: rc = gemv_dispatch<3>(wtype, wb, N, K, rs, xs, ys, ldy, stream); break;
            case 4: rc = gemv_dispatch<4>(wtype, wb, N, K, rs, xs, ys, ldy, stream); break;
            case 5: rc = gemv_dispatch<5>(wtype, wb, N, K, rs, xs, ys, ldy, stream); break;
            case 6: rc = gemv_dispatch<6>(wtype, wb, N, K, rs, xs, ys, ldy, stream); break;
            case 7: rc = gemv_dispatch<7>(wtype, wb, N, K, rs, xs, ys, ldy, stream); break;
            default: rc = gemv_dispatch<8>(wtype, wb, N, K, rs, xs, ys, ldy, stream); break;
        }
        if (rc != MMHIP_OK) {
            return rc;
        }
    }
    return MMHIP_OK;
}

}  // namespace mmhip

using namespace mmhip;

extern "C" int mmhip_mul_mat_q(int type, const void * W, int64_t N, int64_t K, int64_t w_row_stride, const void * xq,
                               int64_t M, float * y, int64_t ldy, void * stream) {
    MMHIP_API_BEGIN();
    const ActLayout L = act_layout(type, K, M);
    if (L.total == 0 || !xq || !W || !y) {
        return set_error(MMHIP_ERR_INVALID, "mul_mat_q: bad arguments (type %d, K=%lld)", type, (long long) K);
    }
    return gemv_q(type, W, N, K, w_row_stride, ActPtrs::from(L, xq), M, y, ldy, (hipStream_t) stream);
}
