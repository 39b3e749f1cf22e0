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
// The quantised activations of the M columns (a few KB) are read through the
// L1/L2 caches by every wave, so HBM carries essentially only the weights.
#include <cstdlib>

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
            // both operands pinned in registers: a select between two array
            // loads would otherwise become one load at a lane-dependent index,
            // which puts the array in scratch memory
            float lo = a[i], hi = a[i + half];
            asm volatile("" : "+v"(lo), "+v"(hi));
            const float send = upper ? lo : hi;
            const float keep = upper ? hi : lo;
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
// With res != nullptr the stored value is total + res[c*ldr + row] (the residual
// ADD of the graph, one f32 rounding as ggml's separate ADD node gives).
template <int NC, int R>
__device__ __forceinline__ void store_rows(float (&acc)[R][NC], int lane, int64_t row0, int64_t N, float * y,
                                           int64_t ldy, const float * res, int64_t ldr) {
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
            y[c * ldy + row] = res ? total + res[c * ldr + row] : total;
        }
    }
}

// 16-byte load from a 16-byte aligned address, or (AL = false) from a 2-byte
// aligned one as eight 16-bit loads.
template <bool AL> __device__ __forceinline__ int4_t ld16a(const uint8_t * p) {
    if constexpr (AL) {
        return *(const int4_t *) p;
    } else {
        const uint16_t * s = (const uint16_t *) p;
        return int4_t{ (int) (s[0] | ((uint32_t) s[1] << 16)), (int) (s[2] | ((uint32_t) s[3] << 16)),
                       (int) (s[4] | ((uint32_t) s[5] << 16)), (int) (s[6] | ((uint32_t) s[7] << 16)) };
    }
}

template <bool AL> __device__ __forceinline__ uint2 ld8a(const uint8_t * p) {
    if constexpr (AL) {
        return *(const uint2 *) p;
    } else {
        const uint16_t * s = (const uint16_t *) p;
        return uint2{ s[0] | ((uint32_t) s[1] << 16), s[2] | ((uint32_t) s[3] << 16) };
    }
}

// Q8_0.  One wave per R consecutive rows.  A row's qs is read in 1024-byte
// chunks (32 blocks; lane l owns bytes 16l .. 16l+15 = half of block l/2);
// the wave issues the loads of CH chunks x R rows before using any, so for
// K <= 1024 * CH one memory round trip covers its whole share (measured on
// the decode shapes: this beats both a per-chunk loop and a split of K over
// the workgroup's waves, which adds a barrier and an LDS reduction).  The
// activation chunks come through L1/L2 (a few KB shared by every wave).
template <int NC, int R, int CH, bool ONE>  // ONE: K <= 1024 * CH, a single pass
__global__ __launch_bounds__(256) void k_gemv_q8_0(const uint8_t * __restrict__ W, int64_t N, int64_t K, int64_t rs,
                                                    const int8_t * __restrict__ xq, const float * __restrict__ xd,
                                                    float * y, int64_t ldy, const float * res, int64_t ldr) {
    const int     lane = threadIdx.x & 63;
    const int64_t g    = (int64_t) blockIdx.x * 4 + (threadIdx.x >> 6);
    if (g * R >= N) {
        return;
    }
    const int       nblk = (int) (K / 32);
    const uint8_t * wr[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        wr[r] = W + (g * R + r < N ? g * R + r : N - 1) * rs;
    }
    float acc[R][NC];
#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            acc[r][c] = 0.0f;
        }
    }
    const int k32   = (int) K;
    const int npass = ONE ? 1 : (k32 + 1024 * CH - 1) / (1024 * CH);
    for (int pass = 0; pass < npass; pass++) {
        const int base = pass * 1024 * CH;
        // every load unconditional (offsets clamped into the row, the lanes
        // past K weighted by zero) so that all of them issue before any use
        int4_t   wq[CH][R], xv[CH][NC];
        uint16_t sw[CH][R];
        float    dx[CH][NC];
#pragma unroll
        for (int u = 0; u < CH; u++) {
            const int o = min(base + 1024 * u + lane * 16, k32 - 16);
#pragma unroll
            for (int r = 0; r < R; r++) {
                wq[u][r] = ld16(wr[r] + o);
                sw[u][r] = *(const uint16_t *) (wr[r] + k32 + 2 * (o >> 5));
            }
#pragma unroll
            for (int c = 0; c < NC; c++) {
                xv[u][c] = ld16(xq + c * k32 + o);
                dx[u][c] = xd[c * nblk + (o >> 5)];
            }
        }
#pragma unroll
        for (int u = 0; u < CH; u++) {
            const bool ok = base + 1024 * u + lane * 16 < k32;
#pragma unroll
            for (int r = 0; r < R; r++) {
                const float dw = ok ? h2f(sw[u][r]) : 0.0f;
#pragma unroll
                for (int c = 0; c < NC; c++) {
                    acc[r][c] += (float) dot16(wq[u][r], xv[u][c]) * (dw * dx[u][c]);
                }
            }
        }
    }
    store_rows<NC, R>(acc, lane, g * R, N, y, ldy, res, ldr);
}

// Persistent Q8_0 GEMVs whose activation rows are made in their prologue:
//   PRO_NORM    the raw rows of an RMS_NORM (+ MUL by the norm weight): sum of
//               squares in double, normalise, times the weight (the arithmetic
//               of k_rms_norm_row);
//   PRO_SWIGLU  silu(gate) * up (the arithmetic of k_swiglu_quant);
// then the Q8_0 activation quantisation of quant_chunk256 into LDS.  This
// removes the separate norm / SwiGLU kernel of the decode graph.
// One 16-wave workgroup per CU.  Each wave streams the weight rows
// it * TW + wave (TW waves in the grid); for K <= 4096 through two register
// buffers, the next iteration's loads in flight while the current one is
// reduced.  Activations are loaded first, then the first weight rows: loads
// return in order, so the prologue runs while the weights are in flight.
constexpr int PG_WAVES   = 16;  // waves per workgroup
constexpr int PRO_NORM   = 0;
constexpr int PRO_SWIGLU = 1;

struct PgArgs {
    const uint8_t * W;
    int64_t         N;
    int             K;
    int64_t         rs;
    const float *   x;  // NORM: raw rows; SWIGLU: gate rows
    int64_t         ldx;
    const float *   u;  // SWIGLU: up rows
    int64_t         ldu;
    const float *   nw;  // NORM: norm weight
    float           eps;
    float *         xo;  // optional f32 activation rows [M, K] (written by workgroup 0)
    float *         y;
    int64_t         ldy;
    const float *   res;
    int64_t         ldr;
    int             nit;  // row iterations (uniform)
};

template <int CH> struct PgBuf {
    int4_t   w[CH];
    uint16_t s[CH];
};

// chunks U0 .. U1 - 1 of a row into b: buffer loads off the row's (uniform)
// base, so each chunk costs one 32-bit offset register; lanes past K re-read
// the row's last 16 bytes and are weighted by zero
template <int CH, int U0 = 0, int U1 = CH>
__device__ __forceinline__ void pg_load(PgBuf<CH> & b, const PgArgs & a, int64_t row, int lane) {
    const uint8_t *              wr = a.W + (row < a.N ? row : a.N - 1) * a.rs;
    const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc((void *) wr, (short) 0, a.K + a.K / 16,
                                                                        0x00020000);
#pragma unroll
    for (int u = U0; u < U1; u++) {
        const unsigned o = min(1024u * u + 16u * lane, (unsigned) a.K - 16u);
        b.w[u]           = __builtin_bit_cast(int4_t, __builtin_amdgcn_raw_buffer_load_b128(rr, (int) o, 0, 0));
        b.s[u]           = __builtin_amdgcn_raw_buffer_load_b16(rr, a.K + 2 * (int) (o >> 5), 0, 0);
    }
}

// one row against the NC quantised rows in LDS (sq: [NC][1024 CH], sd:
// [NC][32 CH]); off is added to the LDS indices (an opaque zero keeps the
// reads inside a loop where the rows do not fit in registers)
template <int NC, int CH>
__device__ __forceinline__ void pg_acc(const PgBuf<CH> & b, const int8_t * sq, const float * sd, int off,
                                       const PgArgs & a, int lane, float (&acc)[1][NC]) {
#pragma unroll
    for (int c = 0; c < NC; c++) {
        acc[0][c] = 0.0f;
    }
#pragma unroll
    for (int u = 0; u < CH; u++) {
        const int  o  = min(1024 * u + lane * 16, a.K - 16);
        const bool ok = 1024 * u + lane * 16 < a.K;
        const float dw = ok ? h2f(b.s[u]) : 0.0f;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const int4_t xq = *(const int4_t *) &sq[c * 1024 * CH + o + off];
            const float  dx = sd[c * 32 * CH + (o >> 5) + off];
            acc[0][c] += (float) dot16(b.w[u], xq) * (dw * dx);
        }
        if constexpr (CH > 4) {
            if (u % 4 == 3) {
                __builtin_amdgcn_sched_barrier(0);  // bounds the LDS reads in flight (registers)
            }
        }
    }
}

template <int NC, int CH>
__device__ __forceinline__ void pg_dot(const PgBuf<CH> & b, const int8_t * sq, const float * sd, int off,
                                       const PgArgs & a, int lane, int64_t row) {
    float acc[1][NC];
    pg_acc<NC, CH>(b, sq, sd, off, a, lane, acc);
    store_rows<NC, 1>(acc, lane, row, a.N, a.y, a.ldy, a.res, a.ldr);
}

// The activation values of the persistent GEMVs' prologue (the separate
// kernels' unfused f32 arithmetic; the dot products keep the plain GEMV's
// FMAs), quantised into LDS (s_q: [NC][MAXK] int8, s_d: [NC][MAXK / 32]).
// xv / xw hold chunk j of thread t: elements 4 t + 4096 j .. + 3.
// Byte position of Q8_K activation byte b in LDS: 16-byte granule g of
// super-block sb = g / 16 stored at g ^ 2 (sb % 4), so that the Q6_K dot's
// 16-byte reads (lanes 4 s + 2 a + b0 at 256 s + 128 a + 16 b0 + 32 t) fall
// in 16 different bank groups per 16 lanes
__device__ __forceinline__ int q8k_swz(int b) {
    const int g = b >> 4;
    return ((g ^ (2 * ((g >> 4) & 3))) << 4) | (b & 15);
}

template <int NC, int J, int MAXK, int PRO, int QT = TYPE_Q8_0>
__device__ __forceinline__ void pg_prologue(const float4_t (&xv)[J][NC], const float4_t (&xw)[J][PRO == PRO_NORM ? 1 : NC],
                                            int8_t * s_q, float * s_d, double (*s_ss)[PG_WAVES], const PgArgs & a,
                                            int lane, int wv, int K, int16_t * s_bs = nullptr) {
#pragma clang fp contract(off)
    float sc[NC];
    if constexpr (PRO == PRO_NORM) {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            double ss = 0.0;
#pragma unroll
            for (int j = 0; j < J; j++) {
                if (4 * (int) threadIdx.x + 256 * PG_WAVES * j < K) {
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        ss += (double) (xv[j][c][k] * xv[j][c][k]);
                    }
                }
            }
            ss = wave_sum_d(ss);
            if (lane == 0) {
                s_ss[c][wv] = ss;
            }
        }
        __syncthreads();
#pragma unroll
        for (int c = 0; c < NC; c++) {
            double tot = 0.0;
#pragma unroll
            for (int w = 0; w < PG_WAVES; w++) {
                tot += s_ss[c][w];
            }
            const float mean = (float) (tot / (double) K);
            sc[c]            = 1.0f / sqrtf(mean + a.eps);
        }
    }
#pragma unroll
    for (int c = 0; c < NC; c++) {
#pragma unroll
        for (int j = 0; j < J; j++) {
            const int e = 4 * (int) threadIdx.x + 256 * PG_WAVES * j;
            float     o[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                if constexpr (PRO == PRO_NORM) {
                    const float t = xv[j][c][k] * sc[c];
                    o[k]          = t * xw[j][0][k];
                } else {
                    const float g    = xv[j][c][k];
                    const float silu = g / (1.0f + expf(-g));
                    o[k]             = silu * xw[j][c][k];
                }
            }
            if constexpr (QT == TYPE_Q8_K) {
                // the wave's 256 elements are one super-block (K % 256 == 0:
                // the condition is uniform over the wave)
                const int ch = e / 256;
                if (e < K) {
                    const char4 q4 = quant_chunk256_q(o, lane, TYPE_Q8_K, s_d + c * (MAXK / 256) + ch,
                                                      s_bs + c * (MAXK / 16) + 16 * ch);
                    *(char4 *) &s_q[c * MAXK + q8k_swz(256 * ch + 4 * lane)] = q4;
                    if (a.xo && blockIdx.x == 0) {
                        *(float4_t *) (a.xo + (int64_t) c * K + e) = float4_t{ o[0], o[1], o[2], o[3] };
                    }
                }
                continue;
            }
            const float m = group8_max(fmaxf(fmaxf(fabsf(o[0]), fabsf(o[1])), fmaxf(fabsf(o[2]), fabsf(o[3]))));
            const float dd = m / 127.0f;
            const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
            if (e < K) {
                char4 q;
                q.x                          = (signed char) roundf(o[0] * id);
                q.y                          = (signed char) roundf(o[1] * id);
                q.z                          = (signed char) roundf(o[2] * id);
                q.w                          = (signed char) roundf(o[3] * id);
                *(char4 *) &s_q[c * MAXK + e] = q;
                if ((lane & 7) == 0) {
                    s_d[c * (MAXK / 32) + e / 32] = h2f(f2h(dd));
                }
                if (a.xo && blockIdx.x == 0) {
                    *(float4_t *) (a.xo + (int64_t) c * K + e) = float4_t{ o[0], o[1], o[2], o[3] };
                }
            }
        }
    }
}

template <int NC, int CH, int PRO>
__global__ __launch_bounds__(64 * PG_WAVES) void k_gemv_q8_0_pro(PgArgs a) {
    constexpr int  MAXK = 1024 * CH;
    constexpr int  J    = MAXK / (256 * PG_WAVES);  // float4 activation chunks per thread
    constexpr bool DB   = CH <= 4;                  // double-buffered row loop
    __shared__ __attribute__((aligned(16))) int8_t s_q[NC * MAXK];
    __shared__ float  s_d[NC * MAXK / 32];
    __shared__ double s_ss[NC][PG_WAVES];
    const int     lane = threadIdx.x & 63;
    const int     wv   = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: row bases in SGPRs
    const int64_t gw   = (int64_t) blockIdx.x * PG_WAVES + wv;
    const int64_t TW   = (int64_t) gridDim.x * PG_WAVES;
    const int     K    = a.K;
    // 1. activations: chunk j of thread t holds elements e = 4 t + 4096 j ..
    // e + 3 (a 32-block is 8 adjacent lanes); past K re-read the row's end
    float4_t xv[J][NC], xw[J][PRO == PRO_NORM ? 1 : NC];
#pragma unroll
    for (int j = 0; j < J; j++) {
        const unsigned e = min(4u * threadIdx.x + 256u * PG_WAVES * j, (unsigned) K - 4u);
#pragma unroll
        for (int c = 0; c < NC; c++) {
            xv[j][c] = *(const float4_t *) (a.x + c * a.ldx + e);
            if constexpr (PRO == PRO_SWIGLU) {
                xw[j][c] = *(const float4_t *) (a.u + c * a.ldu + e);
            }
        }
        if constexpr (PRO == PRO_NORM) {
            xw[j][0] = *(const float4_t *) (a.nw + e);
        }
    }
    // 2. the first weight rows, unconditionally (a row past N re-reads row
    // N - 1 and is not stored); a long row's last chunks after the prologue,
    // whose activation values would not fit in registers beside them
    constexpr int      PRE = DB ? CH : 8;
    PgBuf<CH>          ba;
    PgBuf<DB ? CH : 1> bb;
    pg_load<CH, 0, PRE>(ba, a, gw, lane);
    if constexpr (DB) {
        // the second row once the activations are in: a load returns behind
        // every request the chip has queued before it, so the weights issued
        // ahead of the activations delay them
#pragma unroll
        for (int j = 0; j < J; j++) {
#pragma unroll
            for (int c = 0; c < NC; c++) {
                asm volatile("" ::"v"(xv[j][c][0]), "v"(xw[j][PRO == PRO_NORM ? 0 : c][0]) : "memory");
            }
        }
        pg_load<CH>(bb, a, TW + gw, lane);
    }
    // 3. the activation values, quantised into LDS
    pg_prologue<NC, J, MAXK, PRO>(xv, xw, s_q, s_d, s_ss, a, lane, wv, K);
    if constexpr (PRE < CH) {
        pg_load<CH, PRE, CH>(ba, a, gw, lane);
    }
    __syncthreads();
    // 4. stream the rows
    const int nit = a.nit;
    if constexpr (DB) {
        // reduce one buffer while the other's loads fly; the steady-state
        // loads are unconditional so that each reduction waits for its own
        int it = 0;
        for (; it + 2 < nit; it += 2) {
            pg_dot<NC, CH>(ba, s_q, s_d, 0, a, lane, it * TW + gw);
            pg_load<CH>(ba, a, (it + 2) * TW + gw, lane);
            pg_dot<NC, CH>(bb, s_q, s_d, 0, a, lane, (it + 1) * TW + gw);
            pg_load<CH>(bb, a, (it + 3) * TW + gw, lane);
        }
        pg_dot<NC, CH>(ba, s_q, s_d, 0, a, lane, it * TW + gw);
        if (it + 1 < nit) {
            pg_dot<NC, CH>(bb, s_q, s_d, 0, a, lane, (it + 1) * TW + gw);
        }
    } else {
        // one buffer (a long row fills the registers): load the next row
        // after reducing the current one
        for (int it = 0;;) {
            int off = 0;
            asm volatile("" : "+v"(off));  // the LDS rows are re-read per row
            pg_dot<NC, CH>(ba, s_q, s_d, off, a, lane, it * TW + gw);
            if (++it >= nit) {
                break;
            }
            pg_load<CH>(ba, a, it * TW + gw, lane);
        }
    }
}

// Persistent Q6_K GEMVs with the same prologues, the activation rows
// quantised to Q8_K (super-blocks of 256 with 16-element sums) into LDS.
// A row is read in units of 64 elements as k_gemv_q6_K reads it: lane l owns
// units l + 64 u (u < CH), unit un covering elements eb + 32 t + 0..15
// (t < 4, eb = 256 sb + 128 h + l0 with sb = un / 4, h = un / 2 % 2, l0 =
// 16 (un % 2)) from 16 bytes of ql at 128 sb + 64 h + l0 and + 32, 16 bytes of
// qh at K/2 + 64 sb + 32 h + l0, the half's 8 scales and the super-block's d;
// the row is planar (ql, qh, scales, d), as the backend stores Q6_K.  Each
// lane adds its units in u order and the sums are reduced as store_rows
// reduces them, so the result is k_gemv_q6_K's to the bit.
template <int CH> struct Pg6Buf {
    int4_t   ql0[CH], ql1[CH], qh[CH];
    uint2    sc[CH];
    uint16_t d[CH];
};

template <int CH, int U0 = 0, int U1 = CH>
__device__ __forceinline__ void pg6_load(Pg6Buf<CH> & b, const PgArgs & a, int64_t row, int lane) {
    const uint8_t *              wr = a.W + (row < a.N ? row : a.N - 1) * a.rs;
    const int                    K  = a.K;
    const __amdgpu_buffer_rsrc_t rr =
        __builtin_amdgcn_make_buffer_rsrc((void *) wr, (short) 0, K / 2 + K / 4 + K / 16 + K / 128, 0x00020000);
    // unit lane + 64 u sits 16 super-blocks after unit lane: its offsets are
    // the lane's plus constants (the units past the row read other bytes of
    // the row, or zeros past its end, and are weighted by zero)
    const int sb = lane >> 2, h = (lane >> 1) & 1, l0 = (lane & 1) * 16;
    const int oql = sb * 128 + h * 64 + l0;
    const int oqh = sb * 64 + h * 32 + l0;
    const int osc = sb * 16 + h * 8;
    const int od  = 2 * sb;
#pragma unroll
    for (int u = U0; u < U1; u++) {
        b.ql0[u] = __builtin_bit_cast(int4_t, __builtin_amdgcn_raw_buffer_load_b128(rr, oql + 2048 * u, 0, 0));
        b.ql1[u] = __builtin_bit_cast(int4_t, __builtin_amdgcn_raw_buffer_load_b128(rr, oql + 2048 * u + 32, 0, 0));
        b.qh[u]  = __builtin_bit_cast(int4_t, __builtin_amdgcn_raw_buffer_load_b128(rr, oqh + 1024 * u, K / 2, 0));
        b.sc[u]  = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rr, osc + 256 * u, K / 2 + K / 4, 0));
        b.d[u]   = __builtin_amdgcn_raw_buffer_load_b16(rr, od + 32 * u, K / 2 + K / 4 + K / 16, 0);
    }
}

// The activation operands of one unit: 4 x 16 values, their 16-element sums
// and the super-block scale, per column
template <int NC> struct Pg6X {
    int4_t v[NC][4];
    int    bs[NC][4];
    float  d[NC];
};

template <int NC, int MAXK>
__device__ __forceinline__ void pg6_x(Pg6X<NC> & x, const int8_t * sq, const float * sd, const int16_t * sb16, int un) {
    const int sb = un >> 2, h = (un >> 1) & 1, l0 = (un & 1) * 16;
    const int eb = sb * 256 + h * 128 + l0;
    const int g0 = sb * 16 + h * 8 + (l0 >> 4);
#pragma unroll
    for (int c = 0; c < NC; c++) {
#pragma unroll
        for (int t = 0; t < 4; t++) {
            x.v[c][t]  = *(const int4_t *) &sq[c * MAXK + q8k_swz(eb + 32 * t)];
            x.bs[c][t] = sb16[c * (MAXK / 16) + g0 + 2 * t];
        }
        x.d[c] = sd[c * (MAXK / 256) + sb];
    }
}

// the 6-bit values and scales of one unit (k_gemv_q6_K's unpacking)
template <int CH>
__device__ __forceinline__ void pg6_decode(const Pg6Buf<CH> & b, int u, int un, bool ok, int4_t (&q)[4], int (&sc)[4],
                                           float & dw) {
    const int l0 = (un & 1) * 16;
    dw           = ok ? h2f(b.d[u]) : 0.0f;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int4_t src = (t & 1) ? b.ql1[u] : b.ql0[u];
        const int    sh  = (t < 2) ? 0 : 4;
        q[t].x = ((src.x >> sh) & 0x0F0F0F0F) | (((b.qh[u].x >> (2 * t)) & 0x03030303) << 4);
        q[t].y = ((src.y >> sh) & 0x0F0F0F0F) | (((b.qh[u].y >> (2 * t)) & 0x03030303) << 4);
        q[t].z = ((src.z >> sh) & 0x0F0F0F0F) | (((b.qh[u].z >> (2 * t)) & 0x03030303) << 4);
        q[t].w = ((src.w >> sh) & 0x0F0F0F0F) | (((b.qh[u].w >> (2 * t)) & 0x03030303) << 4);
        const int      bi = (l0 >> 4) + 2 * t;
        const uint32_t wd = bi < 4 ? b.sc[u].x : b.sc[u].y;
        sc[t]             = (int) (int8_t) ((wd >> (8 * (bi & 3))) & 0xff);
    }
}

// column c's share of one unit (k_gemv_q6_K's arithmetic)
template <int NC>
__device__ __forceinline__ void pg6_col(const int4_t (&q)[4], const int (&sc)[4], float dw, const int4_t (&xv)[4],
                                        const int (&bs)[4], float dx, float & acc) {
    int isum = 0;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        isum += sc[t] * (dot16(q[t], xv[t]) - 32 * bs[t]);
    }
    acc += (dw * dx) * (float) isum;
}

template <int NC, int CH>
__device__ __forceinline__ void pg6_unit(const Pg6Buf<CH> & b, int u, const Pg6X<NC> & x, bool ok, int un,
                                         float (&acc)[1][NC]) {
    int4_t q[4];
    int    sc[4];
    float  dw;
    pg6_decode<CH>(b, u, un, ok, q, sc, dw);
#pragma unroll
    for (int c = 0; c < NC; c++) {
        pg6_col<NC>(q, sc, dw, x.v[c], x.bs[c], x.d[c], acc[0][c]);
    }
}

// PRO_NORM / PRO_SWIGLU as k_gemv_q8_0_pro; PRO_NONE: the Q8_K activation
// rows (qs, d, bsums) are copied into LDS instead.  CH = 1 (K <= 4096): a
// lane's activation operands are the same for every row and stay in
// registers, two rows in flight per wave; CH > 1: one row in flight, the
// operands read from LDS per unit.
constexpr int PRO_NONE = 2;

struct Pg6Act {
    const int8_t *  qs;  // PRO_NONE: [NC][K]
    const float *   d;   // [NC][K / 256]
    const int16_t * bs;  // [NC][K / 16]
};

template <int NC, int CH, int PRO>
__global__ __launch_bounds__(64 * PG_WAVES) void k_gemv_q6_K_pro(PgArgs a, Pg6Act xa) {
    constexpr int  MAXK = 4096 * CH;
    constexpr int  J    = MAXK / (256 * PG_WAVES);
    constexpr bool DB   = CH == 1;
    constexpr int  NW   = PRO == PRO_NORM ? 1 : NC;
    __shared__ __attribute__((aligned(16))) int8_t s_q[NC * MAXK];
    __shared__ float   s_d[NC * MAXK / 256];
    __shared__ int16_t s_bs[NC * MAXK / 16];
    __shared__ double  s_ss[NC][PG_WAVES];
    const int     lane  = threadIdx.x & 63;
    const int     wv    = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t gw    = (int64_t) blockIdx.x * PG_WAVES + wv;
    const int64_t TW    = (int64_t) gridDim.x * PG_WAVES;
    const int     K     = a.K;
    const int     units = K / 64;
    // 1. activations (or the quantised rows), then the first weight rows
    float4_t xv[J][NC], xw[J][NW];
    if constexpr (PRO != PRO_NONE) {
#pragma unroll
        for (int j = 0; j < J; j++) {
            const unsigned e = min(4u * threadIdx.x + 256u * PG_WAVES * j, (unsigned) K - 4u);
#pragma unroll
            for (int c = 0; c < NC; c++) {
                xv[j][c] = *(const float4_t *) (a.x + c * a.ldx + e);
                if constexpr (PRO == PRO_SWIGLU) {
                    xw[j][c] = *(const float4_t *) (a.u + c * a.ldu + e);
                }
            }
            if constexpr (PRO == PRO_NORM) {
                xw[j][0] = *(const float4_t *) (a.nw + e);
            }
        }
    } else {
        // int8 values 16 per thread per step, then the scales and sums
        for (int i = threadIdx.x; i < NC * K / 16; i += 64 * PG_WAVES) {
            const int c = i / (K / 16), o = i % (K / 16);
            *(int4_t *) &s_q[c * MAXK + q8k_swz(16 * o)] = *(const int4_t *) (xa.qs + (int64_t) c * K + 16 * o);
            s_bs[c * (MAXK / 16) + o]          = xa.bs[(int64_t) c * (K / 16) + o];
        }
        for (int i = threadIdx.x; i < NC * K / 256; i += 64 * PG_WAVES) {
            const int c = i / (K / 256), o = i % (K / 256);
            s_d[c * (MAXK / 256) + o] = xa.d[(int64_t) c * (K / 256) + o];
        }
    }
    // a long row: its first unit ahead of an f32 prologue, the rest after it
    // (the activation values would not fit in registers beside them); the
    // whole row ahead of a copy of quantised rows
    constexpr int       PRE = DB || PRO == PRO_NONE ? CH : 1;
    Pg6Buf<CH>          ba;
    Pg6Buf<DB ? CH : 1> bb;
    pg6_load<CH, 0, PRE>(ba, a, gw, lane);
    if constexpr (DB) {
        if constexpr (PRO != PRO_NONE) {
#pragma unroll
            for (int j = 0; j < J; j++) {
#pragma unroll
                for (int c = 0; c < NC; c++) {
                    asm volatile("" ::"v"(xv[j][c][0]), "v"(xw[j][PRO == PRO_NORM ? 0 : c][0]) : "memory");
                }
            }
        }
        pg6_load<CH>(bb, a, TW + gw, lane);
    }
    // 2. the activation values, quantised into LDS
    if constexpr (PRO != PRO_NONE) {
        pg_prologue<NC, J, MAXK, PRO, TYPE_Q8_K>(xv, xw, s_q, s_d, s_ss, a, lane, wv, K, s_bs);
    }
    if constexpr (PRE < CH) {
        pg6_load<CH, PRE, CH>(ba, a, gw, lane);
    }
    __syncthreads();
    // 3. stream the rows
    const int nit = a.nit;
    if constexpr (DB) {
        const bool ok = lane < units;
        const int  un = ok ? lane : 0;
        Pg6X<NC>   x;
        pg6_x<NC, MAXK>(x, s_q, s_d, s_bs, un);
        auto dot = [&](const Pg6Buf<CH> & b, int64_t row) {
            float acc[1][NC];
#pragma unroll
            for (int c = 0; c < NC; c++) {
                acc[0][c] = 0.0f;
            }
            pg6_unit<NC, CH>(b, 0, x, ok, un, acc);
            store_rows<NC, 1>(acc, lane, row, a.N, a.y, a.ldy, a.res, a.ldr);
        };
        int it = 0;
        for (; it + 2 < nit; it += 2) {
            dot(ba, it * TW + gw);
            pg6_load<CH>(ba, a, (it + 2) * TW + gw, lane);
            dot(bb, (it + 1) * TW + gw);
            pg6_load<CH>(bb, a, (it + 3) * TW + gw, lane);
        }
        dot(ba, it * TW + gw);
        if (it + 1 < nit) {
            dot(bb, (it + 1) * TW + gw);
        }
    } else {
        // one buffer: the next row's loads after the current row is
        // reduced (N = 4096 rows over 4096 waves: one row each); the
        // activation operands one column at a time from LDS
        for (int it = 0;;) {
            float acc[1][NC];
#pragma unroll
            for (int c = 0; c < NC; c++) {
                acc[0][c] = 0.0f;
            }
#pragma unroll
            for (int u = 0; u < CH; u++) {
                const bool ok = lane + 64 * u < units;
                const int  un = ok ? lane + 64 * u : 0;
                int4_t     q[4];
                int        sc[4];
                float      dw;
                pg6_decode<CH>(ba, u, un, ok, q, sc, dw);
                const int sb = un >> 2, h = (un >> 1) & 1, l0 = (un & 1) * 16;
                const int eb = sb * 256 + h * 128 + l0;
                const int g0 = sb * 16 + h * 8 + (l0 >> 4);
#pragma unroll
                for (int c = 0; c < NC; c++) {
                    int4_t xv[4];
                    int    bs[4];
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        xv[t] = *(const int4_t *) &s_q[c * MAXK + q8k_swz(eb + 32 * t)];
                        bs[t] = s_bs[c * (MAXK / 16) + g0 + 2 * t];
                    }
                    pg6_col<NC>(q, sc, dw, xv, bs, s_d[c * (MAXK / 256) + sb], acc[0][c]);
                    __builtin_amdgcn_sched_barrier(0);  // bounds the LDS operands in flight (registers)
                }
            }
            store_rows<NC, 1>(acc, lane, it * TW + gw, a.N, a.y, a.ldy, a.res, a.ldr);
            if (++it >= nit) {
                break;
            }
            pg6_load<CH>(ba, a, it * TW + gw, lane);
        }
    }
}

// Persistent Q4_K / Q5_K GEMVs (M <= 2, K = 4096 CH) with the structure of
// k_gemv_q6_K_pro: PRO_NORM (the RMS norm and the Q8_K quantisation of the
// activation rows in the prologue) or PRO_NONE (a copy of quantised Q8_K
// rows into LDS).  A row is read in units of 64 elements: unit un = lane +
// 64 u of super-block sb = un / 4 takes the chunk pair c = 2 cp, 2 cp + 1
// (cp = un / 2 % 2) and the column half hf = un % 2, i.e. for each of the two
// chunks the 16 low-nibble elements 256 sb + 64 c + 16 hf + i and the 16
// high-nibble ones 32 further.  Its bytes: 32 of qs at 128 sb + 64 cp + 16 hf
// (and + 32), Q5: the 16 qh bytes K/2 + 32 sb + 16 hf (bits 2c and 2c + 1 of
// byte i are the fifth bits of the low and high nibble), the super-block's 12
// scale bytes and its f16 d, dmin.  Per unit and column ggml's super-block
// form: the integer sums of the four 16-element groups, then
// acc += (d dx) isum - (dmin dx) msum; the lane sums reduce as store_rows
// reduces them.
template <int CH, bool Q5> struct Pg5Buf {
    int4_t   q0[CH], q1[CH];
    int4_t   qh[Q5 ? CH : 1];
    uint32_t s0[CH], s1[CH], s2[CH], dm[CH];
};

typedef uint32_t u32x3_t __attribute__((ext_vector_type(3)));

template <int CH, bool Q5, int U0 = 0, int U1 = CH>
__device__ __forceinline__ void pg5_load(Pg5Buf<CH, Q5> & b, const PgArgs & a, int64_t row, int lane) {
    const uint8_t *              wr    = a.W + (row < a.N ? row : a.N - 1) * a.rs;
    const int                    K     = a.K;
    const int                    qh_sz = Q5 ? K / 8 : 0;
    const int                    sc_at = K / 2 + qh_sz;
    const int                    dm_at = sc_at + 12 * (K / 256);
    const __amdgpu_buffer_rsrc_t rr    = __builtin_amdgcn_make_buffer_rsrc((void *) wr, (short) 0,
                                                                           dm_at + 4 * (K / 256), 0x00020000);
    // unit lane + 64 u sits 16 super-blocks after unit lane: its offsets are
    // the lane's plus constants
    const int sb = lane >> 2, cp = (lane >> 1) & 1, hf = lane & 1;
    const int oq = sb * 128 + cp * 64 + hf * 16;
    const int oh = sb * 32 + hf * 16;
#pragma unroll
    for (int u = U0; u < U1; u++) {
        b.q0[u] = __builtin_bit_cast(int4_t, __builtin_amdgcn_raw_buffer_load_b128(rr, oq + 2048 * u, 0, 0));
        b.q1[u] = __builtin_bit_cast(int4_t, __builtin_amdgcn_raw_buffer_load_b128(rr, oq + 2048 * u + 32, 0, 0));
        if constexpr (Q5) {
            b.qh[u] = __builtin_bit_cast(int4_t, __builtin_amdgcn_raw_buffer_load_b128(rr, oh + 512 * u, K / 2, 0));
        }
        const u32x3_t sc = __builtin_bit_cast(u32x3_t,
                                              __builtin_amdgcn_raw_buffer_load_b96(rr, sb * 12 + 192 * u, sc_at, 0));
        b.s0[u] = sc.x;
        b.s1[u] = sc.y;
        b.s2[u] = sc.z;
        b.dm[u] = __builtin_amdgcn_raw_buffer_load_b32(rr, sb * 4 + 64 * u, dm_at, 0);
    }
}

// The activation operands of one unit: the four 16-value groups (chunk 2cp
// low, high, chunk 2cp + 1 low, high), their sums and the super-block scale
template <int NC> struct Pg5X {
    int4_t v[NC][4];
    int    bs[NC][4];
    float  d[NC];
};

template <int NC, int MAXK>
__device__ __forceinline__ void pg5_x(Pg5X<NC> & x, const int8_t * sq, const float * sd, const int16_t * sb16, int un) {
    const int sb = un >> 2, cp = (un >> 1) & 1, hf = un & 1;
#pragma unroll
    for (int c = 0; c < NC; c++) {
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int e = sb * 256 + (2 * cp + (t >> 1)) * 64 + 32 * (t & 1) + 16 * hf;
            x.v[c][t]   = *(const int4_t *) &sq[c * MAXK + q8k_swz(e)];
            x.bs[c][t]  = sb16[c * (MAXK / 16) + (e >> 4)];
        }
        x.d[c] = sd[c * (MAXK / 256) + sb];
    }
}

// the 4- / 5-bit values of one unit's four groups and their (scale, min):
// pairs j = 4 cp + t, t < 4 (q4k_scale_min_w's fields, computed for both
// halves of the scales and selected by the lane's cp without a branch)
template <int CH, bool Q5>
__device__ __forceinline__ void pg5_decode(const Pg5Buf<CH, Q5> & b, int u, int cp, int4_t (&q)[4], int (&sc)[4],
                                           int (&mn)[4], float & d, float & dmin) {
    const uint32_t w0 = b.s0[u], w1 = b.s1[u], w2 = b.s2[u];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int      lo_sc = (int) ((w0 >> (8 * t)) & 63);
        const int      lo_mn = (int) ((w1 >> (8 * t)) & 63);
        const uint32_t b8    = (w2 >> (8 * t)) & 0xff;
        const int      hi_sc = (int) ((b8 & 0x0f) | (((w0 >> (8 * t + 6)) & 3) << 4));
        const int      hi_mn = (int) ((b8 >> 4) | (((w1 >> (8 * t + 6)) & 3) << 4));
        sc[t]                = cp ? hi_sc : lo_sc;
        mn[t]                = cp ? hi_mn : lo_mn;
    }
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int4_t w = k ? b.q1[u] : b.q0[u];
        const int    c = 2 * cp + k;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int lo = w[i] & 0x0F0F0F0F;
            int hi = (w[i] >> 4) & 0x0F0F0F0F;
            if constexpr (Q5) {
                lo |= ((b.qh[u][i] >> (2 * c)) & 0x01010101) << 4;
                hi |= ((b.qh[u][i] >> (2 * c + 1)) & 0x01010101) << 4;
            }
            q[2 * k][i]     = lo;
            q[2 * k + 1][i] = hi;
        }
    }
    d    = h2f((uint16_t) (b.dm[u] & 0xffff));
    dmin = h2f((uint16_t) (b.dm[u] >> 16));
}

// column c's share of one unit
__device__ __forceinline__ void pg5_col(const int4_t (&q)[4], const int (&sc)[4], const int (&mn)[4], float d,
                                        float dmin, const int4_t (&xv)[4], const int (&bs)[4], float dx, float & acc) {
    int isum = 0, msum = 0;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        isum += sc[t] * dot16(q[t], xv[t]);
        msum += mn[t] * bs[t];
    }
    acc += (d * dx) * (float) isum - (dmin * dx) * (float) msum;
}

template <int NC, int CH, int PRO, bool Q5>
__global__ __launch_bounds__(64 * PG_WAVES) void k_gemv_q45_K_pro(PgArgs a, Pg6Act xa) {
    static_assert(PRO == PRO_NORM || PRO == PRO_NONE, "Q4_K / Q5_K: norm or quantised-row prologue");
    constexpr int  MAXK = 4096 * CH;
    constexpr int  J    = MAXK / (256 * PG_WAVES);
    constexpr bool DB   = CH == 1;
    __shared__ __attribute__((aligned(16))) int8_t s_q[NC * MAXK];
    __shared__ float   s_d[NC * MAXK / 256];
    __shared__ int16_t s_bs[NC * MAXK / 16];
    __shared__ double  s_ss[NC][PG_WAVES];
    const int     lane = threadIdx.x & 63;
    const int     wv   = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t gw   = (int64_t) blockIdx.x * PG_WAVES + wv;
    const int64_t TW   = (int64_t) gridDim.x * PG_WAVES;
    const int     K    = a.K;
    // 1. activations (or the quantised rows), then the first weight rows
    float4_t xv[J][NC], xw[J][1];
    if constexpr (PRO == PRO_NORM) {
#pragma unroll
        for (int j = 0; j < J; j++) {
            const unsigned e = min(4u * threadIdx.x + 256u * PG_WAVES * j, (unsigned) K - 4u);
#pragma unroll
            for (int c = 0; c < NC; c++) {
                xv[j][c] = *(const float4_t *) (a.x + c * a.ldx + e);
            }
            xw[j][0] = *(const float4_t *) (a.nw + e);
        }
    } else {
        for (int i = threadIdx.x; i < NC * K / 16; i += 64 * PG_WAVES) {
            const int c = i / (K / 16), o = i % (K / 16);
            *(int4_t *) &s_q[c * MAXK + q8k_swz(16 * o)] = *(const int4_t *) (xa.qs + (int64_t) c * K + 16 * o);
            s_bs[c * (MAXK / 16) + o]                    = xa.bs[(int64_t) c * (K / 16) + o];
        }
        for (int i = threadIdx.x; i < NC * K / 256; i += 64 * PG_WAVES) {
            const int c = i / (K / 256), o = i % (K / 256);
            s_d[c * (MAXK / 256) + o] = xa.d[(int64_t) c * (K / 256) + o];
        }
    }
    Pg5Buf<CH, Q5>          ba;
    Pg5Buf<DB ? CH : 1, Q5> bb;
    pg5_load<CH, Q5>(ba, a, gw, lane);
    if constexpr (DB) {
        if constexpr (PRO == PRO_NORM) {
            // the second row once the activations are in (loads return in order)
#pragma unroll
            for (int j = 0; j < J; j++) {
#pragma unroll
                for (int c = 0; c < NC; c++) {
                    asm volatile("" ::"v"(xv[j][c][0]), "v"(xw[j][0][0]) : "memory");
                }
            }
        }
        pg5_load<CH, Q5>(bb, a, TW + gw, lane);
    }
    // 2. the activation values, quantised into LDS
    if constexpr (PRO == PRO_NORM) {
        pg_prologue<NC, J, MAXK, PRO, TYPE_Q8_K>(xv, xw, s_q, s_d, s_ss, a, lane, wv, K, s_bs);
    }
    __syncthreads();
    // 3. stream the rows
    const int nit = a.nit;
    const int cp  = (lane >> 1) & 1;
    if constexpr (DB) {
        Pg5X<NC> x;
        pg5_x<NC, MAXK>(x, s_q, s_d, s_bs, lane);
        auto dot = [&](const Pg5Buf<CH, Q5> & b, int64_t row) {
            float acc[1][NC];
            int4_t q[4];
            int    sc[4], mn[4];
            float  d, dmin;
            pg5_decode<CH, Q5>(b, 0, cp, q, sc, mn, d, dmin);
#pragma unroll
            for (int c = 0; c < NC; c++) {
                acc[0][c] = 0.0f;
                pg5_col(q, sc, mn, d, dmin, x.v[c], x.bs[c], x.d[c], acc[0][c]);
            }
            store_rows<NC, 1>(acc, lane, row, a.N, a.y, a.ldy, a.res, a.ldr);
        };
        int it = 0;
        for (; it + 2 < nit; it += 2) {
            dot(ba, it * TW + gw);
            pg5_load<CH, Q5>(ba, a, (it + 2) * TW + gw, lane);
            dot(bb, (it + 1) * TW + gw);
            pg5_load<CH, Q5>(bb, a, (it + 3) * TW + gw, lane);
        }
        dot(ba, it * TW + gw);
        if (it + 1 < nit) {
            dot(bb, (it + 1) * TW + gw);
        }
    } else {
        // one buffer: the next row's loads after the current row is reduced;
        // the activation operands one column at a time from LDS (an opaque
        // zero added to their indices keeps the reads inside the row loop:
        // hoisted, they would not fit in registers beside the row)
        for (int it = 0;;) {
            float acc[1][NC];
#pragma unroll
            for (int c = 0; c < NC; c++) {
                acc[0][c] = 0.0f;
            }
            int off = 0;
            asm volatile("" : "+v"(off));
#pragma unroll
            for (int u = 0; u < CH; u++) {
                int4_t q[4];
                int    sc[4], mn[4];
                float  d, dmin;
                pg5_decode<CH, Q5>(ba, u, cp, q, sc, mn, d, dmin);
#pragma unroll
                for (int c = 0; c < NC; c++) {
                    Pg5X<1> x;
                    pg5_x<1, MAXK>(x, s_q + c * MAXK + off, s_d + c * (MAXK / 256) + off, s_bs + c * (MAXK / 16) + off,
                                   lane + 64 * u);
                    pg5_col(q, sc, mn, d, dmin, x.v[0], x.bs[0], x.d[0], acc[0][c]);
                    __builtin_amdgcn_sched_barrier(0);  // bounds the LDS operands in flight (registers)
                }
            }
            store_rows<NC, 1>(acc, lane, it * TW + gw, a.N, a.y, a.ldy, a.res, a.ldr);
            if (++it >= nit) {
                break;
            }
            pg5_load<CH, Q5>(ba, a, it * TW + gw, lane);
        }
    }
}

// MUL_MAT of Q8_0 weights against 9..16 activation columns already
// quantised (the depth decoder's projections at S x CFG = 16 tokens,
// src/depth-decoder.h:206-257): one 16-wave workgroup per CU copies the
// columns' int8 values and block scales into LDS once (columns past ncv as
// zeros), then streams the weight rows as k_gemv_q8_0_pro does, each byte
// read once in the grid, and dots each row against all 16 columns.  Sums
// and the residual ADD as store_rows<16, 1>; only the ncv real columns are
// stored.
template <int CH>
__global__ __launch_bounds__(64 * PG_WAVES) void k_gemv_q8_0_wide(PgArgs a, const int8_t * __restrict__ xq,
                                                                   const float * __restrict__ xd, int ncv) {
    constexpr int  NC   = 16;
    constexpr int  MAXK = 1024 * CH;
    constexpr bool DB   = CH <= 4;
    extern __shared__ __attribute__((aligned(16))) int8_t g_wide[];
    int8_t *      s_q  = g_wide;                        // [NC][MAXK]
    float *       s_d  = (float *) (g_wide + NC * MAXK);  // [NC][MAXK / 32]
    const int     lane = threadIdx.x & 63;
    const int     wv   = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t gw   = (int64_t) blockIdx.x * PG_WAVES + wv;
    const int64_t TW   = (int64_t) gridDim.x * PG_WAVES;
    const int     K    = a.K;
    // the first rows in flight while the columns are copied
    PgBuf<CH>          ba;
    PgBuf<DB ? CH : 1> bb;
    pg_load<CH>(ba, a, gw, lane);
    if constexpr (DB) {
        pg_load<CH>(bb, a, TW + gw, lane);
    }
    for (int i = threadIdx.x; i < NC * (MAXK / 16); i += 64 * PG_WAVES) {
        const int c = i / (MAXK / 16), e = (i % (MAXK / 16)) * 16;
        int4_t    v = { 0, 0, 0, 0 };
        if (c < ncv && e < K) {
            v = *(const int4_t *) (xq + (int64_t) c * K + e);
        }
        *(int4_t *) (s_q + c * MAXK + e) = v;
    }
    for (int i = threadIdx.x; i < NC * (MAXK / 32); i += 64 * PG_WAVES) {
        const int c = i / (MAXK / 32), b = i % (MAXK / 32);
        s_d[i]      = c < ncv && b < K / 32 ? xd[(int64_t) c * (K / 32) + b] : 0.0f;
    }
    __syncthreads();
    // the 16 waves' rows of one iteration (16 consecutive rows) x 16 columns
    // are staged in LDS and stored by 256 threads, 16 consecutive rows (64
    // bytes) per column: single-float stores to 16 output rows per wave had
    // their lines evicted by the weight stream and written back per store
    __shared__ float s_out[2][NC][PG_WAVES];
    auto dot_stage = [&](const auto & buf, int off, int par) {
        // pg_acc's arithmetic, with the LDS reads bounded to 4 columns at a time
        // (16 columns' operands do not fit in registers beside the row buffers)
        float v[NC];
#pragma unroll
        for (int c = 0; c < NC; c++) {
            v[c] = 0.0f;
        }
#pragma unroll
        for (int u = 0; u < CH; u++) {
            const int   o  = min(1024 * u + lane * 16, K - 16);
            const bool  ok = 1024 * u + lane * 16 < K;
            const float dw = ok ? h2f(buf.s[u]) : 0.0f;
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const int4_t xq = *(const int4_t *) &s_q[c * MAXK + o + off];
                const float  dx = s_d[c * (MAXK / 32) + (o >> 5) + off];
                v[c] += (float) dot16(buf.w[u], xq) * (dw * dx);
                if (c % 4 == 3) {
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
        const float total = wave_reduce_scatter<NC>(v, lane);
        const int   c     = reduce_index<NC>(lane);
        if ((lane & ((64 / NC) - 1)) == 0) {
            s_out[par][c][wv] = total;
        }
    };
    // rows it TW + 16 blockIdx.x + 0..15, columns < ncv (the residual ADD here)
    auto flush = [&](int it) {
        __syncthreads();
        if (threadIdx.x < NC * PG_WAVES) {
            const int     c   = threadIdx.x / PG_WAVES, r = threadIdx.x % PG_WAVES;
            const int64_t row = (int64_t) it * TW + (int64_t) blockIdx.x * PG_WAVES + r;
            if (c < ncv && row < a.N) {
                const float t        = s_out[it & 1][c][r];
                a.y[c * a.ldy + row] = a.res ? t + a.res[c * a.ldr + row] : t;
            }
        }
    };
    const int nit = a.nit;
    if constexpr (DB) {
        for (int it = 0; it < nit; it += 2) {
            dot_stage(ba, 0, 0);
            if (it + 2 < nit) {
                pg_load<CH>(ba, a, (it + 2) * TW + gw, lane);
            }
            flush(it);
            if (it + 1 < nit) {
                dot_stage(bb, 0, 1);
                if (it + 3 < nit) {
                    pg_load<CH>(bb, a, (it + 3) * TW + gw, lane);
                }
                flush(it + 1);
            }
        }
    } else {
        for (int it = 0;;) {
            int off = 0;
            asm volatile("" : "+v"(off));  // the LDS rows are re-read per row
            dot_stage(ba, off, it & 1);
            if (it + 1 < nit) {
                pg_load<CH>(ba, a, (it + 1) * TW + gw, lane);
            }
            flush(it);
            if (++it >= nit) {
                break;
            }
        }
    }
}

// MUL_MAT of Q8_0 weights against 3..16 quantised activation columns on the
// int8 MFMA (the depth decoder's projections at S x CFG tokens,
// src/depth-decoder.h:206-257).  One 16-wave workgroup per CU copies the 16
// columns (past M: zeros) and their block scales into LDS once, then takes
// groups of 16 weight rows in turn, the 16 waves splitting each group's K
// in chunks of two Q8_0 block pairs; the next group's weight loads are in
// flight while the current one is computed.  Per pair, lane (r, q) (r =
// lane % 16, q = lane / 16) loads bytes 16 q .. 16 q + 15 of row r's 64 pair
// bytes; one v_permlane32_swap per dword turns the two halves into the B
// operands of the pair's two v_mfma_i32_16x16x32_i8 (one block each, so
// every block's integer sum is separate, as ggml's vec_dot): operand quad q'
// of either block holds block bytes QMAP[q'] .. + 7, and the activation (A)
// operand is read from LDS with the same map.  A lane's four sums are then
// columns 4 q + i of one weight row, so it loads that row's scales only.  Each block's exact int32 sums
// are scaled as ggml scales them, (float) isum * (d_w * d_x), and added in
// block order per wave; the waves' partial sums are added in wave order.
constexpr int MF_PC   = 2;   // block pairs per chunk
constexpr int MF_PAD  = 32;  // LDS pitch padding of an activation column (bank spread)

__device__ __forceinline__ int mf_qmap(int q) {
    return (q & 1) * 16 + (q >> 1) * 8;  // 0, 16, 8, 24
}

struct MfChunk {
    int4_t w[MF_PC];  // weight bytes of the lane's row, one 16-byte piece per pair
    uint2  sw;        // f16 scales of the lane's row, the chunk's 4 blocks
};
constexpr int MF_LOADS = MF_PC + 1;  // load instructions of mf_load (the DMA wait counts them)

struct MfArgs {
    const uint8_t * W;
    int64_t         N;
    int             K;
    int64_t         rs;
    const int8_t *  xq;  // [M][K]
    const float *   xd;  // [M][K / 32]
    int             M;
    float *         y;
    int64_t         ldy;
    const float *   res;
    int64_t         ldr;
};

// chunk starting at pair p0 of row group g: weight pieces and row scales
// (rows past N re-read row N - 1; chunks past the wave's range are not
// loaded, their buffers not used)
__device__ __forceinline__ void mf_load(MfChunk & b, const MfArgs & a, int64_t g, int p0, int r, int q) {
    const int64_t row0 = g * 16;
    const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
        (void *) (a.W + row0 * a.rs), (short) 0, (int) (min((int64_t) 16, a.N - row0) * a.rs), 0x00020000);
    const int      nr = (int) min((int64_t) 16, a.N - row0);
    const unsigned wo = (unsigned) (min(r, nr - 1) * (int) a.rs + 16 * q);
#pragma unroll
    for (int j = 0; j < MF_PC; j++) {
        const int p = min(p0 + j, (int) (a.K / 64) - 1);
        b.w[j]      = __builtin_bit_cast(int4_t, __builtin_amdgcn_raw_buffer_load_b128(rr, wo, 64 * p, 0));
    }
    // scales of blocks 2 p0 .. 2 p0 + 3 (8-byte aligned: p0 even, K % 256 == 0)
    const unsigned so = (unsigned) (min(r, nr - 1) * (int) a.rs + a.K);
    b.sw              = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rr, so, 4 * p0, 0));
}

// the chunk's four blocks against the LDS columns; pairs at or past pe add
// nothing (computed on a valid pair and not added: every register of the
// chunk is read on every path, so no path leaves its loads outstanding)
__device__ __forceinline__ void mf_acc(const MfChunk & b, const int8_t * s_x, const float * s_xd, int pitch,
                                       int nb, int p0, int pe, int lane, float (&acc)[4]) {
#pragma clang fp contract(off)
    const int c = lane & 15, q = lane >> 4;
#pragma unroll
    for (int j = 0; j < MF_PC; j++) {
        const bool use = p0 + j < pe;
        const int  p   = use ? p0 + j : 0;
        const auto lo = __builtin_amdgcn_permlane32_swap((unsigned) b.w[j].x, (unsigned) b.w[j].z, false, false);
        const auto hi = __builtin_amdgcn_permlane32_swap((unsigned) b.w[j].y, (unsigned) b.w[j].w, false, false);
        const long aa = (long) (((uint64_t) hi[0] << 32) | lo[0]);  // block 2 p
        const long ab = (long) (((uint64_t) hi[1] << 32) | lo[1]);  // block 2 p + 1
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int4_t z   = { 0, 0, 0, 0 };
            const uint2  xv  = *(const uint2 *) (s_x + c * pitch + 64 * p + 32 * h + mf_qmap(q));
            const long   bx  = (long) (((uint64_t) xv.y << 32) | xv.x);
            // D[column 4 q + i][row r]: the activations as the A operand,
            // the weights as B, so a lane's four sums share one weight row
            const int4_t   s   = __builtin_amdgcn_mfma_i32_16x16x32_i8(bx, h ? ab : aa, z, 0, 0, 0);
            const int      blk = 2 * j + h;  // block of the chunk
            const uint32_t wd  = blk >> 1 ? b.sw.y : b.sw.x;
            const float    dw  = h2f((uint16_t) (blk & 1 ? wd >> 16 : wd & 0xffff));
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float dx = s_xd[(4 * q + i) * nb + 2 * p + h];
                const float t  = acc[i] + (float) s[i] * (dw * dx);
                acc[i]         = use ? t : acc[i];
            }
        }
    }
}

// workgroup barrier ordering LDS accesses only (__syncthreads would also
// wait for the output stores and the weight loads in flight)
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int MAXC>  // chunks per wave and row group (K <= 16 waves x MAXC x MF_PC x 64)
__global__ __launch_bounds__(64 * PG_WAVES) void k_gemv_q8_0_mfma(MfArgs a) {
    extern __shared__ __attribute__((aligned(16))) int8_t g_mf[];
    const int pitch = a.K + MF_PAD;
    const int nb    = a.K / 32;
    int8_t *  s_x   = g_mf;                                           // [16][pitch]
    float *   s_xd  = (float *) (g_mf + 16 * pitch);                  // [16][nb]
    float *   s_pt  = s_xd + 16 * nb;                                 // [PG_WAVES][4][64]
    const int lane  = threadIdx.x & 63;
    const int wv    = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r     = lane & 15, q = lane >> 4;
    const int np    = a.K / 64;                                  // block pairs per row
    const int nch   = (np + MF_PC - 1) / MF_PC;                  // chunks per row, split over the waves
    const int cb    = wv * nch / PG_WAVES, ce = (wv + 1) * nch / PG_WAVES;
    const int pe    = min(ce * MF_PC, np);  // the wave's pairs: [cb MF_PC, pe)
    const int64_t ng = (a.N + 15) / 16;
    // 1. the M columns and their block scales DMA'd into LDS (global_load_lds,
    // issued first: they return first), 1 KB of a column or 64 scales per
    // instruction, instructions dealt round-robin to the waves; columns past
    // M are not written (their outputs are not stored)
    // (issued from inline asm, which the compiler does not track: its own
    // tracking would wait for the whole DMA, and every load after it, at
    // the barrier; this wave waits for its DMA itself below)
    const uint32_t lbase = (uint32_t) (uintptr_t) (__attribute__((address_space(3))) int8_t *) g_mf;
    const int      nxi = a.M * (a.K / 1024), nsi = (a.M * nb + 63) / 64;
    int            ndma = 0;
    for (int i = wv; i < nxi + nsi; i += PG_WAVES, ndma++) {
        if (i < nxi) {
            const int c = i / (a.K / 1024), u = i % (a.K / 1024);
            asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
                         ::"v"(a.xq + (int64_t) c * a.K + 1024 * u + 16 * lane), "s"(lbase + c * pitch + 1024 * u)
                         : "memory", "m0");
        } else {
            // the last instruction's lanes past M nb re-read the last scale and
            // land in the scales of column M (< 16 columns of room)
            const int e = min(64 * (i - nxi) + lane, a.M * nb - 1);
            asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off"
                         ::"v"(a.xd + e), "s"(lbase + 16 * pitch + 4 * 64 * (i - nxi)) : "memory", "m0");
        }
    }
    // 2. the first group's rows; every wave issues MAXC chunk loads per group
    // (a chunk past its range re-reads the row's last chunk and is not
    // used), so that the waits on them are the same on every path
    MfChunk ca[MAXC], cn[MAXC];
    int64_t g = blockIdx.x;
#pragma unroll
    for (int k = 0; k < MAXC; k++) {
        mf_load(ca[k], a, g, min(cb + k, nch - 1) * MF_PC, r, q);
    }
    // 3. this wave's DMA done (the row loads issued after it may still fly),
    // then every wave's
    if (ndma > 0) {
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(MAXC * MF_LOADS) : "memory");
    }
    __syncthreads();
    // one group: the next group's loads into nxt, the current from cur
    auto group = [&](MfChunk (&cur)[MAXC], MfChunk (&nxt)[MAXC], int64_t gc) {
        const int64_t gn = gc + gridDim.x;  // past the last group: the last group again
        // output (row lane % 16, column 4 (lane / 16) + i) of lane l and
        // register i is stored by thread t = 16 column + row (consecutive
        // rows per column); its residual is loaded first (loads return in
        // order: loaded after the next group's rows it would wait for them)
        const int     ocol = (int) (threadIdx.x >> 4) & 15, orr = threadIdx.x & 15;
        const int     ol = orr + 16 * (ocol >> 2), oi = ocol & 3;
        const int64_t orow = gc * 16 + orr;
        const bool    ost  = threadIdx.x < 256 && ocol < a.M && orow < a.N;
        const float   ores = ost && a.res ? a.res[ocol * a.ldr + orow] : 0.0f;
#pragma unroll
        for (int k = 0; k < MAXC; k++) {
            mf_load(nxt[k], a, min(gn, ng - 1), min(cb + k, nch - 1) * MF_PC, r, q);
        }
        __builtin_amdgcn_sched_barrier(0);  // the next group's loads issue before this group's arithmetic
        float acc[4] = { 0.0f, 0.0f, 0.0f, 0.0f };
#pragma unroll
        for (int k = 0; k < MAXC; k++) {
            mf_acc(cur[k], s_x, s_xd, pitch, nb, (cb + k) * MF_PC, pe, lane, acc);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            s_pt[(wv * 4 + i) * 64 + lane] = acc[i];
        }
        lds_barrier();
        if (threadIdx.x < 256) {
            float t = s_pt[oi * 64 + ol];
#pragma unroll
            for (int w = 1; w < PG_WAVES; w++) {
                t += s_pt[(w * 4 + oi) * 64 + ol];
            }
            if (ost) {
                a.y[ocol * a.ldy + orow] = a.res ? t + ores : t;
            }
        }
        lds_barrier();  // the partial sums are read before the next group writes them
    };
    // ping-pong between the two buffer sets (no register copies, which would
    // wait for the next group's loads)
    for (;;) {
        group(ca, cn, g);
        g += gridDim.x;
        if (g >= ng) {
            break;
        }
        group(cn, ca, g);
        g += gridDim.x;
        if (g >= ng) {
            break;
        }
    }
}

static int64_t pg_cus();

template <int MAXC> static int launch_mf(const MfArgs & a, hipStream_t stream) {
    const int64_t ng   = (a.N + 15) / 16;
    const int64_t wgs  = std::min<int64_t>(ng, pg_cus());
    const size_t  lds  = (size_t) 16 * (a.K + MF_PAD) + (size_t) 16 * (a.K / 32) * 4 + (size_t) PG_WAVES * 4 * 64 * 4;
    auto          kern = k_gemv_q8_0_mfma<MAXC>;
    if (lds > 64 * 1024 && !ensure_lds_limit((const void *) kern, lds)) {
        return set_error(MMHIP_ERR_HIP, "gemv (int8 MFMA): cannot raise LDS limit to %zu", lds);
    }
    hipLaunchKernelGGL(kern, dim3((unsigned) wgs), dim3(64 * PG_WAVES), lds, stream, a);
    return check_launch("gemv (int8 MFMA, 3-16 columns)");
}

// The MLP's gate_up GEMV with the RMS norm in its prologue (as
// k_gemv_q8_0_pro<PRO_NORM>) and the SwiGLU plus the down GEMV's Q8_0
// activation quantisation in its epilogue: the arithmetic of
// rms_norm_mul_mat followed by swiglu_quant, each SwiGLU value and each
// quantisation block computed once in the grid instead of once per CU in the
// down GEMV's prologue.  Workgroup w owns the Q8_0 blocks [w bpw, (w+1) bpw)
// of the F = N / 2 SwiGLU outputs; per block two units of 16 outputs, wave v
// taking output h = 32 block + 16 half + v, i.e. gate row h and up row F + h
// (swapped halves: F + h and h).  The two rows' sums are reduced as
// store_rows reduces them (same bits as the separate GEMV's y), the SwiGLU of
// each column goes to LDS, and once every unit is done the workgroup
// quantises its blocks, 8 lanes per (block, column) as quant_chunk256.
constexpr int GLU_MAXB = 8;  // blocks per workgroup

struct GluArgs {
    int64_t  F;        // SwiGLU width (N / 2)
    int      swapped;  // gate in the second half
    int      bpw;      // blocks per workgroup
    int8_t * qs;       // Q8_0 activations [NC][F]
    float *  qd;       // their scales [NC][F / 32]
    float *  h;        // optional f32 SwiGLU rows [NC][F]
};

// SwiGLU output of one unit from the gate and up rows' per-lane partial
// sums: each reduced as store_rows<NC, 1> reduces a row, the SwiGLU of
// column c stored at sh[32 c]
template <int NC>
__device__ __forceinline__ void glu_out(float (&ag)[1][NC], float (&au)[1][NC], int lane, float * sh) {
    float vg[NC], vu[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        vg[c] = ag[0][c];
        vu[c] = au[0][c];
    }
    const float g   = wave_reduce_scatter<NC>(vg, lane);
    const float u   = wave_reduce_scatter<NC>(vu, lane);
    const int   idx = reduce_index<NC>(lane);
    if ((lane & ((64 / NC) - 1)) == 0) {
#pragma clang fp contract(off)
        const float silu = g / (1.0f + expf(-g));
        sh[idx * 32]     = silu * u;
    }
}

template <int NC>
__global__ __launch_bounds__(64 * PG_WAVES) void k_gemv_q8_0_norm_glu(PgArgs a, GluArgs gl) {
    constexpr int CH   = 4;
    constexpr int MAXK = 1024 * CH;
    constexpr int J    = MAXK / (256 * PG_WAVES);
    __shared__ __attribute__((aligned(16))) int8_t s_q[NC * MAXK];
    __shared__ float  s_d[NC * MAXK / 32];
    __shared__ double s_ss[NC][PG_WAVES];
    __shared__ __attribute__((aligned(16))) float s_h[GLU_MAXB][NC][32];
    const int     lane = threadIdx.x & 63;
    const int     wv   = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int     K    = a.K;
    const int64_t nblk = gl.F / 32;
    const int     blk0 = (int) blockIdx.x * gl.bpw;
    const int     nu   = 2 * (int) min((int64_t) gl.bpw, nblk - blk0);  // units of this workgroup (even)
    auto          out  = [&](int u) { return (int64_t) (blk0 + u / 2) * 32 + (u & 1) * 16 + wv; };
    auto          grow = [&](int u) { return gl.swapped ? gl.F + out(u) : out(u); };
    auto          urow = [&](int u) { return gl.swapped ? out(u) : gl.F + out(u); };
    // 1. activations, then unit 0's gate row, then (once the activations are
    // in) its up row; the prologue computes while the rows are in flight
    float4_t xv[J][NC], xw[J][1];
#pragma unroll
    for (int j = 0; j < J; j++) {
        const unsigned e = min(4u * threadIdx.x + 256u * PG_WAVES * j, (unsigned) K - 4u);
#pragma unroll
        for (int c = 0; c < NC; c++) {
            xv[j][c] = *(const float4_t *) (a.x + c * a.ldx + e);
        }
        xw[j][0] = *(const float4_t *) (a.nw + e);
    }
    PgBuf<CH> ba, bb;  // gate rows, up rows
    pg_load<CH>(ba, a, grow(0), lane);
#pragma unroll
    for (int j = 0; j < J; j++) {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            asm volatile("" ::"v"(xv[j][c][0]), "v"(xw[j][0][0]) : "memory");
        }
    }
    pg_load<CH>(bb, a, urow(0), lane);
    pg_prologue<NC, J, MAXK, PRO_NORM>(xv, xw, s_q, s_d, s_ss, a, lane, wv, K);
    __syncthreads();
    // 2. the units: the gate row's partial sums wait (unreduced) while the up
    // row is reduced; each buffer is reloaded as soon as it is consumed
    auto slot = [&](int u) { return &s_h[u / 2][0][(u & 1) * 16 + wv]; };
    float ag[1][NC], au[1][NC];
    int   u = 0;
    for (; u + 1 < nu; u++) {
        pg_acc<NC, CH>(ba, s_q, s_d, 0, a, lane, ag);
        pg_load<CH>(ba, a, grow(u + 1), lane);
        pg_acc<NC, CH>(bb, s_q, s_d, 0, a, lane, au);
        glu_out<NC>(ag, au, lane, slot(u));
        pg_load<CH>(bb, a, urow(u + 1), lane);
    }
    pg_acc<NC, CH>(ba, s_q, s_d, 0, a, lane, ag);
    pg_acc<NC, CH>(bb, s_q, s_d, 0, a, lane, au);
    glu_out<NC>(ag, au, lane, slot(u));
    __syncthreads();
    // 3. quantise the workgroup's blocks: 8 lanes per (block, column)
    {
#pragma clang fp contract(off)
        const int p  = wv * 8 + (lane >> 3);
        const int l8 = lane & 7;
        if (p < nu / 2 * NC) {
            const int      b  = p / NC, c = p % NC;
            const float4_t v  = *(const float4_t *) &s_h[b][c][4 * l8];
            const float    m  = group8_max(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
            const float    dd = m / 127.0f;
            const float    id = dd != 0.0f ? 1.0f / dd : 0.0f;
            char4          q;
            q.x                 = (signed char) roundf(v[0] * id);
            q.y                 = (signed char) roundf(v[1] * id);
            q.z                 = (signed char) roundf(v[2] * id);
            q.w                 = (signed char) roundf(v[3] * id);
            const int64_t e     = (int64_t) (blk0 + b) * 32 + 4 * l8;
            *(char4 *) &gl.qs[c * gl.F + e] = q;
            if (l8 == 0) {
                gl.qd[c * (gl.F / 32) + blk0 + b] = h2f(f2h(dd));
            }
            if (gl.h) {
                *(float4_t *) &gl.h[c * gl.F + e] = v;
            }
        }
    }
}

// Q4_K and Q5_K.  Wave-chunk = 1024 bytes of qs (8 super-blocks); lane l
// owns 16 bytes = elements e_lo..e_lo+15 (low nibbles, sub-block 2c) and
// e_lo+32..e_lo+47 (high nibbles, sub-block 2c+1) of super-block sb.  Q5
// adds the 16 qh bytes of the same columns (qh[32sb + (e_lo & 31) + i]), whose
// bits 2c and 2c+1 are the fifth bits of the two nibbles.
template <int NC, int R, int U, bool Q5 = false>
__global__ __launch_bounds__(256) void k_gemv_q4_K(const uint8_t * __restrict__ W, int64_t N, int64_t K, int64_t rs,
                                                    const int8_t * __restrict__ xq, const float * __restrict__ xd,
                                                    const int16_t * __restrict__ xbs, float * y,
                                                    int64_t ldy, const float * res, int64_t ldr) {
    const int     lane = threadIdx.x & 63;
    const int64_t g    = (int64_t) blockIdx.x * 4 + (threadIdx.x >> 6);
    if (g * R >= N) {
        return;
    }
    const int64_t   half_k = K / 2;
    const int64_t   sc_off = half_k + (Q5 ? K / 8 : 0);
    const int       nsb    = (int) (K / 256);
    const int       ngrp   = (int) (K / 16);
    const uint8_t * wr[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        wr[r] = W + (g * R + r < N ? g * R + r : N - 1) * rs;
    }
    float acc[R][NC];
#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            acc[r][c] = 0.0f;
        }
    }
    for (int64_t base = 0; base < half_k; base += 1024 * U) {
        int4_t   wv[U][R];
        int4_t   hv[U][R];
        uint32_t s0[U][R], s1[U][R], s2[U][R], dm[U][R];
        int4_t   xlo[U][NC], xhi[U][NC];
        int      blo[U][NC], bhi[U][NC];
        float    dx[U][NC];
        bool     ok[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int64_t off = base + 1024 * u + lane * 16;
            ok[u]             = off < half_k;
            const int64_t o   = ok[u] ? off : 0;
            const int     sb  = (int) (o >> 7);
            const int     e   = sb * 256 + (int) ((o & 127) >> 5) * 64 + (int) ((o >> 4) & 1) * 16;
#pragma unroll
            for (int r = 0; r < R; r++) {
                wv[u][r]            = ld16(wr[r] + o);
                if constexpr (Q5) {
                    hv[u][r] = ld16(wr[r] + half_k + 32 * sb + (o & 16));
                }
                const uint32_t * sw = (const uint32_t *) (wr[r] + sc_off + 12 * sb);
                s0[u][r]            = sw[0];
                s1[u][r]            = sw[1];
                s2[u][r]            = sw[2];
                dm[u][r]            = *(const uint32_t *) (wr[r] + sc_off + 12 * (int64_t) nsb + 4 * sb);
            }
#pragma unroll
            for (int c = 0; c < NC; c++) {
                xlo[u][c] = ld16(xq + c * K + e);
                xhi[u][c] = ld16(xq + c * K + e + 32);
                blo[u][c] = xbs[c * ngrp + (e >> 4)];
                bhi[u][c] = xbs[c * ngrp + (e >> 4) + 2];
                dx[u][c]  = xd[c * nsb + sb];
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (!ok[u]) {
                continue;
            }
            const int c64 = (int) (((base + 1024 * u + lane * 16) & 127) >> 5);
#pragma unroll
            for (int r = 0; r < R; r++) {
                int sc_lo, mn_lo, sc_hi, mn_hi;
                q4k_scale_min_w(2 * c64, s0[u][r], s1[u][r], s2[u][r], sc_lo, mn_lo);
                q4k_scale_min_w(2 * c64 + 1, s0[u][r], s1[u][r], s2[u][r], sc_hi, mn_hi);
                const float  d    = h2f((uint16_t) (dm[u][r] & 0xffff));
                const float  dmin = h2f((uint16_t) (dm[u][r] >> 16));
                const int4_t w    = wv[u][r];
                int4_t lo = { w.x & 0x0F0F0F0F, w.y & 0x0F0F0F0F, w.z & 0x0F0F0F0F, w.w & 0x0F0F0F0F };
                int4_t hi = { (w.x >> 4) & 0x0F0F0F0F, (w.y >> 4) & 0x0F0F0F0F, (w.z >> 4) & 0x0F0F0F0F,
                              (w.w >> 4) & 0x0F0F0F0F };
                if constexpr (Q5) {
                    const int4_t h = hv[u][r];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        lo[i] |= ((h[i] >> (2 * c64)) & 0x01010101) << 4;
                        hi[i] |= ((h[i] >> (2 * c64 + 1)) & 0x01010101) << 4;
                    }
                }
#pragma unroll
                for (int c = 0; c < NC; c++) {
                    const int isum = sc_lo * dot16(lo, xlo[u][c]) + sc_hi * dot16(hi, xhi[u][c]);
                    const int msum = mn_lo * blo[u][c] + mn_hi * bhi[u][c];
                    acc[r][c] += (d * dx[u][c]) * (float) isum - (dmin * dx[u][c]) * (float) msum;
                }
            }
        }
    }
    store_rows<NC, R>(acc, lane, g * R, N, y, ldy, res, ldr);
}

// Q6_K.  Unit = (super-block sb, half h, 16 columns l0..l0+15): 48 weight
// bytes covering elements 256sb + 128h + l0 + 32t + i (t = 0..3, i < 16),
// whose 16-element scale groups are g0 + 2t.  64 units per wave-chunk.
template <int NC, int R, int U, bool AL>
__global__ __launch_bounds__(256) void k_gemv_q6_K(const uint8_t * __restrict__ W, int64_t N, int64_t K, int64_t rs,
                                                    const int8_t * __restrict__ xq, const float * __restrict__ xd,
                                                    const int16_t * __restrict__ xbs, float * y,
                                                    int64_t ldy, const float * res, int64_t ldr) {
    const int     lane = threadIdx.x & 63;
    const int64_t g    = (int64_t) blockIdx.x * 4 + (threadIdx.x >> 6);
    if (g * R >= N) {
        return;
    }
    const int64_t   qh_off = K / 2;
    const int64_t   sc_off = K / 2 + K / 4;
    const int64_t   d_off  = sc_off + K / 16;
    const int       units  = (int) (K / 64);
    const int       nsb    = (int) (K / 256);
    const int       ngrp   = (int) (K / 16);
    const uint8_t * wr[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        wr[r] = W + (g * R + r < N ? g * R + r : N - 1) * rs;
    }
    float acc[R][NC];
#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            acc[r][c] = 0.0f;
        }
    }
    for (int base = 0; base < units; base += 64 * U) {
        int4_t qa[U][R], qb[U][R], qh[U][R];
        uint2  sw[U][R];
        float  dw[U][R];
        int4_t xv[U][NC][4];
        int    bs[U][NC][4];
        float  dx[U][NC];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int  uu = base + 64 * u + lane;
            const bool ok = uu < units;
            const int  un = ok ? uu : 0;
            const int  sb = un >> 2, h = (un >> 1) & 1, l0 = (un & 1) * 16;
            const int  g0 = sb * 16 + h * 8 + (l0 >> 4);
            const int  eb = sb * 256 + h * 128 + l0;
#pragma unroll
            for (int r = 0; r < R; r++) {
                qa[u][r] = ld16a<AL>(wr[r] + sb * 128 + h * 64 + l0);
                qb[u][r] = ld16a<AL>(wr[r] + sb * 128 + h * 64 + 32 + l0);
                qh[u][r] = ld16a<AL>(wr[r] + qh_off + sb * 64 + h * 32 + l0);
                sw[u][r] = ld8a<AL>(wr[r] + sc_off + sb * 16 + h * 8);
                dw[u][r] = ok ? h2f(*(const uint16_t *) (wr[r] + d_off + 2 * sb)) : 0.0f;
            }
#pragma unroll
            for (int c = 0; c < NC; c++) {
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    xv[u][c][t] = ld16(xq + c * K + eb + 32 * t);
                    bs[u][c][t] = xbs[c * ngrp + g0 + 2 * t];
                }
                dx[u][c] = xd[c * nsb + sb];
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int l0 = ((base + 64 * u + lane) & 1) * 16;
#pragma unroll
            for (int r = 0; r < R; r++) {
                int4_t q[4];
                int    sc[4];
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const int4_t src = (t & 1) ? qb[u][r] : qa[u][r];
                    const int    sh  = (t < 2) ? 0 : 4;
                    q[t].x = ((src.x >> sh) & 0x0F0F0F0F) | (((qh[u][r].x >> (2 * t)) & 0x03030303) << 4);
                    q[t].y = ((src.y >> sh) & 0x0F0F0F0F) | (((qh[u][r].y >> (2 * t)) & 0x03030303) << 4);
                    q[t].z = ((src.z >> sh) & 0x0F0F0F0F) | (((qh[u][r].z >> (2 * t)) & 0x03030303) << 4);
                    q[t].w = ((src.w >> sh) & 0x0F0F0F0F) | (((qh[u][r].w >> (2 * t)) & 0x03030303) << 4);
                    const int      bi = (l0 >> 4) + 2 * t;
                    const uint32_t wd = bi < 4 ? sw[u][r].x : sw[u][r].y;
                    sc[t]             = (int) (int8_t) ((wd >> (8 * (bi & 3))) & 0xff);
                }
#pragma unroll
                for (int c = 0; c < NC; c++) {
                    int isum = 0;
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        isum += sc[t] * (dot16(q[t], xv[u][c][t]) - 32 * bs[u][c][t]);
                    }
                    acc[r][c] += (dw[u][r] * dx[u][c]) * (float) isum;
                }
            }
        }
    }
    store_rows<NC, R>(acc, lane, g * R, N, y, ldy, res, ldr);
}

// ---------------------------------------------------------------------
// host dispatch

template <typename F, typename... Args>
static int launch_gemv(F kern, int R, int64_t N, hipStream_t stream, Args... args) {
    const int64_t waves = (N + R - 1) / R;
    const int64_t wgs   = (waves + 3) / 4;
    if (wgs > 0x7fffffff) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "gemv: N=%lld too large", (long long) N);
    }
    hipLaunchKernelGGL(kern, dim3((unsigned) wgs), dim3(256), 0, stream, args...);
    return check_launch("gemv");
}

// Rows per wave and chunks in flight per lane, by activation count.
// (Measured on the 12288 x 4096 Q8_0 decode GEMV: 2 rows x 2 chunks per wave
// beat 4 x 4 and 1 x 4 by 15-20%; deeper per-wave queues do not help once
// every CU has ~24 waves in flight.)
template <int NC> struct GemvShape {
    static constexpr int R = 2;
    static constexpr int U = NC <= 4 ? 2 : 1;
};

// Q8_0 launch: rows per wave R by matrix height (more waves for the short
// matrices, fewer activation re-reads for the tall ones), chunks per load
// pass CH covering K up to 12288 in one pass for one or two columns.
template <int NC, int R, int CH>
static int launch_q8_0(const uint8_t * W, int64_t N, int64_t K, int64_t rs, const ActPtrs & x, float * y, int64_t ldy,
                       const float * r, int64_t ldr, hipStream_t stream) {
    if (K <= 1024 * CH) {
        auto kern = k_gemv_q8_0<NC, R, CH, true>;
        return launch_gemv(kern, R, N, stream, W, N, K, rs, x.qs, x.d, y, ldy, r, ldr);
    }
    auto kern = k_gemv_q8_0<NC, R, CH, false>;
    return launch_gemv(kern, R, N, stream, W, N, K, rs, x.qs, x.d, y, ldy, r, ldr);
}

template <int NC, int R>
static int launch_q8_0_k(const uint8_t * W, int64_t N, int64_t K, int64_t rs, const ActPtrs & x, float * y,
                         int64_t ldy, const float * r, int64_t ldr, hipStream_t stream) {
    const int64_t nch = (K + 1023) / 1024;
    if constexpr (NC > 4) {
        return launch_q8_0<NC, R, 2>(W, N, K, rs, x, y, ldy, r, ldr, stream);
    } else if constexpr (NC > 2) {
        return launch_q8_0<NC, R, 4>(W, N, K, rs, x, y, ldy, r, ldr, stream);
    } else {
        if (nch <= 4) {
            return launch_q8_0<NC, R, 4>(W, N, K, rs, x, y, ldy, r, ldr, stream);
        }
        if (nch <= 12) {
            return launch_q8_0<NC, R, 12>(W, N, K, rs, x, y, ldy, r, ldr, stream);
        }
        return launch_q8_0<NC, R, 8>(W, N, K, rs, x, y, ldy, r, ldr, stream);
    }
}

template <int NC>
static int gemv_dispatch(int wtype, const uint8_t * W, int64_t N, int64_t K, int64_t rs, const ActPtrs & x, float * y,
                         int64_t ldy, const float * r, int64_t ldr, hipStream_t stream) {
    constexpr int R = GemvShape<NC>::R;
    constexpr int U = GemvShape<NC>::U;
    if (wtype == TYPE_Q8_0) {
        if constexpr (NC <= 2) {
            // long rows (the down projection, K = 12288): two rows per wave
            // in passes of two 1 KB chunks (4096 x 12288, M = 2: 12.1 us
            // against 13.6 us for one pass over twelve chunks of one row;
            // the same sums in the same order)
            if (K > 4096) {
                return launch_q8_0<NC, 2, 2>(W, N, K, rs, x, y, ldy, r, ldr, stream);
            }
        }
        // one row per wave for the short matrices (more waves in flight; with
        // two rows a 12-chunk pass needs 256 VGPRs and one wave per SIMD)
        if (N <= 8192) {
            return launch_q8_0_k<NC, 1>(W, N, K, rs, x, y, ldy, r, ldr, stream);
        }
        return launch_q8_0_k<NC, 2>(W, N, K, rs, x, y, ldy, r, ldr, stream);
    }
    if (wtype == TYPE_Q4_K) {
        constexpr int U4 = U > 2 ? 2 : U;
        return launch_gemv(k_gemv_q4_K<NC, R, U4>, R, N, stream, W, N, K, rs, x.qs, x.d, x.bs, y, ldy, r, ldr);
    }
    if (wtype == TYPE_Q5_K) {
        constexpr int U5 = U > 2 ? 2 : U;
        return launch_gemv(k_gemv_q4_K<NC, R, U5, true>, R, N, stream, W, N, K, rs, x.qs, x.d, x.bs, y, ldy, r,
                           ldr);
    }
    constexpr int U6 = 1;
    if (rs % 16 == 0 && ((uintptr_t) W) % 16 == 0) {
        return launch_gemv(k_gemv_q6_K<NC, R, U6, true>, R, N, stream, W, N, K, rs, x.qs, x.d, x.bs, y, ldy, r, ldr);
    }
    return launch_gemv(k_gemv_q6_K<NC, R, U6, false>, R, N, stream, W, N, K, rs, x.qs, x.d, x.bs, y, ldy, r, ldr);
}

bool gemv_supported(int wtype, int64_t N, int64_t K, int64_t rs, const void * W) {
    if (!is_repacked_type(wtype) || K % 256 != 0 || N <= 0 || K > ((int64_t) 1 << 30) ||
        rs < row_bytes(wtype, K)) {
        return false;
    }
    // Q8_0 / Q4_K / Q5_K rows are read with 16-byte loads; Q6_K rows may be
    // 2-byte aligned
    const int64_t align = wtype == TYPE_Q6_K ? 2 : 16;
    return rs % align == 0 && ((uintptr_t) W) % align == 0;
}

// GGML_OP_MUL_MAT over BF16 weights at 1..16 activation rows (the BF16 files
// of the depth decoder and the LM, src/depth-decoder.h:206-257): ggml's BF16
// dot rounds the activations to bf16 and sums the f32 products of the pairs.
// One wave per weight row; lane l takes the 8-element chunks l, l + 64, ..;
// the activation chunks come from cache.  Sums: per-lane f32, then a
// symmetric wave reduction.  At most BF16_GEMV_MAXM activation rows.
__global__ __launch_bounds__(256) void k_gemv_bf16(const uint16_t * __restrict__ W, int64_t N, int64_t K, int64_t ldw,
                                                   const float * __restrict__ x, int64_t ldx, int M,
                                                   float * __restrict__ y, int64_t ldy) {
#pragma clang fp contract(off)
    const int64_t row  = (int64_t) blockIdx.x * 4 + (threadIdx.x >> 6);
    const int     lane = threadIdx.x & 63;
    if (row >= N) {
        return;  // wave-uniform
    }
    const uint16_t * wr = W + row * ldw;
    float            acc[BF16_GEMV_MAXM];
#pragma unroll
    for (int c = 0; c < BF16_GEMV_MAXM; c++) {
        acc[c] = 0.0f;
    }
    for (int64_t k = (int64_t) lane * 8; k < K; k += 512) {
        const uint4 wv = *(const uint4 *) (wr + k);
        float       wf[8];
        const uint32_t ww[4] = { wv.x, wv.y, wv.z, wv.w };
#pragma unroll
        for (int e = 0; e < 4; e++) {
            wf[2 * e]     = __uint_as_float(ww[e] << 16);
            wf[2 * e + 1] = __uint_as_float(ww[e] & 0xffff0000u);
        }
#pragma unroll
        for (int c = 0; c < BF16_GEMV_MAXM; c++) {
            if (c < M) {
                const float4_t a = *(const float4_t *) (x + c * ldx + k);
                const float4_t b = *(const float4_t *) (x + c * ldx + k + 4);
                float          s = acc[c];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    s = s + wf[e] * round_bf16(a[e]);
                }
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    s = s + wf[4 + e] * round_bf16(b[e]);
                }
                acc[c] = s;
            }
        }
    }
#pragma unroll
    for (int c = 0; c < BF16_GEMV_MAXM; c++) {
        if (c < M) {
            const float v = wave_sum(acc[c]);
            if (lane == 0) {
                y[c * ldy + row] = v;
            }
        }
    }
}

static int gemv_wide(const uint8_t * W, int64_t N, int64_t K, int64_t rs, const ActPtrs & x, int64_t M, float * y,
                     int64_t ldy, hipStream_t stream, const float * r, int64_t ldr);

static bool gemv_q45_pro_ok(int64_t K, int64_t M, int64_t rs, const void * W);
static int  gemv_q45_pro(int wtype, const void * W, int64_t N, int64_t K, int64_t rs, const ActPtrs & x, int64_t M,
                         float * y, int64_t ldy, hipStream_t stream, const float * r, int64_t ldr);
static bool gemv_q6_pro_ok(int64_t K, int64_t M, int64_t rs, const void * W);
static int  gemv_q6_pro(const void * W, int64_t N, int64_t K, int64_t rs, const ActPtrs & x, int64_t M, float * y,
                        int64_t ldy, hipStream_t stream, const float * r, int64_t ldr);

int gemv_q(int wtype, const void * W, int64_t N, int64_t K, int64_t rs, const ActPtrs & x, int64_t M, float * y,
           int64_t ldy, hipStream_t stream, const float * r, int64_t ldr) {
    if (!gemv_supported(wtype, N, K, rs, W) || M < 1 || ldy < N) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "gemv: type %d N=%lld K=%lld M=%lld rs=%lld not supported", wtype,
                         (long long) N, (long long) K, (long long) M, (long long) rs);
    }
    if (wtype == TYPE_Q6_K && gemv_q6_pro_ok(K, M, rs, W) && getenv("GGML_MI355X_DISABLE_Q6_PRO") == nullptr) {
        return gemv_q6_pro(W, N, K, rs, x, M, y, ldy, stream, r, ldr);
    }
    if ((wtype == TYPE_Q4_K || wtype == TYPE_Q5_K) && gemv_q45_pro_ok(K, M, rs, W) &&
        getenv("GGML_MI355X_DISABLE_Q45_PRO") == nullptr) {
        return gemv_q45_pro(wtype, W, N, K, rs, x, M, y, ldy, stream, r, ldr);
    }
    const uint8_t * wb = (const uint8_t *) W;
    // the int8-MFMA GEMV at 9..16 columns, and at 3..8 columns for rows longer
    // than 4096 (shorter rows at <= 8 columns: the column-group GEMV below is
    // faster, one row per wave with no LDS staging or cross-wave sum)
    static const bool mfma = getenv("GGML_MI355X_DISABLE_GEMV_MFMA") == nullptr;
    if (mfma && wtype == TYPE_Q8_0 && (M >= 9 || (M >= 3 && K > 4096)) && M <= 16 && K % 1024 == 0 &&
        K <= 16 * 3 * MF_PC * 64 &&
        rs % 16 == 0 &&
        (uintptr_t) W % 16 == 0 && (uintptr_t) x.qs % 16 == 0 && (uintptr_t) x.d % 16 == 0) {
        const MfArgs a{ wb, N, (int) K, rs, x.qs, x.d, (int) M, y, ldy, r, ldr };
        return K <= 16 * 2 * MF_PC * 64 ? launch_mf<2>(a, stream) : launch_mf<3>(a, stream);
    }
    if (wtype == TYPE_Q8_0 && M > 8 && M <= 16 && K <= 8192 && K % 32 == 0) {
        return gemv_wide(wb, N, K, rs, x, M, y, ldy, stream, r, ldr);
    }
    const int mc = 8;  // column groups of up to 8
    for (int64_t c0 = 0; c0 < M; c0 += mc) {
        const int64_t nc = std::min<int64_t>(mc, M - c0);
        ActPtrs       xs = x.slice(c0, K);
        float *       ys = y + c0 * ldy;
        const float * rsl = r ? r + c0 * ldr : nullptr;
        int           rc;
        switch (nc) {
            case 1: rc = gemv_dispatch<1>(wtype, wb, N, K, rs, xs, ys, ldy, rsl, ldr, stream); break;
            case 2: rc = gemv_dispatch<2>(wtype, wb, N, K, rs, xs, ys, ldy, rsl, ldr, stream); break;
            case 3: rc = gemv_dispatch<3>(wtype, wb, N, K, rs, xs, ys, ldy, rsl, ldr, stream); break;
            case 4: rc = gemv_dispatch<4>(wtype, wb, N, K, rs, xs, ys, ldy, rsl, ldr, stream); break;
            case 5: rc = gemv_dispatch<5>(wtype, wb, N, K, rs, xs, ys, ldy, rsl, ldr, stream); break;
            case 6: rc = gemv_dispatch<6>(wtype, wb, N, K, rs, xs, ys, ldy, rsl, ldr, stream); break;
            case 7: rc = gemv_dispatch<7>(wtype, wb, N, K, rs, xs, ys, ldy, rsl, ldr, stream); break;
            default: rc = gemv_dispatch<8>(wtype, wb, N, K, rs, xs, ys, ldy, rsl, ldr, stream); break;
        }
        if (rc != MMHIP_OK) {
            return rc;
        }
    }
    return MMHIP_OK;
}

// ---------------------------------------------------------------------------
// BF16 weights at decode (1-2 activation columns): the LM's projections from a
// BF16 model file (qwen3_linear, src/qwen3-enc.h:67-69, in qw3lm_forward_batch,
// src/qwen3-lm.h:742-856) with the block's RMS norm (src/qwen3-enc.h:87-93) in
// the prologue, the residual ADD in the store, or the SwiGLU of the fused
// gate|up rows (src/qwen3-enc.h:106-108) in the epilogue.  Persistent: one
// 8-wave workgroup per CU (two register buffers of a 4096-element segment per
// wave: 128 KB of loads in flight per CU).  The prologue computes the activation columns once
// per workgroup -- the RMS norm as k_rms_norm_row does (double sum of the f32
// squares, the mean rounded to f32, 1 / sqrtf(mean + eps), x * scale, then
// * w), rounded to bf16 as ggml rounds the src1 of a BF16 MUL_MAT -- into LDS.
// Each wave streams whole rows in segments of 4096 elements (lane l holds the
// 16-byte chunks l + 64 i, i < 8), the next segment's loads in flight while
// the current one is multiplied: exact products of bf16 values summed in f32
// by pairs (v_dot2_f32_bf16; ggml-CPU's vec_dot_bf16 sums the same products
// in another order), reduced across the wave.  EPI 0: store; 1: residual ADD (one f32 rounding, as the
// ADD node); 2: SwiGLU pairs, gate row j and up row N / 2 + j -> silu(g) * u
// (k_swiglu's arithmetic).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

struct BfDecArgs {
    const uint16_t * W;
    int64_t          N, K, ldw;  // rows, row length, row stride (elements)
    const float *    x;
    int64_t          ldx;
    const float *    nw;  // norm weight (NORM)
    float            eps;
    const float *    r;  // residual (EPI 1)
    int64_t          ldr;
    float *          y;
    int64_t          ldy;
};

template <int NC, bool NORM, int EPI>
__global__ __launch_bounds__(512) void k_gemv_bf16_dec(BfDecArgs a) {
#pragma clang fp contract(off)
    extern __shared__ __attribute__((aligned(16))) uint16_t s_x[];  // [NC][K] bf16 activation columns
    __shared__ double s_ss[8];
    const int     tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t K   = a.K;
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const float * xc = a.x + c * a.ldx;
        float         sc = 1.0f;
        if constexpr (NORM) {
            double ss = 0.0;
            for (int64_t k = 4 * (int64_t) tid; k < K; k += 2048) {
                const float4_t v = *(const float4_t *) (xc + k);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    ss += (double) (v[e] * v[e]);
                }
            }
            ss = wave_sum_d(ss);
            if (lane == 0) {
                s_ss[wave] = ss;
            }
            __syncthreads();
            double t = 0.0;
#pragma unroll
            for (int w = 0; w < 8; w++) {
                t += s_ss[w];
            }
            __syncthreads();  // s_ss is reused by the next column
            const float mean = (float) (t / (double) K);
            sc               = 1.0f / sqrtf(mean + a.eps);
        }
        for (int64_t k = 4 * (int64_t) tid; k < K; k += 2048) {
            const float4_t v = *(const float4_t *) (xc + k);
            float4_t       w = { 1.0f, 1.0f, 1.0f, 1.0f };
            if constexpr (NORM) {
                w = *(const float4_t *) (a.nw + k);
            }
            uint32_t h[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float o = NORM ? (v[e] * sc) * w[e] : v[e];
                h[e]          = __float_as_uint(round_bf16(o)) >> 16;
            }
            *(uint2 *) (s_x + c * K + k) = uint2{ h[0] | (h[1] << 16), h[2] | (h[3] << 16) };
        }
    }
    __syncthreads();

    const int64_t items = EPI == 2 ? a.N / 2 : a.N;
    constexpr int64_t seg = 4096;  // elements per segment: 8 chunks of 16 bytes per lane
    const int     nseg  = (int) (K / seg);
    const int     nrow  = EPI == 2 ? 2 : 1;
    const int     spi   = nrow * nseg;  // segments per item
    const int64_t W     = (int64_t) gridDim.x * 8;
    int64_t       it    = (int64_t) blockIdx.x * 8 + wave;
    if (it >= items) {
        return;  // wave-uniform; no barrier follows
    }
    auto seg_ptr = [&](int64_t item, int t) {
        const int     rr  = t / nseg;
        const int64_t row = rr ? item + a.N / 2 : item;
        return a.W + row * a.ldw + (int64_t) (t - rr * nseg) * seg + 8 * lane;
    };
    // unconditional loads (a finished wave reloads its last segment): the
    // compiler's wait counts then leave the next segment in flight
    auto load = [&](uint4 (&b)[8], const uint16_t * p) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            b[i] = *(const uint4 *) (p + 512 * i);
        }
    };
    // per-lane sums of the current row, and (SwiGLU) of the pair's gate row;
    // no runtime-indexed arrays, so both stay in registers
    float acc[NC], gacc[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        acc[c]  = 0.0f;
        gacc[c] = 0.0f;
    }
    // v_dot2_f32_bf16: two exact bf16 products added to an f32 sum per
    // instruction, on the packed pairs as loaded (the dot of ggml-CPU's
    // AVX512-BF16 path, vdpbf16ps, sums the same pairs the same way)
    auto compute = [&](const uint4 (&b)[8], int t) {
        const int64_t k0 = (int64_t) (t % nseg) * seg + 8 * lane;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t ww[4] = { b[i].x, b[i].y, b[i].z, b[i].w };
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const uint4    xv    = *(const uint4 *) (s_x + c * K + k0 + 512 * i);
                const uint32_t xx[4] = { xv.x, xv.y, xv.z, xv.w };
                float          s     = acc[c];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, ww[e]),
                                                        __builtin_bit_cast(bf16x2_t, xx[e]), s, false);
                }
                acc[c] = s;
            }
        }
    };
    // after segment t of an item: at the end of the gate row keep its sums,
    // at the end of the item reduce and store
    auto row_end = [&](int64_t item, int t) {
        if (t % nseg != nseg - 1) {
            return;
        }
        if (EPI == 2 && t < nseg) {
#pragma unroll
            for (int c = 0; c < NC; c++) {
                gacc[c] = acc[c];
                acc[c]  = 0.0f;
            }
            return;
        }
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const float v = wave_sum(acc[c]);
            const float g = EPI == 2 ? wave_sum(gacc[c]) : 0.0f;
            if (lane == 0) {
                float o;
                if constexpr (EPI == 2) {
                    const float silu = g / (1.0f + expf(-g));
                    o                = silu * v;
                } else if constexpr (EPI == 1) {
                    o = a.r[c * a.ldr + item] + v;
                } else {
                    o = v;
                }
                a.y[c * a.ldy + item] = o;
            }
            acc[c] = 0.0f;
        }
    };
    // the wave's stream: items it, it + W, ...; within an item its rows, each
    // in nseg segments; two register buffers alternate
    uint4 b0[8], b1[8];
    int   t = 0;
    load(b0, seg_ptr(it, 0));
    // the segment after (it, t), or (it, t) itself at the end of the stream
    auto next = [&](int64_t & i2, int & t2) {
        i2 = it;
        t2 = t + 1;
        if (t2 == spi) {
            t2 = 0;
            i2 += W;
        }
        const bool more = i2 < items;
        if (!more) {
            i2 = it;
            t2 = t;
        }
        return more;
    };
    for (;;) {
        int64_t    it1;
        int        t1;
        const bool more = next(it1, t1);
        load(b1, seg_ptr(it1, t1));
        compute(b0, t);
        row_end(it, t);
        if (!more) {
            break;
        }
        it              = it1;
        t               = t1;
        const bool more2 = next(it1, t1);
        load(b0, seg_ptr(it1, t1));
        compute(b1, t);
        row_end(it, t);
        if (!more2) {
            break;
        }
        it = it1;
        t  = t1;
    }
}

bool bf16_dec_supported(int64_t N, int64_t K, int64_t M, bool glu) {
    return N > 0 && K > 0 && M >= 1 && M <= 2 && K % 4096 == 0 && (size_t) M * K * 2 <= 64 * 1024 &&
           (!glu || N % 2 == 0);
}

static int64_t pg_cus();

template <int NC, bool NORM, int EPI>
static int launch_bf16_dec(const BfDecArgs & a, hipStream_t stream) {
    const size_t lds = (size_t) NC * a.K * 2;
    if (lds > 64 * 1024 || !ensure_lds_limit((const void *) k_gemv_bf16_dec<NC, NORM, EPI>, lds)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "bf16 decode GEMV: %zu bytes of LDS", lds);
    }
    const int64_t items = EPI == 2 ? a.N / 2 : a.N;
    const int64_t wgs   = std::max<int64_t>(1, std::min<int64_t>((items + 7) / 8, pg_cus()));
    hipLaunchKernelGGL((k_gemv_bf16_dec<NC, NORM, EPI>), dim3((unsigned) wgs), dim3(512), lds, stream, a);
    return check_launch("bf16 decode GEMV");
}

template <int NC>
static int bf16_dec_dispatch(const BfDecArgs & a, bool norm, int epi, hipStream_t stream) {
    if (norm) {
        return epi == 2 ? launch_bf16_dec<NC, true, 2>(a, stream)
                        : epi == 1 ? launch_bf16_dec<NC, true, 1>(a, stream) : launch_bf16_dec<NC, true, 0>(a, stream);
    }
    return epi == 2 ? launch_bf16_dec<NC, false, 2>(a, stream)
                    : epi == 1 ? launch_bf16_dec<NC, false, 1>(a, stream) : launch_bf16_dec<NC, false, 0>(a, stream);
}

}  // namespace mmhip

using namespace mmhip;

extern "C" int mmhip_mul_mat_bf16(const void * W, int64_t N, int64_t K, int64_t ldw, const float * x, int64_t ldx,
                                  int64_t M, float * y, int64_t ldy, void * stream) {
    MMHIP_API_BEGIN();
    if (!W || !x || !y || N <= 0 || K <= 0 || M <= 0 || ldw < K || ldx < K || ldy < N) {
        return set_error(MMHIP_ERR_INVALID, "mul_mat_bf16: bad arguments N=%lld K=%lld M=%lld", (long long) N,
                         (long long) K, (long long) M);
    }
    if (M > BF16_GEMV_MAXM || K % 8 != 0 || ldw % 8 != 0 || ldx % 4 != 0 || ((uintptr_t) W) % 16 != 0 ||
        ((uintptr_t) x) % 16 != 0) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "mul_mat_bf16: M=%lld K=%lld (M <= 16, K %% 8 == 0, aligned rows)",
                         (long long) M, (long long) K);
    }
    const int64_t nwg = (N + 3) / 4;
    if (nwg > 0x7fffffff) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "mul_mat_bf16: too many rows");
    }
    hipLaunchKernelGGL(k_gemv_bf16, dim3((unsigned) nwg), dim3(256), 0, (hipStream_t) stream, (const uint16_t *) W, N,
                       K, ldw, x, ldx, (int) M, y, ldy);
    return check_launch("mul_mat_bf16");
}

extern "C" int mmhip_mul_mat_bf16_dec_supported(int64_t N, int64_t K, int64_t M, int glu) {
    return bf16_dec_supported(N, K, M, glu != 0) ? 1 : 0;
}

extern "C" int mmhip_mul_mat_bf16_dec(const void * W, int64_t N, int64_t K, int64_t ldw, const float * x, int64_t ldx,
                                      int64_t M, const float * norm_w, float eps, const float * r, int64_t ldr, int glu,
                                      float * y, int64_t ldy, void * stream) {
    MMHIP_API_BEGIN();
    const int64_t nout = glu ? N / 2 : N;
    if (!W || !x || !y || ldw < K || ldx < K || ldy < nout || (r && ldr < nout) || (r && glu)) {
        return set_error(MMHIP_ERR_INVALID, "mul_mat_bf16_dec: bad arguments N=%lld K=%lld M=%lld", (long long) N,
                         (long long) K, (long long) M);
    }
    if (!bf16_dec_supported(N, K, M, glu != 0) || ldw % 8 != 0 || ldx % 4 != 0 || ((uintptr_t) W) % 16 != 0 ||
        ((uintptr_t) x) % 16 != 0 || (norm_w && ((uintptr_t) norm_w) % 16 != 0)) {
        return set_error(MMHIP_ERR_UNSUPPORTED,
                         "mul_mat_bf16_dec: N=%lld K=%lld M=%lld (M <= 2, K %% 4096 == 0, M K bf16 in 64 KB, aligned rows)",
                         (long long) N, (long long) K, (long long) M);
    }
    BfDecArgs a{ (const uint16_t *) W, N, K, ldw, x, ldx, norm_w, eps, r, ldr, y, ldy };
    const int epi = glu ? 2 : r ? 1 : 0;
    return M == 1 ? bf16_dec_dispatch<1>(a, norm_w != nullptr, epi, (hipStream_t) stream)
                  : bf16_dec_dispatch<2>(a, norm_w != nullptr, epi, (hipStream_t) stream);
}

extern "C" int mmhip_mul_mat_q(int type, const void * W, int64_t N, int64_t K, int64_t w_row_stride, const void * xq,
                               int64_t M, float * y, int64_t ldy, void * stream) {
    MMHIP_API_BEGIN();
    const ActLayout L = act_layout(type, K, M);
    if (L.total == 0 || !xq || !W || !y) {
        return set_error(MMHIP_ERR_INVALID, "mul_mat_q: bad arguments (type %d, K=%lld)", type, (long long) K);
    }
    return gemv_q(type, W, N, K, w_row_stride, ActPtrs::from(L, xq), M, y, ldy, (hipStream_t) stream);
}

extern "C" int mmhip_mul_mat_q_add(int type, const void * W, int64_t N, int64_t K, int64_t w_row_stride,
                                   const void * xq, int64_t M, const float * r, int64_t ldr, float * y, int64_t ldy,
                                   void * stream) {
    MMHIP_API_BEGIN();
    const ActLayout L = act_layout(type, K, M);
    if (L.total == 0 || !xq || !W || !y || !r || ldr < N) {
        return set_error(MMHIP_ERR_INVALID, "mul_mat_q_add: bad arguments (type %d, K=%lld)", type, (long long) K);
    }
    return gemv_q(type, W, N, K, w_row_stride, ActPtrs::from(L, xq), M, y, ldy, (hipStream_t) stream, r, ldr);
}

namespace mmhip {
// compute units of the current device (the persistent grid's size)
static int64_t pg_cus() {
    static int cached[64] = {};
    int        dev        = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        return 256;
    }
    if (!cached[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
            n = 256;
        }
        cached[dev] = n;
    }
    return cached[dev];
}

template <int NC, int CH, int PRO> static int launch_pro(PgArgs a, hipStream_t stream, const char * what) {
    // one resident workgroup per CU; the rows split evenly over the iterations
    const int64_t need = (a.N + PG_WAVES - 1) / PG_WAVES;  // workgroups for one iteration
    const int64_t nit  = (need + pg_cus() - 1) / pg_cus();
    const int64_t wgs  = (need + nit - 1) / nit;
    if (nit > 0x7fffffff) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "%s: N=%lld too large", what, (long long) a.N);
    }
    a.nit     = (int) nit;
    auto kern = k_gemv_q8_0_pro<NC, CH, PRO>;
    hipLaunchKernelGGL(kern, dim3((unsigned) wgs), dim3(64 * PG_WAVES), 0, stream, a);
    return check_launch(what);
}

template <int CH>
static int launch_wide(PgArgs a, const int8_t * xq, const float * xd, int ncv, hipStream_t stream) {
    const int64_t need = (a.N + PG_WAVES - 1) / PG_WAVES;
    const int64_t nit  = (need + pg_cus() - 1) / pg_cus();
    const int64_t wgs  = (need + nit - 1) / nit;
    if (nit > 0x7fffffff) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "gemv (16 columns): N=%lld too large", (long long) a.N);
    }
    a.nit             = (int) nit;
    const size_t lds  = (size_t) 16 * 1024 * CH + (size_t) 16 * 32 * CH * sizeof(float);
    auto         kern = k_gemv_q8_0_wide<CH>;
    if (lds > 64 * 1024 && !ensure_lds_limit((const void *) kern, lds)) {
        return set_error(MMHIP_ERR_HIP, "gemv (16 columns): cannot raise LDS limit to %zu", lds);
    }
    hipLaunchKernelGGL(kern, dim3((unsigned) wgs), dim3(64 * PG_WAVES), lds, stream, a, xq, xd, ncv);
    return check_launch("gemv (16 columns)");
}

static int gemv_wide(const uint8_t * W, int64_t N, int64_t K, int64_t rs, const ActPtrs & x, int64_t M, float * y,
                     int64_t ldy, hipStream_t stream, const float * r, int64_t ldr) {
    const PgArgs a{ W, N, (int) K, rs, nullptr, 0, nullptr, 0, nullptr, 0.0f, nullptr, y, ldy, r, ldr, 1 };
    const int    ch = (int) ((K + 1023) / 1024);
    switch (ch) {
        case 1: return launch_wide<1>(a, x.qs, x.d, (int) M, stream);
        case 2: return launch_wide<2>(a, x.qs, x.d, (int) M, stream);
        case 3:
        case 4: return launch_wide<4>(a, x.qs, x.d, (int) M, stream);
        case 5:
        case 6: return launch_wide<6>(a, x.qs, x.d, (int) M, stream);
        default: return launch_wide<8>(a, x.qs, x.d, (int) M, stream);
    }
}

template <int NC, int CH, int PRO>
static int launch_pro6(PgArgs a, Pg6Act xa, hipStream_t stream, const char * what) {
    const int64_t need = (a.N + PG_WAVES - 1) / PG_WAVES;
    const int64_t nit  = (need + pg_cus() - 1) / pg_cus();
    const int64_t wgs  = (need + nit - 1) / nit;
    if (nit > 0x7fffffff) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "%s: N=%lld too large", what, (long long) a.N);
    }
    a.nit     = (int) nit;
    auto kern = k_gemv_q6_K_pro<NC, CH, PRO>;
    hipLaunchKernelGGL(kern, dim3((unsigned) wgs), dim3(64 * PG_WAVES), 0, stream, a, xa);
    return check_launch(what);
}

// Q6_K GEMV on quantised activations (M <= 2) through the persistent kernel:
// the Q8_K rows copied into LDS once per workgroup instead of re-read per wave
static bool gemv_q6_pro_ok(int64_t K, int64_t M, int64_t rs, const void * W) {
    return M >= 1 && M <= 2 && K % 2048 == 0 && K <= 12288 && rs % 16 == 0 && ((uintptr_t) W) % 16 == 0;
}

static int gemv_q6_pro(const void * W, int64_t N, int64_t K, int64_t rs, const ActPtrs & x, int64_t M, float * y,
                       int64_t ldy, hipStream_t stream, const float * r, int64_t ldr) {
    const PgArgs a{ (const uint8_t *) W, N, (int) K, rs, nullptr, 0, nullptr, 0, nullptr, 0.0f, nullptr, y, ldy, r,
                    ldr, 1 };
    const Pg6Act xa{ x.qs, x.d, x.bs };
    const char * what = "gemv q6_K";
    if (K <= 4096) {
        return M == 1 ? launch_pro6<1, 1, PRO_NONE>(a, xa, stream, what)
                      : launch_pro6<2, 1, PRO_NONE>(a, xa, stream, what);
    }
    return M == 1 ? launch_pro6<1, 3, PRO_NONE>(a, xa, stream, what) : launch_pro6<2, 3, PRO_NONE>(a, xa, stream, what);
}

template <int NC, int CH, int PRO, bool Q5>
static int launch_pro45(PgArgs a, Pg6Act xa, hipStream_t stream, const char * what) {
    const int64_t need = (a.N + PG_WAVES - 1) / PG_WAVES;
    const int64_t nit  = (need + pg_cus() - 1) / pg_cus();
    const int64_t wgs  = (need + nit - 1) / nit;
    if (nit > 0x7fffffff) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "%s: N=%lld too large", what, (long long) a.N);
    }
    a.nit     = (int) nit;
    auto kern = k_gemv_q45_K_pro<NC, CH, PRO, Q5>;
    hipLaunchKernelGGL(kern, dim3((unsigned) wgs), dim3(64 * PG_WAVES), 0, stream, a, xa);
    return check_launch(what);
}

template <int NC, int PRO>
static int launch_pro45_k(int type, const PgArgs & a, const Pg6Act & xa, hipStream_t stream, const char * what) {
    const bool q5 = type == TYPE_Q5_K;
    switch (a.K / 4096) {
        case 1: return q5 ? launch_pro45<NC, 1, PRO, true>(a, xa, stream, what)
                          : launch_pro45<NC, 1, PRO, false>(a, xa, stream, what);
        case 2:
            if constexpr (PRO == PRO_NONE) {
                return q5 ? launch_pro45<NC, 2, PRO, true>(a, xa, stream, what)
                          : launch_pro45<NC, 2, PRO, false>(a, xa, stream, what);
            }
            break;
        case 3:
            if constexpr (PRO == PRO_NONE) {
                return q5 ? launch_pro45<NC, 3, PRO, true>(a, xa, stream, what)
                          : launch_pro45<NC, 3, PRO, false>(a, xa, stream, what);
            }
            break;
        default: break;
    }
    return set_error(MMHIP_ERR_UNSUPPORTED, "%s: K=%d", what, a.K);
}

// Q4_K / Q5_K GEMV on quantised activations (M <= 2, K = 4096, 8192 or 12288)
// through the persistent kernel: the Q8_K rows copied into LDS once per
// workgroup instead of re-read per wave
static bool gemv_q45_pro_ok(int64_t K, int64_t M, int64_t rs, const void * W) {
    return M >= 1 && M <= 2 && K % 4096 == 0 && K <= 12288 && rs % 16 == 0 && ((uintptr_t) W) % 16 == 0;
}

static int gemv_q45_pro(int wtype, const void * W, int64_t N, int64_t K, int64_t rs, const ActPtrs & x, int64_t M,
                        float * y, int64_t ldy, hipStream_t stream, const float * r, int64_t ldr) {
    const PgArgs a{ (const uint8_t *) W, N, (int) K, rs, nullptr, 0, nullptr, 0, nullptr, 0.0f, nullptr, y, ldy, r,
                    ldr, 1 };
    const Pg6Act xa{ x.qs, x.d, x.bs };
    return M == 1 ? launch_pro45_k<1, PRO_NONE>(wtype, a, xa, stream, "gemv q4_K / q5_K")
                  : launch_pro45_k<2, PRO_NONE>(wtype, a, xa, stream, "gemv q4_K / q5_K");
}

template <int PRO>
static int dispatch_pro(int type, const PgArgs & a, int64_t M, hipStream_t stream, const char * what) {
    if (type == TYPE_Q4_K || type == TYPE_Q5_K) {
        if constexpr (PRO == PRO_NORM) {
            const Pg6Act xa{};
            return M == 1 ? launch_pro45_k<1, PRO>(type, a, xa, stream, what)
                          : launch_pro45_k<2, PRO>(type, a, xa, stream, what);
        }
        return set_error(MMHIP_ERR_UNSUPPORTED, "%s: type %d", what, type);
    }
    if (type == TYPE_Q6_K) {
        const Pg6Act xa{};
        if (a.K <= 4096) {
            return M == 1 ? launch_pro6<1, 1, PRO>(a, xa, stream, what) : launch_pro6<2, 1, PRO>(a, xa, stream, what);
        }
        return set_error(MMHIP_ERR_UNSUPPORTED, "%s: K=%d", what, a.K);
    }
    if (a.K <= 4096) {
        return M == 1 ? launch_pro<1, 4, PRO>(a, stream, what) : launch_pro<2, 4, PRO>(a, stream, what);
    }
    if constexpr (PRO == PRO_SWIGLU) {
        return M == 1 ? launch_pro<1, 12, PRO>(a, stream, what) : launch_pro<2, 12, PRO>(a, stream, what);
    }
    return set_error(MMHIP_ERR_UNSUPPORTED, "%s: K=%d", what, a.K);
}

// M <= 2 (two activation columns in registers); the norm over K <= 4096 (the
// model widths), the SwiGLU over K <= 12288 (the FFN widths).  Q6_K rows are
// read with 16-byte loads: K % 2048 == 0 makes the packed row 16-byte sized.
static bool pro_supported(int pro, int type, int64_t N, int64_t K, int64_t M) {
    // Q6_K SwiGLU prologue at K <= 4096 only: over the FFN's 12288 the
    // gate / up reads of every workgroup (196 KB each at M = 2) cost more
    // than the separate SwiGLU + quantisation pass they replace
    // Q4_K / Q5_K: the RMS norm over K = 4096 rows
    return (type == TYPE_Q8_0 || (type == TYPE_Q6_K && K % 2048 == 0 && (pro == PRO_NORM || K <= 4096)) ||
            ((type == TYPE_Q4_K || type == TYPE_Q5_K) && pro == PRO_NORM && K == 4096)) && N > 0 &&
           M >= 1 && M <= 2 && K >= 256 && K <= (pro == PRO_NORM ? 4096 : 12288) && K % 256 == 0;
}

// the 16-byte row loads of the persistent Q4_K / Q5_K / Q6_K GEMVs
static bool pro_rows_ok(int type, int64_t rs, const void * W) {
    return type == TYPE_Q8_0 || (rs % 16 == 0 && ((uintptr_t) W) % 16 == 0);
}
}  // namespace mmhip

extern "C" int mmhip_rms_norm_mul_mat_supported(int type, int64_t N, int64_t K, int64_t M) {
    return pro_supported(PRO_NORM, type, N, K, M);
}

extern "C" int mmhip_rms_norm_mul_mat(int type, const void * W, int64_t N, int64_t K, int64_t w_row_stride,
                                      const float * x, int64_t ldx, int64_t M, const float * norm_w, float eps,
                                      float * xn_out, const float * res, int64_t ldr, float * y, int64_t ldy,
                                      void * stream) {
    MMHIP_API_BEGIN();
    if (!pro_supported(PRO_NORM, type, N, K, M)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "rms_norm_mul_mat: type %d N=%lld K=%lld M=%lld", type, (long long) N,
                         (long long) K, (long long) M);
    }
    if (!W || !x || !norm_w || !y || ldx < K || ldy < N || (res && ldr < N) ||
        !gemv_supported(type, N, K, w_row_stride, W) || !pro_rows_ok(type, w_row_stride, W) ||
        ((uintptr_t) x | (uintptr_t) norm_w | (uintptr_t) xn_out) % 16 != 0 || (ldx % 4) != 0) {
        return set_error(MMHIP_ERR_INVALID, "rms_norm_mul_mat: bad arguments / alignment");
    }
    const PgArgs a{ (const uint8_t *) W, N, (int) K, w_row_stride, x, ldx, nullptr, 0, norm_w, eps, xn_out, y, ldy,
                    res, ldr, 1 };
    return dispatch_pro<PRO_NORM>(type, a, M, (hipStream_t) stream, "rms_norm_mul_mat");
}

extern "C" int mmhip_swiglu_mul_mat_supported(int type, int64_t N, int64_t K, int64_t M) {
    return pro_supported(PRO_SWIGLU, type, N, K, M);
}

extern "C" int mmhip_swiglu_mul_mat(int type, const void * W, int64_t N, int64_t K, int64_t w_row_stride,
                                    const float * g, int64_t ldg, const float * u, int64_t ldu, int64_t M,
                                    float * h_out, const float * res, int64_t ldr, float * y, int64_t ldy,
                                    void * stream) {
    MMHIP_API_BEGIN();
    if (!pro_supported(PRO_SWIGLU, type, N, K, M)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "swiglu_mul_mat: type %d N=%lld K=%lld M=%lld", type, (long long) N,
                         (long long) K, (long long) M);
    }
    if (!W || !g || !u || !y || ldg < K || ldu < K || ldy < N || (res && ldr < N) ||
        !gemv_supported(type, N, K, w_row_stride, W) || !pro_rows_ok(type, w_row_stride, W) ||
        ((uintptr_t) g | (uintptr_t) u | (uintptr_t) h_out) % 16 != 0 || (ldg % 4) != 0 || (ldu % 4) != 0) {
        return set_error(MMHIP_ERR_INVALID, "swiglu_mul_mat: bad arguments / alignment");
    }
    const PgArgs a{ (const uint8_t *) W, N, (int) K, w_row_stride, g, ldg, u, ldu, nullptr, 0.0f, h_out, y, ldy,
                    res, ldr, 1 };
    return dispatch_pro<PRO_SWIGLU>(type, a, M, (hipStream_t) stream, "swiglu_mul_mat");
}

extern "C" int mmhip_rms_norm_mul_mat_glu_supported(int type, int64_t N, int64_t K, int64_t M) {
    if (!(type == TYPE_Q8_0 && M >= 1 && M <= 2 && K >= 256 && K <= 4096 && K % 256 == 0 && N > 0 && N % 512 == 0)) {
        return 0;
    }
    const int64_t nblk = N / 64;  // Q8_0 blocks of the N / 2 SwiGLU outputs
    return (nblk + pg_cus() - 1) / pg_cus() <= GLU_MAXB;
}

extern "C" int mmhip_rms_norm_mul_mat_glu(int type, const void * W, int64_t N, int64_t K, int64_t w_row_stride,
                                          const float * x, int64_t ldx, int64_t M, const float * norm_w, float eps,
                                          int swapped, void * xq, float * h_out, void * stream) {
    MMHIP_API_BEGIN();
    if (!mmhip_rms_norm_mul_mat_glu_supported(type, N, K, M)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "rms_norm_mul_mat_glu: type %d N=%lld K=%lld M=%lld", type,
                         (long long) N, (long long) K, (long long) M);
    }
    if (!W || !x || !norm_w || !xq || ldx < K || !gemv_supported(type, N, K, w_row_stride, W) ||
        ((uintptr_t) x | (uintptr_t) norm_w | (uintptr_t) h_out | (uintptr_t) xq) % 16 != 0 || (ldx % 4) != 0) {
        return set_error(MMHIP_ERR_INVALID, "rms_norm_mul_mat_glu: bad arguments / alignment");
    }
    const int64_t   F    = N / 2;
    const ActLayout L    = act_layout(TYPE_Q8_0, F, M);
    const int64_t   nblk = F / 32;
    const int64_t   bpw  = (nblk + pg_cus() - 1) / pg_cus();
    const int64_t   wgs  = (nblk + bpw - 1) / bpw;
    const PgArgs    a{ (const uint8_t *) W, N, (int) K, w_row_stride, x, ldx, nullptr, 0, norm_w, eps, nullptr,
                       nullptr, 0, nullptr, 0, 1 };
    const GluArgs   gl{ F, swapped ? 1 : 0, (int) bpw, (int8_t *) xq + L.qs_off, (float *) ((char *) xq + L.d_off),
                        h_out };
    if (M == 1) {
        hipLaunchKernelGGL(k_gemv_q8_0_norm_glu<1>, dim3((unsigned) wgs), dim3(64 * PG_WAVES), 0,
                           (hipStream_t) stream, a, gl);
    } else {
        hipLaunchKernelGGL(k_gemv_q8_0_norm_glu<2>, dim3((unsigned) wgs), dim3(64 * PG_WAVES), 0,
                           (hipStream_t) stream, a, gl);
    }
    return check_launch("rms_norm_mul_mat_glu");
}
