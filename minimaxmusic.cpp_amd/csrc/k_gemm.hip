// k_gemm.hip - MUL_MAT at token counts (M > 8): MFMA GEMM with the weight
// tile dequantised into LDS.
//
//   y[m, n] = sum_k x[m, k] * deq(W)[n, k]
//
// Workgroup tile: 256 tokens x 256 weight rows (8 waves, each 128 x 64 with
// eight v_mfma_f32_32x32x16_f16 accumulators) when the problem has at least
// 256 such tiles, else 128 x 128 (4 waves, each 64 x 64); K step 64.  Per K step the x tile (f32) is rounded to f16 and the weight
// tile is dequantised exactly as the GGUF definitions (f32, no contraction)
// and then rounded to f16; both are stored row-major (k contiguous) in LDS,
// which is the operand order of the MFMA A (tokens) and B (weight rows)
// inputs.  The output accumulator layout gives each lane one weight row, so
// stores of 32 lanes are 128 contiguous bytes of a y row.
//
// The next K step's global loads are issued before the current step's MFMAs
// (register double buffering), so HBM/L2 latency overlaps the matrix work.
#include "mmhip_device.h"
#include "mmhip_internal.h"

namespace mmhip {

constexpr int GM_BK = 64;
constexpr int GM_LS = GM_BK + 8;  // LDS row stride in halves (144 bytes)

__device__ __forceinline__ float16_t gm_mfma(half8_t a, half8_t b, float16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Raw bytes a thread needs for its half row (32 weights) of one K step.
struct WRaw {
    int4_t   q0, q1;     // quant bytes
    uint32_t s0, s1, s2;  // Q4_K scales / Q6_K scales (s0, s1) / unused
    uint32_t dm;          // f16 scale(s)
};

// Thread t of the workgroup owns weight row (t / 2) of the tile and the half
// (t % 2) of the 64-wide K step.
template <int WT>
__device__ __forceinline__ void w_load(WRaw & w, const uint8_t * row, int64_t K, int k0, int half) {
    if constexpr (WT == TYPE_Q8_0) {
        // one Q8_0 block: 32 quants at k0 + 32*half
        const int kb = k0 + 32 * half;
        w.q0         = *(const int4_t *) (row + kb);
        w.q1         = *(const int4_t *) (row + kb + 16);
        w.dm         = *(const uint16_t *) (row + K + 2 * (kb >> 5));
    } else if constexpr (WT == TYPE_Q4_K) {
        // 16 bytes of the 32-byte chunk holding sub-blocks 2c, 2c+1
        const int sb = k0 >> 8, c = (k0 & 255) >> 6;
        w.q0         = *(const int4_t *) (row + sb * 128 + c * 32 + half * 16);
        const uint32_t * sc = (const uint32_t *) (row + K / 2 + 12 * sb);
        w.s0         = sc[0];
        w.s1         = sc[1];
        w.s2         = sc[2];
        w.dm         = *(const uint32_t *) (row + K / 2 + 12 * (K / 256) + 4 * sb);
    } else {
        // Q6_K: K step = quarter pair (t, t+1) of half hf; 16 columns l0..l0+15
        const int sb = k0 >> 8, hf = (k0 & 255) >> 7, tq = (k0 & 127) >> 5;  // tq in {0, 2}
        const int l0 = half * 16;
        const uint8_t * ql = row + sb * 128 + hf * 64;
        // t = tq uses ql[l] (tq = 0: low nibble; tq = 2: high nibble) and
        // t = tq + 1 uses ql[l + 32]
        w.q0 = *(const int4_t *) (ql + l0);
        w.q1 = *(const int4_t *) (ql + 32 + l0);
        const int4_t qh = *(const int4_t *) (row + K / 2 + sb * 64 + hf * 32 + l0);
        w.s0 = (uint32_t) qh.x;
        w.s1 = (uint32_t) qh.y;
        w.s2 = (uint32_t) qh.z;
        w.dm = (uint32_t) qh.w;
    }
}

// Dequantise the thread's 32 weights (f32 exact, then f16) into LDS row
// `wrow` of the tile at K columns [32*half, 32*half+32) (Q8_0) or the column
// sets given by the format (Q4_K, Q6_K).
template <int WT>
__device__ __forceinline__ void w_store(const WRaw & w, _Float16 * sW, const uint8_t * row, int64_t K, int k0,
                                        int half) {
#pragma clang fp contract(off)
    if constexpr (WT == TYPE_Q8_0) {
        const float d = h2f((uint16_t) w.dm);
        half8_t     o[4];
        const int8_t * q = (const int8_t *) &w.q0;
        const int8_t * r = (const int8_t *) &w.q1;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            o[i / 8][i % 8]     = (_Float16) (d * (float) q[i]);
            o[2 + i / 8][i % 8] = (_Float16) (d * (float) r[i]);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            *(half8_t *) &sW[32 * half + 8 * j] = o[j];
        }
    } else if constexpr (WT == TYPE_Q4_K) {
        const int c = (k0 & 255) >> 6;
        int       sc_lo, mn_lo, sc_hi, mn_hi;
        q4k_scale_min_w(2 * c, w.s0, w.s1, w.s2, sc_lo, mn_lo);
        q4k_scale_min_w(2 * c + 1, w.s0, w.s1, w.s2, sc_hi, mn_hi);
        const float     d    = h2f((uint16_t) (w.dm & 0xffff));
        const float     dmin = h2f((uint16_t) (w.dm >> 16));
        const float     d1 = d * (float) sc_lo, m1 = dmin * (float) mn_lo;
        const float     d2 = d * (float) sc_hi, m2 = dmin * (float) mn_hi;
        const uint8_t * q  = (const uint8_t *) &w.q0;
        half8_t         lo[2], hi[2];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            lo[i / 8][i % 8] = (_Float16) (d1 * (float) (q[i] & 15) - m1);
            hi[i / 8][i % 8] = (_Float16) (d2 * (float) (q[i] >> 4) - m2);
        }
        // low nibbles: columns 16*half + 0..15; high nibbles: 32 + 16*half + 0..15
        *(half8_t *) &sW[16 * half]          = lo[0];
        *(half8_t *) &sW[16 * half + 8]      = lo[1];
        *(half8_t *) &sW[32 + 16 * half]     = hi[0];
        *(half8_t *) &sW[32 + 16 * half + 8] = hi[1];
    } else {
        const int       sb = k0 >> 8, hf = (k0 & 255) >> 7, tq = (k0 & 127) >> 5;
        const float     d  = h2f(*(const uint16_t *) (row + K / 2 + K / 4 + K / 16 + 2 * sb));
        const int8_t *  sc = (const int8_t *) (row + K / 2 + K / 4) + sb * 16 + hf * 8;
        const uint8_t * qa = (const uint8_t *) &w.q0;
        const uint8_t * qb = (const uint8_t *) &w.q1;
        const uint32_t  qhw[4] = { w.s0, w.s1, w.s2, w.dm };
        const uint8_t * qh = (const uint8_t *) qhw;
        // element l0 + i of quarter t has scale index 2t + (l0 + i) / 16 = 2t + half
        const float ds0 = d * (float) sc[2 * tq + half];
        const float ds1 = d * (float) sc[2 * (tq + 1) + half];
        half8_t     o0[2], o1[2];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int lo0 = tq == 0 ? (qa[i] & 15) : (qa[i] >> 4);
            const int lo1 = tq == 0 ? (qb[i] & 15) : (qb[i] >> 4);
            const int h0  = (qh[i] >> (2 * tq)) & 3;
            const int h1  = (qh[i] >> (2 * tq + 2)) & 3;
            o0[i / 8][i % 8] = (_Float16) (ds0 * (float) ((lo0 | (h0 << 4)) - 32));
            o1[i / 8][i % 8] = (_Float16) (ds1 * (float) ((lo1 | (h1 << 4)) - 32));
        }
        // quarter t -> columns 0..31, quarter t+1 -> 32..63 of the K step
        *(half8_t *) &sW[16 * half]          = o0[0];
        *(half8_t *) &sW[16 * half + 8]      = o0[1];
        *(half8_t *) &sW[32 + 16 * half]     = o1[0];
        *(half8_t *) &sW[32 + 16 * half + 8] = o1[1];
    }
}

// Consecutive work items go to one XCD (workgroups are dealt round-robin over
// the 8 XCDs), so the workgroups sharing an activation tile share an L2.
__device__ __forceinline__ int64_t gm_xcd_remap(int64_t lin, int64_t total) {
    const int64_t per = total / 8;
    return lin >= per * 8 ? lin : (lin % 8) * per + lin / 8;
}

// NW waves; tile BM x BN with BM = BN = 32 * NW (staging: thread t owns row
// t / 2 of both tiles and half t % 2 of the K step); waves in a WM x (NW/WM)
// grid, each computing MB x NB blocks of 32 x 32.
template <int WT, int NW, int WM>
__global__ __launch_bounds__(NW * 64) void k_gemm_q(const uint8_t * __restrict__ W, int64_t N, int64_t K, int64_t rs,
                                                     const float * __restrict__ x, int64_t ldx, int64_t M,
                                                     float * __restrict__ y, int64_t ldy, int64_t n_ntiles,
                                                     int64_t n_tiles) {
    constexpr int BM = 32 * NW;
    constexpr int BN = 32 * NW;
    constexpr int WN = NW / WM;
    constexpr int MB = BM / WM / 32;
    constexpr int NB = BN / WN / 32;
    extern __shared__ __attribute__((aligned(16))) _Float16 g_lds[];
    _Float16 * sX = g_lds;
    _Float16 * sW = g_lds + BM * GM_LS;

    const int64_t work = gm_xcd_remap(blockIdx.x, n_tiles);
    const int64_t nt   = work % n_ntiles;
    const int64_t mt   = work / n_ntiles;
    const int64_t m0   = mt * BM;
    const int64_t n0   = nt * BN;
    const int     tid  = threadIdx.x;
    const int     wave = tid >> 6;
    const int     lane = tid & 63;
    const int     wm   = wave / WN;
    const int     wn   = wave % WN;
    const int     lq   = lane & 31;
    const int     hh   = lane >> 5;

    const int       srow  = tid >> 1;
    const int       shalf = tid & 1;
    const int64_t   xm    = m0 + srow;
    const bool      x_ok  = xm < M;
    const float *   xrow  = x + (x_ok ? xm : 0) * ldx + shalf * 32;
    const int64_t   wn_   = n0 + srow;
    const bool      w_ok  = wn_ < N;
    const uint8_t * wrow  = W + (w_ok ? wn_ : 0) * rs;

    float16_t acc[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; i++) {
#pragma unroll
        for (int j = 0; j < NB; j++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                acc[i][j][r] = 0.0f;
            }
        }
    }

    float4_t xr[8];
    WRaw     wr;
    auto     load = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            xr[i] = x_ok ? *(const float4_t *) (xrow + k0 + 4 * i) : float4_t{ 0.0f, 0.0f, 0.0f, 0.0f };
        }
        w_load<WT>(wr, wrow, K, k0, shalf);
    };

    load(0);
    for (int k0 = 0; k0 < K; k0 += GM_BK) {
        __syncthreads();
        {
            half8_t o[4];
#pragma unroll
            for (int i = 0; i < 8; i++) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    o[i / 2][(i % 2) * 4 + j] = (_Float16) xr[i][j];
                }
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                *(half8_t *) &sX[srow * GM_LS + shalf * 32 + 8 * j] = o[j];
            }
        }
        if (w_ok) {
            w_store<WT>(wr, &sW[srow * GM_LS], wrow, K, k0, shalf);
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                *(half8_t *) &sW[srow * GM_LS + shalf * 32 + 8 * j] = half8_t{};
            }
        }
        __syncthreads();
        if (k0 + GM_BK < K) {
            load(k0 + GM_BK);
        }
#pragma unroll
        for (int kk = 0; kk < GM_BK / 16; kk++) {
            half8_t a[MB], b[NB];
#pragma unroll
            for (int i = 0; i < MB; i++) {
                a[i] = *(const half8_t *) &sX[(wm * (BM / WM) + i * 32 + lq) * GM_LS + kk * 16 + 8 * hh];
            }
#pragma unroll
            for (int j = 0; j < NB; j++) {
                b[j] = *(const half8_t *) &sW[(wn * (BN / WN) + j * 32 + lq) * GM_LS + kk * 16 + 8 * hh];
            }
#pragma unroll
            for (int i = 0; i < MB; i++) {
#pragma unroll
                for (int j = 0; j < NB; j++) {
                    acc[i][j] = gm_mfma(a[i], b[j], acc[i][j]);
                }
            }
        }
    }

    // C[i = token][j = weight row]: lane holds row j = lq, tokens 8(r/4) + 4hh + r%4
#pragma unroll
    for (int i = 0; i < MB; i++) {
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const int64_t n = n0 + wn * (BN / WN) + j * 32 + lq;
            if (n >= N) {
                continue;
            }
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int64_t m = m0 + wm * (BM / WM) + i * 32 + 8 * (r / 4) + 4 * hh + (r % 4);
                if (m < M) {
                    y[m * ldy + n] = acc[i][j][r];
                }
            }
        }
    }
}

bool gemm_supported(int wtype, int64_t N, int64_t K, int64_t rs, const void * W, const float * x, int64_t ldx) {
    if (!(wtype == TYPE_Q8_0 || wtype == TYPE_Q4_K || wtype == TYPE_Q6_K) || N <= 0 || K % GM_BK != 0 ||
        rs < row_bytes(wtype, K)) {
        return false;
    }
    if ((wtype == TYPE_Q4_K || wtype == TYPE_Q6_K) && K % 256 != 0) {
        return false;
    }
    // 16-byte weight and activation loads
    return rs % 16 == 0 && ((uintptr_t) W) % 16 == 0 && ((uintptr_t) x) % 16 == 0 && ldx % 4 == 0;
}

template <int NW, int WM>
static int launch_gemm(int wtype, const uint8_t * W, int64_t N, int64_t K, int64_t rs, const float * x, int64_t ldx,
                       int64_t M, float * y, int64_t ldy, hipStream_t stream) {
    constexpr int BT   = 32 * NW;
    const int64_t n_nt = (N + BT - 1) / BT;
    const int64_t n_mt = (M + BT - 1) / BT;
    const int64_t n    = n_nt * n_mt;
    if (n > 0x7fffffff) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "mul_mat gemm: too many tiles");
    }
    const size_t lds = (size_t) 2 * BT * GM_LS * sizeof(_Float16);
    auto go = [&](auto kern) -> int {
        if (lds > 64 * 1024 && !ensure_lds_limit((const void *) kern, lds)) {
            return set_error(MMHIP_ERR_HIP, "mul_mat gemm: cannot raise LDS limit to %zu", lds);
        }
        hipLaunchKernelGGL(kern, dim3((unsigned) n), dim3(NW * 64), lds, stream, W, N, K, rs, x, ldx, M, y, ldy, n_nt,
                           n);
        return check_launch("mul_mat gemm");
    };
    switch (wtype) {
        case TYPE_Q8_0: return go(k_gemm_q<TYPE_Q8_0, NW, WM>);
        case TYPE_Q4_K: return go(k_gemm_q<TYPE_Q4_K, NW, WM>);
        default: return go(k_gemm_q<TYPE_Q6_K, NW, WM>);
    }
}

int gemm_q(int wtype, const void * W, int64_t N, int64_t K, int64_t rs, const float * x, int64_t ldx, int64_t M,
           float * y, int64_t ldy, hipStream_t stream) {
    if (!gemm_supported(wtype, N, K, rs, W, x, ldx)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "mul_mat gemm: type %d N=%lld K=%lld rs=%lld not supported", wtype,
                         (long long) N, (long long) K, (long long) rs);
    }
    const uint8_t * wb       = (const uint8_t *) W;
    const int64_t   tiles256 = ((N + 255) / 256) * ((M + 255) / 256);
    if (tiles256 >= 256) {
        return launch_gemm<8, 2>(wtype, wb, N, K, rs, x, ldx, M, y, ldy, stream);
    }
    return launch_gemm<4, 2>(wtype, wb, N, K, rs, x, ldx, M, y, ldy, stream);
}

}  // namespace mmhip
