// k_gemm.hip - MUL_MAT at token counts (M > 16): MFMA GEMM with the weight
// tile dequantised into LDS.
//
//   y[m, n] = sum_k x[m, k] * deq(W)[n, k]
//
// The activations are first rounded to f16 into a packed copy (workspace):
// every workgroup along N reads them, so they are converted once and moved at
// half the bytes.  Workgroup tile: 256 tokens x 256 weight rows (8 waves,
// each 128 x 64 with eight v_mfma_f32_32x32x16_f16 accumulators) when the
// problem has at least 256 such tiles, else 64 tokens x 128 weight rows (4
// waves, each 32 x 64); K step 64.  The weight tile is dequantised exactly as the GGUF
// definitions (f32, no contraction) and then rounded to f16; both tiles are
// k-contiguous rows in LDS, the operand order of the MFMA A (tokens) and B
// (weight rows) inputs.  The output accumulator layout gives each lane one
// weight row, so stores of 32 lanes are 128 contiguous bytes of a y row.
#include <cstdlib>
#include <mutex>
#include <type_traits>
#include <unordered_map>

#include "mmhip_device.h"
#include "mmhip_internal.h"

namespace mmhip {

constexpr int GM_BK = 64;
constexpr int GM_LS = GM_BK + 8;  // LDS row stride in halves (144 bytes)

__device__ __forceinline__ float16_t gm_mfma(half8_t a, half8_t b, float16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// The same product on bf16 operands (carried as 16-bit patterns in half8_t):
// bf16 x bf16 products are exact in f32 and accumulate in f32.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float16_t gm_mfma_bf16(half8_t a, half8_t b, float16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                   0, 0, 0);
}

// Raw bytes a thread needs for its half row (32 weights) of one K step.
struct WRaw {
    int4_t   q0, q1;     // quant bytes (Q5_K: q1 = the fifth-bit bytes)
    uint32_t s0, s1, s2;  // Q4_K / Q5_K scales; Q6_K high bits (with dm)
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
    } else if constexpr (WT == TYPE_Q4_K || WT == TYPE_Q5_K) {
        // 16 bytes of the 32-byte chunk holding sub-blocks 2c, 2c+1; Q5_K:
        // the qh bytes of the same 16 columns (bits 2c, 2c+1)
        const int64_t qh_sz = WT == TYPE_Q5_K ? K / 8 : 0;
        const int     sb = k0 >> 8, c = (k0 & 255) >> 6;
        w.q0         = *(const int4_t *) (row + sb * 128 + c * 32 + half * 16);
        if constexpr (WT == TYPE_Q5_K) {
            w.q1 = *(const int4_t *) (row + K / 2 + sb * 32 + half * 16);
        }
        const uint32_t * sc = (const uint32_t *) (row + K / 2 + qh_sz + 12 * sb);
        w.s0         = sc[0];
        w.s1         = sc[1];
        w.s2         = sc[2];
        w.dm         = *(const uint32_t *) (row + K / 2 + qh_sz + 12 * (K / 256) + 4 * sb);
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

// Byte e of a 16-byte load, as the format's signed / unsigned value.  The
// bytes are taken from the 32-bit words with shifts at the point of use: a
// byte-pointer view of the loaded vector makes the compiler unpack it right
// after the load, which forces the wait for that load before the MFMA work
// that should hide it.
__device__ __forceinline__ int byte_s(const int4_t & v, int e) {
    return (int) (int8_t) (v[e >> 2] >> (8 * (e & 3)));
}

__device__ __forceinline__ int byte_u(const int4_t & v, int e) {
    return (v[e >> 2] >> (8 * (e & 3))) & 0xff;
}

__device__ __forceinline__ int byte_u32(const uint32_t (&w)[4], int e) {
    return (int) ((w[e >> 2] >> (8 * (e & 3))) & 0xff);
}

// Dequantise the thread's 32 weights (f32 exact, then f16) into four 16-byte
// chunks o[0..3] and name the chunk index (0..7) of the 64-wide K step each
// one belongs to (Q8_0: 4*half + c; Q4_K / Q6_K: low nibbles or first
// quarter at 2*half + {0,1}, high nibbles or second quarter at 4 + 2*half +
// {0,1}).
template <int WT>
__device__ __forceinline__ void w_dequant(const WRaw & w, const uint8_t * row, int64_t K, int k0, int half,
                                          half8_t (&o)[4], int (&chunk)[4]) {
#pragma clang fp contract(off)
    if constexpr (WT == TYPE_Q8_0) {
        const float d = h2f((uint16_t) w.dm);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            o[i / 8][i % 8]     = (_Float16) (d * (float) byte_s(w.q0, i));
            o[2 + i / 8][i % 8] = (_Float16) (d * (float) byte_s(w.q1, i));
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            chunk[j] = 4 * half + j;
        }
    } else if constexpr (WT == TYPE_Q4_K || WT == TYPE_Q5_K) {
        const int c = (k0 & 255) >> 6;
        int       sc_lo, mn_lo, sc_hi, mn_hi;
        q4k_scale_min_w(2 * c, w.s0, w.s1, w.s2, sc_lo, mn_lo);
        q4k_scale_min_w(2 * c + 1, w.s0, w.s1, w.s2, sc_hi, mn_hi);
        const float d    = h2f((uint16_t) (w.dm & 0xffff));
        const float dmin = h2f((uint16_t) (w.dm >> 16));
        const float d1 = d * (float) sc_lo, m1 = dmin * (float) mn_lo;
        const float d2 = d * (float) sc_hi, m2 = dmin * (float) mn_hi;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int q  = byte_u(w.q0, i);
            int       ql = q & 15, qh = q >> 4;
            if constexpr (WT == TYPE_Q5_K) {
                const int h = byte_u(w.q1, i);
                ql |= ((h >> (2 * c)) & 1) << 4;
                qh |= ((h >> (2 * c + 1)) & 1) << 4;
            }
            o[i / 8][i % 8]     = (_Float16) (d1 * (float) ql - m1);
            o[2 + i / 8][i % 8] = (_Float16) (d2 * (float) qh - m2);
        }
        chunk[0] = 2 * half;
        chunk[1] = 2 * half + 1;
        chunk[2] = 4 + 2 * half;
        chunk[3] = 4 + 2 * half + 1;
    } else {
        const int       sb = k0 >> 8, hf = (k0 & 255) >> 7, tq = (k0 & 127) >> 5;
        const float     d  = h2f(*(const uint16_t *) (row + K / 2 + K / 4 + K / 16 + 2 * sb));
        const int8_t *  sc = (const int8_t *) (row + K / 2 + K / 4) + sb * 16 + hf * 8;
        const uint32_t  qhw[4] = { w.s0, w.s1, w.s2, w.dm };
        // element l0 + i of quarter t has scale index 2t + (l0 + i) / 16 = 2t + half
        const float ds0 = d * (float) sc[2 * tq + half];
        const float ds1 = d * (float) sc[2 * (tq + 1) + half];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int qa = byte_u(w.q0, i), qb = byte_u(w.q1, i), qh = byte_u32(qhw, i);
            const int lo0 = tq == 0 ? (qa & 15) : (qa >> 4);
            const int lo1 = tq == 0 ? (qb & 15) : (qb >> 4);
            const int h0  = (qh >> (2 * tq)) & 3;
            const int h1  = (qh >> (2 * tq + 2)) & 3;
            o[i / 8][i % 8]     = (_Float16) (ds0 * (float) ((lo0 | (h0 << 4)) - 32));
            o[2 + i / 8][i % 8] = (_Float16) (ds1 * (float) ((lo1 | (h1 << 4)) - 32));
        }
        chunk[0] = 2 * half;
        chunk[1] = 2 * half + 1;
        chunk[2] = 4 + 2 * half;
        chunk[3] = 4 + 2 * half + 1;
    }
}

// Consecutive work items go to one XCD (workgroups are dealt round-robin over
// the 8 XCDs), so the workgroups sharing an activation tile share an L2.
__device__ __forceinline__ int64_t gm_xcd_remap(int64_t lin, int64_t total) {
    const int64_t per = total / 8;
    return lin >= per * 8 ? lin : (lin % 8) * per + lin / 8;
}

// The activation tile reaches LDS without passing through registers:
// global_load_lds_dwordx4 writes the 16 bytes of lane l at M0 + 16 l, so one
// wave instruction fills 1 KB of LDS.  It is issued from inline asm so that
// the compiler's wait-count bookkeeping (which would wait for every such load
// before any LDS read it cannot prove disjoint) leaves the prefetch alone; the
// kernel waits for it explicitly before the barrier that publishes a stage.
typedef __attribute__((address_space(3))) _Float16 lds_half_t;

__device__ __forceinline__ void dma16(const void * src, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds_addr) : "memory", "m0");
}

// Tiles in LDS are unpadded rows of 64 halves (8 chunks of 16 bytes) with
// chunk c of row r stored at chunk c ^ (r & 7): the 32 rows an MFMA operand
// read touches then spread over all banks.
template <int BK>
__device__ __forceinline__ int swz(int r, int c) {
    return r * BK + 8 * (c ^ (r & 7));
}

// Rows of 32 halves (the f16-weight ring's K step): chunk c of row r at
// c ^ ((r >> 2) & 3), so the 16 rows one 16-lane operand read touches fall in
// 16 different bank groups.
__device__ __forceinline__ int swz32(int r, int c) {
    return r * 32 + 8 * (c ^ ((r >> 2) & 3));
}

// NW waves; tile BT x BT with BT = 32 * NW tokens x weight rows.  Waves in a
// WM x (NW/WM) grid, each computing MB x NB blocks of 32 x 32.  Per 64-wide K
// step: the activation tile (f16, from the converted copy) is DMA'd into one
// of two LDS stages; thread t dequantises half (t % 2) of weight row t / 2
// into one of two LDS weight buffers.  The next step's DMA and weight loads
// are issued before the current step's MFMAs, so one step of MFMA work hides
// their latency; one barrier per step.
//
// GLU: the N = 2 F weight rows are the value and gate halves of a SwiGLU
// (swiglu_split(gate, value) over the two halves of the product, with the
// bias ADD before it).  A tile then covers BT / 2 SwiGLU columns j: in each
// wave's NB blocks of 32 rows, block 2p holds value rows and block 2p + 1 the
// gate rows of the same 32 columns, so the accumulators of a (value, gate)
// pair sit in the same lane and register.  The epilogue adds both biases, forms
// silu(g) * v with k_swiglu's arithmetic and stores the SwiGLU rows [M, F]
// in f32 and / or f16 (the next GEMM's activation format).
//
// WH: the weights come as 16-bit rows rs bytes apart, so both tiles are
// DMA'd: a ring of GM_NS stages of 32-wide K steps, each stage's DMA issued
// GM_NS - 1 steps ahead, one barrier per step.  WT = TYPE_F16: the quantised
// weights dequantised once by k_w_to_f16 with the same arithmetic (the MFMAs
// run in the same k order, so the sums are the register-staged kernel's to the
// bit).  WT = TYPE_BF16: BF16 weight rows as stored, bf16 activations, the
// bf16 MFMA.
//
// WIDE (WH, NW = 4, BM = 256): 256 x 256 tiles on four waves, one per SIMD,
// each computing 128 x 128 (256 accumulators, in the AGPRs).  With no second
// wave on the SIMD to cover LDS latency, the operands of step ks + 1 are read
// into a second register set while the MFMAs of step ks run, and this
// thread's DMA instructions for step ks + 3 sit between those reads, so the
// MFMA pipe never waits on an LDS read or a DMA issue.  Per K step a wave
// reads (128 + 128) rows from LDS where the eight-wave layout read
// (128 + 64) rows per wave, a third less LDS traffic per MFMA.
constexpr int GM_NS = 4;

template <int WT, int NW, int WM, int BK, int BM, bool GLU, bool WH = false, bool WIDE = false>
__global__ __launch_bounds__(NW * 64) void k_gemm_q(const uint8_t * __restrict__ W, int64_t N, int64_t K, int64_t rs,
                                                     const _Float16 * __restrict__ xh, int64_t M,
                                                     const float * __restrict__ bias, const float * res, int64_t ldr,
                                                     float * y, int64_t ldy, GemmGlu glu, GemmMulti mul,
                                                     GemmSplit spl, int64_t n_ntiles, int64_t n_tiles) {
#pragma clang fp contract(off)
    constexpr int BT  = WIDE ? 256 : 32 * NW;  // weight rows per tile (thread t stages row t / 2)
    constexpr int T   = NW * 64;
    constexpr int WN  = NW / WM;
    constexpr int MB  = BM / WM / 32;
    constexpr int NB  = BT / WN / 32;
    constexpr int CPR = BK / 8;        // 16-byte chunks per tile row
    constexpr int SUB = BK / GM_BK > 0 ? BK / GM_BK : 1;  // 64-wide weight sub-steps per K step (register path)
    constexpr int XI  = BM * CPR / T;  // DMA instructions per thread per stage
    constexpr int TIX = BM * BK;       // halves per activation tile
    constexpr int TIL = BT * BK;       // halves per weight tile
    static_assert(MB >= 1 && XI >= 1, "tile shape");
    static_assert(!WH || BK == 32, "the f16-weight ring steps 32 columns");
    static_assert(!GLU || NB % 2 == 0, "GLU tiles pair value and gate blocks in each wave");
    static_assert(!WIDE || (WH && NW == 4 && (BM == 256 || BM == 192)), "the wide tiles run on the DMA ring, four waves");
    extern __shared__ __attribute__((aligned(16))) _Float16 g_lds[];
    _Float16 * sX = g_lds;            // 2 stages
    _Float16 * sW = g_lds + 2 * TIX;  // 2 buffers

    // consecutive work items (one XCD, one L2) share the operand that is
    // re-read most: the weight tile when there are more weight tiles than
    // token tiles (m_fast: its token tiles run together), else the
    // activation tiles, in groups of GM_GROUP token tiles with the token tile
    // fastest, so that the workgroups running together on an XCD cover a
    // block of GM_GROUP token tiles by several weight tiles and each weight
    // tile is fetched once per group rather than once per token tile
    // split-K: work items (part, tile), the parts of one tile n_base apart
    constexpr int GM_GROUP = 4;
    const int64_t n_base  = n_tiles / spl.n;
    const int64_t lin     = gm_xcd_remap(blockIdx.x, n_tiles);
    const int     kpart   = (int) (lin / n_base);
    const int64_t work    = lin % n_base;
    const int64_t n_mt    = n_base / n_ntiles;
    const bool    m_fast  = n_ntiles > n_mt;
    int64_t       tm, tn;  // token tile, weight tile
    if (m_fast) {
        tm = work % n_mt;
        tn = work / n_mt;
    } else {
        const int64_t gsz = (int64_t) GM_GROUP * n_ntiles;
        const int64_t g   = work / gsz, r = work % gsz;
        const int64_t gw  = min((int64_t) GM_GROUP, n_mt - g * GM_GROUP);
        tm                = g * GM_GROUP + r % gw;
        tn                = r / gw;
    }
    const int64_t m0 = tm * BM;
    int64_t       n0 = tn * BT;
    if (mul.n > 0) {
        // several weight matrices: this tile's rows come from matrix n0 / Nper
        const int mi = (int) (n0 / mul.Nper);
        n0 -= mi * mul.Nper;
        W    = mul.W[mi];
        y    = mul.y[mi];
        ldy  = mul.ldy[mi];
        bias = mul.bias[mi];
        N    = mul.Nper;
    }
    const int     tid  = threadIdx.x;
    const int     wave = tid >> 6;
    const int     lane = tid & 63;
    const int     wm   = wave / WN;
    const int     wn   = wave % WN;
    const int     lq   = lane & 31;
    const int     hh   = lane >> 5;

    // DMA sources: instruction i of wave w fills stage chunks (w XI + i) 64 + lane
    const int        wave_s = __builtin_amdgcn_readfirstlane(wave);
    const _Float16 * xsrc[XI];
#pragma unroll
    for (int i = 0; i < XI; i++) {
        const int     c = (wave * XI + i) * 64 + lane, r = c / CPR;
        const int64_t m = m0 + r < M ? m0 + r : M - 1;  // rows past M: any valid row, never stored
        xsrc[i]         = xh + m * K + 8 * ((c % CPR) ^ (r & 7));
    }
    const uint32_t lds_x = (uint32_t) (uintptr_t) (lds_half_t *) sX;
    auto           dma   = [&](int stage, int k0) {
#pragma unroll
        for (int i = 0; i < XI; i++) {
            dma16(xsrc[i] + k0, lds_x + 2u * (uint32_t) (stage * TIX + (wave_s * XI + i) * 512));
        }
    };

    const int       srow  = tid >> 1;
    const int       shalf = tid & 1;
    // the weight row of local tile row r (valid: inside the matrix)
    auto wrow_of = [&](int r, bool & valid) -> int64_t {
        if constexpr (GLU) {
            // local row (wave block, value / gate, 32-row offset) -> SwiGLU column j
            const int     wq = r / (BT / WN), blk = (r % (BT / WN)) / 32;
            const int64_t j  = n0 / 2 + wq * (BT / WN / 2) + (blk / 2) * 32 + (r % 32);
            valid            = j < glu.F;
            return (blk & 1) != (glu.swapped != 0) ? glu.F + j : j;
        } else {
            valid = n0 + r < N;
            return n0 + r;
        }
    };
    bool          w_ok;
    const int64_t wsel = wrow_of(srow, w_ok);  // weight row staged by this thread
    const uint8_t * wrow = W + (w_ok ? wsel : 0) * rs;
    WRaw            wr[SUB];
    auto            wload = [&](int k0) {
#pragma unroll
        for (int u = 0; u < SUB; u++) {
            w_load<WT>(wr[u], wrow, K, k0 + GM_BK * u, shalf);
        }
    };
    auto wstore = [&](int buf, int k0) {
#pragma unroll
        for (int u = 0; u < SUB; u++) {
            half8_t o[4];
            int     ch[4];
            w_dequant<WT>(wr[u], wrow, K, k0 + GM_BK * u, shalf, o, ch);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                *(half8_t *) &sW[buf * TIL + swz<BK>(srow, ch[j] + 8 * u)] = w_ok ? o[j] : half8_t{};
            }
        }
    };

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
    auto compute = [&](int buf) {
        const _Float16 * bx = sX + buf * TIX;
        const _Float16 * bw = sW + buf * TIL;
#pragma unroll
        for (int kk = 0; kk < BK / 16; kk++) {
            half8_t a[MB], b[NB];
#pragma unroll
            for (int i = 0; i < MB; i++) {
                a[i] = *(const half8_t *) &bx[swz<BK>(wm * (BM / WM) + i * 32 + lq, 2 * kk + hh)];
            }
#pragma unroll
            for (int j = 0; j < NB; j++) {
                b[j] = *(const half8_t *) &bw[swz<BK>(wn * (BT / WN) + j * 32 + lq, 2 * kk + hh)];
            }
#pragma unroll
            for (int i = 0; i < MB; i++) {
#pragma unroll
                for (int j = 0; j < NB; j++) {
                    acc[i][j] = gm_mfma(a[i], b[j], acc[i][j]);
                }
            }
        }
    };

    const int nk = (int) (K / BK / spl.n);  // K steps of this part
    const int kb = kpart * nk * BK;         // its first column
    if constexpr (WH) {
        // stage s: the activation tile then the weight tile; rows outside
        // the matrices read a valid row and are never stored
        constexpr int STG = TIX + TIL;
        constexpr int WI  = BT * CPR / T;  // weight DMA instructions per thread per stage
        constexpr int PER = XI + WI;
        static_assert(WI >= 1, "tile shape");
        const _Float16 * wsrc[WI];
#pragma unroll
        for (int i = 0; i < WI; i++) {
            const int     c = (wave * WI + i) * 64 + lane, r = c / CPR;
            bool          ok;
            const int64_t n = wrow_of(r, ok);
            wsrc[i]         = (const _Float16 *) (W + (ok ? n : 0) * rs) + 8 * ((c % CPR) ^ ((r >> 2) & 3));
        }
        const _Float16 * xs[XI];
#pragma unroll
        for (int i = 0; i < XI; i++) {
            const int     c = (wave * XI + i) * 64 + lane, r = c / CPR;
            const int64_t m = m0 + r < M ? m0 + r : M - 1;
            xs[i]           = xh + m * K + 8 * ((c % CPR) ^ ((r >> 2) & 3));
        }
        auto dma2 = [&](int st, int k0) {
#pragma unroll
            for (int i = 0; i < XI; i++) {
                dma16(xs[i] + k0, lds_x + 2u * (uint32_t) (st * STG + (wave_s * XI + i) * 512));
            }
#pragma unroll
            for (int i = 0; i < WI; i++) {
                dma16(wsrc[i] + k0, lds_x + 2u * (uint32_t) (st * STG + TIX + (wave_s * WI + i) * 512));
            }
        };
        auto compute2 = [&](int st) {
            const _Float16 * bx = g_lds + st * STG;
            const _Float16 * bw = bx + TIX;
#pragma unroll
            for (int kk = 0; kk < BK / 16; kk++) {
                half8_t a[MB], b[NB];
#pragma unroll
                for (int i = 0; i < MB; i++) {
                    a[i] = *(const half8_t *) &bx[swz32(wm * (BM / WM) + i * 32 + lq, 2 * kk + hh)];
                }
#pragma unroll
                for (int j = 0; j < NB; j++) {
                    b[j] = *(const half8_t *) &bw[swz32(wn * (BT / WN) + j * 32 + lq, 2 * kk + hh)];
                }
#pragma unroll
                for (int i = 0; i < MB; i++) {
#pragma unroll
                    for (int j = 0; j < NB; j++) {
                        if constexpr (WT == TYPE_BF16) {
                            acc[i][j] = gm_mfma_bf16(a[i], b[j], acc[i][j]);
                        } else {
                            acc[i][j] = gm_mfma(a[i], b[j], acc[i][j]);
                        }
                    }
                }
            }
        };
        if constexpr (WIDE) {
        constexpr int KK = BK / 16;
        half8_t ra0[KK][MB], rb0[KK][NB], ra1[KK][MB], rb1[KK][NB];
        auto mf = [&](const half8_t (&a)[KK][MB], const half8_t (&b)[KK][NB]) {
#pragma unroll
            for (int kk = 0; kk < KK; kk++) {
#pragma unroll
                for (int i = 0; i < MB; i++) {
#pragma unroll
                    for (int j = 0; j < NB; j++) {
                        if constexpr (WT == TYPE_BF16) {
                            acc[i][j] = gm_mfma_bf16(a[kk][i], b[kk][j], acc[i][j]);
                        } else {
                            acc[i][j] = gm_mfma(a[kk][i], b[kk][j], acc[i][j]);
                        }
                    }
                }
            }
        };
        // the operand reads of the step in stage sr, with this thread's DMA
        // of columns kd into stage sd spread between them (one instruction
        // every SP reads)
        auto rd = [&](half8_t (&a)[KK][MB], half8_t (&b)[KK][NB], int sr, auto dma_c, int sd, int kd) {
            constexpr bool D  = decltype(dma_c)::value;
            constexpr int  SP = KK * (MB + NB) / PER;
            static_assert(SP >= 1 && KK * (MB + NB) % PER == 0, "DMA spread");
            const _Float16 * bx = g_lds + sr * STG;
            const _Float16 * bw = bx + TIX;
#pragma unroll
            for (int g = 0; g < KK * (MB + NB); g++) {
                const int kk = g / (MB + NB), e = g % (MB + NB);
                if (e < MB) {
                    a[kk][e] = *(const half8_t *) &bx[swz32(wm * (BM / WM) + e * 32 + lq, 2 * kk + hh)];
                } else {
                    b[kk][e - MB] = *(const half8_t *) &bw[swz32(wn * (BT / WN) + (e - MB) * 32 + lq, 2 * kk + hh)];
                }
                if constexpr (D) {
                    if (g % SP == 0) {
                        const int d = g / SP;
                        if (d < XI) {
                            dma16(xs[d] + kd, lds_x + 2u * (uint32_t) (sd * STG + (wave_s * XI + d) * 512));
                        } else {
                            dma16(wsrc[d - XI] + kd,
                                  lds_x + 2u * (uint32_t) (sd * STG + TIX + (wave_s * WI + d - XI) * 512));
                        }
                    }
                }
            }
        };
        // every DMA runs, past the last step on the last step's columns into a
        // stage no step reads, so that the waits below count a fixed number
        // of instructions
#pragma unroll
        for (int st = 0; st < GM_NS - 1; st++) {
            dma2(st, kb + min(st, nk - 1) * BK);
        }
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"((GM_NS - 2) * PER) : "memory");
        __syncthreads();
        rd(ra0, rb0, 0, std::false_type{}, 0, 0);
        auto step = [&](auto cur_c, int ks) {
            // this thread's DMA of step ks + 1 in; the barrier publishes every
            // thread's and retires all reads of the stage the next DMA fills
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PER) : "memory");
            __syncthreads();
            __builtin_amdgcn_sched_barrier(0);
            const int sd = (ks + GM_NS - 1) % GM_NS, kd = kb + min(ks + GM_NS - 1, nk - 1) * BK;
            // past the last step the reads fetch a stage no step uses
            if constexpr (decltype(cur_c)::value == 0) {
                rd(ra1, rb1, (ks + 1) % GM_NS, std::true_type{}, sd, kd);
                mf(ra0, rb0);
            } else {
                rd(ra0, rb0, (ks + 1) % GM_NS, std::true_type{}, sd, kd);
                mf(ra1, rb1);
            }
            // one LDS read (and its DMA) between consecutive MFMA pairs
#pragma unroll
            for (int g = 0; g < KK * (MB + NB); g++) {
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
            }
            __builtin_amdgcn_sched_barrier(0);
        };
        int ks = 0;
        for (; ks + 1 < nk; ks += 2) {
            step(std::integral_constant<int, 0>{}, ks);
            step(std::integral_constant<int, 1>{}, ks + 1);
        }
        if (ks < nk) {
            step(std::integral_constant<int, 0>{}, ks);
        }
        } else {
#pragma unroll
        for (int st = 0; st < GM_NS - 1; st++) {
            if (st < nk) {
                dma2(st, kb + st * BK);
            }
        }
        // stage 0 in (the later stages may fly); every wait counts this
        // thread's own DMA instructions, loads returning in issue order
        if (nk >= GM_NS - 1) {
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"((GM_NS - 2) * PER) : "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        __syncthreads();
        for (int ks = 0; ks < nk; ks++) {
            const bool more = ks + GM_NS - 1 < nk;
            if (more) {
                dma2((ks + GM_NS - 1) % GM_NS, kb + (ks + GM_NS - 1) * BK);
            }
            __builtin_amdgcn_sched_barrier(0);
            compute2(ks % GM_NS);
            // step ks + 1's stage in before the barrier that publishes it
            if (more) {
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"((GM_NS - 2) * PER) : "memory");
            } else {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            }
            __syncthreads();
        }
        }
    } else {
    dma(0, kb);
    wload(kb);
    wstore(0, kb);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int ks = 0; ks < nk; ks++) {
        const int nxt = (ks + 1) & 1;
        if (ks + 1 < nk) {
            dma(nxt, kb + (ks + 1) * BK);
            __builtin_amdgcn_sched_barrier(0);
            wload(kb + (ks + 1) * BK);
            __builtin_amdgcn_sched_barrier(0);
        }
        compute(ks & 1);
        if (ks + 1 < nk) {
            wstore(nxt, kb + (ks + 1) * BK);
        }
        __builtin_amdgcn_s_waitcnt(0);  // this thread's DMA and LDS writes
        __syncthreads();
    }
    }

    // C[i = token][j = weight row]: lane holds row j = lq, tokens 8(r/4) + 4hh + r%4.
    // Each epilogue runs branch-free on whole tiles (all but the last row and
    // column of tiles): at the joins of per-element bounds branches the
    // compiler waits for every store in flight, one wait per element.
    const int64_t mw     = m0 + wm * (BM / WM) + 4 * hh;  // token of register 0 in block i = 0
    const bool    full_m = m0 + BM <= M;
    if constexpr (GLU) {
        // pair p of this wave: value block 2p, gate block 2p + 1, SwiGLU column j
        constexpr int NP = NB / 2;
        int64_t       jp[NP];
        float         bv[NP], bg[NP];
#pragma unroll
        for (int q = 0; q < NP; q++) {
            jp[q]            = n0 / 2 + wn * (BT / WN / 2) + q * 32 + lq;
            const bool    ok = jp[q] < glu.F;
            const int64_t rv = glu.swapped ? glu.F + jp[q] : jp[q];  // value row
            const int64_t rg = glu.swapped ? jp[q] : glu.F + jp[q];  // gate row
            bv[q]            = bias && ok ? bias[rv] : 0.0f;
            bg[q]            = bias && ok ? bias[rg] : 0.0f;
        }
        // the bias in registers before any store: a use behind a store's
        // bounds branch would otherwise wait for all stores in flight
        __builtin_amdgcn_s_waitcnt(0);
        auto go = [&](auto full_c) {
            constexpr bool FULL = decltype(full_c)::value;
#pragma unroll
            for (int q = 0; q < NP; q++) {
                const int64_t j = jp[q];
                if (j >= glu.F) {
                    continue;
                }
#pragma unroll
                for (int i = 0; i < MB; i++) {
                    float o[16];
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        float v = acc[i][2 * q][r], g = acc[i][2 * q + 1][r];
                        if (bias) {
                            v = v + bv[q];
                            g = g + bg[q];
                        }
                        const float silu = g / (1.0f + expf(-g));
                        o[r]             = silu * v;
                    }
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int64_t m = mw + i * 32 + 8 * (r / 4) + (r % 4);
                        if (FULL || m < M) {
                            if (glu.h) {
                                glu.h[m * glu.F + j] = o[r];
                            }
                            if (glu.hh) {
                                glu.hh[m * glu.F + j] = (_Float16) o[r];
                            }
                        }
                    }
                }
            }
        };
        if (full_m) {
            go(std::integral_constant<bool, true>{});
        } else {
            go(std::integral_constant<bool, false>{});
        }
        return;
    }
    const int64_t nl   = n0 + wn * (BT / WN) + lq;  // this lane's column in weight block 0
    const bool    full = full_m && n0 + BT <= N;
    if (spl.n > 1) {
        // partial sums of this K part; the reduce kernel adds the ADDs
        float * pp = spl.part + (int64_t) kpart * M * N;
        auto    go = [&](auto full_c) {
            constexpr bool FULL = decltype(full_c)::value;
#pragma unroll
            for (int i = 0; i < MB; i++) {
#pragma unroll
                for (int j = 0; j < NB; j++) {
                    const int64_t n = nl + 32 * j;
                    if (!FULL && n >= N) {
                        continue;
                    }
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int64_t m = mw + i * 32 + 8 * (r / 4) + (r % 4);
                        if (FULL || m < M) {
                            pp[m * N + n] = acc[i][j][r];
                        }
                    }
                }
            }
        };
        if (full) {
            go(std::integral_constant<bool, true>{});
        } else {
            go(std::integral_constant<bool, false>{});
        }
        return;
    }
    // Epilogue: the bias ADD, then the residual ADD, each rounded as its op.
    // The bias is loaded once per column, and each 32 x 32 block's residual
    // values are loaded before the previous block's stores are issued (loads
    // and stores share one completion counter, so a load issued behind
    // stores would wait for them too).  In place (res == y) every element is
    // read before this thread writes it, and no other thread touches it.
    float bn[NB];
#pragma unroll
    for (int j = 0; j < NB; j++) {
        bn[j] = bias && nl + 32 * j < N ? bias[nl + 32 * j] : 0.0f;
    }
    __builtin_amdgcn_s_waitcnt(0);  // the bias in registers before any store
    auto go = [&](auto full_c) {
        constexpr bool FULL = decltype(full_c)::value;
        float          rv[16];
        auto           rload = [&](int b) {
            const int64_t n = nl + 32 * (b % NB);
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int64_t m = mw + (b / NB) * 32 + 8 * (r / 4) + (r % 4);
                rv[r]           = FULL || (m < M && n < N) ? res[m * ldr + n] : 0.0f;
            }
        };
        if (res) {
            rload(0);
        }
#pragma unroll
        for (int b = 0; b < MB * NB; b++) {
            const int     i = b / NB, j = b % NB;
            const int64_t n = nl + 32 * j;
            float         v[16];
#pragma unroll
            for (int r = 0; r < 16; r++) {
                v[r] = bias ? acc[i][j][r] + bn[j] : acc[i][j][r];
            }
            if (res) {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    v[r] = rv[r] + v[r];
                }
                if (b + 1 < MB * NB) {
                    rload(b + 1);
                }
            }
            if (!FULL && n >= N) {
                continue;
            }
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int64_t m = mw + i * 32 + 8 * (r / 4) + (r % 4);
                if (FULL || m < M) {
                    y[m * ldy + n] = v[r];
                }
            }
        }
    };
    if (full) {
        go(std::integral_constant<bool, true>{});
    } else {
        go(std::integral_constant<bool, false>{});
    }
}

// Split-K reduction: y[m, n] = ((part_0 + part_1 + ...) + bias[n]) + res[m, n],
// the parts summed in order, each ADD rounded as its op; 4 columns per thread.
__global__ void k_splitk_reduce(const float * __restrict__ part, int nparts, int64_t M, int64_t N,
                                const float * __restrict__ bias, const float * res, int64_t ldr, float * y,
                                int64_t ldy) {
#pragma clang fp contract(off)
    const int64_t n4 = N / 4;
    for (int64_t t = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; t < M * n4; t += (int64_t) gridDim.x * blockDim.x) {
        const int64_t m = t / n4, n = (t % n4) * 4;
        float4_t      v = *(const float4_t *) (part + m * N + n);
        for (int p = 1; p < nparts; p++) {
            const float4_t w = *(const float4_t *) (part + ((int64_t) p * M + m) * N + n);
            v[0]             = v[0] + w[0];
            v[1]             = v[1] + w[1];
            v[2]             = v[2] + w[2];
            v[3]             = v[3] + w[3];
        }
#pragma unroll
        for (int k = 0; k < 4; k++) {
            if (bias) {
                v[k] = v[k] + bias[n + k];
            }
            if (res) {
                v[k] = res[m * ldr + n + k] + v[k];
            }
            y[m * ldy + n + k] = v[k];
        }
    }
}

// Activations f32 -> f16 (round to nearest even), rows of K into a packed
// [M, K] copy: 8 elements per thread per pass.
__device__ __forceinline__ void x_to_f16_part(const float * __restrict__ x, int64_t ldx, int64_t K, int64_t n8,
                                              _Float16 * __restrict__ xh, int64_t t0, int64_t stride) {
    for (int64_t t = t0; t < n8; t += stride) {
        const int64_t  e = t * 8, m = e / K, k = e % K;
        const float4_t a = *(const float4_t *) (x + m * ldx + k);
        const float4_t b = *(const float4_t *) (x + m * ldx + k + 4);
        half8_t        o;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            o[j]     = (_Float16) a[j];
            o[4 + j] = (_Float16) b[j];
        }
        *(half8_t *) (xh + e) = o;
    }
}

__global__ void k_x_to_f16(const float * __restrict__ x, int64_t ldx, int64_t K, int64_t n8,
                           _Float16 * __restrict__ xh) {
    x_to_f16_part(x, ldx, K, n8, xh, blockIdx.x * (int64_t) blockDim.x + threadIdx.x, (int64_t) gridDim.x * blockDim.x);
}

// Activations f32 -> bf16 (ggml's rounding: nearest-even, NaN quiet) into a
// packed [M, K] copy of 16-bit patterns, 8 elements per thread per pass.
__global__ void k_x_to_bf16(const float * __restrict__ x, int64_t ldx, int64_t K, int64_t n8,
                            uint16_t * __restrict__ xb) {
    for (int64_t t = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; t < n8; t += (int64_t) gridDim.x * blockDim.x) {
        const int64_t  e = t * 8, m = e / K, k = e % K;
        const float4_t a = *(const float4_t *) (x + m * ldx + k);
        const float4_t b = *(const float4_t *) (x + m * ldx + k + 4);
        uint32_t       o[4];
#pragma unroll
        for (int j = 0; j < 2; j++) {
            o[j]     = (__float_as_uint(round_bf16(a[2 * j])) >> 16) | (__float_as_uint(round_bf16(a[2 * j + 1])) & 0xffff0000u);
            o[2 + j] = (__float_as_uint(round_bf16(b[2 * j])) >> 16) | (__float_as_uint(round_bf16(b[2 * j + 1])) & 0xffff0000u);
        }
        *(int4_t *) (xb + e) = int4_t{ (int) o[0], (int) o[1], (int) o[2], (int) o[3] };
    }
}

// Weights -> f16 rows [N][K] (row stride K), the register-staged kernel's
// dequantisation: thread (row, 64-wide K step, half) dequantises its 32
// values exactly (f32, then f16) and writes them as four 16-byte chunks.
template <int WT>
__device__ __forceinline__ void w_to_f16_part(const uint8_t * __restrict__ W, int64_t N, int64_t K, int64_t rs,
                                              _Float16 * __restrict__ wh, int64_t t) {
    const int64_t nsteps = K / GM_BK;
    if (t >= N * nsteps * 2) {
        return;
    }
    const int       half = (int) (t & 1);
    const int64_t   st   = (t >> 1) % nsteps;
    const int64_t   row  = (t >> 1) / nsteps;
    const uint8_t * wr   = W + row * rs;
    const int       k0   = (int) (st * GM_BK);
    WRaw            w;
    w_load<WT>(w, wr, K, k0, half);
    half8_t o[4];
    int     ch[4];
    w_dequant<WT>(w, wr, K, k0, half, o, ch);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        *(half8_t *) (wh + row * K + k0 + 8 * ch[j]) = o[j];
    }
}

template <int WT>
__global__ __launch_bounds__(256) void k_w_to_f16(const uint8_t * __restrict__ W, int64_t N, int64_t K, int64_t rs,
                                                   _Float16 * __restrict__ wh) {
    w_to_f16_part<WT>(W, N, K, rs, wh, (int64_t) blockIdx.x * 256 + threadIdx.x);
}

// Both conversions of a GEMM call in one launch: workgroups [0, nbw) convert
// the weight rows, the rest the activations (grid-stride over them), so the
// two streams share one launch; the dequantising weight workgroups, the
// slower per byte, are dispatched first and run beside the activation stream
// instead of after it.
template <int WT>
__global__ __launch_bounds__(256) void k_xw_to_f16(const float * __restrict__ x, int64_t ldx, int64_t K, int64_t n8,
                                                    _Float16 * __restrict__ xh, int nbw,
                                                    const uint8_t * __restrict__ W, int64_t N, int64_t rs,
                                                    _Float16 * __restrict__ wh) {
    if ((int) blockIdx.x < nbw) {
        w_to_f16_part<WT>(W, N, K, rs, wh, (int64_t) blockIdx.x * 256 + threadIdx.x);
    } else {
        const int64_t nbx = (int64_t) gridDim.x - nbw;
        x_to_f16_part(x, ldx, K, n8, xh, (blockIdx.x - nbw) * (int64_t) 256 + threadIdx.x, nbx * 256);
    }
}

static int weights_to_f16(int wtype, const uint8_t * W, int64_t N, int64_t K, int64_t rs, _Float16 * wh,
                          hipStream_t stream) {
    const int64_t n  = N * (K / GM_BK) * 2;
    const int64_t nb = (n + 255) / 256;
    if (nb > 0x7fffffff) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "mul_mat gemm: weight rows too large");
    }
    switch (wtype) {
        case TYPE_Q8_0: hipLaunchKernelGGL(k_w_to_f16<TYPE_Q8_0>, dim3((unsigned) nb), dim3(256), 0, stream, W, N, K, rs, wh); break;
        case TYPE_Q4_K: hipLaunchKernelGGL(k_w_to_f16<TYPE_Q4_K>, dim3((unsigned) nb), dim3(256), 0, stream, W, N, K, rs, wh); break;
        case TYPE_Q5_K: hipLaunchKernelGGL(k_w_to_f16<TYPE_Q5_K>, dim3((unsigned) nb), dim3(256), 0, stream, W, N, K, rs, wh); break;
        default: hipLaunchKernelGGL(k_w_to_f16<TYPE_Q6_K>, dim3((unsigned) nb), dim3(256), 0, stream, W, N, K, rs, wh); break;
    }
    return check_launch("mul_mat gemm: weights to f16");
}

bool gemm_supported(int wtype, int64_t N, int64_t K, int64_t rs, const void * W, const float * x, int64_t ldx) {
    if (!is_repacked_type(wtype) || N <= 0 || K % GM_BK != 0 || rs < row_bytes(wtype, K)) {
        return false;
    }
    if (wtype != TYPE_Q8_0 && K % 256 != 0) {
        return false;
    }
    // 16-byte weight and activation loads
    return rs % 16 == 0 && ((uintptr_t) W) % 16 == 0 && ((uintptr_t) x) % 16 == 0 && ldx % 4 == 0;
}

size_t gemm_workspace(int64_t K, int64_t M) {
    return (size_t) M * (size_t) K * sizeof(_Float16);
}

template <int NW, int WM, int BK, int BM = 32 * NW, bool WH = false, bool WIDE = false>
static int launch_gemm(int wtype, const uint8_t * W, int64_t N, int64_t K, int64_t rs, const _Float16 * xh, int64_t M,
                       const float * bias, const float * res, int64_t ldr, float * y, int64_t ldy, const GemmGlu & glu,
                       const GemmMulti & mul, const GemmSplit & spl, hipStream_t stream) {
    constexpr int BT   = WIDE ? 256 : 32 * NW;
    const int64_t n_nt = (N + BT - 1) / BT;
    const int64_t n_mt = (M + BM - 1) / BM;
    const int64_t n    = n_nt * n_mt * spl.n;
    if (n > 0x7fffffff) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "mul_mat gemm: too many tiles");
    }
    if (K / BK / spl.n < 1) {
        // every K part holds at least one step (the ring's prologue loads step 0)
        return set_error(MMHIP_ERR_UNSUPPORTED, "mul_mat gemm: K = %lld too short for %d parts", (long long) K, spl.n);
    }
    const size_t lds = (size_t) (WH ? GM_NS : 2) * (BM + BT) * BK * sizeof(_Float16);
    auto         go  = [&](auto kern) -> int {
        if (lds > 64 * 1024 && !ensure_lds_limit((const void *) kern, lds)) {
            return set_error(MMHIP_ERR_HIP, "mul_mat gemm: cannot raise LDS limit to %zu", lds);
        }
        hipLaunchKernelGGL(kern, dim3((unsigned) n), dim3(NW * 64), lds, stream, W, N, K, rs, xh, M, bias, res, ldr, y,
                           ldy, glu, mul, spl, n_nt, n);
        return check_launch("mul_mat gemm");
    };
    if constexpr (WH) {
        // 16-bit weight rows: f16 copies of any block type, or BF16 as stored
        if (wtype == TYPE_BF16) {
            return go(k_gemm_q<TYPE_BF16, NW, WM, BK, BM, false, true, WIDE>);
        }
        return glu.F > 0 ? go(k_gemm_q<TYPE_F16, NW, WM, BK, BM, true, true, WIDE>)
                         : go(k_gemm_q<TYPE_F16, NW, WM, BK, BM, false, true, WIDE>);
    } else {
        if (glu.F > 0) {
            switch (wtype) {
                case TYPE_Q8_0: return go(k_gemm_q<TYPE_Q8_0, NW, WM, BK, BM, true>);
                case TYPE_Q4_K: return go(k_gemm_q<TYPE_Q4_K, NW, WM, BK, BM, true>);
                case TYPE_Q5_K: return go(k_gemm_q<TYPE_Q5_K, NW, WM, BK, BM, true>);
                default: return go(k_gemm_q<TYPE_Q6_K, NW, WM, BK, BM, true>);
            }
        }
        switch (wtype) {
            case TYPE_Q8_0: return go(k_gemm_q<TYPE_Q8_0, NW, WM, BK, BM, false>);
            case TYPE_Q4_K: return go(k_gemm_q<TYPE_Q4_K, NW, WM, BK, BM, false>);
            case TYPE_Q5_K: return go(k_gemm_q<TYPE_Q5_K, NW, WM, BK, BM, false>);
            default: return go(k_gemm_q<TYPE_Q6_K, NW, WM, BK, BM, false>);
        }
    }
}

// Tile configuration by shape (activations already f16, rows of K).
static int gemm_launch(int wtype, const uint8_t * wb, int64_t N, int64_t K, int64_t rs, const _Float16 * xh, int64_t M,
                       const float * bias, const float * res, int64_t ldr, float * y, int64_t ldy, const GemmGlu & glu,
                       const GemmMulti & mul, const GemmSplit & spl, hipStream_t stream, bool wh = false) {
    const int64_t tiles256 = ((N + 255) / 256) * ((M + 255) / 256);
    if (wh) {
        // f16 weight rows (row stride K): the DMA ring on the same tile choice.
        // 192-token tiles (3/4 of the work of a 256-token tile) where they
        // take fewer rounds of the 256 CUs by that weight: the DiT's 1380
        // tokens fill 8 of them (5.4 of 256) and its projections' grids of
        // 144 to 384 tiles of 256 run a partly filled round
        const int64_t nn     = (N + 255) / 256;
        const int64_t r256   = (nn * ((M + 255) / 256) * spl.n + 255) / 256;
        const int64_t r192   = (nn * ((M + 191) / 192) * spl.n + 255) / 256;
        const bool    bm192  = 3 * r192 < 4 * r256;
        auto          wide   = [&](const float * bi, const float * re, int64_t lr, float * yy, int64_t ly) {
            return bm192 ? launch_gemm<4, 2, 32, 192, true, true>(wtype, wb, N, K, K * 2, xh, M, bi, re, lr, yy, ly, glu,
                                                                   mul, spl, stream)
                         : launch_gemm<4, 2, 32, 256, true, true>(wtype, wb, N, K, K * 2, xh, M, bi, re, lr, yy, ly, glu,
                                                                   mul, spl, stream);
        };
        if (spl.n > 1) {
            int rc = wide(nullptr, nullptr, 0, nullptr, N);
            if (rc != MMHIP_OK) {
                return rc;
            }
            const int64_t nt = M * (N / 4);
            const int64_t nb = (nt + 255) / 256;
            hipLaunchKernelGGL(k_splitk_reduce, dim3((unsigned) (nb < 16384 ? nb : 16384)), dim3(256), 0, stream,
                               (const float *) spl.part, spl.n, M, N, bias, res, ldr, y, ldy);
            return check_launch("mul_mat gemm: split-K reduce");
        }
        if (tiles256 >= 256 || (mul.n > 0 && tiles256 >= 128)) {
            return wide(bias, res, ldr, y, ldy);
        }
        return launch_gemm<4, 2, 32, 64, true>(wtype, wb, N, K, K * 2, xh, M, bias, res, ldr, y, ldy, glu, mul, spl,
                                               stream);
    }
    if (spl.n > 1) {
        // 256 x 256 tiles over K parts, then the ordered reduction with the ADDs
        const GemmSplit sp = spl;
        int rc = launch_gemm<8, 2, 64>(wtype, wb, N, K, rs, xh, M, nullptr, nullptr, 0, nullptr, N, glu, mul, sp, stream);
        if (rc != MMHIP_OK) {
            return rc;
        }
        const int64_t nt = M * (N / 4);
        const int64_t nb = (nt + 255) / 256;
        hipLaunchKernelGGL(k_splitk_reduce, dim3((unsigned) (nb < 16384 ? nb : 16384)), dim3(256), 0, stream,
                           (const float *) spl.part, spl.n, M, N, bias, res, ldr, y, ldy);
        return check_launch("mul_mat gemm: split-K reduce");
    }
    // several weight matrices in one launch: 256 x 256 tiles once they fill
    // half the CUs (the DiT's q / k / v: 144 tiles), where three launches of
    // small tiles ran at half the MFMA rate
    if (tiles256 >= 256 || (mul.n > 0 && tiles256 >= 128)) {
        return launch_gemm<8, 2, 64>(wtype, wb, N, K, rs, xh, M, bias, res, ldr, y, ldy, glu, mul, spl, stream);
    }
    // small grids (the DiT's 2048-row projections at 1380 tokens: 176 tiles of
    // 128 x 128): 64-token x 128-row tiles, twice the workgroups, three per CU
    // in LDS (a 128-wide K step on 128 x 128 tiles: 2.6 % slower per DiT block;
    // 32 x 128 and 128 x 256 tiles: 1 % and 25 % slower)
    return launch_gemm<4, 2, 64, 64>(wtype, wb, N, K, rs, xh, M, bias, res, ldr, y, ldy, glu, mul, spl, stream);
}

// K parts for a shape: few 256 x 256 tiles (under half the CUs) and a long
// K (the DiT's ff_out: 48 tiles, K = 8192) split K four ways.
int gemm_split(int64_t N, int64_t K, int64_t M) {
    const int64_t tiles256 = ((N + 255) / 256) * ((M + 255) / 256);
    return tiles256 < 128 && K >= 4096 && K % (4 * GM_BK) == 0 && N % 4 == 0 ? 4 : 1;
}

size_t gemm_split_bytes(int64_t N, int64_t K, int64_t M) {
    const int s = gemm_split(N, K, M);
    return s > 1 ? (size_t) s * (size_t) M * (size_t) N * sizeof(float) : 0;
}

// Whether the weights go to f16 once before the GEMM.  In the register-staged
// kernel every token tile dequantises the whole weight tile again, and that
// VALU work, not the MFMAs, sets its pace; the f16 ring kernel runs 10-25 %
// faster on the same shapes, which pays for the extra pass over the weights
// (their bytes plus 2 per value) from about 1500 tokens on (measured: 8192
// tokens x 6144 x 2048 Q4_K 270 -> 229 + 8 us; 1380 tokens x 16384 x 2048
// Q8_0 147 -> 133 + 25 us).
bool gemm_use_wh(int64_t N, int64_t K, int64_t M) {
    (void) N;
    (void) K;
    return M >= 2048 && getenv("GGML_MI355X_DISABLE_GEMM_WH") == nullptr;
}

size_t gemm_wh_bytes(int64_t N, int64_t K, int64_t M) {
    return gemm_use_wh(N, K, M) ? ((size_t) N * (size_t) K * sizeof(_Float16) + 255) / 256 * 256 : 0;
}

size_t gemm_q_workspace(int64_t N, int64_t K, int64_t M) {
    const size_t xo = (gemm_workspace(K, M) + 255) / 256 * 256;
    return xo + gemm_wh_bytes(N, K, M) + gemm_split_bytes(N, K, M);
}

// f16 copies of quantised weights (rows [N][K], k_w_to_f16's values) that a
// caller made once and registered, keyed by the quantised weight's address:
// the token-count GEMMs then run the DMA ring on them with no conversion.
// The results are the register-staged kernel's to the bit either way.
struct F16Weights {
    int64_t      N, K;
    const void * wh;
};

static std::mutex                                     g_f16w_mu;
static std::unordered_map<const void *, F16Weights> g_f16w;

int register_f16_weights(const void * W, int64_t N, int64_t K, const void * wh) {
    if (!W || !wh || N <= 0 || K <= 0 || K % 32 != 0 || ((uintptr_t) wh) % 16 != 0) {
        return set_error(MMHIP_ERR_INVALID, "register_weights_f16: bad arguments N=%lld K=%lld", (long long) N,
                         (long long) K);
    }
    std::lock_guard<std::mutex> lk(g_f16w_mu);
    g_f16w[W] = F16Weights{ N, K, wh };
    return MMHIP_OK;
}

int unregister_f16_weights(const void * W) {
    std::lock_guard<std::mutex> lk(g_f16w_mu);
    return g_f16w.erase(W) ? MMHIP_OK : set_error(MMHIP_ERR_INVALID, "unregister_weights_f16: not registered");
}

// The registered copy of W (N rows of K), or null.
static const void * f16_weights(const void * W, int64_t N, int64_t K) {
    std::lock_guard<std::mutex> lk(g_f16w_mu);
    if (g_f16w.empty()) {
        return nullptr;
    }
    const auto it = g_f16w.find(W);
    return it != g_f16w.end() && it->second.N == N && it->second.K == K ? it->second.wh : nullptr;
}

int weights_to_f16_checked(int wtype, const void * W, int64_t N, int64_t K, int64_t rs, void * wh, hipStream_t stream) {
    if (!W || !wh || !gemm_supported(wtype, N, K, rs, W, (const float *) wh, K)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "weights_to_f16: type %d N=%lld K=%lld rs=%lld", wtype, (long long) N,
                         (long long) K, (long long) rs);
    }
    return weights_to_f16(wtype, (const uint8_t *) W, N, K, rs, (_Float16 *) wh, stream);
}

int gemm_q_h(int wtype, const void * W, int64_t N, int64_t K, int64_t rs, const void * xh, int64_t M, float * y,
             int64_t ldy, hipStream_t stream, const float * bias, const float * res, int64_t ldr, const GemmGlu * glu,
             const GemmMulti * mul, void * split_ws, size_t split_ws_bytes) {
    if (!gemm_supported(wtype, N, K, rs, W, (const float *) xh, K) || ((uintptr_t) xh) % 16 != 0) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "mul_mat gemm (f16 activations): type %d N=%lld K=%lld rs=%lld not supported",
                         wtype, (long long) N, (long long) K, (long long) rs);
    }
    const GemmGlu   none{};
    const GemmMulti single{};
    GemmSplit       spl;
    if (!glu && !mul && split_ws && split_ws_bytes >= gemm_split_bytes(N, K, M) && ((uintptr_t) split_ws) % 16 == 0) {
        spl.n    = gemm_split(N, K, M);
        spl.part = (float *) split_ws;
    }
    // registered f16 copies (every matrix of a multi call): the DMA ring
    GemmMulti    mf = mul ? *mul : single;
    const void * wh = nullptr;
    if (mul) {
        bool all = mul->n > 0;
        for (int i = 0; i < mul->n && all; i++) {
            const void * p = f16_weights(mul->W[i], mul->Nper, K);
            all            = p != nullptr;
            mf.W[i]        = (const uint8_t *) p;
        }
        wh = all ? mf.W[0] : nullptr;
        if (!all) {
            mf = *mul;
        }
    } else {
        wh = f16_weights(W, N, K);
    }
    return gemm_launch(wtype, (const uint8_t *) (wh ? wh : W), N, K, rs, (const _Float16 *) xh, M, bias, res, ldr, y,
                       ldy, glu ? *glu : none, mf, spl, stream, wh != nullptr);
}

int convert_act_f16(const float * x, int64_t ldx, int64_t K, int64_t M, void * xh, hipStream_t stream) {
    const int64_t n8 = M * K / 8;
    const int64_t nb = (n8 + 255) / 256;
    hipLaunchKernelGGL(k_x_to_f16, dim3((unsigned) (nb < 8192 ? nb : 8192)), dim3(256), 0, stream, x, ldx, K, n8,
                       (_Float16 *) xh);
    return check_launch("mul_mat gemm: convert");
}

int gemm_q(int wtype, const void * W, int64_t N, int64_t K, int64_t rs, const float * x, int64_t ldx, int64_t M,
           float * y, int64_t ldy, void * ws, size_t ws_bytes, hipStream_t stream, const float * bias,
           const float * res, int64_t ldr, const GemmGlu * glu) {
    if (!gemm_supported(wtype, N, K, rs, W, x, ldx)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "mul_mat gemm: type %d N=%lld K=%lld rs=%lld not supported", wtype,
                         (long long) N, (long long) K, (long long) rs);
    }
    const size_t need = gemm_workspace(K, M);
    if (!ws || ws_bytes < need || ((uintptr_t) ws) % 16 != 0) {
        return set_error(MMHIP_ERR_WORKSPACE, "mul_mat gemm: workspace %zu < %zu (16-byte aligned)", ws_bytes, need);
    }
    _Float16 *    xh  = (_Float16 *) ws;
    const int64_t n8  = M * K / 8;
    const int64_t nb  = (n8 + 255) / 256;
    const int     nbx = (int) (nb < 8192 ? nb : 8192);
    int           rc  = MMHIP_OK;
    const GemmGlu   none{};
    const GemmMulti single{};
    GemmSplit       spl;
    // workspace: the f16 activations, [the f16 weights,] [the partial sums]
    const size_t    xo  = (need + 255) / 256 * 256;
    const size_t    whb = gemm_wh_bytes(N, K, M);
    const bool      wh  = whb && ws_bytes >= xo + whb;
    const size_t    so  = xo + (wh ? whb : 0);
    const size_t    sb  = gemm_split_bytes(N, K, M);
    if (!glu && sb && ws_bytes >= so + sb) {
        spl.n    = gemm_split(N, K, M);
        spl.part = (float *) ((char *) ws + so);
    }
    const uint8_t * wb  = (const uint8_t *) W;
    const void *    reg = f16_weights(W, N, K);  // a registered f16 copy: no conversion
    const int64_t   nw  = (N * (K / GM_BK) * 2 + 255) / 256;  // weight-conversion workgroups
    if (!reg && wh && nbx + nw <= 0x7fffffff) {
        // the activations and the weights to f16 in one launch
        _Float16 * whp = (_Float16 *) ((char *) ws + xo);
        const dim3 g((unsigned) (nbx + nw));
        switch (wtype) {
            case TYPE_Q8_0: hipLaunchKernelGGL(k_xw_to_f16<TYPE_Q8_0>, g, dim3(256), 0, stream, x, ldx, K, n8, xh, (int) nw, wb, N, rs, whp); break;
            case TYPE_Q4_K: hipLaunchKernelGGL(k_xw_to_f16<TYPE_Q4_K>, g, dim3(256), 0, stream, x, ldx, K, n8, xh, (int) nw, wb, N, rs, whp); break;
            case TYPE_Q5_K: hipLaunchKernelGGL(k_xw_to_f16<TYPE_Q5_K>, g, dim3(256), 0, stream, x, ldx, K, n8, xh, (int) nw, wb, N, rs, whp); break;
            default: hipLaunchKernelGGL(k_xw_to_f16<TYPE_Q6_K>, g, dim3(256), 0, stream, x, ldx, K, n8, xh, (int) nw, wb, N, rs, whp); break;
        }
        rc = check_launch("mul_mat gemm: convert");
        if (rc != MMHIP_OK) {
            return rc;
        }
        wb = (const uint8_t *) whp;
    } else {
        hipLaunchKernelGGL(k_x_to_f16, dim3((unsigned) nbx), dim3(256), 0, stream, x, ldx, K, n8, xh);
        rc = check_launch("mul_mat gemm: convert");
        if (rc != MMHIP_OK) {
            return rc;
        }
        if (reg) {
            wb = (const uint8_t *) reg;
        } else if (wh) {
            _Float16 * whp = (_Float16 *) ((char *) ws + xo);
            rc             = weights_to_f16(wtype, wb, N, K, rs, whp, stream);
            if (rc != MMHIP_OK) {
                return rc;
            }
            wb = (const uint8_t *) whp;
        }
    }
    return gemm_launch(wtype, wb, N, K, rs, xh, M, bias, res, ldr, y, ldy, glu ? *glu : none, single, spl, stream,
                       wh || reg);
}

// BF16 weights at token counts: rows rs bytes apart read in place by the
// 16-bit DMA ring (K % 32 == 0, 16-byte rows), activations rounded to bf16
// into the workspace first.
bool gemm_bf16_supported(int64_t N, int64_t K, int64_t rs, const void * W, const float * x, int64_t ldx) {
    return N > 0 && K > 0 && K % 32 == 0 && rs >= 2 * K && rs % 16 == 0 && ((uintptr_t) W) % 16 == 0 &&
           ((uintptr_t) x) % 16 == 0 && ldx % 4 == 0;
}

size_t gemm_bf16_workspace(int64_t K, int64_t M) {
    return (size_t) M * (size_t) K * sizeof(uint16_t);
}

int gemm_bf16(const void * W, int64_t N, int64_t K, int64_t rs, const float * x, int64_t ldx, int64_t M, float * y,
              int64_t ldy, void * ws, size_t ws_bytes, hipStream_t stream) {
    if (!gemm_bf16_supported(N, K, rs, W, x, ldx)) {
        return set_error(MMHIP_ERR_UNSUPPORTED,
                         "mul_mat bf16 gemm: N=%lld K=%lld rs=%lld (K %% 32 == 0, 16-byte aligned rows)",
                         (long long) N, (long long) K, (long long) rs);
    }
    const size_t need = gemm_bf16_workspace(K, M);
    if (!ws || ws_bytes < need || ((uintptr_t) ws) % 16 != 0) {
        return set_error(MMHIP_ERR_WORKSPACE, "mul_mat bf16 gemm: workspace %zu < %zu (16-byte aligned)", ws_bytes,
                         need);
    }
    const int64_t n8 = M * K / 8;
    const int64_t nb = (n8 + 255) / 256;
    hipLaunchKernelGGL(k_x_to_bf16, dim3((unsigned) (nb < 8192 ? nb : 8192)), dim3(256), 0, stream, x, ldx, K, n8,
                       (uint16_t *) ws);
    int rc = check_launch("mul_mat bf16 gemm: convert");
    if (rc != MMHIP_OK) {
        return rc;
    }
    const GemmGlu   none{};
    const GemmMulti single{};
    const GemmSplit one{};
    const uint8_t * wb       = (const uint8_t *) W;
    const auto *    xb       = (const _Float16 *) ws;  // 16-bit patterns
    const int64_t   tiles256 = ((N + 255) / 256) * ((M + 255) / 256);
    if (tiles256 >= 256) {
        // 192-token tiles where they take fewer rounds by work (gemm_launch's rule)
        const int64_t nn = (N + 255) / 256;
        if (3 * ((nn * ((M + 191) / 192) + 255) / 256) < 4 * ((tiles256 + 255) / 256)) {
            return launch_gemm<4, 2, 32, 192, true, true>(TYPE_BF16, wb, N, K, rs, xb, M, nullptr, nullptr, 0, y, ldy,
                                                          none, single, one, stream);
        }
        return launch_gemm<4, 2, 32, 256, true, true>(TYPE_BF16, wb, N, K, rs, xb, M, nullptr, nullptr, 0, y, ldy, none,
                                                      single, one, stream);
    }
    return launch_gemm<4, 2, 32, 64, true>(TYPE_BF16, wb, N, K, rs, xb, M, nullptr, nullptr, 0, y, ldy, none, single,
                                           one, stream);
}

// F32 weights at token counts (the DiT's k = 1 convs, src/dit.h:258 and
// :285, which the quantiser leaves in F32): y[m, n] = sum_k x[m, k] * W[n, k]
// on v_mfma_f32_32x32x2f32, f32 products summed in f32 as ggml-CPU's f32 dot
// sums them (in another order).  One wave per 64 tokens x 64 weight rows,
// four 32 x 32 accumulators (tokens are the A operand, so a lane's outputs
// share one weight row and 32 lanes store 128 contiguous bytes of a y row).
// Per 32-wide K chunk lane l reads 16 consecutive floats (64 bytes) of token
// row / weight row l % 32 at k offset 16 (l / 32); MFMA step s (0..15) takes
// element s, so the two lane halves supply k = s and k = 16 + s: every k of
// the chunk once, the same k for both operands.  Rows past M or N are read as
// the last row (in bounds) and not stored.  The next chunk's loads are in
// flight while the current chunk's 64 MFMAs run.
__global__ __launch_bounds__(64) void k_gemm_f32(const float * __restrict__ W, int64_t ldw, const float * __restrict__ x,
                                                 int64_t ldx, int64_t N, int64_t K, int64_t M, float * __restrict__ y,
                                                 int64_t ldy) {
    const int     l = threadIdx.x, li = l & 31, h = l >> 5;
    const int64_t n0 = (int64_t) blockIdx.x * 64, m0 = (int64_t) blockIdx.y * 64;
    const float * pw[2];
    const float * px[2];
#pragma unroll
    for (int b = 0; b < 2; b++) {
        const int64_t n = n0 + 32 * b + li, m = m0 + 32 * b + li;
        pw[b]           = W + (n < N ? n : N - 1) * ldw + 16 * h;
        px[b]           = x + (m < M ? m : M - 1) * ldx + 16 * h;
    }
    float16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                acc[i][j][r] = 0.0f;
            }
        }
    }
    float4_t ca[2][4], cw[2][4];
#pragma unroll
    for (int b = 0; b < 2; b++) {
#pragma unroll
        for (int c = 0; c < 4; c++) {
            ca[b][c] = *(const float4_t *) (px[b] + 4 * c);
            cw[b][c] = *(const float4_t *) (pw[b] + 4 * c);
        }
    }
    for (int64_t k0 = 0; k0 < K; k0 += 32) {
        float4_t na[2][4], nw[2][4];
        const int64_t kn = k0 + 32 < K ? k0 + 32 : k0;  // the last chunk reloads itself (in bounds)
#pragma unroll
        for (int b = 0; b < 2; b++) {
#pragma unroll
            for (int c = 0; c < 4; c++) {
                na[b][c] = *(const float4_t *) (px[b] + kn + 4 * c);
                nw[b][c] = *(const float4_t *) (pw[b] + kn + 4 * c);
            }
        }
#pragma unroll
        for (int s = 0; s < 16; s++) {
#pragma unroll
            for (int i = 0; i < 2; i++) {
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(ca[i][s >> 2][s & 3], cw[j][s >> 2][s & 3],
                                                                      acc[i][j], 0, 0, 0);
                }
            }
        }
#pragma unroll
        for (int b = 0; b < 2; b++) {
#pragma unroll
            for (int c = 0; c < 4; c++) {
                ca[b][c] = na[b][c];
                cw[b][c] = nw[b][c];
            }
        }
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int64_t n = n0 + 32 * j + li;
        if (n >= N) {
            continue;
        }
#pragma unroll
        for (int i = 0; i < 2; i++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int64_t m = m0 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
                if (m < M) {
                    y[m * ldy + n] = acc[i][j][r];
                }
            }
        }
    }
}

bool gemm_f32_supported(int64_t N, int64_t K, int64_t ldw, const void * W, const float * x, int64_t ldx) {
    return N > 0 && K > 0 && K % 32 == 0 && ldw >= K && ldw % 4 == 0 && ldx >= K && ldx % 4 == 0 &&
           ((uintptr_t) W) % 16 == 0 && ((uintptr_t) x) % 16 == 0;
}

int gemm_f32(const float * W, int64_t ldw, const float * x, int64_t ldx, int64_t N, int64_t K, int64_t M, float * y,
             int64_t ldy, hipStream_t stream) {
    if (!gemm_f32_supported(N, K, ldw, W, x, ldx) || M <= 0 || ldy < N) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "mul_mat f32 gemm: N=%lld K=%lld M=%lld (K %% 32 == 0, 16-byte rows)",
                         (long long) N, (long long) K, (long long) M);
    }
    const int64_t gx = (N + 63) / 64, gy = (M + 63) / 64;
    if (gx > INT32_MAX || gy > 65535) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "mul_mat f32 gemm: grid too large");
    }
    hipLaunchKernelGGL(k_gemm_f32, dim3((unsigned) gx, (unsigned) gy), dim3(64), 0, stream, W, ldw, x, ldx, N, K, M, y,
                       ldy);
    return check_launch("mul_mat f32 gemm");
}

}  // namespace mmhip
