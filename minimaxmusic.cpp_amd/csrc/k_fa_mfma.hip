// k_fa_mfma.hip - flash attention on MFMA for many query rows: causal prefill
// (src/qwen3-lm.h:432-436) and the DiT's bidirectional attention
// (src/dit.h:221-222).
//
// Workgroup = NW waves = 32*NW query rows of one (head, batch); each wave owns
// 32 query rows (with 8 waves: two 128-row ranges from opposite ends of the
// sequence, which evens out causal work).  KV is walked in tiles of 64 keys staged in LDS (K as rows, V
// transposed).  Per tile a wave computes S^T = K Q^T (keys x queries) with
// v_mfma_f32_32x32x16_f16, so each lane owns one query column: the online
// softmax (max, sum, rescale) is lane-local apart from one exchange with the
// lane holding the other half of the keys.  P^T stays in registers and feeds
// O^T = V^T P^T directly as the B operand; the V^T tile stores keys with bits 2
// and 3 swapped inside each 16-key group, which is the order in which the S^T
// accumulator registers hold them.
//
// Arithmetic: Q, K, V and P are f16 MFMA operands with f32 accumulation
// (GGML_PREC_F32); the softmax runs in f32 base 2 with log2(e) folded into the
// scale.  A prepass over the mask finds, per query row, the last key the row
// can see; a workgroup stops at the last key any of its rows can see, so fully
// masked KV tiles (the causal upper triangle, the -inf padding of the cache
// window) are never read.
//
// The unmasked D = 128 case on a full grid (the DiT) runs k_fa_dma instead,
// described above its definition below.
#include <type_traits>

#include "k_fa_common.h"
#include "mmhip_device.h"
#include "mmhip_internal.h"

namespace mmhip {

constexpr int FA_BK = 64;

__device__ __forceinline__ float16_t mfma32(half8_t a, half8_t b, float16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// LDS position of key k (0..63) inside a V^T row: bits 2 and 3 swapped.
__device__ __forceinline__ int vt_pos(int k) {
    return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1);
}

// Bank swizzle of V^T row r: the 8-key groups of the row are XOR-permuted by
// (r / 16) % 8.  Staging writes (4 bytes: 16 lanes on rows 8 apart x 4
// lanes on adjacent key pairs) and A-operand reads (16 bytes: 16 lanes on
// adjacent rows, one position) then both hit 64 distinct banks per pass;
// reads of 8 consecutive positions stay contiguous.
__device__ __forceinline__ int vt_swz(int r) {
    return ((r >> 4) & 7) << 3;
}

// Work item of linear workgroup id `lin` out of `total`: workgroups are
// dispatched round-robin over the 8 XCDs (id % 8), so consecutive work items
// are dealt to one XCD at a time; all query tiles of a (head, batch) then
// share that XCD's L2 for their K/V tiles.
__device__ __forceinline__ int xcd_remap(int lin, int total) {
    const int per = total / 8;
    if (lin >= per * 8) {
        return lin;  // the remainder keeps its own index
    }
    return (lin % 8) * per + lin / 8;
}

template <int D, int NW>
__global__ __launch_bounds__(NW * 64) void k_fa_mfma(FaArgs a, const int * __restrict__ row_end,
                                                     const int * __restrict__ zero_end, int n_qtiles,
                                                     float * __restrict__ out) {
    constexpr int NT  = NW * 64;
    constexpr int BQ  = NW * 32;
    constexpr int KS  = D + 8;      // K row stride (halves)
    constexpr int VS  = FA_BK + 8;  // V^T row stride (halves)
    constexpr int NQK = D / 16;     // MFMA k-steps for Q.K
    constexpr int NDB = D / 32;     // 32-row blocks of O^T
    constexpr int KCH = FA_BK * (D / 8) / NT;        // 16-byte K chunks per thread per tile
    constexpr int VCH = (FA_BK / 2) * (D / 8) / NT;  // V key pairs x 8 dims per thread per tile
    static_assert(KCH >= 1 && VCH >= 1, "tile too small for the workgroup");
    __shared__ __attribute__((aligned(16))) _Float16 sK[FA_BK * KS];
    __shared__ __attribute__((aligned(16))) _Float16 sV[D * VS];

    const int total = n_qtiles * a.Hq * a.B;
    const int lin   = xcd_remap((int) (blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z)), total);
    const int qt    = n_qtiles - 1 - lin % n_qtiles;  // longest (causal) tiles first
    const int h     = (lin / n_qtiles) % a.Hq;
    const int b     = lin / (n_qtiles * a.Hq);
    const int G     = a.Hq / a.Hkv;
    const int hk    = h / G;
    const int bk    = b / (a.B / a.Bk);
    const int tid   = threadIdx.x;
    const int wave  = tid >> 6;
    const int lane  = tid & 63;
    const int lq    = lane & 31;
    const int hh    = lane >> 5;
    // query rows: with 8 waves the workgroup pairs 128-row tile qt (waves 0-3)
    // with tile n128 - 1 - qt (waves 4-7), so that under a causal mask every
    // workgroup gets one short and one long row range (the middle tile of an
    // odd count goes alone); otherwise 32 NW consecutive rows
    int my_q;
    if constexpr (NW == 8) {
        const int n128 = (a.nq + 127) / 128;
        const int half = wave >> 2;
        const int t128 = half ? n128 - 1 - qt : qt;
        my_q           = half && t128 <= qt ? a.nq : t128 * 128 + (wave & 3) * 32 + lq;
    } else {
        my_q = qt * BQ + wave * 32 + lq;
    }
    const bool q_ok = my_q < a.nq;

    // Q^T operand: this lane's query, dims 16kk + 8hh + 0..7, rounded to f16
    half8_t      qreg[NQK];
    const float * qp = (const float *) (a.q + (int64_t) (q_ok ? my_q : 0) * a.qnb1 + h * a.qnb2 + b * a.qnb3);
#pragma unroll
    for (int kk = 0; kk < NQK; kk++) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            qreg[kk][i] = (_Float16) qp[16 * kk + 8 * hh + i];
        }
    }
    const char * mrow = a.mask ? a.mask + (int64_t) (q_ok ? my_q : 0) * a.mnb1 + (h % a.mne2) * a.mnb2 +
                                     (b % a.mne3) * a.mnb3
                               : nullptr;

    float16_t oacc[NDB];
#pragma unroll
    for (int i = 0; i < NDB; i++) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            oacc[i][r] = 0.0f;
        }
    }
    float       m     = -INFINITY;
    float       l     = 0.0f;
    const float log2e = 1.4426950408889634f;
    const float sl2   = a.scale * log2e;

    // last visible key of each wave's rows (max of the per-row ends) and of
    // the workgroup's (max over waves: the K / V staging walks that far, a
    // wave computes up to its own end); keys below every row's all-zero mask
    // prefix take the unmasked path
    int kv_end = a.nkv, w_end = __any(q_ok) ? a.nkv : 0, zfast = a.nkv;
    if (row_end) {
        __shared__ int s_end[NW];
        const int      plane = (b % a.mne3) * a.mne2 + (h % a.mne2);
        const int      e     = q_ok ? row_end[(int64_t) plane * a.nq + my_q] : 0;
        const int      z     = q_ok ? zero_end[(int64_t) plane * a.nq + my_q] : a.nkv;
        w_end                = min(a.nkv, (int) wave_max((float) e));
        zfast                = -(int) wave_max((float) -z);
        if (lane == 0) {
            s_end[wave] = w_end;
        }
        __syncthreads();
        int te = 0;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            te = max(te, s_end[w]);
        }
        kv_end = min(kv_end, te);
    }

    const char * kbase = a.k + hk * a.knb2 + bk * a.knb3;
    const char * vbase = a.v + hk * a.vnb2 + bk * a.vnb3;

    // register stage of the next tile
    half8_t rk[KCH], rv0[VCH], rv1[VCH];
    auto    fetch = [&](int k0) {
#pragma unroll
        for (int i = 0; i < KCH; i++) {
            const int c = tid + i * NT, key = c / (D / 8), seg = c % (D / 8), kg = k0 + key;
            rk[i] = kg < a.nkv ? *(const half8_t *) (kbase + (int64_t) kg * a.knb1 + seg * 16) : half8_t{};
        }
#pragma unroll
        for (int i = 0; i < VCH; i++) {
            // the pair whose keys land at positions 2 kp, 2 kp + 1 of the V^T rows
            const int c = tid + i * NT, kp = c / (D / 8), seg = c % (D / 8), kg = k0 + vt_pos(2 * kp);
            rv0[i] = kg < a.nkv ? *(const half8_t *) (vbase + (int64_t) kg * a.vnb1 + seg * 16) : half8_t{};
            rv1[i] = kg + 1 < a.nkv ? *(const half8_t *) (vbase + (int64_t) (kg + 1) * a.vnb1 + seg * 16)
                                    : half8_t{};
        }
    };

    if (kv_end > 0) {
        fetch(0);
    }
    for (int k0 = 0; k0 < kv_end; k0 += FA_BK) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < KCH; i++) {
            const int c = tid + i * NT, key = c / (D / 8), seg = c % (D / 8);
            *(half8_t *) &sK[key * KS + seg * 8] = rk[i];
        }
#pragma unroll
        for (int i = 0; i < VCH; i++) {
            const int c = tid + i * NT, kp = c / (D / 8), seg = c % (D / 8);
            const int pos = 2 * kp;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int r = seg * 8 + j;
                *(half2_t *) &sV[r * VS + (pos ^ vt_swz(r))] = half2_t{ rv0[i][j], rv1[i][j] };
            }
        }
        __syncthreads();
        if (k0 + FA_BK < kv_end) {
            fetch(k0 + FA_BK);
        }
        if (k0 >= w_end) {
            continue;  // past every key this wave's rows can see (it keeps staging)
        }

        // S^T (64 keys x 32 queries) = K Q^T.  Raised wave priority while
        // issuing MFMAs: of two waves on a SIMD, the one with matrix work
        // goes first and the other's softmax fills the gaps.
        __builtin_amdgcn_s_setprio(1);
        float16_t s[2];
#pragma unroll
        for (int kb = 0; kb < 2; kb++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                s[kb][r] = 0.0f;
            }
#pragma unroll
            for (int kk = 0; kk < NQK; kk++) {
                const half8_t ak = *(const half8_t *) &sK[(kb * 32 + lq) * KS + 16 * kk + 8 * hh];
                s[kb]            = mfma32(ak, qreg[kk], s[kb]);
            }
        }
        __builtin_amdgcn_s_setprio(0);
        // scale, mask, out-of-range keys; tile max for this lane's query.
        // Without a mask on a full tile the raw scores are kept: their max
        // is scaled once, and the scale folds into the exp2 argument below.
        const bool fast = (!mrow || k0 + FA_BK <= zfast) && k0 + FA_BK <= a.nkv;
        float      mx   = -INFINITY;
        if (fast) {
#pragma unroll
            for (int kb = 0; kb < 2; kb++) {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    mx = fmaxf(mx, s[kb][r]);
                }
            }
            mx *= sl2;
        } else {
#pragma unroll
        for (int kb = 0; kb < 2; kb++) {
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                const int key0 = k0 + kb * 32 + 8 * g4 + 4 * hh;
                float     mv[4] = { 0.0f, 0.0f, 0.0f, 0.0f };
                if (mrow) {
                    if (key0 + 3 < a.nkv && (((uintptr_t) mrow) & 7) == 0) {
                        const uint2 w = *(const uint2 *) (mrow + (int64_t) key0 * 2);
                        mv[0]         = h2f((uint16_t) (w.x & 0xffff));
                        mv[1]         = h2f((uint16_t) (w.x >> 16));
                        mv[2]         = h2f((uint16_t) (w.y & 0xffff));
                        mv[3]         = h2f((uint16_t) (w.y >> 16));
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            mv[i] = key0 + i < a.nkv ? h2f(((const uint16_t *) mrow)[key0 + i]) : 0.0f;
                        }
                    }
                }
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = 4 * g4 + i;
                    float     v = (key0 + i < a.nkv) ? s[kb][r] * sl2 + mv[i] * log2e : -INFINITY;
                    s[kb][r]    = v;
                    mx          = fmaxf(mx, v);
                }
            }
        }
        }
        mx = max_xor32(mx);
        // the reference max moves only when a score exceeds it by more than
        // 8 (log2 units): p = exp2(s - m) then stays <= 2^8 (well inside f16
        // and f32), O / l is unchanged in exact arithmetic, and most tiles
        // need no rescale of the accumulators
        const float mnew = mx > m + 8.0f ? mx : m;
        // No divergent control flow from here on: the MFMAs below combine the
        // operands of all 64 lanes.  A query with nothing visible yet keeps
        // its state (alpha = 1) and contributes p = exp2(-inf) = 0.
        const bool  live  = mnew != -INFINITY;
        const float mref  = live ? mnew : 0.0f;
        const float smul  = fast ? sl2 : 1.0f;
        const float alpha = live ? __builtin_amdgcn_exp2f(m - mnew) : 1.0f;
        float       rs    = 0.0f;
        l                 = l * alpha;
        m                 = mnew;
        if (__any(alpha != 1.0f)) {  // wave-uniform: no lane's running max moved -> nothing to rescale
#pragma unroll
            for (int i = 0; i < NDB; i++) {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    oacc[i][r] *= alpha;
                }
            }
        }
        // P^T -> f16 B operands, then O^T (D x 32 queries) += V^T P^T
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int kb = 0; kb < 2; kb++) {
#pragma unroll
            for (int t = 0; t < 2; t++) {
                half8_t pb;
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    // fast path: raw score * scale - max in one rounding; masked
                    // path: already scaled, s * 1 - max == s - max exactly
                    const float p = __builtin_amdgcn_exp2f(fmaf(s[kb][8 * t + u], smul, -mref));
                    rs += p;
                    pb[u] = (_Float16) p;
                }
#pragma unroll
                for (int db = 0; db < NDB; db++) {
                    const int     r  = db * 32 + lq;
                    const half8_t av = *(const half8_t *) &sV[r * VS + ((kb * 32 + 16 * t + 8 * hh) ^ vt_swz(r))];
                    oacc[db]         = mfma32(av, pb, oacc[db]);
                }
            }
        }
        __builtin_amdgcn_s_setprio(0);
        l += sum_xor32(rs);
    }

    if (q_ok) {
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        float *     op  = out + (((int64_t) b * a.nq + my_q) * a.Hq + h) * D;
#pragma unroll
        for (int db = 0; db < NDB; db++) {
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                const int d = db * 32 + 8 * g4 + 4 * hh;
                float4_t  v = { oacc[db][4 * g4] * inv, oacc[db][4 * g4 + 1] * inv, oacc[db][4 * g4 + 2] * inv,
                                oacc[db][4 * g4 + 3] * inv };
                *(float4_t *) (op + d) = v;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Unmasked D = 128 with a full grid (the DiT's attention, src/dit.h:221-222):
// k_fa_dma.  The chip runs MFMA work at a power-limited clock that drops
// further with every VALU op and LDS byte issued beside it, so this kernel
// minimises both per MFMA:
//  - K / V tiles (64 keys, 16 KB each) go from global memory straight into a
//    double-buffered LDS ring with global_load_lds (no register staging, no
//    transposing stores); K rows store 16-byte chunk c at c ^ (row & 15), V
//    rows at c ^ 2 (row & 3), which keeps both read patterns bank-conflict
//    free;
//  - V^T operands come from ds_read_b64_tr_b16: within each 16-lane group,
//    lane i receives element i % 4 of the 4-element rows addressed by lanes
//    4 j + i / 4 (j = 0..3), so the lanes address V rows in exactly the key
//    order the S^T accumulator registers hold (bits 2 and 3 of the key swapped);
//  - Q is scaled by scale * log2(e) before its f16 rounding, and every QK
//    accumulator starts at -m (the running row max, log2 units): the scores
//    come out as s - m and p = exp2(s - m) is one v_exp per score; the row
//    sum adds the f16 p pairs with v_dot2 (the same values the PV MFMA uses);
//  - the running max moves only on a slow path: on a row's first 32 keys, or
//    when a lane's partial sum exceeds 2^14 (some score more than 14 above
//    m); O and l are then rescaled by exp2(-shift).  p stays below 2^15,
//    inside f16.
// Pipeline per wave (32 query rows, 8 waves, two per SIMD): unit u = 32 keys;
// unit u runs the softmax of unit u (VALU) between the MFMAs of QK(u + 1) and
// PV(u - 1), with the LDS operands of MFMA step i + 2 read during step i.  One
// barrier per 64-key tile.
__device__ __forceinline__ void fa_dma16(const void * src, uint32_t lds_addr) {
    // issued from inline asm: the compiler's wait-count tracking would
    // otherwise wait for the DMA before unrelated LDS reads; the kernel waits
    // for it itself before the barrier that publishes a tile
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds_addr) : "memory", "m0");
}

typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4_t lds_short4_t;

// Masked form (MASK: the LM's causal prefill, src/qwen3-lm.h:432-436, or any
// f16 mask), with the mask prepass's per-row ends: one 128-row query tile per
// workgroup of four waves, two workgroups per CU; the K / V tiles are staged
// up to the last key any row of the workgroup can see, and a wave computes
// up to the last key its own rows can see, then only takes part in the
// staging.  A unit past the wave's all-zero mask prefix adds the mask (log2
// units) to its scores, loaded while the unit before it runs.  A row's
// running max is set on its first unit with a visible key.
//
// The unmasked form stages K and V through 4-tile rings (128 KB of LDS, one
// workgroup per CU as the registers allow anyway), each tile issued three
// 64-key steps before its first reader and waited for by count, so the
// loads of the two younger steps stay in flight across a barrier.  The
// masked form's rings hold 2 tiles (64 KB, two workgroups per CU): the K
// tile of the next step and the V tile of this one are waited for at each
// step's barrier.
template <bool MASK, int NW = 8, int KR = 4>
__global__ __launch_bounds__(NW * 64, 2) void k_fa_dma(FaArgs a, const int * __restrict__ row_end,
                                                       const int * __restrict__ zero_end, int n_qtiles,
                                                       float * __restrict__ out) {
    constexpr int D = 128, NQK = 8, NDB = 4, TILE = FA_BK * 256;
    constexpr int US  = 1;         // unit stride of a wave
    constexpr int PPW = 16 / NW;   // 1 KB pieces of a 16 KB tile each wave DMAs
    static_assert(MASK ? (NW == 4 && KR == 2) : (NW == 8 && KR == 4), "configurations");
    extern __shared__ __attribute__((aligned(1024))) char smem[];  // K ring, then V ring
    const int  total = n_qtiles * a.Hq * a.B;
    // one 128-row tile per workgroup (masked, four waves): workgroups in
    // order of falling row ends (the longest tiles first, every XCD a share
    // of each length), two per CU, so that a CU takes the next tile as soon
    // as one of its two finishes
    const int  lin   = MASK ? (int) blockIdx.x : xcd_remap((int) blockIdx.x, total);
    const int  qt    = MASK ? n_qtiles - 1 - lin / (a.Hq * a.B) : lin % n_qtiles;
    const int  h     = MASK ? lin % a.Hq : (lin / n_qtiles) % a.Hq;
    const int  b     = MASK ? (lin / a.Hq) % a.B : lin / (n_qtiles * a.Hq);
    const int  hk    = h / (a.Hq / a.Hkv);
    const int  bk    = b / (a.B / a.Bk);
    const int  tid   = threadIdx.x;
    const int  wave  = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int  lane  = tid & 63;
    const int  lq    = lane & 31;
    const int  hh    = lane >> 5;
    const int   par  = 0;  // the wave's first unit
    int         my_q;
    if constexpr (MASK) {
        my_q = qt * 128 + wave * 32 + lq;
    } else {
        my_q = qt * 256 + wave * 32 + lq;
    }
    const bool  q_ok = my_q < a.nq;
    const float log2e = 1.4426950408889634f;
    const float sl2   = a.scale * log2e;

    // keys: the workgroup stages [0, kv_end), this wave computes [0, w_end),
    // and units wholly inside [0, zfast) need no mask (all-zero prefix)
    int          kv_end = a.nkv, w_end = a.nkv, zfast = a.nkv;
    const char * mrow   = nullptr;
    if constexpr (MASK) {
        __shared__ int s_end[NW];
        const int      plane = (b % a.mne3) * a.mne2 + (h % a.mne2);
        const int      e     = q_ok ? row_end[(int64_t) plane * a.nq + my_q] : 0;
        const int      z     = q_ok ? zero_end[(int64_t) plane * a.nq + my_q] : a.nkv;
        // wave-uniform values (readfirstlane: the loop bounds and DMA
        // addresses below must live in scalar registers)
        w_end = __builtin_amdgcn_readfirstlane(min(a.nkv, (int) wave_max((float) e)));
        zfast = __builtin_amdgcn_readfirstlane(-(int) wave_max((float) -z));
        if (lane == 0) {
            s_end[wave] = w_end;
        }
        __syncthreads();
        int te = 0;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            te = max(te, s_end[w]);
        }
        kv_end = __builtin_amdgcn_readfirstlane(te);
        mrow   = a.mask + (int64_t) (q_ok ? my_q : 0) * a.mnb1 + (h % a.mne2) * a.mnb2 + (b % a.mne3) * a.mnb3;
    }

    // Q^T operand: dims 16 kk + 8 hh + 0..7 of this lane's query, scaled, f16
    half8_t qreg[NQK];
    {
        const float * qp = (const float *) (a.q + (int64_t) (q_ok ? my_q : 0) * a.qnb1 + h * a.qnb2 + b * a.qnb3);
#pragma unroll
        for (int kk = 0; kk < NQK; kk++) {
            const float4_t x0 = *(const float4_t *) (qp + 16 * kk + 8 * hh);
            const float4_t x1 = *(const float4_t *) (qp + 16 * kk + 8 * hh + 4);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                qreg[kk][i]     = (_Float16) (x0[i] * sl2);
                qreg[kk][i + 4] = (_Float16) (x1[i] * sl2);
            }
        }
    }
    float16_t oacc[NDB];
#pragma unroll
    for (int i = 0; i < NDB; i++) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            oacc[i][r] = 0.0f;
        }
    }
    float m = 0.0f;  // running row max (log2 units)
    float l = 0.0f;  // this lane's half of the row sum
    bool  mset = false;                           // (MASK) the running max is set for this lane's row
    const int n     = (kv_end + FA_BK - 1) / FA_BK;  // 64-key tiles staged
    const int nu_wg = (kv_end + 31) / 32;            // 32-key units staged
    const int nu    = (w_end + 31) / 32;             // 32-key units the wave's rows see
    const int nk    = nu;                            // units this wave computes

    // the mask of this lane's query at the 16 keys of unit u it holds
    // (k0 + 8 g4 + 4 hh + i, i = 0..3), f16 bits; -inf past the keys
    uint2      mw[4];
    const bool m8 = MASK && ((((uintptr_t) mrow) & 7) == 0);
    auto mask_need = [&](int u) { return MASK && u * 32 + 32 > zfast; };
    auto mask_load = [&](int u) {
#pragma unroll
        for (int g4 = 0; g4 < 4; g4++) {
            const int key0 = u * 32 + 8 * g4 + 4 * hh;
            if (m8 && key0 + 3 < a.nkv) {
                mw[g4] = *(const uint2 *) (mrow + (int64_t) key0 * 2);
            } else {
                uint16_t hv[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    hv[i] = key0 + i < a.nkv ? ((const uint16_t *) mrow)[key0 + i] : (uint16_t) 0xfc00;
                }
                mw[g4] = uint2{ (uint32_t) hv[0] | ((uint32_t) hv[1] << 16), (uint32_t) hv[2] | ((uint32_t) hv[3] << 16) };
            }
        }
    };
    auto mask_apply = [&](float16_t & s) {
#pragma unroll
        for (int g4 = 0; g4 < 4; g4++) {
            s[4 * g4 + 0] += h2f((uint16_t) (mw[g4].x & 0xffff)) * log2e;
            s[4 * g4 + 1] += h2f((uint16_t) (mw[g4].x >> 16)) * log2e;
            s[4 * g4 + 2] += h2f((uint16_t) (mw[g4].y & 0xffff)) * log2e;
            s[4 * g4 + 3] += h2f((uint16_t) (mw[g4].y >> 16)) * log2e;
        }
    };

    // DMA: this wave fills 1 KB pieces PPW wave .. PPW wave + PPW - 1 (4 rows
    // each) of a K and a V tile; lane -> row 4 piece + lane / 16, stored chunk
    // lane % 16
    const char *   kbase = a.k + hk * a.knb2 + bk * a.knb3;
    const char *   vbase = a.v + hk * a.vnb2 + bk * a.vnb3;
    const uint32_t sbase = (uint32_t) (uintptr_t) (__attribute__((address_space(3))) char *) smem;
    const int      drow = lane >> 4, dpc = lane & 15;
    auto dma_k = [&](int j) {
#pragma unroll
        for (int i = 0; i < PPW; i++) {
            const int piece = PPW * wave + i, r = 4 * piece + drow;
            const int key   = min(j * FA_BK + r, a.nkv - 1);  // rows past the end repeat the last key (masked below)
            fa_dma16(kbase + (int64_t) key * a.knb1 + ((dpc ^ (r & 15)) << 4),
                     sbase + (j & (KR - 1)) * TILE + piece * 1024);
        }
    };
    auto dma_v = [&](int j) {
#pragma unroll
        for (int i = 0; i < PPW; i++) {
            const int piece = PPW * wave + i, r = 4 * piece + drow;
            const int key   = min(j * FA_BK + r, a.nkv - 1);
            fa_dma16(vbase + (int64_t) key * a.vnb1 + ((dpc ^ (2 * (r & 3))) << 4),
                     sbase + (KR + (j & (KR - 1))) * TILE + piece * 1024);
        }
    };
    // K operand of k-step kk: row lq of the 32-key unit, logical chunk 2 kk + hh
    uint32_t ka[NQK];
#pragma unroll
    for (int kk = 0; kk < NQK; kk++) {
        ka[kk] = lq * 256 + (((2 * kk + hh) ^ (lq & 15)) << 4);
    }
    // V^T operand: source lane (tg, tj, tq) of a transposed read addresses
    // V[key0 + 4 (tg / 2) + tj][32 db + 16 (tg & 1) + 4 tq]; the V swizzle
    // 2 (key & 3) = 2 tj folds into +-64 bytes on even / odd db
    const int      tg = lane >> 4, tj = (lane >> 2) & 3, tq = lane & 3;
    const int      vx = (tj >> 1) * 64;
    const uint32_t vlane =
        (4 * (tg >> 1) + tj) * 256 + 16 * ((2 * (tg & 1) + (tq >> 1)) ^ (2 * (tj & 1))) + 8 * (tq & 1);
    const uint32_t vb[2] = { vlane + vx, vlane - vx };
    auto qk_op = [&](int u, int kk) -> half8_t {
        const char * kt = smem + ((u >> 1) & (KR - 1)) * TILE;
        return *(const half8_t *) (kt + ka[kk] + (u & 1) * 8192);
    };
    // PV step i of a unit: key half t = i / 4 (16 keys), output block db = i % 4
    auto pv_op = [&](int u, int i) -> half8_t {
        const uint32_t vt = sbase + (KR + ((u >> 1) & (KR - 1))) * TILE;
        const int      t = i >> 2, db = i & 3;
        half8_t        av;
#pragma unroll
        for (int hf = 0; hf < 2; hf++) {
            const uint32_t ad = vt + vb[db & 1] + ((u & 1) * 32 + 16 * t + 8 * hf) * 256 + 64 * db;
            const half4_t  x  = __builtin_bit_cast(
                half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t *) (uintptr_t) ad));
#pragma unroll
            for (int e = 0; e < 4; e++) {
                av[4 * hf + e] = x[e];
            }
        }
        return av;
    };

    float16_t zero16, negm;  // negm: -m in every register, the C operand of a unit's first QK MFMA
#pragma unroll
    for (int r = 0; r < 16; r++) {
        zero16[r] = 0.0f;
        negm[r]   = 0.0f;
    }
    float16_t sc, sn;         // s - m of unit u (softmax input) and of unit u + 1 (being computed)
    half8_t   pp[2], pn[2];   // P of unit u - 1 (PV input) and of unit u (softmax output)
    float     m_sn = 0.0f;    // the m that sn was computed against
    const half2_t ones2 = { (_Float16) 1.0f, (_Float16) 1.0f };
    auto exp_pack = [&](float & rs) {
        rs = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
            const half2_t pk = { (_Float16) __builtin_amdgcn_exp2f(sc[r]), (_Float16) __builtin_amdgcn_exp2f(sc[r + 1]) };
            rs                        = __builtin_amdgcn_fdot2(pk, ones2, rs, false);
            pn[r >> 3][r & 7]         = pk[0];
            pn[r >> 3][(r & 7) + 1]   = pk[1];
        }
    };
    // move m to the row max (first unit: exactly; later: upwards only),
    // rescale O and l, redo the unit's p
    auto slow = [&](float & rs, bool first_unit) {
        float mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            mx = fmaxf(mx, sc[r]);
        }
        mx = max_xor32(mx);
        // first: nothing visible accumulated yet (O and l zero), m goes to
        // the unit's max exactly; otherwise it moves up only
        const bool  first = MASK ? !mset : first_unit;
        const float d     = first ? (mx == -INFINITY ? 0.0f : mx) : (mx > 0.0f ? mx : 0.0f);
        if constexpr (MASK) {
            mset = mset || mx != -INFINITY;
        }
        if (__any(d != 0.0f)) {
            if (__any(!first)) {
                const float alpha = first ? 1.0f : __builtin_amdgcn_exp2f(-d);
                l *= alpha;
#pragma unroll
                for (int q = 0; q < NDB; q++) {
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        oacc[q][r] *= alpha;
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < 16; r++) {
                sc[r] -= d;
            }
            m += d;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                negm[r] = -m;
            }
        }
        exp_pack(rs);
    };
    // unit u: softmax(u) (SM), QK(u + US) (QK), PV(u - US) (PV); which parts
    // are present is a compile-time choice, so the steady-state unit is
    // branch-free and the compiler interleaves its VALU work with the MFMAs
    auto unit = [&](int u, auto QKc, auto PVc, auto SMc) {
        constexpr bool do_qk = decltype(QKc)::value, do_pv = decltype(PVc)::value, do_sm = decltype(SMc)::value;
        if constexpr (do_sm) {
            const int k0 = u * 32;
            if (k0 + 32 > a.nkv) {  // the last, partial unit
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    if (k0 + 8 * (r / 4) + 4 * hh + (r % 4) >= a.nkv) {
                        sc[r] = -INFINITY;
                    }
                }
            }
        }
        const float m_used = m;
        float       rs     = 0.0f;
        // operands three MFMA steps ahead; the scheduling barrier keeps each
        // step's LDS reads above it (left alone, the scheduler sank them to
        // just before their MFMA, reusing one register set, so every MFMA
        // waited out a whole LDS read).  Masked: nothing crosses it (the
        // lone long-row waves of a causal workgroup: 50.1 -> 44.8 us at B = 2,
        // S = 1024); unmasked: ALU, MFMA and transcendental work may
        // (the DiT shape: 295 -> 291 us)
        half8_t     av[4], ak[4];
        if constexpr (do_pv) {
            av[0] = pv_op(u - US, 0);
            av[1] = pv_op(u - US, 1);
            av[2] = pv_op(u - US, 2);
        }
        if constexpr (do_qk) {
            ak[0] = qk_op(u + US, 0);
            ak[1] = qk_op(u + US, 1);
            ak[2] = qk_op(u + US, 2);
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            if (i + 3 < 8) {
                if constexpr (do_pv) {
                    av[(i + 3) % 4] = pv_op(u - US, i + 3);
                }
                if constexpr (do_qk) {
                    ak[(i + 3) % 4] = qk_op(u + US, i + 3);
                }
            }
            __builtin_amdgcn_sched_barrier(MASK ? 0 : 0x040F);
            if constexpr (do_pv) {
                oacc[i & 3] = mfma32(av[i % 4], pp[i >> 2], oacc[i & 3]);
            }
            if constexpr (do_qk) {
                sn = mfma32(ak[i % 4], qreg[i], i == 0 ? negm : sn);
            }
            if constexpr (do_sm) {
                const int     r  = 2 * i;
                const half2_t pk = { (_Float16) __builtin_amdgcn_exp2f(sc[r]),
                                     (_Float16) __builtin_amdgcn_exp2f(sc[r + 1]) };
                rs                      = __builtin_amdgcn_fdot2(pk, ones2, rs, false);
                pn[r >> 3][r & 7]       = pk[0];
                pn[r >> 3][(r & 7) + 1] = pk[1];
            }
        }
        if constexpr (do_sm) {
            if ((MASK ? __any(!mset) : u == 0) || __any(rs > 16384.0f)) {
                slow(rs, u == 0);
            }
            l += rs;
        }
        if constexpr (do_qk) {
            m_sn = m_used;
        }
    };
    // DMA group g (g >= -KR / 2): K tile g + KR and V tile g + KR - 1, each
    // PPW loads per wave when the tile exists; the groups before 0 go out
    // after the prologue, group j after the barrier that follows unit 2 j
    auto group_loads = [&](int g) { return PPW * (g + KR < n) + PPW * (g + KR - 1 < n); };
    auto issue_group = [&](int g) {
        if (g + KR < n) {
            dma_k(g + KR);
        }
        if (g + KR - 1 < n) {
            dma_v(g + KR - 1);
        }
    };
    // after unit u: sn becomes the next softmax input (shifted if m moved
    // since it was computed); after an even unit 2 j: the wait for K tile
    // j + 1 and V tile j (group j - 3: only the loads of groups j - 2 and
    // j - 1 may still be in flight), the barrier, then group j: K tile j + 4
    // into the buffer of K tile j (last read in unit 2 j), V tile j + 3 into
    // that of V tile j - 1 (last read in unit 2 j)
    auto after = [&](int u) {
        sc = sn;
        if (__any(m_sn != m)) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                sc[r] += m_sn - m;
            }
        }
        if (mask_need(u + US) && u + US < nu) {
            mask_apply(sc);
        }
        pp[0] = pn[0];
        pp[1] = pn[1];
        if ((u & 1) == 0) {
            const int j = u >> 1;
            if constexpr (KR == 2) {
                // K tile j + 1 and V tile j: group j - 1, the last one issued
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            } else {
                switch (group_loads(j - 2) + group_loads(j - 1)) {
                    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
                    case 2: asm volatile("s_waitcnt vmcnt(2)" ::: "memory"); break;
                    case 4: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
                    case 6: asm volatile("s_waitcnt vmcnt(6)" ::: "memory"); break;
                    default: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
                }
            }
            asm volatile("s_barrier" ::: "memory");
            issue_group(j);
        }
    };

    // prologue: K tiles 0 and 1, V tile 0 resident, groups -2 and -1 issued
    // behind the barrier; the scores of the wave's first unit (m = 0)
    const int u0 = par;
    dma_k(0);
    if constexpr (KR == 4) {
        if (n > 1) {
            dma_k(1);
        }
        if (n > 0) {
            dma_v(0);
        }
    }
    if (mask_need(u0) && nk > 0) {
        mask_load(u0);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    asm volatile("s_barrier" ::: "memory");
    if constexpr (KR == 4) {
        issue_group(-2);
    }
    issue_group(-1);
    sc = zero16;
    if (nk > 0) {
#pragma unroll
        for (int kk = 0; kk < NQK; kk++) {
            sc = mfma32(qk_op(u0, kk), qreg[kk], sc);
        }
        if (mask_need(u0)) {
            mask_apply(sc);
        }
    }
    using T_ = std::integral_constant<bool, true>;
    using F_ = std::integral_constant<bool, false>;
    // the wave's own units u0, u0 + US, ... (nk of them, each followed by
    // after(u): the barrier and the wave's share of the staging), the PV of
    // its last unit, then (masked: a wave whose rows see fewer keys than the
    // workgroup stages) after() alone for the remaining staged tiles.  The
    // drained PV reads a V tile that is restaged after the next step at the
    // earliest.
    if (nk > 0) {
        if (nk > 1 && mask_need(u0 + US)) {
            mask_load(u0 + US);
        }
        if (nk > 1) {
            unit(u0, T_{}, F_{}, T_{});
        } else {
            unit(u0, F_{}, F_{}, T_{});
        }
        after(u0);
        for (int i = 1; i + 1 < nk; i++) {
            const int u = u0 + i * US;
            if (mask_need(u + US)) {
                mask_load(u + US);
            }
            unit(u, T_{}, T_{}, T_{});
            after(u);
        }
        if (nk > 1) {
            const int u = u0 + (nk - 1) * US;
            unit(u, F_{}, T_{}, T_{});
            after(u);
        }
        unit(u0 + nk * US, F_{}, T_{}, F_{});
    }
    if constexpr (MASK) {
        for (int u = nu; u < nu_wg; u++) {
            after(u);
        }
    }

    l += __shfl_xor(l, 32);
    if (q_ok) {
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        float *     op  = out + (((int64_t) b * a.nq + my_q) * a.Hq + h) * D;
#pragma unroll
        for (int db = 0; db < NDB; db++) {
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                const int d = db * 32 + 8 * g4 + 4 * hh;
                float4_t  v = { oacc[db][4 * g4] * inv, oacc[db][4 * g4 + 1] * inv, oacc[db][4 * g4 + 2] * inv,
                                oacc[db][4 * g4 + 3] * inv };
                *(float4_t *) (op + d) = v;
            }
        }
    }
}

// k_fa_dma's preconditions: 16-byte aligned Q rows (float4 loads) and K / V
// rows (16-byte DMA), D = 128, and at least one workgroup of 256 rows per CU
// (MMHIP_DISABLE_FA_DMA=1 takes the register-staged kernel instead)
constexpr size_t FA_DMA_LDS  = 8 * FA_BK * 256;  // K and V rings of 4 tiles
constexpr size_t FA_DMA_LDS2 = 4 * FA_BK * 256;  // K and V rings of 2 tiles (two workgroups per CU)

static int fa_dma_qtiles(const FaArgs & a) {
    return a.mask ? (a.nq + 127) / 128 : (a.nq + 255) / 256;
}

static bool fa_dma_ok(const FaArgs & a, int D) {
    auto al16 = [](int64_t v) { return (v & 15) == 0; };
    const int64_t tiles = (int64_t) fa_dma_qtiles(a) * a.Hq * a.B;
    return D == 128 && !getenv("MMHIP_DISABLE_FA_DMA") && tiles >= 256 && a.nkv >= 1 &&
           al16((int64_t) (uintptr_t) a.q) && al16(a.qnb1) &&
           al16(a.qnb2) && al16(a.qnb3) && al16((int64_t) (uintptr_t) a.k) && al16(a.knb1) && al16(a.knb2) &&
           al16(a.knb3) && al16((int64_t) (uintptr_t) a.v) && al16(a.vnb1) && al16(a.vnb2) && al16(a.vnb3);
}

// Mask prepass: for every mask plane (mask batch x mask head) and query row,
// one past the last key whose mask value is not -inf (0 if the row is fully
// masked), and the length of the row's leading run of exact zeros (+-0: no
// bias, so those keys need no mask).  One wave per row, 16-byte loads.
__global__ __launch_bounds__(256) void k_fa_row_end(FaArgs a, int * __restrict__ row_end, int * __restrict__ zero_end) {
    const int64_t row   = (int64_t) blockIdx.x * 4 + (threadIdx.x >> 6);  // plane * nq + q
    const int     lane  = threadIdx.x & 63;
    const int64_t nrows = (int64_t) a.nq * a.mne2 * a.mne3;
    if (row >= nrows) {
        return;
    }
    const int        q     = (int) (row % a.nq);
    const int        plane = (int) (row / a.nq);
    const uint16_t * mr    = (const uint16_t *) (a.mask + (int64_t) q * a.mnb1 + (plane % a.mne2) * a.mnb2 +
                                                 (plane / a.mne2) * a.mnb3);
    int best = -1, first_nz = a.nkv;
    auto see = [&](uint16_t hv, int k) {
        if (hv != 0xfc00) {  // f16 -inf
            best = max(best, k);
        }
        if ((hv & 0x7fff) != 0) {
            first_nz = min(first_nz, k);
        }
    };
    if ((((uintptr_t) mr) & 15) == 0) {
        const int nvec = a.nkv / 8;
        for (int i = lane; i < nvec; i += 64) {
            const int4_t w = *(const int4_t *) (mr + 8 * i);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const uint32_t word = (uint32_t) w[j / 2];
                see((uint16_t) ((j & 1) ? (word >> 16) : (word & 0xffff)), 8 * i + j);
            }
        }
        for (int k = nvec * 8 + lane; k < a.nkv; k += 64) {
            see(mr[k], k);
        }
    } else {
        for (int k = lane; k < a.nkv; k += 64) {
            see(mr[k], k);
        }
    }
    best     = (int) wave_max((float) best);
    first_nz = -(int) wave_max((float) -first_nz);
    if (lane == 0) {
        row_end[row]  = best + 1;
        zero_end[row] = first_nz;
    }
}

// Query rows per workgroup: 256 (8 waves) for D = 128 when that still gives
// every CU work, else 128 (4 waves).
static int fa_mfma_waves(const FaArgs & a, int D) {
    const int64_t tiles256 = (int64_t) ((a.nq + 255) / 256) * a.Hq * a.B;
    return D == 128 && tiles256 >= 256 ? 8 : 4;
}

size_t fa_mfma_workspace(const FaArgs & a) {
    // per-row ends and zero-prefix lengths for up to Hq * B mask planes
    return 2 * align_up((size_t) a.nq * a.Hq * a.B * sizeof(int), 256);
}

bool fa_mfma_supported(const FaArgs & a, int D) {
    return (D == 64 || D == 128) && a.nq >= 1;
}

template <int D, int NW>
static void launch_fa_mfma(const FaArgs & a, const int * row_end, const int * zero_end, int n_qtiles, float * out,
                           hipStream_t stream) {
    const int64_t total = (int64_t) n_qtiles * a.Hq * a.B;
    hipLaunchKernelGGL((k_fa_mfma<D, NW>), dim3((unsigned) total), dim3(NW * 64), 0, stream, a, row_end, zero_end,
                       n_qtiles, out);
}

int fa_mfma(const FaArgs & a, int D, float * out, void * ws, size_t ws_bytes, hipStream_t stream) {
    const int NW       = fa_mfma_waves(a, D);
    const int BQ       = NW * 32;
    const int n_qtiles = (a.nq + BQ - 1) / BQ;
    if ((int64_t) n_qtiles * a.Hq * a.B > 0x7fffffff) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "flash_attn mfma: grid too large");
    }
    int * row_end  = nullptr;
    int * zero_end = nullptr;
    if (a.mask) {
        const size_t need = fa_mfma_workspace(a);
        if (!ws || ws_bytes < need) {
            return set_error(MMHIP_ERR_WORKSPACE, "flash_attn mfma: workspace %zu < %zu", ws_bytes, need);
        }
        row_end             = (int *) ws;
        zero_end            = (int *) ((char *) ws + need / 2);
        const int64_t nrows = (int64_t) a.nq * a.mne2 * a.mne3;
        hipLaunchKernelGGL(k_fa_row_end, dim3((unsigned) ((nrows + 3) / 4)), dim3(256), 0, stream, a, row_end,
                           zero_end);
        int rc = check_launch("flash_attn mask prepass");
        if (rc != MMHIP_OK) {
            return rc;
        }
    }
    if (fa_dma_ok(a, D)) {
        const int    nqt = fa_dma_qtiles(a);
        const size_t lds = FA_DMA_LDS;
        if (a.mask) {
            if (!ensure_lds_limit((const void *) k_fa_dma<true, 4, 2>, FA_DMA_LDS2)) {
                return set_error(MMHIP_ERR_HIP, "flash_attn dma: cannot raise the LDS limit");
            }
            hipLaunchKernelGGL((k_fa_dma<true, 4, 2>), dim3((unsigned) (nqt * a.Hq * a.B)), dim3(256), FA_DMA_LDS2,
                               stream, a, row_end, zero_end, nqt, out);
        } else {
            if (!ensure_lds_limit((const void *) k_fa_dma<false>, lds)) {
                return set_error(MMHIP_ERR_HIP, "flash_attn dma: cannot raise the LDS limit");
            }
            hipLaunchKernelGGL(k_fa_dma<false>, dim3((unsigned) (nqt * a.Hq * a.B)), dim3(512), lds, stream, a,
                               nullptr, nullptr, nqt, out);
        }
    } else if (D == 128) {
        NW == 8 ? launch_fa_mfma<128, 8>(a, row_end, zero_end, n_qtiles, out, stream)
                : launch_fa_mfma<128, 4>(a, row_end, zero_end, n_qtiles, out, stream);
    } else if (D == 64) {
        launch_fa_mfma<64, 4>(a, row_end, zero_end, n_qtiles, out, stream);
    } else {
        return set_error(MMHIP_ERR_UNSUPPORTED, "flash_attn mfma: head dim %d", D);
    }
    return check_launch("flash_attn mfma");
}

}  // namespace mmhip
