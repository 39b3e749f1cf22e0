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
    if (D == 128) {
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
