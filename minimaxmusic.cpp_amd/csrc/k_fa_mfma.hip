// k_fa_mfma.hip - flash attention on MFMA for many query rows: causal prefill
// (src/qwen3-lm.h:432-436) and the DiT's bidirectional attention
// (src/dit.h:221-222).
//
// Workgroup = 4 waves = 128 query rows of one (head, batch); each wave owns 32
// query rows.  KV is walked in tiles of 64 keys staged in LDS (K as rows, V
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
// scale.  A prepass over the mask finds, per 128-query tile, the last key any
// query of the tile can see, so fully masked KV tiles (the causal upper
// triangle, the -inf padding of the cache window) are never read.
#include "k_fa_common.h"
#include "mmhip_device.h"
#include "mmhip_internal.h"

namespace mmhip {

constexpr int FA_BQ = 128;
constexpr int FA_BK = 64;

__device__ __forceinline__ float16_t mfma32(half8_t a, half8_t b, float16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// LDS position of key k (0..63) inside a V^T row: bits 2 and 3 swapped.
__device__ __forceinline__ int vt_pos(int k) {
    return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1);
}

template <int D>
__global__ __launch_bounds__(256) void k_fa_mfma(FaArgs a, const int * __restrict__ kv_end_tab, int n_qtiles,
                                                 float * __restrict__ out) {
    constexpr int KS = D + 8;       // K row stride (halves)
    constexpr int VS = FA_BK + 8;   // V^T row stride (halves)
    constexpr int NQK = D / 16;     // MFMA k-steps for Q.K
    constexpr int NDB = D / 32;     // 32-row blocks of O^T
    __shared__ __attribute__((aligned(16))) _Float16 sK[FA_BK * KS];
    __shared__ __attribute__((aligned(16))) _Float16 sV[D * VS];

    const int qt   = n_qtiles - 1 - (int) blockIdx.x;  // longest (causal) tiles first
    const int h    = blockIdx.y;
    const int b    = blockIdx.z;
    const int G    = a.Hq / a.Hkv;
    const int hk   = h / G;
    const int bk   = b / (a.B / a.Bk);
    const int tid  = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int lq   = lane & 31;
    const int hh   = lane >> 5;
    const int my_q = qt * FA_BQ + wave * 32 + lq;
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

    int kv_end = a.nkv;
    if (kv_end_tab) {
        const int plane = (b % a.mne3) * a.mne2 + (h % a.mne2);
        kv_end          = min(kv_end, kv_end_tab[plane * n_qtiles + qt]);
    }

    const char * kbase = a.k + hk * a.knb2 + bk * a.knb3;
    const char * vbase = a.v + hk * a.vnb2 + bk * a.vnb3;

    for (int k0 = 0; k0 < kv_end; k0 += FA_BK) {
        __syncthreads();
        // stage K rows
        for (int c = tid; c < FA_BK * (D / 8); c += 256) {
            const int key = c / (D / 8), seg = c % (D / 8);
            const int kg  = k0 + key;
            half8_t   v   = {};
            if (kg < a.nkv) {
                v = *(const half8_t *) (kbase + (int64_t) kg * a.knb1 + seg * 16);
            }
            *(half8_t *) &sK[key * KS + seg * 8] = v;
        }
        // stage V transposed, two keys per 32-bit LDS write
        for (int c = tid; c < (FA_BK / 2) * (D / 8); c += 256) {
            const int kp = c / (D / 8), seg = c % (D / 8);
            const int key = 2 * kp;
            const int kg  = k0 + key;
            half8_t   v0 = {}, v1 = {};
            if (kg < a.nkv) {
                v0 = *(const half8_t *) (vbase + (int64_t) kg * a.vnb1 + seg * 16);
            }
            if (kg + 1 < a.nkv) {
                v1 = *(const half8_t *) (vbase + (int64_t) (kg + 1) * a.vnb1 + seg * 16);
            }
            const int pos = vt_pos(key);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                half2_t pr = { v0[i], v1[i] };
                *(half2_t *) &sV[(seg * 8 + i) * VS + pos] = pr;
            }
        }
        __syncthreads();

        // S^T (64 keys x 32 queries) = K Q^T
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
        // scale, mask, out-of-range keys; tile max for this lane's query
        float mx = -INFINITY;
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
        mx               = fmaxf(mx, __shfl_xor(mx, 32, WAVE));
        const float mnew = fmaxf(m, mx);
        float       alpha = 1.0f, rs = 0.0f;
        half8_t     pb[2][2];
        if (mnew == -INFINITY) {
#pragma unroll
            for (int kb = 0; kb < 2; kb++) {
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    pb[kb][t] = half8_t{};
                }
            }
        } else {
            alpha = __builtin_amdgcn_exp2f(m - mnew);
#pragma unroll
            for (int kb = 0; kb < 2; kb++) {
#pragma unroll
                for (int t = 0; t < 2; t++) {
#pragma unroll
                    for (int u = 0; u < 8; u++) {
                        const float p = __builtin_amdgcn_exp2f(s[kb][8 * t + u] - mnew);
                        rs += p;
                        pb[kb][t][u] = (_Float16) p;
                    }
                }
            }
        }
        rs = rs + __shfl_xor(rs, 32, WAVE);
        l  = l * alpha + rs;
        m  = mnew;
#pragma unroll
        for (int i = 0; i < NDB; i++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                oacc[i][r] *= alpha;
            }
        }
        // O^T (D x 32 queries) += V^T P^T
#pragma unroll
        for (int db = 0; db < NDB; db++) {
#pragma unroll
            for (int kb = 0; kb < 2; kb++) {
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const half8_t av = *(const half8_t *) &sV[(db * 32 + lq) * VS + kb * 32 + 16 * t + 8 * hh];
                    oacc[db]         = mfma32(av, pb[kb][t], oacc[db]);
                }
            }
        }
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

// Mask prepass: for every mask plane (mask batch x mask head) and 128-query
// tile, one past the last key with a finite mask value in any of the tile's
// queries (0 if the whole tile is masked).
__global__ __launch_bounds__(256) void k_fa_kv_end(FaArgs a, int n_qtiles, int * __restrict__ kv_end_tab) {
    __shared__ int s_max[4];
    const int      qt    = blockIdx.x;
    const int      plane = blockIdx.y;
    const int      m3    = plane / a.mne2;
    const int      m2    = plane % a.mne2;
    int            best  = -1;
    const int      q_end = min(a.nq, (qt + 1) * FA_BQ);
    for (int q = qt * FA_BQ; q < q_end; q++) {
        const uint16_t * mr = (const uint16_t *) (a.mask + (int64_t) q * a.mnb1 + m2 * a.mnb2 + m3 * a.mnb3);
        for (int k = a.nkv - 1 - (int) threadIdx.x; k > best; k -= 256) {
            if (mr[k] != 0xfc00) {  // f16 -inf
                best = max(best, k);
                break;
            }
        }
    }
    best = (int) wave_max((float) best);
    if ((threadIdx.x & 63) == 0) {
        s_max[threadIdx.x >> 6] = best;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const int v = max(max(s_max[0], s_max[1]), max(s_max[2], s_max[3]));
        kv_end_tab[plane * n_qtiles + qt] = v + 1;
    }
}

size_t fa_mfma_workspace(const FaArgs & a) {
    const int n_qtiles = (a.nq + FA_BQ - 1) / FA_BQ;
    return align_up((size_t) n_qtiles * a.Hq * a.B * sizeof(int), 256);
}

bool fa_mfma_supported(const FaArgs & a, int D) {
    return (D == 64 || D == 128) && a.nq >= 1;
}

int fa_mfma(const FaArgs & a, int D, float * out, void * ws, size_t ws_bytes, hipStream_t stream) {
    const int n_qtiles = (a.nq + FA_BQ - 1) / FA_BQ;
    if (a.Hq > 65535 || a.B > 65535) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "flash_attn mfma: grid too large");
    }
    int * kv_end = nullptr;
    if (a.mask) {
        const size_t need = fa_mfma_workspace(a);
        if (!ws || ws_bytes < need) {
            return set_error(MMHIP_ERR_WORKSPACE, "flash_attn mfma: workspace %zu < %zu", ws_bytes, need);
        }
        kv_end = (int *) ws;
        hipLaunchKernelGGL(k_fa_kv_end, dim3(n_qtiles, a.mne2 * a.mne3), dim3(256), 0, stream, a, n_qtiles, kv_end);
        int rc = check_launch("flash_attn mask prepass");
        if (rc != MMHIP_OK) {
            return rc;
        }
    }
    const dim3 grid(n_qtiles, a.Hq, a.B);
    if (D == 128) {
        hipLaunchKernelGGL(k_fa_mfma<128>, grid, dim3(256), 0, stream, a, kv_end, n_qtiles, out);
    } else if (D == 64) {
        hipLaunchKernelGGL(k_fa_mfma<64>, grid, dim3(256), 0, stream, a, kv_end, n_qtiles, out);
    } else {
        return set_error(MMHIP_ERR_UNSUPPORTED, "flash_attn mfma: head dim %d", D);
    }
    return check_launch("flash_attn mfma");
}

}  // namespace mmhip
