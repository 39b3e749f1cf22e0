// k_fa_decode.hip - split-KV flash attention for few query rows per KV head
// (the LM's CFG-batched decode: n_q = 1, 4 query heads per KV head).
//
// Grid (splits, Hkv, B * row_groups).  A workgroup reads one KV range of one
// KV head once and serves all query rows of that head group (GQA), so K/V
// bytes cross HBM once.  D/8 lanes share a key (16-byte K and V loads, keys
// contiguous in the cache), 64/(D/8) keys per wave step; every lane keeps its
// own online-softmax state (max, sum, 8 output dims) and states are merged
// across lanes, waves and splits with the log-sum-exp rule.
//
// Arithmetic: Q is rounded to f16 and Q.K uses f16 products with f32
// accumulation (v_dot2_f32_f16), as ggml-CPU converts Q to K's type; the
// softmax and the V accumulation are f32 (GGML_PREC_F32), in base 2 with
// log2(e) folded into the scale.
#include "mmhip_device.h"
#include "mmhip_internal.h"
#include <cstdlib>

#include "k_fa_common.h"

namespace mmhip {

template <int D, int QR, int U>
__global__ __launch_bounds__(256) void k_fa_decode(FaArgs a, int chunk, int nsplit, float * __restrict__ part_o,
                                                   float * __restrict__ part_ml, float * __restrict__ out) {
    constexpr int LPK = D / 8;
    constexpr int KPW = 64 / LPK;
    __shared__ float s_m[4][QR], s_l[4][QR];
    __shared__ float s_o[4][QR][D];

    const int split = blockIdx.x;
    const int g     = blockIdx.y;
    const int b     = blockIdx.z % a.B;
    const int rg    = blockIdx.z / a.B;
    const int G     = a.Hq / a.Hkv;
    const int nrows = G * a.nq;
    const int r0    = rg * QR;
    const int bk    = b / (a.B / a.Bk);
    const int wave  = threadIdx.x >> 6;
    const int lane  = threadIdx.x & 63;
    const int seg   = lane % LPK;
    const int ks    = lane / LPK;
    const int kbeg  = split * chunk;
    const int kend  = min(a.nkv, kbeg + chunk);

    const char * mrow[QR];
    const float * qrow[QR];
    bool         rvalid[QR];
#pragma unroll
    for (int r = 0; r < QR; r++) {
        const int rr  = r0 + r;
        rvalid[r]     = rr < nrows;
        const int rrc = rvalid[r] ? rr : r0;
        const int hq  = g * G + rrc % G;
        const int iq  = rrc / G;
        qrow[r]       = (const float *) (a.q + iq * a.qnb1 + hq * a.qnb2 + b * a.qnb3) + seg * 8;
        mrow[r] = a.mask ? a.mask + iq * a.mnb1 + (hq % a.mne2) * a.mnb2 + (b % a.mne3) * a.mnb3 : nullptr;
    }

    const char * kbase = a.k + g * a.knb2 + bk * a.knb3 + seg * 16;
    const char * vbase = a.v + g * a.vnb2 + bk * a.vnb3 + seg * 16;

    // mask rows shared by every query row of the group (the LM's causal /
    // padding mask is one row per token): one mask load per key
    bool mask_shared = true;
#pragma unroll
    for (int r = 1; r < QR; r++) {
        mask_shared = mask_shared && (!rvalid[r] || mrow[r] == mrow[0]);
    }
    // without a mask, the loads read K's first bytes (in bounds: 2 * nkv <=
    // the K rows) and the value is dropped, keeping every load unconditional
    const char * mbase = mrow[0] ? mrow[0] : a.k;
    const bool   has_m = mrow[0] != nullptr;

    // One pass = U keys per lane.  All K / V / mask loads of a pass are issued
    // together (those of the first pass even before Q's), then all scores,
    // one running-max update per row, and the exp2-weighted V sums.
    half8_t  kk[U], vv[U];
    int      jc[U];
    uint16_t mk[U];  // raw f16 mask bits: converted at use, so no load waits here
    auto     load_pass = [&](int base) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int j = base + 4 * KPW * u + ks;
            jc[u]       = j < kend ? j : kend - 1;
            kk[u]       = *(const half8_t *) (kbase + (int64_t) jc[u] * a.knb1);
            vv[u]       = *(const half8_t *) (vbase + (int64_t) jc[u] * a.vnb1);
            mk[u]       = *(const uint16_t *) (mbase + jc[u] * 2);
        }
    };
    const int step = 4 * KPW * U;
    int       base = kbeg + wave * KPW;
    if (base < kend) {
        load_pass(base);
    }

    half8_t qv[QR];
#pragma unroll
    for (int r = 0; r < QR; r++) {
#pragma unroll
        for (int d = 0; d < 8; d++) {
            qv[r][d] = (_Float16) qrow[r][d];  // q is only 4-byte aligned
        }
    }

    float m[QR], l[QR], o[QR][8];
#pragma unroll
    for (int r = 0; r < QR; r++) {
        m[r] = -INFINITY;
        l[r] = 0.0f;
#pragma unroll
        for (int d = 0; d < 8; d++) {
            o[r][d] = 0.0f;
        }
    }
    const float log2e = 1.4426950408889634f;

    for (; base < kend; base += step) {
        float sc[QR][U];
#pragma unroll
        for (int u = 0; u < U; u++) {
#pragma unroll
            for (int r = 0; r < QR; r++) {
                float dot = 0.0f;
                dot = __builtin_amdgcn_fdot2(half2_t{ kk[u][0], kk[u][1] }, half2_t{ qv[r][0], qv[r][1] }, dot, false);
                dot = __builtin_amdgcn_fdot2(half2_t{ kk[u][2], kk[u][3] }, half2_t{ qv[r][2], qv[r][3] }, dot, false);
                dot = __builtin_amdgcn_fdot2(half2_t{ kk[u][4], kk[u][5] }, half2_t{ qv[r][4], qv[r][5] }, dot, false);
                dot = __builtin_amdgcn_fdot2(half2_t{ kk[u][6], kk[u][7] }, half2_t{ qv[r][6], qv[r][7] }, dot, false);
                dot = group_sum<LPK>(dot);
                const float mv = !has_m ? 0.0f
                                 : (mask_shared || r == 0) ? h2f(mk[u])
                                                           : h2f(*(const uint16_t *) (mrow[r] + jc[u] * 2));
                const bool kv = base + 4 * KPW * u + ks < kend;
                sc[r][u]      = (kv && rvalid[r]) ? (dot * a.scale + mv) * log2e : -INFINITY;
            }
        }
        half8_t vcur[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            vcur[u] = vv[u];
        }
        if (base + step < kend) {
            load_pass(base + step);  // next pass's loads overlap this pass's softmax
        }
#pragma unroll
        for (int r = 0; r < QR; r++) {
            float mn = m[r];
#pragma unroll
            for (int u = 0; u < U; u++) {
                mn = fmaxf(mn, sc[r][u]);
            }
            if (mn == -INFINITY) {
                continue;  // nothing finite yet for this row (per-lane state, no cross-lane op below)
            }
            const float alpha = __builtin_amdgcn_exp2f(m[r] - mn);
            float       psum  = 0.0f;
            float       pv[8];
#pragma unroll
            for (int d = 0; d < 8; d++) {
                pv[d] = 0.0f;
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                const float p = __builtin_amdgcn_exp2f(sc[r][u] - mn);
                psum += p;
#pragma unroll
                for (int d = 0; d < 8; d++) {
                    pv[d] += p * (float) vcur[u][d];
                }
            }
            l[r] = l[r] * alpha + psum;
#pragma unroll
            for (int d = 0; d < 8; d++) {
                o[r][d] = o[r][d] * alpha + pv[d];
            }
            m[r] = mn;
        }
    }

    // merge the KPW key slots of the wave (lanes with equal seg)
#pragma unroll
    for (int off = LPK; off < 64; off <<= 1) {
#pragma unroll
        for (int r = 0; r < QR; r++) {
            const float m2 = __shfl_xor(m[r], off, WAVE);
            const float l2 = __shfl_xor(l[r], off, WAVE);
            const float M  = fmaxf(m[r], m2);
            const float a1 = m[r] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m[r] - M);
            const float a2 = m2 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m2 - M);
            l[r]           = l[r] * a1 + l2 * a2;
#pragma unroll
            for (int d = 0; d < 8; d++) {
                const float o2 = __shfl_xor(o[r][d], off, WAVE);
                o[r][d]        = o[r][d] * a1 + o2 * a2;
            }
            m[r] = M;
        }
    }
    if (ks == 0) {
#pragma unroll
        for (int r = 0; r < QR; r++) {
#pragma unroll
            for (int d = 0; d < 8; d++) {
                s_o[wave][r][seg * 8 + d] = o[r][d];
            }
            if (seg == 0) {
                s_m[wave][r] = m[r];
                s_l[wave][r] = l[r];
            }
        }
    }
    __syncthreads();

    for (int idx = threadIdx.x; idx < QR * D; idx += 256) {
        const int r  = idx / D;
        const int d  = idx % D;
        const int rr = r0 + r;
        if (rr >= nrows) {
            continue;
        }
        float M = s_m[0][r];
#pragma unroll
        for (int w = 1; w < 4; w++) {
            M = fmaxf(M, s_m[w][r]);
        }
        float L = 0.0f, O = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const float sc = s_m[w][r] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s_m[w][r] - M);
                L += s_l[w][r] * sc;
                O += s_o[w][r][d] * sc;
            }
        }
        const int hq = g * G + rr % G;
        const int iq = rr / G;
        if (nsplit == 1) {
            out[(((int64_t) b * a.nq + iq) * a.Hq + hq) * D + d] = L > 0.0f ? O / L : 0.0f;
        } else {
            const int64_t pr = (((int64_t) b * a.Hq + hq) * a.nq + iq) * nsplit + split;
            part_o[pr * D + d] = O;
            if (d == 0) {
                part_ml[pr * 2 + 0] = M;
                part_ml[pr * 2 + 1] = L;
            }
        }
    }
}

// ---------------------------------------------------------------------
// MFMA decode: the G * nq (<= 16) query rows of one KV head are the columns
// of 16 x 16 MFMA tiles.  Workgroup = (split, KV head, batch), NW waves; the
// split's keys are dealt to the waves in 16-key tiles (wave w: tiles w,
// w + NW, ...), each wave keeping its own online-softmax state.  A wave
// issues the loads of TP tiles at once: with the split sized to NW * TP
// tiles every load of the workgroup is in flight before the first use.
//   S^T (16 keys x 16 cols) = K Q^T with mfma_f32_16x16x32_f16: lane l owns
//     key l % 16 and dims 32s + 8(l / 16) .. +7 of the A operand, a 16-byte
//     load straight from the cache; Q^T is the B operand, held in registers.
//   The S^T accumulator (lane l: keys 4(l / 16) + i, column l % 16) is
//     exactly the B-operand layout of mfma_f32_16x16x16f16, so P^T feeds
//     O^T (dims x cols) = V^T P^T without leaving registers.
//   V^T (the A operand: lane l needs dim l % 16 of keys 4(l / 16) .. +3) goes
//     through a per-wave LDS tile written transposed.
// Scores, softmax and the partial format are those of k_fa_decode, and the
// same combine kernel merges the splits.

#ifndef DEC_NW
#define DEC_NW 8  // waves per MFMA decode workgroup
#endif
// waves per workgroup at head size D (the merge buffer is NW * 16 * D floats)
constexpr int dec_nw(int D) {
    return D >= 256 && DEC_NW > 8 ? 8 : DEC_NW;
}

// One row of the fused head prologue (HD): the RMS norm, weight and NeoX
// RoPE of k_head_rows' head_row, lane l holding elements EPL l .. (the rotate
// pairs lanes l and l ^ 32).
template <int D>
__device__ __forceinline__ void fa_head_row(float (&v)[D / 64], const float (&w)[D / 64], bool norm, bool has_w,
                                            float eps, bool rope, int32_t pos, float ts, int lane) {
#pragma clang fp contract(off)
    constexpr int EPL = D / 64;
    if (norm) {
        double ss = 0.0;
#pragma unroll
        for (int k = 0; k < EPL; k++) {
            ss += (double) (v[k] * v[k]);
        }
        ss               = wave_sum_d(ss);
        const float mean = (float) (ss / (double) D);
        const float sc   = 1.0f / sqrtf(mean + eps);
#pragma unroll
        for (int k = 0; k < EPL; k++) {
            const float y = v[k] * sc;
            v[k]          = has_w ? y * w[k] : y;
        }
    }
    if (rope) {
        const int i0    = EPL * (lane & 31);
        float     theta = (float) pos;
        for (int k = 0; k < i0; k++) {
            theta *= ts;
        }
        const bool upper = lane >= 32;
#pragma unroll
        for (int k = 0; k < EPL; k++) {
            const float other = __shfl_xor(v[k], 32, WAVE);
            const float c = cosf(theta), sn = sinf(theta);
            v[k]  = upper ? other * sn + v[k] * c : v[k] * c - other * sn;
            theta *= ts;
        }
    }
}

template <int D, int NW, int TP, bool HD>
__global__ __launch_bounds__(64 * NW) void k_fa_dec_mfma(FaArgs a, FaHead h, int chunk, int nsplit,
                                                         float * __restrict__ part_o, float * __restrict__ part_ml,
                                                         float * __restrict__ out) {
    constexpr int NS  = D / 32;  // k-steps of Q.K (32 dims each)
    constexpr int NDB = D / 16;  // 16-dim blocks of O^T
    constexpr int VTS = 16 + 4;  // V^T row stride (halves): 16 keys + pad
    constexpr int SVT = NW * D * VTS;     // halves of the waves' V^T tiles
    constexpr int OS  = D + 4;             // merge-buffer row stride (floats): rows 4 banks apart
    constexpr int SO  = NW * 16 * OS * 2;  // halves of the merge buffer (floats)
    __shared__ __attribute__((aligned(16))) _Float16 s_buf[SVT > SO ? SVT : SO];
    __shared__ float s_m[NW][16], s_l[NW][16];
    // HD: the processed query rows (f32) and the new key / value rows (f16)
    __shared__ __attribute__((aligned(16))) float    s_qrow[HD ? 16 : 1][HD ? D : 4];
    __shared__ __attribute__((aligned(16))) _Float16 s_new[2][HD ? D : 8];

    const int split = blockIdx.x;
    const int g     = blockIdx.y;
    const int b     = blockIdx.z;
    const int G     = a.Hq / a.Hkv;
    const int ncol  = G * a.nq;
    const int bk    = b / (a.B / a.Bk);
    const int wave  = threadIdx.x >> 6;
    const int lane  = threadIdx.x & 63;
    const int col   = lane & 15;
    const int kq    = lane >> 4;
    const int kbeg  = split * chunk;
    const int kend  = min(a.nkv, kbeg + chunk);
    const int ntile = (kend - kbeg + 15) / 16;

    const bool   cvalid = col < ncol;
    const int    cc     = cvalid ? col : 0;
    const int    hq     = g * G + cc % G;
    const int    iq     = cc / G;
    const char * mrow   = a.mask ? a.mask + iq * a.mnb1 + (hq % a.mne2) * a.mnb2 + (b % a.mne3) * a.mnb3 : nullptr;

    const char * kbase = a.k + g * a.knb2 + bk * a.knb3 + 16 * kq;
    const char * vbase = a.v + g * a.vnb2 + bk * a.vnb3 + 16 * kq;
    _Float16 *   svt   = s_buf + wave * D * VTS;

    // without a mask the mask loads read the cache's first bytes (in bounds:
    // 2 * nkv <= the K rows) and are dropped, so every load is unconditional
    const char * mbase = mrow ? mrow : a.k;

    // loads of TP tiles: K and V fragments (lane: key l % 16, dims 32s + 8kq
    // ..) and the raw mask bits of the lane's score keys 4kq .. 4kq+3
    half8_t  kf[TP][NS], vf[TP][NS];
    uint16_t mk[TP][4];
    auto     load_tiles = [&](int t0) {
#pragma unroll
        for (int p = 0; p < TP; p++) {
            const int t   = t0 + NW * p;
            const int key = min(kbeg + 16 * t + col, kend - 1);
#pragma unroll
            for (int s = 0; s < NS; s++) {
                kf[p][s] = *(const half8_t *) (kbase + (int64_t) key * a.knb1 + 64 * s);
                vf[p][s] = *(const half8_t *) (vbase + (int64_t) key * a.vnb1 + 64 * s);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                mk[p][i] = *(const uint16_t *) (mbase + (int64_t) min(kbeg + 16 * t + 4 * kq + i, kend - 1) * 2);
            }
        }
    };
    // HD: wave w < ncol processes query column w, wave ncol the new key row,
    // wave ncol + 1 the new value row (further waves redo the value row and
    // drop it).  Their loads go first, ahead of the tiles: loads return in
    // order, so the prologue runs while the tiles are in flight.
    constexpr int EPL  = D / 64;
    const int     task = min(wave, ncol + 1);
    float         tv[EPL], tw[EPL];
    int32_t       tpos = 0;
    int64_t       id   = -1;  // the new rows' cache row
    if constexpr (HD) {
        const char *    src;
        const float *   wp;
        const int32_t * pp;
        if (task < ncol) {
            const int     hq_t = g * G + task % G;
            const int     iq_t = task / G;
            const int64_t r    = h.qr0 + iq_t * h.qr1 + hq_t * h.qr2 + b * h.qr3;
            src                = h.q_src + (r / h.q_H) * h.q_nbt + (r % h.q_H) * h.q_nbh;
            wp                 = h.q_w ? h.q_w : (const float *) src;
            pp                 = h.q_pos ? h.q_pos + r / h.q_H : (const int32_t *) src;
        } else if (task == ncol) {
            src = h.k_src + b * h.k_nbt + g * h.k_nbh;
            wp  = h.k_w ? h.k_w : (const float *) src;
            pp  = h.k_pos ? h.k_pos + b : (const int32_t *) src;
        } else {
            src = h.v_src + b * h.v_nbt + g * h.v_nbh;
            wp  = (const float *) src;
            pp  = (const int32_t *) src;
        }
#pragma unroll
        for (int k = 0; k < EPL; k++) {
            tv[k] = ((const float *) src)[EPL * lane + k];
            tw[k] = wp[EPL * lane + k];
        }
        tpos             = *pp;
        const char * ip  = h.ids + (g % h.ids_ne1) * h.ids_nb1 + (b % h.ids_ne2) * h.ids_nb2;
        id               = h.ids_type == 27 ? *(const int64_t *) ip : (int64_t) *(const int32_t *) ip;
        // wait for them before the tile loads go out: issued together, these
        // few small loads return behind the whole KV stream of the GPU
#pragma unroll
        for (int k = 0; k < EPL; k++) {
            asm volatile("" ::"v"(tv[k]), "v"(tw[k]));
        }
        asm volatile("" ::"v"(tpos), "v"(id));
    }
    // HD: the rows are processed before the tile loads go out as well: the
    // tile loads fill the memory request queues, so a wave issuing them
    // stalls until earlier requests drain, and the rows are on the critical
    // path (every wave needs the query rows before its first tile)
    if constexpr (HD) {
        if (task <= ncol + 1) {
            const bool is_q = task < ncol;
            fa_head_row<D>(tv, tw, is_q ? h.q_norm != 0 : task == ncol && h.k_norm != 0,
                           is_q ? h.q_w != nullptr : h.k_w != nullptr, is_q ? h.q_eps : h.k_eps,
                           is_q ? h.q_pos != nullptr : task == ncol && h.k_pos != nullptr, tpos, is_q ? h.q_ts : h.k_ts,
                           lane);
            const bool writer = split == ((id >= 0 && id < a.nkv) ? (int) (id / chunk) : 0);
            if (is_q) {
#pragma unroll
                for (int k = 0; k < EPL; k++) {
                    s_qrow[task][EPL * lane + k] = tv[k];
                }
            } else if (wave == task) {
                const int  nr = task - ncol;  // 0 key, 1 value
                char *     dp = (char *) (nr == 0 ? a.k : a.v) + id * (nr == 0 ? a.knb1 : a.vnb1) +
                            g * (nr == 0 ? a.knb2 : a.vnb2) + b * (nr == 0 ? a.knb3 : a.vnb3);
#pragma unroll
                for (int k = 0; k < EPL; k++) {
                    const uint16_t hb = f2h(tv[k]);
                    s_new[nr][EPL * lane + k] = __builtin_bit_cast(_Float16, hb);
                    if (writer && id >= 0) {
                        ((uint16_t *) dp)[EPL * lane + k] = hb;
                    }
                }
            }
        }
    }
    // the first tiles, unconditionally (keys are clamped into the split):
    // a load under a condition makes the compiler wait for everything
    // issued before it
    int t0 = wave;
    load_tiles(t0);
    // Q^T B operand: column col, dims 32s + 8kq .. +7 (zero for unused
    // columns; an unused column reads column 0's row)
    half8_t qb[NS];
    // HD: the key tile / column holding the new row (tn = -1: not in this
    // split); the writer is the split holding it (split 0 when none does)
    int tn = -1, kc = 0;
    if constexpr (HD) {
        __syncthreads();
#pragma unroll
        for (int s = 0; s < NS; s++) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                qb[s][i] = cvalid ? (_Float16) s_qrow[cc][32 * s + 8 * kq + i] : (_Float16) 0.0f;
            }
        }
        if (id >= kbeg && id < kend) {
            tn = (int) (id - kbeg) / 16;
            kc = (int) (id - kbeg) % 16;
        }
    } else {
    float         qf[NS][8];
    const float * qp  = (const float *) (a.q + iq * a.qnb1 + hq * a.qnb2 + b * a.qnb3) + 8 * kq;
    const bool    q16 = (((uintptr_t) a.q | (uintptr_t) a.qnb1 | (uintptr_t) a.qnb2 | (uintptr_t) a.qnb3) & 15) == 0;
    if (q16) {  // uniform
#pragma unroll
        for (int s = 0; s < NS; s++) {
            const float4_t lo = *(const float4_t *) (qp + 32 * s);
            const float4_t hi = *(const float4_t *) (qp + 32 * s + 4);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                qf[s][i]     = lo[i];
                qf[s][4 + i] = hi[i];
            }
        }
    } else {
#pragma unroll
        for (int s = 0; s < NS; s++) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                qf[s][i] = qp[32 * s + i];
            }
        }
    }
#pragma unroll
    for (int s = 0; s < NS; s++) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            qb[s][i] = cvalid ? (_Float16) qf[s][i] : (_Float16) 0.0f;
        }
    }
    }

    float4_t oacc[NDB];
#pragma unroll
    for (int i = 0; i < NDB; i++) {
        oacc[i] = float4_t{ 0.0f, 0.0f, 0.0f, 0.0f };
    }
    float       m     = -INFINITY;
    float       l     = 0.0f;
    const float log2e = 1.4426950408889634f;
    const float sl2   = a.scale * log2e;

    for (; t0 < ntile; t0 += NW * TP) {
#pragma unroll
        for (int p = 0; p < TP; p++) {
            const int t = t0 + NW * p;
            if (t >= ntile) {
                break;  // uniform over the wave
            }
            if constexpr (HD) {
                // the new row replaces what the cache held at its position
                if (t == tn && col == kc) {
#pragma unroll
                    for (int s = 0; s < NS; s++) {
                        kf[p][s] = *(const half8_t *) &s_new[0][32 * s + 8 * kq];
                        vf[p][s] = *(const half8_t *) &s_new[1][32 * s + 8 * kq];
                    }
                }
            }
            // S^T tile
            float4_t sacc = { 0.0f, 0.0f, 0.0f, 0.0f };
#pragma unroll
            for (int s = 0; s < NS; s++) {
                sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[p][s], qb[s], sacc, 0, 0, 0);
            }
            // V^T tile into LDS: dim 32s + 8kq + j, key col
#pragma unroll
            for (int s = 0; s < NS; s++) {
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    svt[(32 * s + 8 * kq + j) * VTS + col] = vf[p][s][j];
                }
            }
            // scores of keys 4kq + i for this lane's column
            const int key0 = kbeg + 16 * t + 4 * kq;
            float     sc[4];
            float     mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int   key = key0 + i;
                const bool  ok  = key < kend && cvalid;
                const float mv  = mrow ? h2f(mk[p][i]) : 0.0f;
                sc[i]           = ok ? sacc[i] * sl2 + mv * log2e : -INFINITY;
                mx              = fmaxf(mx, sc[i]);
            }
            mx = max_xor32(max_xor16(mx));
            // no divergent control flow around the MFMAs: a column with
            // nothing visible yet keeps alpha = 1 and p = exp2(-inf) = 0
            const float mnew  = fmaxf(m, mx);
            const bool  live  = mnew != -INFINITY;
            const float mref  = live ? mnew : 0.0f;
            const float alpha = live ? __builtin_amdgcn_exp2f(m - mnew) : 1.0f;
            half4_t     pb;
            float       rs = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float pv = __builtin_amdgcn_exp2f(sc[i] - mref);
                rs += pv;
                pb[i] = (_Float16) pv;
            }
            rs = sum_xor32(sum_xor16(rs));
            l = l * alpha + rs;
            m = mnew;
            // the transposed V tile written above by this wave's lanes
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int db = 0; db < NDB; db++) {
                const half4_t av = *(const half4_t *) &svt[(16 * db + col) * VTS + 4 * kq];
                oacc[db]         = oacc[db] * alpha;
                oacc[db]         = __builtin_amdgcn_mfma_f32_16x16x16f16(av, pb, oacc[db], 0, 0, 0);
            }
            __builtin_amdgcn_wave_barrier();
        }
        if (t0 + NW * TP < ntile) {
            load_tiles(t0 + NW * TP);
        }
    }

    // merge the NW waves (LDS reused: V^T tiles are done)
    __syncthreads();
    float * s_o = (float *) s_buf;  // [NW][16][OS]
    if (kq == 0) {
        s_m[wave][col] = m;
        s_l[wave][col] = l;
    }
    if (cvalid) {  // the merge reads the ncol used columns only
#pragma unroll
        for (int db = 0; db < NDB; db++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                s_o[(wave * 16 + col) * OS + 16 * db + 4 * kq + i] = oacc[db][i];
            }
        }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < ncol * D; idx += 64 * NW) {
        const int c = idx / D;
        const int d = idx % D;
        float     M = s_m[0][c];
#pragma unroll
        for (int w = 1; w < NW; w++) {
            M = fmaxf(M, s_m[w][c]);
        }
        float L = 0.0f, O = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < NW; w++) {
                const float f = s_m[w][c] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s_m[w][c] - M);
                L += s_l[w][c] * f;
                O += s_o[(w * 16 + c) * OS + d] * f;
            }
        }
        const int h  = g * G + c % G;
        const int qi = c / G;
        if (nsplit == 1) {
            out[(((int64_t) b * a.nq + qi) * a.Hq + h) * D + d] = L > 0.0f ? O / L : 0.0f;
        } else {
            const int64_t pr = (((int64_t) b * a.Hq + h) * a.nq + qi) * nsplit + split;
            part_o[pr * D + d] = O;
            if (d == 0) {
                part_ml[pr * 2 + 0] = M;
                part_ml[pr * 2 + 1] = L;
            }
        }
    }
}

// ---------------------------------------------------------------------
// The split combine of one output element (a head's dim d; its splits'
// partial rows at pr0 .. pr0 + nsplit - 1): the weights exp2(m_s - M) from
// the split maxima sm[] and sums sl[], the weighted sums in split order
// without contraction, then O / L (k_fa_combine_q's arithmetic).
__device__ __forceinline__ float fa_combine_elem(const float * __restrict__ part_o, int64_t pr0, int D, int d,
                                                 int nsplit, const float * sm, const float * sl) {
#pragma clang fp contract(off)
    float M = -INFINITY;
    for (int sidx = 0; sidx < nsplit; sidx++) {
        M = fmaxf(M, sm[sidx]);
    }
    float L = 0.0f, O = 0.0f;
    if (M != -INFINITY) {
#pragma unroll 8
        for (int sidx = 0; sidx < nsplit; sidx++) {
            const float ms = sm[sidx];
            const float f  = ms == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ms - M);
            L += sl[sidx] * f;
            O += part_o[(pr0 + sidx) * D + d] * f;
        }
    }
    return L > 0.0f ? O / L : 0.0f;
}

// Quantisation of an output element v (element e of activation row `row`,
// K elements a row) into the activation layout of qtype, with k_quant.hip's
// arithmetic.  Q8_0: a block is 32 consecutive lanes.  Q8_K: a super-block
// is the 256 threads of 4 consecutive waves, t the thread's index among them,
// s_red / s_idx / s_amax 4 LDS entries of theirs; every thread of the
// workgroup calls it together (it synchronises the workgroup), and only the
// valid ones store.
__device__ __forceinline__ void fa_quant_elem(float v, bool valid, int t, int64_t row, int e, int K, int qtype,
                                              int8_t * __restrict__ xq_qs, float * __restrict__ xq_d,
                                              int16_t * __restrict__ xq_bs, float * s_red, int * s_idx,
                                              float * s_amax) {
#pragma clang fp contract(off)
    int8_t * qs = xq_qs + row * K + e;
    if (qtype == TYPE_Q8_0) {
        const float a  = group32_max(fabsf(v));
        const float dd = a / 127.0f;
        const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
        if (valid) {
            *qs = (int8_t) roundf(v * id);
            if ((t & 31) == 0) {
                xq_d[row * (K / 32) + e / 32] = h2f(f2h(dd));
            }
        }
        return;
    }
    // Q8_K super-block of 256: the first element of largest |x|
    const int lane = t & 63;
    float     a    = fabsf(v);
    float     vm   = v;
    int       ix   = t;
    wave_argmax_abs(a, vm, ix);
    if (lane == 0) {
        s_red[t >> 6]  = vm;
        s_idx[t >> 6]  = ix;
        s_amax[t >> 6] = a;
    }
    __syncthreads();
    float bestA = s_amax[0], bestV = s_red[0];
    int   bestI = s_idx[0];
    for (int w = 1; w < 4; w++) {
        const float aw = s_amax[w];
        if (aw > bestA || (aw == bestA && s_idx[w] < bestI)) {
            bestA = aw;
            bestV = s_red[w];
            bestI = s_idx[w];
        }
    }
    int   q  = 0;
    float dd = 0.0f;
    if (bestA != 0.0f) {
        const float iscale = -127.0f / bestV;
        const int   qi     = (int) rintf(iscale * v);
        q                  = qi > 127 ? 127 : qi;
        dd                 = 1.0f / iscale;
    }
    const int sb = group16_sum_i(q);
    if (valid) {
        *qs = (int8_t) q;
        if ((t & 15) == 0) {
            xq_bs[row * (K / 16) + e / 16] = (int16_t) sb;
        }
        if (t == 0) {
            xq_d[row * (K / 256) + e / 256] = dd;
        }
    }
}

// ---------------------------------------------------------------------
// Decode with the head prologue and the split's whole KV range in LDS
// (D = 128, <= 256 keys per split, one query row, one mask row per
// workgroup: the LM's batched CFG decode, src/qwen3-lm.h:762-826).  The waves
// the prologue leaves free DMA the split's K and V rows into LDS with
// global_load_lds at kernel start, so the KV stream runs while
// the query / key / value rows are loaded, normalised and rotated; the
// prologue waves issue no DMA, so their waits are on their own row loads
// only.  Then the new key / value row replaces the stale cache row in LDS and
// every wave computes its 16-key tiles from LDS: K as the A operand of
// mfma_f32_16x16x32_f16 (chunk c of key row r stored at c ^ (r & 15)), V^T by
// ds_read_b64_tr_b16 as the A operand of mfma_f32_16x16x16f16 (chunk c of V
// row r at c ^ 2 (r & 3)).  Scores, softmax, wave merge and the partial
// format are those of k_fa_dec_mfma.
constexpr int DD_D     = 128;
constexpr int DD_NW    = 8;
constexpr int DD_MAXK  = 256;                       // keys per split
constexpr int DD_ROW   = DD_D * 2;                  // bytes per K / V row
constexpr int DD_KV    = DD_MAXK * DD_ROW;          // bytes of the K (or V) range
constexpr int DD_OS    = DD_D + 4;                  // merge-buffer row stride (floats)
constexpr int DD_LDS   = 2 * DD_KV + DD_MAXK * 2;   // K, V, mask row
typedef short dd_short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) dd_short4_t dd_lds_short4_t;

__device__ __forceinline__ void dd_dma16(const void * src, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds_addr) : "memory", "m0");
}

__global__ __launch_bounds__(64 * DD_NW) void k_fa_dec_dma(FaArgs a, FaHead h, int chunk, int nsplit,
                                                            float * __restrict__ part_o, float * __restrict__ part_ml,
                                                            float * __restrict__ out) {
    constexpr int D = DD_D, NW = DD_NW, NS = D / 32, NDB = D / 16, EPL = D / 64;
    extern __shared__ __attribute__((aligned(1024))) char dd_lds[];  // K [256][256 B], V [256][256 B], mask [256] f16
    __shared__ float s_m[NW][16], s_l[NW][16];
    __shared__ __attribute__((aligned(16))) float    s_qrow[16][D];
    __shared__ __attribute__((aligned(16))) _Float16 s_new[2][D];

    const int split = blockIdx.x;
    const int g     = blockIdx.y;
    const int b     = blockIdx.z;
    const int G     = a.Hq / a.Hkv;
    const int ncol  = G * a.nq;
    const int wave  = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane  = threadIdx.x & 63;
    const int col   = lane & 15;
    const int kq    = lane >> 4;
    const int kbeg  = split * chunk;
    const int kend  = min(a.nkv, kbeg + chunk);
    const int nkey  = kend - kbeg;
    const int ntile = (nkey + 15) / 16;
    const bool cvalid = col < ncol;
    const int  cc     = cvalid ? col : 0;
    const uint32_t lbase = (uint32_t) (uintptr_t) (__attribute__((address_space(3))) char *) dd_lds;

    // 1. the DMA waves (past the prologue's tasks): K and V rows of the
    // split, 1 KB (4 rows) per instruction, then the mask row
    const int ndma = NW - (ncol + 2);
    if (wave >= ncol + 2) {
        const int    dw    = wave - (ncol + 2);
        const char * kbase = a.k + g * a.knb2 + b * a.knb3;
        const char * vbase = a.v + g * a.vnb2 + b * a.vnb3;
        const int    npc   = (nkey + 3) / 4;  // 1 KB pieces per tensor
        const int    r4 = lane >> 4, c16 = lane & 15;
        for (int pc = dw; pc < 2 * npc; pc += ndma) {
            const bool isv = pc >= npc;
            const int  p   = isv ? pc - npc : pc;
            const int  r   = 4 * p + r4;
            const int  key = kbeg + min(r, nkey - 1);
            const int  ch  = isv ? (c16 ^ (2 * (r & 3))) : (c16 ^ (r & 15));
            const char * src = (isv ? vbase + (int64_t) key * a.vnb1 : kbase + (int64_t) key * a.knb1) + 16 * ch;
            dd_dma16(src, lbase + (isv ? DD_KV : 0) + p * 1024);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }

    // 2. the head prologue (waves 0 .. ncol + 1), as k_fa_dec_mfma's: all
    // of a wave's loads (cache row id, row, weight, position, mask) go out
    // together, then the wave computes
    int64_t id = -1;  // the new rows' cache row (prologue waves)
    if (wave < ncol + 2) {
        const int       task = wave;
        const char *    src;
        const float *   wp;
        const int32_t * pp;
        if (task < ncol) {
            const int     hq_t = g * G + task % G;
            const int     iq_t = task / G;
            const int64_t r    = h.qr0 + iq_t * h.qr1 + hq_t * h.qr2 + b * h.qr3;
            src                = h.q_src + (r / h.q_H) * h.q_nbt + (r % h.q_H) * h.q_nbh;
            wp                 = h.q_w ? h.q_w : (const float *) src;
            pp                 = h.q_pos ? h.q_pos + r / h.q_H : (const int32_t *) src;
        } else if (task == ncol) {
            src = h.k_src + b * h.k_nbt + g * h.k_nbh;
            wp  = h.k_w ? h.k_w : (const float *) src;
            pp  = h.k_pos ? h.k_pos + b : (const int32_t *) src;
        } else {
            src = h.v_src + b * h.v_nbt + g * h.v_nbh;
            wp  = (const float *) src;
            pp  = (const int32_t *) src;
        }
        // the id as one or two words, without a branch on its type (an i32
        // id reads its one word twice)
        const bool      i64  = h.ids_type == 27;
        const int32_t * ip   = (const int32_t *) (h.ids + (g % h.ids_ne1) * h.ids_nb1 + (b % h.ids_ne2) * h.ids_nb2);
        const int32_t   idlo = ip[0];
        const int32_t   idhi = ip[i64 ? 1 : 0];
        float           tv[EPL], tw[EPL];
#pragma unroll
        for (int k = 0; k < EPL; k++) {
            tv[k] = ((const float *) src)[EPL * lane + k];
            tw[k] = wp[EPL * lane + k];
        }
        const int32_t tpos = *pp;
        // the value-row wave (no norm, no rope) also brings the split's mask
        // row into LDS: keys kbeg + 4 lane + i, clamped into the split
        if (a.mask && task == ncol + 1) {
            const char * mrow = a.mask + (b % a.mne3) * a.mnb3;
            uint16_t     mk[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                mk[i] = *(const uint16_t *) (mrow + (int64_t) min(kbeg + 4 * lane + i, kend - 1) * 2);
            }
            uint16_t * sm = (uint16_t *) (dd_lds + 2 * DD_KV);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sm[4 * lane + i] = mk[i];
            }
        }
        id                = i64 ? (int64_t) (((uint64_t) (uint32_t) idhi << 32) | (uint32_t) idlo) : (int64_t) idlo;
        const bool is_q   = task < ncol;
        fa_head_row<D>(tv, tw, is_q ? h.q_norm != 0 : task == ncol && h.k_norm != 0,
                       is_q ? h.q_w != nullptr : h.k_w != nullptr, is_q ? h.q_eps : h.k_eps,
                       is_q ? h.q_pos != nullptr : task == ncol && h.k_pos != nullptr, tpos, is_q ? h.q_ts : h.k_ts,
                       lane);
        const bool writer = split == ((id >= 0 && id < a.nkv) ? (int) (id / chunk) : 0);
        if (is_q) {
#pragma unroll
            for (int k = 0; k < EPL; k++) {
                s_qrow[task][EPL * lane + k] = tv[k];
            }
        } else {
            const int nr = task - ncol;  // 0 key, 1 value
            char *    dp = (char *) (nr == 0 ? a.k : a.v) + id * (nr == 0 ? a.knb1 : a.vnb1) +
                        g * (nr == 0 ? a.knb2 : a.vnb2) + b * (nr == 0 ? a.knb3 : a.vnb3);
#pragma unroll
            for (int k = 0; k < EPL; k++) {
                const uint16_t hb         = f2h(tv[k]);
                s_new[nr][EPL * lane + k] = __builtin_bit_cast(_Float16, hb);
                if (writer && id >= 0) {
                    ((uint16_t *) dp)[EPL * lane + k] = hb;
                }
            }
        }
    }
    __syncthreads();
    // 3. the new rows over the stale cache rows (LDS, swizzled as the DMA stores)
    if (id >= kbeg && id < kend && wave < 2 && lane < 16) {
        const int r  = (int) (id - kbeg);
        const int ch = wave == 0 ? (lane ^ (r & 15)) : (lane ^ (2 * (r & 3)));
        *(int4_t *) (dd_lds + wave * DD_KV + r * DD_ROW + 16 * ch) = *(const int4_t *) &s_new[wave][8 * lane];
    }
    // Q^T B operand: column col, dims 32s + 8kq .. +7
    half8_t qb[NS];
#pragma unroll
    for (int s = 0; s < NS; s++) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            qb[s][i] = cvalid ? (_Float16) s_qrow[cc][32 * s + 8 * kq + i] : (_Float16) 0.0f;
        }
    }
    __syncthreads();

    // 4. the wave's tiles (t = wave, wave + NW, ...) from LDS
    float4_t oacc[NDB];
#pragma unroll
    for (int i = 0; i < NDB; i++) {
        oacc[i] = float4_t{ 0.0f, 0.0f, 0.0f, 0.0f };
    }
    float       m     = -INFINITY;
    float       l     = 0.0f;
    const float log2e = 1.4426950408889634f;
    const float sl2   = a.scale * log2e;
    const _Float16 * smask = (const _Float16 *) (dd_lds + 2 * DD_KV);
    // V^T tr-read source lane: group tg = lane / 16 (keys 4 tg + tj), tq: dims 4 tq
    const int tg = lane >> 4, tj = (lane >> 2) & 3, tq = lane & 3;
    for (int t = wave; t < ntile; t += NW) {
        // S^T tile: K rows 16 t + col, dims 32s + 8kq
        float4_t sacc = { 0.0f, 0.0f, 0.0f, 0.0f };
        const int rk  = 16 * t + col;
#pragma unroll
        for (int s = 0; s < NS; s++) {
            const half8_t kf = *(const half8_t *) (dd_lds + rk * DD_ROW + 16 * ((4 * s + kq) ^ (rk & 15)));
            sacc             = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qb[s], sacc, 0, 0, 0);
        }
        // scores of keys 4kq + i for this lane's column
        float sc[4];
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int   kr = 16 * t + 4 * kq + i;  // key row in the split
            const bool  ok = kr < nkey && cvalid;
            const float mv = a.mask ? (float) smask[kr] : 0.0f;
            sc[i]          = ok ? sacc[i] * sl2 + mv * log2e : -INFINITY;
            mx             = fmaxf(mx, sc[i]);
        }
        mx                = max_xor32(max_xor16(mx));
        const float mnew  = fmaxf(m, mx);
        const bool  live  = mnew != -INFINITY;
        const float mref  = live ? mnew : 0.0f;
        const float alpha = live ? __builtin_amdgcn_exp2f(m - mnew) : 1.0f;
        half4_t     pb;
        float       rs = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float pv = __builtin_amdgcn_exp2f(sc[i] - mref);
            rs += pv;
            pb[i] = (_Float16) pv;
        }
        rs = sum_xor32(sum_xor16(rs));
        l  = l * alpha + rs;
        m  = mnew;
        // O^T += V^T P^T: lane (dim 16db + i, keys 4 tg ..) via transposed reads
        const int rv = 16 * t + 4 * tg + tj;
#pragma unroll
        for (int db = 0; db < NDB; db++) {
            const int      d  = 16 * db + 4 * tq;
            const uint32_t ad = lbase + DD_KV + rv * DD_ROW + 16 * ((d >> 3) ^ (2 * (rv & 3))) + 2 * (d & 7);
            const half4_t  av = __builtin_bit_cast(
                half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((dd_lds_short4_t *) (uintptr_t) ad));
            oacc[db] = oacc[db] * alpha;
            oacc[db] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, pb, oacc[db], 0, 0, 0);
        }
    }

    // 5. merge the NW waves (the K / V space reused) and write the partials
    __syncthreads();
    float * s_o = (float *) dd_lds;  // [NW][16][DD_OS]
    if (kq == 0) {
        s_m[wave][col] = m;
        s_l[wave][col] = l;
    }
    if (cvalid) {
#pragma unroll
        for (int db = 0; db < NDB; db++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                s_o[(wave * 16 + col) * DD_OS + 16 * db + 4 * kq + i] = oacc[db][i];
            }
        }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < ncol * D; idx += 64 * NW) {
        const int c = idx / D;
        const int d = idx % D;
        float     M = s_m[0][c];
#pragma unroll
        for (int w = 1; w < NW; w++) {
            M = fmaxf(M, s_m[w][c]);
        }
        float L = 0.0f, O = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < NW; w++) {
                const float f = s_m[w][c] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s_m[w][c] - M);
                L += s_l[w][c] * f;
                O += s_o[(w * 16 + c) * DD_OS + d] * f;
            }
        }
        const int hh = g * G + c % G;
        const int qi = c / G;
        if (nsplit == 1) {
            out[(((int64_t) b * a.nq + qi) * a.Hq + hh) * D + d] = L > 0.0f ? O / L : 0.0f;
        } else {
            const int64_t pr = (((int64_t) b * a.Hq + hh) * a.nq + qi) * nsplit + split;
            part_o[pr * D + d] = O;
            if (d == 0) {
                part_ml[pr * 2 + 0] = M;
                part_ml[pr * 2 + 1] = L;
            }
        }
    }
}

// k_fa_dec_dma's preconditions
static bool dec_dma_ok(const FaArgs & a, int D, int chunk, const FaHead * hd) {
    auto al16 = [](int64_t v) { return (v & 15) == 0; };
    const int G = a.Hq / a.Hkv;
    return hd && D == DD_D && chunk <= DD_MAXK && a.nq == 1 && G * a.nq + 3 <= DD_NW && a.Bk == a.B &&
           (!a.mask || a.mne2 == 1) &&
           al16((int64_t) (uintptr_t) a.k) && al16(a.knb1) && al16(a.knb2) && al16(a.knb3) &&
           al16((int64_t) (uintptr_t) a.v) && al16(a.vnb1) && al16(a.vnb2) && al16(a.vnb3) &&
           getenv("GGML_MI355X_DISABLE_DEC_DMA") == nullptr;
}

// One workgroup of D threads per output row (b, hq, iq): the split weights
// exp2(m_s - M) / L are formed once in LDS, then every thread sums its dim.
__global__ __launch_bounds__(256) void k_fa_combine(const float * __restrict__ part_o,
                                                    const float * __restrict__ part_ml, int nsplit, int D, int nq,
                                                    int Hq, float * __restrict__ out) {
    __shared__ float s_w[256];
    __shared__ float s_red[2];
    const int     hq  = blockIdx.x / nq;
    const int     iq  = blockIdx.x % nq;
    const int     b   = blockIdx.y;
    const int     t   = threadIdx.x;
    const int64_t pr0 = (((int64_t) b * Hq + hq) * nq + iq) * nsplit;
    // blockDim.x == D >= 64 and nsplit <= D: thread t < nsplit owns split t
    float ms = -INFINITY, ls = 0.0f;
    if (t < nsplit) {
        ms = part_ml[(pr0 + t) * 2];
        ls = part_ml[(pr0 + t) * 2 + 1];
    }
    float M = wave_max(ms);
    if (blockDim.x > 64) {
        if ((t & 63) == 0) {
            s_w[t >> 6] = M;
        }
        __syncthreads();
        for (int w = 0; w < (int) blockDim.x / 64; w++) {
            M = fmaxf(M, s_w[w]);
        }
        __syncthreads();
    }
    const float sc = (ms == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(ms - M);
    float       L  = wave_sum(ls * sc);
    if (blockDim.x > 64) {
        if ((t & 63) == 0) {
            s_w[t >> 6] = L;
        }
        __syncthreads();
        L = 0.0f;
        for (int w = 0; w < (int) blockDim.x / 64; w++) {
            L += s_w[w];
        }
        __syncthreads();
    }
    if (t == 0) {
        s_red[0] = L;
    }
    if (t < nsplit) {
        s_w[t] = sc;
    }
    __syncthreads();
    const float inv = s_red[0] > 0.0f ? 1.0f / s_red[0] : 0.0f;
    float       O   = 0.0f;
    int         s   = 0;
    for (; s + 4 <= nsplit; s += 4) {
        const float o0 = part_o[(pr0 + s) * D + t], o1 = part_o[(pr0 + s + 1) * D + t];
        const float o2 = part_o[(pr0 + s + 2) * D + t], o3 = part_o[(pr0 + s + 3) * D + t];
        O += o0 * s_w[s] + o1 * s_w[s + 1] + o2 * s_w[s + 2] + o3 * s_w[s + 3];
    }
    for (; s < nsplit; s++) {
        O += part_o[(pr0 + s) * D + t] * s_w[s];
    }
    out[(((int64_t) b * nq + iq) * Hq + hq) * D + t] = O * inv;
}

// Split combine that also quantises the output rows for the GEMV that
// consumes them (the attention output projection): one 256-thread workgroup
// per 256-element chunk of an output row (b, iq), thread t owning element t
// (head e / D, dim e % D), so a workgroup holds whole Q8_0 blocks and a whole
// Q8_K super-block.  The quantisation arithmetic is k_quant.hip's.  With
// xq_qs null it is the plain combine (the decode's default: the same
// arithmetic as the decode kernel's own combine).
__global__ __launch_bounds__(256) void k_fa_combine_q(const float * __restrict__ part_o,
                                                      const float * __restrict__ part_ml, int nsplit, int D, int nq,
                                                      int Hq, float * __restrict__ out, int qtype,
                                                      int8_t * __restrict__ xq_qs, float * __restrict__ xq_d,
                                                      int16_t * __restrict__ xq_bs) {
    __shared__ float s_m[4][128], s_l[4][128];
    __shared__ float s_red[4], s_amax[4];
    __shared__ int   s_idx[4];
    const int t    = threadIdx.x;
    const int e    = 256 * blockIdx.x + t;  // element of the output row
    const int iq   = blockIdx.y;
    const int b    = blockIdx.z;
    const int hq   = e / D;
    const int d    = e % D;
    const int hl   = t / D;                 // head within the workgroup (256 / D heads)
    const int64_t pr0 = (((int64_t) b * Hq + hq) * nq + iq) * nsplit;
    // split maxima and sums of this workgroup's heads into LDS
    for (int sidx = d; sidx < nsplit; sidx += D) {
        s_m[hl][sidx] = part_ml[(pr0 + sidx) * 2];
        s_l[hl][sidx] = part_ml[(pr0 + sidx) * 2 + 1];
    }
    __syncthreads();
    const float   v   = fa_combine_elem(part_o, pr0, D, d, nsplit, s_m[hl], s_l[hl]);
    const int64_t row = (int64_t) b * nq + iq;
    const int     K   = Hq * D;
    out[row * K + e]  = v;
    if (xq_qs) {
        fa_quant_elem(v, true, t, row, e, K, qtype, xq_qs, xq_d, xq_bs, s_red, s_idx, s_amax);
    }
}

// ---------------------------------------------------------------------

// keys per lane per pass (D = 128, QR = 4: 128 keys per workgroup pass)
constexpr int dec_u(int QR) {
    return QR <= 4 ? 8 : 4;
}

static int dec_qr(const FaArgs & a) {
    return (a.Hq / a.Hkv) * a.nq <= 4 ? 4 : 8;
}

static bool dec_mfma(const FaArgs & a);

static void decode_plan(const FaArgs & a, int D, int & nsplit, int & chunk, int & rowgroups) {
    const int G    = a.Hq / a.Hkv;
    const int QR   = dec_qr(a);
    rowgroups      = dec_mfma(a) ? 1 : (G * a.nq + QR - 1) / QR;
    const int kpw  = 64 / (D / 8);
    // keys one workgroup pass covers (MFMA kernel: one 16-key tile per wave)
    const int step = dec_mfma(a) ? 16 * dec_nw(D) : 4 * kpw * dec_u(QR);
    const int base_wgs = a.Hkv * a.B * rowgroups;
    const int target   = 256;  // workgroups (measured: 256 vs 512 splits, a few % on the decode step)
    int       ns       = (target + base_wgs - 1) / base_wgs;
    // the combine kernel gives one thread per split: nsplit <= D
    const int max_ns   = std::max(1, std::min(D, (a.nkv + step - 1) / step));
    ns                 = std::max(1, std::min(ns, max_ns));
    chunk              = ((a.nkv + ns - 1) / ns + step - 1) / step * step;
    nsplit             = (a.nkv + chunk - 1) / chunk;
}

size_t fa_decode_workspace(const FaArgs & a, int D) {
    int nsplit, chunk, rg;
    decode_plan(a, D, nsplit, chunk, rg);
    if (nsplit <= 1) {
        return 0;
    }
    const size_t rows = (size_t) a.B * a.Hq * a.nq * nsplit;
    return align_up(rows * D * sizeof(float), 256) + align_up(rows * 2 * sizeof(float), 256);
}

template <int D>
static void launch_decode(const FaArgs & a, int QR, dim3 grid, int chunk, int nsplit, float * po, float * pml,
                          float * out, hipStream_t stream) {
    if (QR == 4) {
        hipLaunchKernelGGL((k_fa_decode<D, 4, dec_u(4)>), grid, dim3(256), 0, stream, a, chunk, nsplit, po, pml, out);
    } else {
        hipLaunchKernelGGL((k_fa_decode<D, 8, dec_u(8)>), grid, dim3(256), 0, stream, a, chunk, nsplit, po, pml, out);
    }
}

template <int D, bool HD>
static int launch_dec_mfma(dim3 g3, int tiles, const FaArgs & a, const FaHead & h, int chunk, int nsplit, float * po,
                           float * pml, float * out, hipStream_t stream) {
    // D = 256 holds twice the fragments per tile: one tile per load round
    constexpr int NW = dec_nw(D);
    if constexpr (D <= 128) {
        if (tiles >= 2) {
            hipLaunchKernelGGL((k_fa_dec_mfma<D, NW, 2, HD>), g3, dim3(64 * NW), 0, stream, a, h, chunk, nsplit, po, pml,
                               out);
            return check_launch("flash_attn decode");
        }
    }
    hipLaunchKernelGGL((k_fa_dec_mfma<D, NW, 1, HD>), g3, dim3(64 * NW), 0, stream, a, h, chunk, nsplit, po, pml, out);
    return check_launch("flash_attn decode");
}

// The MFMA decode kernel serves up to 16 query rows per KV head.
static bool dec_mfma(const FaArgs & a) {
    return (a.Hq / a.Hkv) * a.nq <= 16;
}

bool fa_decode_head_supported(const FaArgs & a, int D) {
    // the query columns and the two new rows one wave each; one cache set
    // per attention batch
    return dec_mfma(a) && (a.Hq / a.Hkv) * a.nq + 2 <= dec_nw(D) && a.Bk == a.B && (D == 64 || D == 128 || D == 256);
}

int fa_decode(const FaArgs & a, int D, float * out, void * ws, size_t ws_bytes, hipStream_t stream, int qtype,
              void * xq, bool * quantised, const FaHead * hd) {
    if (quantised) {
        *quantised = false;
    }
    if (hd && !fa_decode_head_supported(a, D)) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "flash_attn decode: fused head prologue does not fit these shapes");
    }
    int nsplit, chunk, rg;
    decode_plan(a, D, nsplit, chunk, rg);
    float * part_o  = nullptr;
    float * part_ml = nullptr;
    if (nsplit > 1) {
        const size_t need = fa_decode_workspace(a, D);
        if (!ws || ws_bytes < need) {
            return set_error(MMHIP_ERR_WORKSPACE, "flash_attn decode: workspace %zu < %zu", ws_bytes, need);
        }
        const size_t rows = (size_t) a.B * a.Hq * a.nq * nsplit;
        part_o            = (float *) ws;
        part_ml           = (float *) ((char *) ws + align_up(rows * D * sizeof(float), 256));
    }
    if ((int64_t) a.B * rg > 65535) {
        return set_error(MMHIP_ERR_UNSUPPORTED, "flash_attn decode: B * row groups too large");
    }
    // the split combine: quantising for xq's weights where its layout allows,
    // by k_fa_combine_q's arithmetic wherever the rows are whole 256-chunks
    const int64_t   K      = (int64_t) a.Hq * D;
    const ActLayout L      = xq ? act_layout(qtype, K, (int64_t) a.B * a.nq) : ActLayout{};
    const bool      comb_q = K % 256 == 0 && nsplit <= 128;
    const bool      quant  = xq && L.total != 0 && comb_q;
    if (dec_dma_ok(a, D, chunk, hd)) {
        const dim3 g3(nsplit, a.Hkv, a.B);
        if (!ensure_lds_limit((const void *) k_fa_dec_dma, DD_LDS)) {
            return set_error(MMHIP_ERR_HIP, "flash_attn decode: cannot raise LDS limit to %d", DD_LDS);
        }
        hipLaunchKernelGGL(k_fa_dec_dma, g3, dim3(64 * DD_NW), DD_LDS, stream, a, *hd, chunk, nsplit, part_o, part_ml,
                           out);
    } else if (dec_mfma(a)) {
        const dim3 g3(nsplit, a.Hkv, a.B);
        // tiles per wave: the split's tiles in one load round where that fits
        const int tiles = (chunk / 16 + dec_nw(D) - 1) / dec_nw(D);
        int          rc    = MMHIP_OK;
        const FaHead h0{};
        const FaHead & h   = hd ? *hd : h0;
#define MM_DEC(DD)                                                                                               \
    rc = hd ? launch_dec_mfma<DD, true>(g3, tiles, a, h, chunk, nsplit, part_o, part_ml, out, stream)             \
            : launch_dec_mfma<DD, false>(g3, tiles, a, h, chunk, nsplit, part_o, part_ml, out, stream)
        switch (D) {
            case 64: MM_DEC(64); break;
            case 128: MM_DEC(128); break;
            case 256: MM_DEC(256); break;
            default: return set_error(MMHIP_ERR_UNSUPPORTED, "flash_attn decode: head dim %d", D);
        }
#undef MM_DEC
        if (rc != MMHIP_OK) {
            return rc;
        }
    } else {
    const dim3 grid(nsplit, a.Hkv, a.B * rg);
    const int  QR = dec_qr(a);
    switch (D) {
        case 64: launch_decode<64>(a, QR, grid, chunk, nsplit, part_o, part_ml, out, stream); break;
        case 128: launch_decode<128>(a, QR, grid, chunk, nsplit, part_o, part_ml, out, stream); break;
        case 256: launch_decode<256>(a, QR, grid, chunk, nsplit, part_o, part_ml, out, stream); break;
        default: return set_error(MMHIP_ERR_UNSUPPORTED, "flash_attn decode: head dim %d", D);
    }
    }
    int rc = check_launch("flash_attn decode");
    if (rc != MMHIP_OK || nsplit == 1) {
        return rc;
    }
    if (comb_q) {
        hipLaunchKernelGGL(k_fa_combine_q, dim3((unsigned) (K / 256), a.nq, a.B), dim3(256), 0, stream, part_o, part_ml,
                           nsplit, D, a.nq, a.Hq, out, L.vec_type, quant ? (int8_t *) xq + L.qs_off : nullptr,
                           quant ? (float *) ((char *) xq + L.d_off) : nullptr,
                           quant && L.vec_type == TYPE_Q8_K ? (int16_t *) ((char *) xq + L.bs_off) : nullptr);
        if (quantised) {
            *quantised = quant;
        }
        return check_launch("flash_attn combine");
    }
    hipLaunchKernelGGL(k_fa_combine, dim3(a.Hq * a.nq, a.B), dim3(D), 0, stream, part_o, part_ml, nsplit, D, a.nq, a.Hq,
                       out);
    return check_launch("flash_attn combine");
}

}  // namespace mmhip
