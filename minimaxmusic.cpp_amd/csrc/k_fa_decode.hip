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

    half8_t      qv[QR];
    const char * mrow[QR];
    bool         rvalid[QR];
#pragma unroll
    for (int r = 0; r < QR; r++) {
        const int rr  = r0 + r;
        rvalid[r]     = rr < nrows;
        const int rrc = rvalid[r] ? rr : r0;
        const int hq  = g * G + rrc % G;
        const int iq  = rrc / G;
        const float * qp = (const float *) (a.q + iq * a.qnb1 + hq * a.qnb2 + b * a.qnb3) + seg * 8;
#pragma unroll
        for (int d = 0; d < 8; d++) {
            qv[r][d] = (_Float16) qp[d];
        }
        mrow[r] = a.mask ? a.mask + iq * a.mnb1 + (hq % a.mne2) * a.mnb2 + (b % a.mne3) * a.mnb3 : nullptr;
    }

    const char * kbase = a.k + g * a.knb2 + bk * a.knb3 + seg * 16;
    const char * vbase = a.v + g * a.vnb2 + bk * a.vnb3 + seg * 16;

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

    // U keys per lane in flight: all K/V loads of an iteration are issued
    // before the first use.
    for (int base = kbeg + wave * KPW; base < kend; base += 4 * KPW * U) {
        half8_t kk[U], vv[U];
        int64_t jc[U];
        bool    jv[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int j = base + 4 * KPW * u + ks;
            jv[u]       = j < kend;
            jc[u]       = jv[u] ? j : kend - 1;
            kk[u]       = *(const half8_t *) (kbase + jc[u] * a.knb1);
            vv[u]       = *(const half8_t *) (vbase + jc[u] * a.vnb1);
        }
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
                const float mv = mrow[r] ? h2f(*(const uint16_t *) (mrow[r] + jc[u] * 2)) : 0.0f;
                const float s  = (jv[u] && rvalid[r]) ? (dot * a.scale + mv) * log2e : -INFINITY;
                const float mn = fmaxf(m[r], s);
                float       alpha = 1.0f, p = 0.0f;
                if (mn != -INFINITY) {
                    alpha = __builtin_amdgcn_exp2f(m[r] - mn);
                    p     = __builtin_amdgcn_exp2f(s - mn);
                }
                l[r] = l[r] * alpha + p;
#pragma unroll
                for (int d = 0; d < 8; d++) {
                    o[r][d] = o[r][d] * alpha + p * (float) vv[u][d];
                }
                m[r] = mn;
            }
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

// ---------------------------------------------------------------------

constexpr int DEC_U = 4;

static int dec_qr(const FaArgs & a) {
    return (a.Hq / a.Hkv) * a.nq <= 4 ? 4 : 8;
}

static void decode_plan(const FaArgs & a, int D, int & nsplit, int & chunk, int & rowgroups) {
    const int G    = a.Hq / a.Hkv;
    const int QR   = dec_qr(a);
    rowgroups      = (G * a.nq + QR - 1) / QR;
    const int kpw  = 64 / (D / 8);
    const int step = 4 * kpw * DEC_U;  // keys one workgroup iteration covers
    const int base_wgs = a.Hkv * a.B * rowgroups;
    const int target   = 512;
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
        hipLaunchKernelGGL((k_fa_decode<D, 4, DEC_U>), grid, dim3(256), 0, stream, a, chunk, nsplit, po, pml, out);
    } else {
        hipLaunchKernelGGL((k_fa_decode<D, 8, DEC_U>), grid, dim3(256), 0, stream, a, chunk, nsplit, po, pml, out);
    }
}

int fa_decode(const FaArgs & a, int D, float * out, void * ws, size_t ws_bytes, hipStream_t stream) {
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
    const dim3 grid(nsplit, a.Hkv, a.B * rg);
    const int  QR = dec_qr(a);
    switch (D) {
        case 64: launch_decode<64>(a, QR, grid, chunk, nsplit, part_o, part_ml, out, stream); break;
        case 128: launch_decode<128>(a, QR, grid, chunk, nsplit, part_o, part_ml, out, stream); break;
        case 256: launch_decode<256>(a, QR, grid, chunk, nsplit, part_o, part_ml, out, stream); break;
        default: return set_error(MMHIP_ERR_UNSUPPORTED, "flash_attn decode: head dim %d", D);
    }
    int rc = check_launch("flash_attn decode");
    if (rc != MMHIP_OK || nsplit == 1) {
        return rc;
    }
    hipLaunchKernelGGL(k_fa_combine, dim3(a.Hq * a.nq, a.B), dim3(D), 0, stream, part_o, part_ml, nsplit, D, a.nq, a.Hq,
                       out);
    return check_launch("flash_attn combine");
}

}  // namespace mmhip
