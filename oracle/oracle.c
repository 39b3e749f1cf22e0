/*
 * oracle.c - CPU restatement of ggml-CPU arithmetic for the attention +
 * quantized-matmul hot path.  TEST INFRASTRUCTURE ONLY (the checker): see
 * oracle.h.  Built with -ffp-contract=off so every float operation below is
 * rounded exactly as written.
 *
 * Pinning (what independently checks each function; tests/test_oracle_*.py):
 *   fp16/bf16 conversions  exhaustive fp16->fp32 and 2^20 random fp32->fp16
 *                          against numpy's IEEE conversions; bf16 vs the torch
 *                          rounding of the same values.
 *   dequantize Q8_0/Q4_K/Q5_K/Q6_K
 *                          hand-built known-answer blocks with literal expected
 *                          values (tests/golden/known_blocks.json), covering
 *                          d = 1, q = -127..127; Q4_K 6-bit scale packing for
 *                          sub-blocks j < 4 and j >= 4; dmin != 0; Q5_K's fifth
 *                          bit from qh (bit j of byte l for sub-block j); Q6_K's
 *                          -32 offset and all 16 scales; plus an independent
 *                          numpy bit-field decoder on random blocks.
 *   quantize_row_q8_0/_q8_K
 *                          closed forms: x = d*q exactly representable round-
 *                          trips; all-zero rows; the Q8_K max element maps to
 *                          -127 and bsums equal the 16-element sums.
 *   vec_dot / mul_mat_ggml integer dots checked against numpy int64 dots of
 *                          the dequantised blocks (exact); one-hot x returns
 *                          column k of deq(W) to the activation quantum.
 *   mul_mat_f64            brute-force numpy float64 matmul of the
 *                          dequantised weights; one-hot, linearity, CFG-row
 *                          swap.
 *   flash_attn_ext_f64     torch.nn.functional.scaled_dot_product_attention in
 *                          float64 on CPU; closed forms (constant K -> mean V,
 *                          single allowed key -> that V row, causal prefix
 *                          invariance, GQA head map, padded -inf tail).
 *   flash_attn_ext_ggml    against _f64 within the f16-accumulator bound; its
 *                          exact bits against real ggml stay unpinned (ggml is
 *                          not present): "parity unpinned" for bit-identity,
 *                          pinned to tolerance only.
 *   rms_norm / rope / swiglu
 *                          numpy float64 closed forms (rope against the direct
 *                          pow form within 1e-5 at position <= 8192).
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* scalar conversions                                                   */
/* ------------------------------------------------------------------ */

uint16_t orc_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax   = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                       /* inf / nan */
        if (ax > 0x7f800000u) {
            return (uint16_t) (sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
        }
        return (uint16_t) (sign | 0x7c00u);
    }
    if (ax >= 0x477ff000u) {                       /* >= 65520 rounds to inf */
        return (uint16_t) (sign | 0x7c00u);
    }
    if (ax < 0x38800000u) {                        /* result is subnormal or zero */
        const uint32_t e = ax >> 23;
        if (e < 102) {
            return (uint16_t) sign;
        }
        const uint32_t m     = (ax & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126 - e;            /* >= 14 */
        uint32_t       q     = m >> shift;
        const uint32_t rem   = m & ((1u << shift) - 1);
        const uint32_t half  = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) {
            q++;
        }
        return (uint16_t) (sign | q);
    }
    uint32_t       h   = (((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) {
        h++;
    }
    return (uint16_t) (sign | h);
}

float orc_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = ((uint32_t) h & 0x8000u) << 16;
    const uint32_t e    = ((uint32_t) h >> 10) & 0x1fu;
    const uint32_t m    = (uint32_t) h & 0x3ffu;
    uint32_t       x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else {
            const float f = (float) m * 5.9604644775390625e-08f; /* m * 2^-24, exact */
            memcpy(&x, &f, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float r;
    memcpy(&r, &x, 4);
    return r;
}

uint16_t orc_fp32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) {
        return (uint16_t) ((x >> 16) | 64u);
    }
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t) (x >> 16);
}

float orc_bf16_to_fp32(uint16_t h) {
    const uint32_t x = (uint32_t) h << 16;
    float          r;
    memcpy(&r, &x, 4);
    return r;
}

void orc_fp32_to_fp16_row(const float * x, uint16_t * y, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        y[i] = orc_fp32_to_fp16(x[i]);
    }
}

void orc_fp16_to_fp32_row(const uint16_t * x, float * y, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        y[i] = orc_fp16_to_fp32(x[i]);
    }
}

/* ------------------------------------------------------------------ */
/* block formats                                                        */
/* ------------------------------------------------------------------ */

size_t orc_type_size(int type) {
    switch (type) {
        case ORC_TYPE_F32:  return 4;
        case ORC_TYPE_F16:  return 2;
        case ORC_TYPE_BF16: return 2;
        case ORC_TYPE_I32:  return 4;
        case ORC_TYPE_I64:  return 8;
        case ORC_TYPE_Q8_0: return sizeof(orc_block_q8_0);
        case ORC_TYPE_Q4_K: return sizeof(orc_block_q4_K);
        case ORC_TYPE_Q5_K: return sizeof(orc_block_q5_K);
        case ORC_TYPE_Q6_K: return sizeof(orc_block_q6_K);
        case ORC_TYPE_Q8_K: return sizeof(orc_block_q8_K);
        default:            return 0;
    }
}

int orc_blck_size(int type) {
    switch (type) {
        case ORC_TYPE_Q8_0: return ORC_QK8_0;
        case ORC_TYPE_Q4_K:
        case ORC_TYPE_Q5_K:
        case ORC_TYPE_Q6_K:
        case ORC_TYPE_Q8_K: return ORC_QK_K;
        default:            return 1;
    }
}

size_t orc_row_size(int type, int64_t ne0) {
    return orc_type_size(type) * (size_t) (ne0 / orc_blck_size(type));
}

/* Q4_K packs eight 6-bit (scale, min) pairs into 12 bytes: pairs 0-3 sit in
 * the low 6 bits of bytes 0-3 (scale) and 4-7 (min); pairs 4-7 take their low
 * 4 bits from the nibbles of bytes 8-11 and their top 2 bits from the spare
 * top bits of bytes 0-3 (scale) and 4-7 (min). */
static void q4k_scale_min(int j, const uint8_t * s, int * sc, int * mn) {
    if (j < 4) {
        *sc = s[j] & 63;
        *mn = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 0x0f) | ((s[j - 4] >> 6) << 4);
        *mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* Q4_K element e (0..255) of a super-block: 64-element chunk c = e/64 reads
 * bytes qs[32c .. 32c+31], low nibble for e%64 < 32, high nibble otherwise. */
static int q4k_quant(const orc_block_q4_K * b, int e) {
    const int c = e >> 6, r = e & 63;
    const uint8_t byte = b->qs[32 * c + (r & 31)];
    return r < 32 ? (byte & 0x0f) : (byte >> 4);
}

/* Q5_K element e (0..255): the Q4_K nibble of e (qs laid out as Q4_K's) plus
 * 16 times bit j = e/32 of qh[e%32] (dequantize_row_q5_K walks qh with one
 * mask bit per 32-element sub-block). */
static int q5k_quant(const orc_block_q5_K * b, int e) {
    const int c = e >> 6, r = e & 63, l = e & 31;
    const uint8_t byte = b->qs[32 * c + l];
    const int     lo   = r < 32 ? (byte & 0x0f) : (byte >> 4);
    return lo + (((b->qh[l] >> (e >> 5)) & 1) << 4);
}

/* Q6_K element e (0..255): half h = e/128, within the half quarter t = r/32,
 * column l = r%32.  Low 4 bits from ql[64h + l + 32*(t&1)] (low nibble for
 * t < 2), high 2 bits from qh[32h + l] bits 2t..2t+1; value offset by -32;
 * scale index e/16. */
static int q6k_quant(const orc_block_q6_K * b, int e) {
    const int h = e >> 7, r = e & 127, t = r >> 5, l = r & 31;
    const uint8_t lo_byte = b->ql[64 * h + l + 32 * (t & 1)];
    const int     lo      = (t < 2) ? (lo_byte & 0x0f) : (lo_byte >> 4);
    const int     hi      = (b->qh[32 * h + l] >> (2 * t)) & 3;
    return (lo | (hi << 4)) - 32;
}

void orc_dequantize_row(int type, const void * src, float * dst, int64_t k) {
    switch (type) {
        case ORC_TYPE_F32:
            memcpy(dst, src, (size_t) k * 4);
            return;
        case ORC_TYPE_F16:
            orc_fp16_to_fp32_row((const uint16_t *) src, dst, k);
            return;
        case ORC_TYPE_BF16:
            for (int64_t i = 0; i < k; i++) {
                dst[i] = orc_bf16_to_fp32(((const uint16_t *) src)[i]);
            }
            return;
        case ORC_TYPE_Q8_0: {
            const orc_block_q8_0 * b = (const orc_block_q8_0 *) src;
            for (int64_t i = 0; i < k / ORC_QK8_0; i++) {
                const float d = orc_fp16_to_fp32(b[i].d);
                for (int j = 0; j < ORC_QK8_0; j++) {
                    dst[i * ORC_QK8_0 + j] = d * (float) b[i].qs[j];
                }
            }
            return;
        }
        case ORC_TYPE_Q4_K: {
            const orc_block_q4_K * b = (const orc_block_q4_K *) src;
            for (int64_t i = 0; i < k / ORC_QK_K; i++) {
                const float d    = orc_fp16_to_fp32(b[i].d);
                const float dmin = orc_fp16_to_fp32(b[i].dmin);
                for (int j = 0; j < 8; j++) {
                    int sc, mn;
                    q4k_scale_min(j, b[i].scales, &sc, &mn);
                    const float d1 = d * (float) sc;
                    const float m1 = dmin * (float) mn;
                    for (int l = 0; l < 32; l++) {
                        const int e = 32 * j + l;
                        dst[i * ORC_QK_K + e] = d1 * (float) q4k_quant(&b[i], e) - m1;
                    }
                }
            }
            return;
        }
        case ORC_TYPE_Q5_K: {
            const orc_block_q5_K * b = (const orc_block_q5_K *) src;
            for (int64_t i = 0; i < k / ORC_QK_K; i++) {
                const float d    = orc_fp16_to_fp32(b[i].d);
                const float dmin = orc_fp16_to_fp32(b[i].dmin);
                for (int j = 0; j < 8; j++) {
                    int sc, mn;
                    q4k_scale_min(j, b[i].scales, &sc, &mn);
                    const float d1 = d * (float) sc;
                    const float m1 = dmin * (float) mn;
                    for (int l = 0; l < 32; l++) {
                        const int e = 32 * j + l;
                        dst[i * ORC_QK_K + e] = d1 * (float) q5k_quant(&b[i], e) - m1;
                    }
                }
            }
            return;
        }
        case ORC_TYPE_Q6_K: {
            const orc_block_q6_K * b = (const orc_block_q6_K *) src;
            for (int64_t i = 0; i < k / ORC_QK_K; i++) {
                const float d = orc_fp16_to_fp32(b[i].d);
                for (int e = 0; e < ORC_QK_K; e++) {
                    const float ds = d * (float) b[i].scales[e >> 4];
                    dst[i * ORC_QK_K + e] = ds * (float) q6k_quant(&b[i], e);
                }
            }
            return;
        }
        case ORC_TYPE_Q8_K: {
            const orc_block_q8_K * b = (const orc_block_q8_K *) src;
            for (int64_t i = 0; i < k / ORC_QK_K; i++) {
                for (int j = 0; j < ORC_QK_K; j++) {
                    dst[i * ORC_QK_K + j] = b[i].d * (float) b[i].qs[j];
                }
            }
            return;
        }
        default:
            abort();
    }
}

/* ggml's reference Q8_0 activation quantiser [ext]: d = amax/127 stored as
 * f16, q = roundf(x / d) (round half away from zero) with the f32 d. */
void orc_quantize_row_q8_0(const float * x, void * y, int64_t k) {
    orc_block_q8_0 * b = (orc_block_q8_0 *) y;
    for (int64_t i = 0; i < k / ORC_QK8_0; i++) {
        float amax = 0.0f;
        for (int j = 0; j < ORC_QK8_0; j++) {
            const float a = fabsf(x[i * ORC_QK8_0 + j]);
            amax          = a > amax ? a : amax;
        }
        const float d  = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        b[i].d         = orc_fp32_to_fp16(d);
        for (int j = 0; j < ORC_QK8_0; j++) {
            b[i].qs[j] = (int8_t) roundf(x[i * ORC_QK8_0 + j] * id);
        }
    }
}

/* ggml's Q8_K activation quantiser [ext]: the element of largest magnitude
 * (first one on ties) maps to -127 via iscale = -127/max, q = nearest-even
 * of iscale*x capped at 127, d = 1/iscale (f32), bsums = 16-element sums. */
void orc_quantize_row_q8_K(const float * x, void * y, int64_t k) {
    orc_block_q8_K * b = (orc_block_q8_K *) y;
    for (int64_t i = 0; i < k / ORC_QK_K; i++) {
        const float * xb   = x + i * ORC_QK_K;
        float         amax = 0.0f, vmax = 0.0f;
        for (int j = 0; j < ORC_QK_K; j++) {
            const float a = fabsf(xb[j]);
            if (a > amax) {
                amax = a;
                vmax = xb[j];
            }
        }
        if (amax == 0.0f) {
            memset(&b[i], 0, sizeof(b[i]));
            continue;
        }
        const float iscale = -127.0f / vmax;
        for (int j = 0; j < ORC_QK_K; j++) {
            int v = (int) rintf(iscale * xb[j]);
            b[i].qs[j] = (int8_t) (v > 127 ? 127 : v);
        }
        for (int g = 0; g < 16; g++) {
            int s = 0;
            for (int j = 0; j < 16; j++) {
                s += b[i].qs[16 * g + j];
            }
            b[i].bsums[g] = (int16_t) s;
        }
        b[i].d = 1.0f / iscale;
    }
}

/* Integer-exact block dots, combined per block in f32 [ext]. */
float orc_vec_dot(int type, int64_t k, const void * wrow, const void * xq) {
    float sumf = 0.0f;
    switch (type) {
        case ORC_TYPE_Q8_0: {
            const orc_block_q8_0 * w = (const orc_block_q8_0 *) wrow;
            const orc_block_q8_0 * x = (const orc_block_q8_0 *) xq;
            for (int64_t i = 0; i < k / ORC_QK8_0; i++) {
                int sumi = 0;
                for (int j = 0; j < ORC_QK8_0; j++) {
                    sumi += (int) w[i].qs[j] * (int) x[i].qs[j];
                }
                const float dd = orc_fp16_to_fp32(w[i].d) * orc_fp16_to_fp32(x[i].d);
                sumf += (float) sumi * dd;
            }
            return sumf;
        }
        case ORC_TYPE_Q4_K: {
            const orc_block_q4_K * w = (const orc_block_q4_K *) wrow;
            const orc_block_q8_K * x = (const orc_block_q8_K *) xq;
            for (int64_t i = 0; i < k / ORC_QK_K; i++) {
                int isum = 0, msum = 0;
                for (int j = 0; j < 8; j++) {
                    int sc, mn;
                    q4k_scale_min(j, w[i].scales, &sc, &mn);
                    int s = 0;
                    for (int l = 0; l < 32; l++) {
                        s += q4k_quant(&w[i], 32 * j + l) * (int) x[i].qs[32 * j + l];
                    }
                    isum += sc * s;
                    msum += mn * ((int) x[i].bsums[2 * j] + (int) x[i].bsums[2 * j + 1]);
                }
                const float d    = orc_fp16_to_fp32(w[i].d) * x[i].d;
                const float dmin = orc_fp16_to_fp32(w[i].dmin) * x[i].d;
                sumf += d * (float) isum;
                sumf -= dmin * (float) msum;
            }
            return sumf;
        }
        case ORC_TYPE_Q5_K: {
            const orc_block_q5_K * w = (const orc_block_q5_K *) wrow;
            const orc_block_q8_K * x = (const orc_block_q8_K *) xq;
            for (int64_t i = 0; i < k / ORC_QK_K; i++) {
                int isum = 0, msum = 0;
                for (int j = 0; j < 8; j++) {
                    int sc, mn;
                    q4k_scale_min(j, w[i].scales, &sc, &mn);
                    int s = 0;
                    for (int l = 0; l < 32; l++) {
                        s += q5k_quant(&w[i], 32 * j + l) * (int) x[i].qs[32 * j + l];
                    }
                    isum += sc * s;
                    msum += mn * ((int) x[i].bsums[2 * j] + (int) x[i].bsums[2 * j + 1]);
                }
                const float d    = orc_fp16_to_fp32(w[i].d) * x[i].d;
                const float dmin = orc_fp16_to_fp32(w[i].dmin) * x[i].d;
                sumf += d * (float) isum;
                sumf -= dmin * (float) msum;
            }
            return sumf;
        }
        case ORC_TYPE_Q6_K: {
            const orc_block_q6_K * w = (const orc_block_q6_K *) wrow;
            const orc_block_q8_K * x = (const orc_block_q8_K *) xq;
            for (int64_t i = 0; i < k / ORC_QK_K; i++) {
                int isum = 0;
                for (int g = 0; g < 16; g++) {
                    int s = 0;
                    for (int l = 0; l < 16; l++) {
                        s += q6k_quant(&w[i], 16 * g + l) * (int) x[i].qs[16 * g + l];
                    }
                    isum += (int) w[i].scales[g] * s;
                }
                const float d = orc_fp16_to_fp32(w[i].d) * x[i].d;
                sumf += d * (float) isum;
            }
            return sumf;
        }
        default:
            abort();
    }
}

/* ------------------------------------------------------------------ */
/* thread pool helper                                                   */
/* ------------------------------------------------------------------ */

typedef void (*orc_range_fn)(void * ctx, int64_t begin, int64_t end);

typedef struct {
    orc_range_fn fn;
    void *       ctx;
    int64_t      begin, end;
} orc_job;

static void * orc_job_run(void * p) {
    orc_job * j = (orc_job *) p;
    j->fn(j->ctx, j->begin, j->end);
    return NULL;
}

static void orc_parallel_for(int64_t n, int nthreads, orc_range_fn fn, void * ctx) {
    if (nthreads <= 1 || n < 2) {
        fn(ctx, 0, n);
        return;
    }
    if (nthreads > 256) {
        nthreads = 256;
    }
    if (nthreads > n) {
        nthreads = (int) n;
    }
    pthread_t th[256];
    orc_job   jobs[256];
    for (int t = 0; t < nthreads; t++) {
        jobs[t].fn    = fn;
        jobs[t].ctx   = ctx;
        jobs[t].begin = n * t / nthreads;
        jobs[t].end   = n * (t + 1) / nthreads;
        if (t > 0) {
            pthread_create(&th[t], NULL, orc_job_run, &jobs[t]);
        }
    }
    orc_job_run(&jobs[0]);
    for (int t = 1; t < nthreads; t++) {
        pthread_join(th[t], NULL);
    }
}

/* ------------------------------------------------------------------ */
/* mul_mat                                                              */
/* ------------------------------------------------------------------ */

typedef struct {
    int           type;
    const void *  W;
    int64_t       N, K, M;
    size_t        wrow, xrow;
    const void *  xq;      /* quantised activations (ggml flavour) */
    const float * x;       /* raw activations (f64 flavour) */
    int64_t       x_stride;
    float *       y;
    double *      y64;
} orc_mm_ctx;

static void orc_mm_ggml_range(void * p, int64_t n0, int64_t n1) {
    orc_mm_ctx * c = (orc_mm_ctx *) p;
    for (int64_t n = n0; n < n1; n++) {
        const char * w = (const char *) c->W + (size_t) n * c->wrow;
        for (int64_t m = 0; m < c->M; m++) {
            c->y[m * c->N + n] = orc_vec_dot(c->type, c->K, w, (const char *) c->xq + (size_t) m * c->xrow);
        }
    }
}

void orc_mul_mat_ggml(int type, const void * W, int64_t N, int64_t K,
                      const float * x, int64_t x_stride, int64_t M, float * y, int nthreads) {
    const int    vtype = (type == ORC_TYPE_Q8_0) ? ORC_TYPE_Q8_0 : ORC_TYPE_Q8_K;
    const size_t xrow  = orc_row_size(vtype, K);
    char *       xq    = (char *) malloc(xrow * (size_t) M);
    for (int64_t m = 0; m < M; m++) {
        if (vtype == ORC_TYPE_Q8_0) {
            orc_quantize_row_q8_0(x + m * x_stride, xq + (size_t) m * xrow, K);
        } else {
            orc_quantize_row_q8_K(x + m * x_stride, xq + (size_t) m * xrow, K);
        }
    }
    orc_mm_ctx c = { type, W, N, K, M, orc_row_size(type, K), xrow, xq, x, x_stride, y, NULL };
    orc_parallel_for(N, nthreads, orc_mm_ggml_range, &c);
    free(xq);
}

static void orc_mm_f64_range(void * p, int64_t n0, int64_t n1) {
    orc_mm_ctx * c   = (orc_mm_ctx *) p;
    float *      deq = (float *) malloc((size_t) c->K * sizeof(float));
    for (int64_t n = n0; n < n1; n++) {
        orc_dequantize_row(c->type, (const char *) c->W + (size_t) n * c->wrow, deq, c->K);
        for (int64_t m = 0; m < c->M; m++) {
            const float * xm = c->x + m * c->x_stride;
            double        s  = 0.0;
            for (int64_t k = 0; k < c->K; k++) {
                s += (double) deq[k] * (double) xm[k];
            }
            c->y64[m * c->N + n] = s;
        }
    }
    free(deq);
}

void orc_mul_mat_f64(int type, const void * W, int64_t N, int64_t K,
                     const float * x, int64_t x_stride, int64_t M, double * y, int nthreads) {
    orc_mm_ctx c = { type, W, N, K, M, orc_row_size(type, K), 0, NULL, x, x_stride, NULL, y };
    orc_parallel_for(N, nthreads, orc_mm_f64_range, &c);
}

/* ------------------------------------------------------------------ */
/* flash_attn_ext                                                       */
/* ------------------------------------------------------------------ */

typedef struct {
    const orc_tensor *q, *k, *v, *mask;
    float             scale;
    float *           out;
    double *          out64;
} orc_fa_ctx;

static const void * orc_at(const orc_tensor * t, int64_t i1, int64_t i2, int64_t i3) {
    return (const char *) t->data + i1 * t->nb[1] + i2 * t->nb[2] + i3 * t->nb[3];
}

/* One query row per work item: r = ((b * Hq) + h) * n_q + i. */
static void orc_fa_ggml_range(void * p, int64_t r0, int64_t r1) {
    orc_fa_ctx *       c   = (orc_fa_ctx *) p;
    const orc_tensor * q   = c->q;
    const orc_tensor * k   = c->k;
    const orc_tensor * v   = c->v;
    const int64_t      D   = q->ne[0], DV = v->ne[0];
    const int64_t      nq  = q->ne[1], Hq = q->ne[2];
    const int64_t      nkv = k->ne[1];
    const int64_t      rk2 = Hq / k->ne[2], rk3 = q->ne[3] / k->ne[3];
    uint16_t *         Qh  = (uint16_t *) malloc((size_t) D * 2);
    uint16_t *         acc = (uint16_t *) malloc((size_t) DV * 2);
    for (int64_t r = r0; r < r1; r++) {
        const int64_t iq1 = r % nq, iq2 = (r / nq) % Hq, iq3 = r / (nq * Hq);
        const float * qr  = (const float *) orc_at(q, iq1, iq2, iq3);
        for (int64_t d = 0; d < D; d++) {
            Qh[d] = orc_fp32_to_fp16(qr[d]);
        }
        memset(acc, 0, (size_t) DV * 2);
        const uint16_t * mp = NULL;
        if (c->mask && c->mask->data) {
            mp = (const uint16_t *) orc_at(c->mask, iq1, iq2 % c->mask->ne[2], iq3 % c->mask->ne[3]);
        }
        const int64_t ik2 = iq2 / rk2, ik3 = iq3 / rk3;
        float         S = 0.0f, M = -INFINITY;
        for (int64_t ic = 0; ic < nkv; ic++) {
            const float mv = mp ? orc_fp16_to_fp32(mp[ic]) : 0.0f;
            if (mv == -INFINITY) {
                continue;
            }
            const uint16_t * kr  = (const uint16_t *) orc_at(k, ic, ik2, ik3);
            double           dot = 0.0;
            for (int64_t d = 0; d < D; d++) {
                dot += (double) (orc_fp16_to_fp32(kr[d]) * orc_fp16_to_fp32(Qh[d]));
            }
            float s = (float) dot;
            s       = s * c->scale;
            s       = s + mv;
            float ms = 1.0f, vs = 1.0f;
            if (s > M) {
                const float Mold = M;
                M                = s;
                ms               = expf(Mold - M);
                for (int64_t d = 0; d < DV; d++) {
                    acc[d] = orc_fp32_to_fp16(orc_fp16_to_fp32(acc[d]) * ms);
                }
            } else {
                vs = expf(s - M);
            }
            const uint16_t * vr = (const uint16_t *) orc_at(v, ic, ik2, ik3);
            for (int64_t d = 0; d < DV; d++) {
                acc[d] = orc_fp32_to_fp16(fmaf(orc_fp16_to_fp32(vr[d]), vs, orc_fp16_to_fp32(acc[d])));
            }
            S = S * ms + vs;
        }
        const float S_inv = S == 0.0f ? 0.0f : 1.0f / S;
        float *     o     = c->out + ((iq3 * nq + iq1) * Hq + iq2) * DV;
        for (int64_t d = 0; d < DV; d++) {
            o[d] = orc_fp16_to_fp32(acc[d]) * S_inv;
        }
    }
    free(Qh);
    free(acc);
}

static void orc_fa_f64_range(void * p, int64_t r0, int64_t r1) {
    orc_fa_ctx *       c   = (orc_fa_ctx *) p;
    const orc_tensor * q   = c->q;
    const orc_tensor * k   = c->k;
    const orc_tensor * v   = c->v;
    const int64_t      D   = q->ne[0], DV = v->ne[0];
    const int64_t      nq  = q->ne[1], Hq = q->ne[2];
    const int64_t      nkv = k->ne[1];
    const int64_t      rk2 = Hq / k->ne[2], rk3 = q->ne[3] / k->ne[3];
    double *           s   = (double *) malloc((size_t) nkv * sizeof(double));
    double *           acc = (double *) malloc((size_t) DV * sizeof(double));
    for (int64_t r = r0; r < r1; r++) {
        const int64_t iq1 = r % nq, iq2 = (r / nq) % Hq, iq3 = r / (nq * Hq);
        const float * qr  = (const float *) orc_at(q, iq1, iq2, iq3);
        const uint16_t * mp = NULL;
        if (c->mask && c->mask->data) {
            mp = (const uint16_t *) orc_at(c->mask, iq1, iq2 % c->mask->ne[2], iq3 % c->mask->ne[3]);
        }
        const int64_t ik2 = iq2 / rk2, ik3 = iq3 / rk3;
        double        mx  = -INFINITY;
        for (int64_t ic = 0; ic < nkv; ic++) {
            const double mv = mp ? (double) orc_fp16_to_fp32(mp[ic]) : 0.0;
            if (mv == -INFINITY) {
                s[ic] = -INFINITY;
                continue;
            }
            const uint16_t * kr  = (const uint16_t *) orc_at(k, ic, ik2, ik3);
            double           dot = 0.0;
            for (int64_t d = 0; d < D; d++) {
                dot += (double) qr[d] * (double) orc_fp16_to_fp32(kr[d]);
            }
            s[ic] = dot * (double) c->scale + mv;
            mx    = s[ic] > mx ? s[ic] : mx;
        }
        for (int64_t d = 0; d < DV; d++) {
            acc[d] = 0.0;
        }
        double l = 0.0;
        if (mx != -INFINITY) {
            for (int64_t ic = 0; ic < nkv; ic++) {
                if (s[ic] == -INFINITY) {
                    continue;
                }
                const double     pw = exp(s[ic] - mx);
                const uint16_t * vr = (const uint16_t *) orc_at(v, ic, ik2, ik3);
                l += pw;
                for (int64_t d = 0; d < DV; d++) {
                    acc[d] += pw * (double) orc_fp16_to_fp32(vr[d]);
                }
            }
        }
        double * o = c->out64 + ((iq3 * nq + iq1) * Hq + iq2) * DV;
        for (int64_t d = 0; d < DV; d++) {
            o[d] = l > 0.0 ? acc[d] / l : 0.0;
        }
    }
    free(s);
    free(acc);
}

void orc_flash_attn_ext_ggml(const orc_tensor * q, const orc_tensor * k, const orc_tensor * v,
                             const orc_tensor * mask, float scale, float * out, int nthreads) {
    orc_fa_ctx c = { q, k, v, mask, scale, out, NULL };
    orc_parallel_for(q->ne[1] * q->ne[2] * q->ne[3], nthreads, orc_fa_ggml_range, &c);
}

void orc_flash_attn_ext_f64(const orc_tensor * q, const orc_tensor * k, const orc_tensor * v,
                            const orc_tensor * mask, float scale, double * out, int nthreads) {
    orc_fa_ctx c = { q, k, v, mask, scale, NULL, out };
    orc_parallel_for(q->ne[1] * q->ne[2] * q->ne[3], nthreads, orc_fa_f64_range, &c);
}

/* ------------------------------------------------------------------ */
/* glue                                                                 */
/* ------------------------------------------------------------------ */

/* ggml rms_norm: mean of squares accumulated in double, scale = 1/sqrtf in
 * f32 [ext]; then the elementwise MUL by the norm weight. */
void orc_rms_norm_mul(const float * x, const float * w, float * y, int64_t n, int64_t rows, float eps) {
    for (int64_t r = 0; r < rows; r++) {
        const float * xr  = x + r * n;
        double        sum = 0.0;
        for (int64_t i = 0; i < n; i++) {
            sum += (double) (xr[i] * xr[i]);
        }
        const float mean  = (float) (sum / (double) n);
        const float scale = 1.0f / sqrtf(mean + eps);
        for (int64_t i = 0; i < n; i++) {
            const float t = xr[i] * scale;
            y[r * n + i]  = w ? t * w[i] : t;
        }
    }
}

void orc_layer_norm(const float * x, float * y, int64_t n, int64_t rows, float eps) {
    for (int64_t r = 0; r < rows; r++) {
        const float * xr  = x + r * n;
        float *       yr  = y + r * n;
        double        sum = 0.0;
        for (int64_t i = 0; i < n; i++) {
            sum += (double) xr[i];
        }
        const float mean = (float) (sum / (double) n);
        double      sum2 = 0.0;
        for (int64_t i = 0; i < n; i++) {
            const float v = xr[i] - mean;
            yr[i]         = v;
            sum2 += (double) (v * v);
        }
        const float variance = (float) (sum2 / (double) n);
        const float scale    = 1.0f / sqrtf(variance + eps);
        for (int64_t i = 0; i < n; i++) {
            yr[i] *= scale;
        }
    }
}

/* NeoX RoPE: pair (i, i + n_dims/2) rotates by theta_i, with theta_0 = pos
 * and theta_{i+1} = theta_i * base^(-2/n_dims) accumulated in f32 (the
 * iterative cache of ggml's rope [ext]). */
void orc_rope_neox(const float * x, float * y, int64_t head_dim, int64_t n_dims, int64_t heads,
                   int64_t tokens, const int32_t * positions, float freq_base) {
    const float theta_scale = powf(freq_base, -2.0f / (float) n_dims);
    const int64_t half      = n_dims / 2;
    for (int64_t t = 0; t < tokens; t++) {
        for (int64_t h = 0; h < heads; h++) {
            const float * xr    = x + (t * heads + h) * head_dim;
            float *       yr    = y + (t * heads + h) * head_dim;
            float         theta = (float) positions[t];
            for (int64_t i = 0; i < half; i++) {
                const float c = cosf(theta), s = sinf(theta);
                const float x0 = xr[i], x1 = xr[i + half];
                yr[i]        = x0 * c - x1 * s;
                yr[i + half] = x0 * s + x1 * c;
                theta *= theta_scale;
            }
            for (int64_t i = n_dims; i < head_dim; i++) {
                yr[i] = xr[i];
            }
        }
    }
}

void orc_swiglu(const float * x, float * y, int64_t n, int64_t rows) {
    for (int64_t r = 0; r < rows; r++) {
        const float * g = x + r * 2 * n;
        const float * u = g + n;
        for (int64_t i = 0; i < n; i++) {
            const float silu = g[i] / (1.0f + expf(-g[i]));
            y[r * n + i]     = silu * u[i];
        }
    }
}
