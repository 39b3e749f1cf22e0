// mmhip_device.h - device-side helpers shared by the gfx950 kernels.
//
// Weight layout on the device ("row-grouped layout"): a quantized row keeps
// exactly its GGUF byte size (ggml_row_size), so row strides, views and
// ggml_nbytes are unchanged, but inside each row the fields of all blocks are
// grouped so that every field streams with aligned 16-byte loads:
//   Q8_0 : qs[K] (int8)        | d[K/32] (f16)
//   Q4_K : qs[K/2] (nibbles)   | scales[12*K/256] | dm[2*K/256] (f16 d, dmin)
//   Q5_K : qs[K/2] (nibbles)   | qh[K/8] | scales[12*K/256] | dm[2*K/256]
//   Q6_K : ql[K/2] | qh[K/4]   | sc[K/16] (int8)  | d[K/256] (f16)
// Within a field, blocks keep their GGUF order and their GGUF byte order.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace mmhip {

constexpr int TYPE_F32  = 0;
constexpr int TYPE_F16  = 1;
constexpr int TYPE_Q8_0 = 8;
constexpr int TYPE_Q4_K = 12;
constexpr int TYPE_Q5_K = 13;
constexpr int TYPE_Q6_K = 14;
constexpr int TYPE_Q8_K = 15;
constexpr int TYPE_BF16 = 30;

// f32 -> bf16 as ggml rounds it (ggml_compute_fp32_to_bf16): nearest-even on
// the upper 16 bits, NaN kept quiet; returned as the f32 of the bf16 value.
__device__ __forceinline__ float round_bf16(float v) {
    uint32_t u = __float_as_uint(v);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        u = (u | 0x00400000u) & 0xffff0000u;
    } else {
        u = (u + (0x7fffu + ((u >> 16) & 1u))) & 0xffff0000u;
    }
    return __uint_as_float(u);
}

constexpr int QK8_0 = 32;
constexpr int QK_K  = 256;

constexpr int WAVE = 64;

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float    float16_t __attribute__((ext_vector_type(16)));
typedef float    float4_t __attribute__((ext_vector_type(4)));
typedef int      int4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float) v;
}

__device__ __forceinline__ uint16_t f2h(float f) {
    _Float16 v = (_Float16) f;  // round to nearest even
    uint16_t h;
    __builtin_memcpy(&h, &v, 2);
    return h;
}

// Signed 4-byte dot product with int32 accumulate (v_dot4_i32_i8).
__device__ __forceinline__ int dot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

// Reductions across the 16-lane rows of a wave with the gfx950 row swaps
// (one VALU op instead of an LDS permute): v_permlane16_swap exchanges rows
// 1 / 3 of its first operand with rows 0 / 2 of its second, v_permlane32_swap
// rows 2-3 with rows 0-1; with the value in both operands each lane ends up
// holding its own value and that of lane ^ 16 (^ 32), in some order, so a
// symmetric op of the pair is the xor reduction (a + b == b + a in IEEE).
__device__ __forceinline__ float2 lanes_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return float2{ __uint_as_float(r[0]), __uint_as_float(r[1]) };
}

__device__ __forceinline__ float2 lanes_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return float2{ __uint_as_float(r[0]), __uint_as_float(r[1]) };
}

__device__ __forceinline__ float max_xor16(float x) {
    const float2 p = lanes_xor16(x);
    return fmaxf(p.x, p.y);
}

__device__ __forceinline__ float max_xor32(float x) {
    const float2 p = lanes_xor32(x);
    return fmaxf(p.x, p.y);
}

__device__ __forceinline__ float sum_xor16(float x) {
    const float2 p = lanes_xor16(x);
    return p.x + p.y;
}

__device__ __forceinline__ float sum_xor32(float x) {
    const float2 p = lanes_xor32(x);
    return p.x + p.y;
}

// DPP row moves used below (all lanes of every row take part):
// quad_perm [1,0,3,2] (lane ^ 1), quad_perm [2,3,0,1] (lane ^ 2),
// row_half_mirror (lane i of an 8-lane half <-> 7 - i: the other quad) and
// row_mirror (lane i of a 16-lane row <-> 15 - i: the other half).  Once
// every lane of a quad (half) holds the same value, the mirrors pair it
// with the other quad (half), so a symmetric op reduces over 8 (16) lanes.
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;

template <int CTRL> __device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

template <int CTRL> __device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}

template <int CTRL> __device__ __forceinline__ double dpp_d(double v) {
    const int2 p = __builtin_bit_cast(int2, v);
    return __builtin_bit_cast(double, int2{ __builtin_amdgcn_mov_dpp(p.x, CTRL, 0xF, 0xF, false),
                                            __builtin_amdgcn_mov_dpp(p.y, CTRL, 0xF, 0xF, false) });
}

// both halves of a double through the row swaps: element k of the two
// results comes from the same lane, so {lo[k], hi[k]} are that lane's double
__device__ __forceinline__ double sum_xor16_d(double v) {
    const int2 p  = __builtin_bit_cast(int2, v);
    const auto lo = __builtin_amdgcn_permlane16_swap(p.x, p.x, false, false);
    const auto hi = __builtin_amdgcn_permlane16_swap(p.y, p.y, false, false);
    return __builtin_bit_cast(double, int2{ (int) lo[0], (int) hi[0] }) +
           __builtin_bit_cast(double, int2{ (int) lo[1], (int) hi[1] });
}

__device__ __forceinline__ double sum_xor32_d(double v) {
    const int2 p  = __builtin_bit_cast(int2, v);
    const auto lo = __builtin_amdgcn_permlane32_swap(p.x, p.x, false, false);
    const auto hi = __builtin_amdgcn_permlane32_swap(p.y, p.y, false, false);
    return __builtin_bit_cast(double, int2{ (int) lo[0], (int) hi[0] }) +
           __builtin_bit_cast(double, int2{ (int) lo[1], (int) hi[1] });
}

// Max over aligned groups of 8 lanes (a Q8_0 block of 4-value lanes);
// every lane of the group receives it.
__device__ __forceinline__ float group8_max(float v) {
    v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    return fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
}

// Max over aligned groups of 32 lanes (a Q8_0 block of one value per lane).
__device__ __forceinline__ float group32_max(float v) {
    v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f<DPP_MIRROR>(v));
    return max_xor16(v);
}

// Sum over aligned groups of 16 lanes (a Q8_K 16-element block sum).
__device__ __forceinline__ int group16_sum_i(int v) {
    v += dpp_i<DPP_XOR1>(v);
    v += dpp_i<DPP_XOR2>(v);
    v += dpp_i<DPP_HALF_MIRROR>(v);
    return v + dpp_i<DPP_MIRROR>(v);
}

// The element of largest |x| over the wave, lowest index on ties: a (its
// |x|), vm (its x) and ix (its index) hold each lane's candidate on entry and
// the winner in every lane on return.  (largest a, lowest ix) is a total
// order, so any reduction tree selects the same element.
__device__ __forceinline__ void wave_argmax_abs(float & a, float & vm, int & ix) {
    auto take = [&](float a2, float vm2, int ix2) {
        if (a2 > a || (a2 == a && ix2 < ix)) {
            a  = a2;
            vm = vm2;
            ix = ix2;
        }
    };
    take(dpp_f<DPP_XOR1>(a), dpp_f<DPP_XOR1>(vm), dpp_i<DPP_XOR1>(ix));
    take(dpp_f<DPP_XOR2>(a), dpp_f<DPP_XOR2>(vm), dpp_i<DPP_XOR2>(ix));
    take(dpp_f<DPP_HALF_MIRROR>(a), dpp_f<DPP_HALF_MIRROR>(vm), dpp_i<DPP_HALF_MIRROR>(ix));
    take(dpp_f<DPP_MIRROR>(a), dpp_f<DPP_MIRROR>(vm), dpp_i<DPP_MIRROR>(ix));
    {
        const auto pa = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(a), false, false);
        const auto pv = __builtin_amdgcn_permlane16_swap(__float_as_uint(vm), __float_as_uint(vm), false, false);
        const auto pi = __builtin_amdgcn_permlane16_swap((unsigned) ix, (unsigned) ix, false, false);
        a = __uint_as_float(pa[0]), vm = __uint_as_float(pv[0]), ix = (int) pi[0];
        take(__uint_as_float(pa[1]), __uint_as_float(pv[1]), (int) pi[1]);
    }
    {
        const auto pa = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(a), false, false);
        const auto pv = __builtin_amdgcn_permlane32_swap(__float_as_uint(vm), __float_as_uint(vm), false, false);
        const auto pi = __builtin_amdgcn_permlane32_swap((unsigned) ix, (unsigned) ix, false, false);
        a = __uint_as_float(pa[0]), vm = __uint_as_float(pv[0]), ix = (int) pi[0];
        take(__uint_as_float(pa[1]), __uint_as_float(pv[1]), (int) pi[1]);
    }
}

// Sum over all 64 lanes; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<DPP_XOR1>(v);
    v += dpp_f<DPP_XOR2>(v);
    v += dpp_f<DPP_HALF_MIRROR>(v);
    v += dpp_f<DPP_MIRROR>(v);
    return sum_xor32(sum_xor16(v));
}

// double-precision wave sum (ggml-CPU accumulates RMS_NORM's squares in double)
__device__ __forceinline__ double wave_sum_d(double v) {
    v += dpp_d<DPP_XOR1>(v);
    v += dpp_d<DPP_XOR2>(v);
    v += dpp_d<DPP_HALF_MIRROR>(v);
    v += dpp_d<DPP_MIRROR>(v);
    return sum_xor32_d(sum_xor16_d(v));
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f<DPP_MIRROR>(v));
    return max_xor32(max_xor16(v));
}

// Sum over aligned groups of G lanes (G a power of two <= 64), using
// row-local DPP where the group fits a 16-lane row; every lane of the group
// receives the total.
template <int G> __device__ __forceinline__ float group_sum(float v) {
    if constexpr (G >= 64) {
        v += __shfl_xor(v, 32, WAVE);
    }
    if constexpr (G >= 32) {
        v += __shfl_xor(v, 16, WAVE);
    }
    if constexpr (G >= 16) {
        v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false));
    }
    if constexpr (G >= 8) {
        v += __shfl_xor(v, 4, WAVE);
    }
    if constexpr (G >= 4) {
        v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    }
    if constexpr (G >= 2) {
        v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    }
    return v;
}

// Q4_K 6-bit (scale, min) pair j of a 12-byte scales field.
__device__ __forceinline__ void q4k_scale_min(int j, const uint8_t * s, int & sc, int & mn) {
    if (j < 4) {
        sc = s[j] & 63;
        mn = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 0x0f) | ((s[j - 4] >> 6) << 4);
        mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

// Same, from the three 32-bit words of the scales field (register form).
__device__ __forceinline__ void q4k_scale_min_w(int j, uint32_t w0, uint32_t w1, uint32_t w2, int & sc, int & mn) {
    // bytes 0-3 = w0, 4-7 = w1, 8-11 = w2
    if (j < 4) {
        sc = (w0 >> (8 * j)) & 63;
        mn = (w1 >> (8 * j)) & 63;
    } else {
        const int      jj = j - 4;
        const uint32_t b8 = (w2 >> (8 * jj)) & 0xff;
        sc = (int) ((b8 & 0x0f) | (((w0 >> (8 * jj + 6)) & 3) << 4));
        mn = (int) ((b8 >> 4) | (((w1 >> (8 * jj + 6)) & 3) << 4));
    }
}

__host__ __device__ constexpr int64_t row_bytes(int type, int64_t k) {
    return type == TYPE_Q8_0 ? (k / 32) * 34
         : type == TYPE_Q4_K ? (k / 256) * 144
         : type == TYPE_Q5_K ? (k / 256) * 176
         : type == TYPE_Q6_K ? (k / 256) * 210
         : type == TYPE_F16 || type == TYPE_BF16 ? k * 2
         : type == TYPE_F32 ? k * 4
         : 0;
}

// Activation quantisation of a 256-element chunk held in registers, lane l
// owning elements 4l .. 4l+3, with exactly the arithmetic of k_quant.hip
// (ggml quantize_row_q8_0_ref / quantize_row_q8_K_ref):
//   Q8_0: eight blocks of 32 (8 lanes each); d = amax/127 rounded to f16,
//         q = roundf(x / d)
//   Q8_K: one super-block; the first element of largest |x| gives
//         iscale = -127 / x_max, q = min(127, nearest-even(iscale * x)),
//         d = 1 / iscale, plus the sixteen 16-element sums of q.
// qs, d, bs point at the chunk's first element / scale / sum.

// The lane's four values (the caller stores them); the scales and sums are
// stored here.
__device__ __forceinline__ char4 quant_chunk256_q(const float (&v)[4], int lane, int qtype, float * __restrict__ d,
                                                  int16_t * __restrict__ bs) {
#pragma clang fp contract(off)
    char4 q4;
    if (qtype == TYPE_Q8_0) {
        const float a = group8_max(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
        const float dd = a / 127.0f;
        const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
        q4.x           = (signed char) roundf(v[0] * id);
        q4.y           = (signed char) roundf(v[1] * id);
        q4.z           = (signed char) roundf(v[2] * id);
        q4.w           = (signed char) roundf(v[3] * id);
        if ((lane & 7) == 0) {
            d[lane >> 3] = h2f(f2h(dd));
        }
    } else {
        float a = 0.0f, vm = 0.0f;
        int   ix = 4 * lane;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float t = fabsf(v[k]);
            if (t > a) {
                a  = t;
                vm = v[k];
                ix = 4 * lane + k;
            }
        }
        wave_argmax_abs(a, vm, ix);
        int   qv[4] = { 0, 0, 0, 0 };
        float dd    = 0.0f;
        if (a != 0.0f) {
            const float iscale = -127.0f / vm;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int q = (int) rintf(iscale * v[k]);
                qv[k]       = q > 127 ? 127 : q;
            }
            dd = 1.0f / iscale;
        }
        q4.x   = (signed char) qv[0];
        q4.y   = (signed char) qv[1];
        q4.z   = (signed char) qv[2];
        q4.w   = (signed char) qv[3];
        int sb = qv[0] + qv[1] + qv[2] + qv[3];
        sb += dpp_i<DPP_XOR1>(sb);
        sb += dpp_i<DPP_XOR2>(sb);
        if ((lane & 3) == 0) {
            bs[lane >> 2] = (int16_t) sb;
        }
        if (lane == 0) {
            d[0] = dd;
        }
    }
    return q4;
}

__device__ __forceinline__ void quant_chunk256(const float (&v)[4], int lane, int qtype, int8_t * __restrict__ qs,
                                               float * __restrict__ d, int16_t * __restrict__ bs) {
    *(char4 *) (qs + 4 * lane) = quant_chunk256_q(v, lane, qtype, d, bs);
}

}  // namespace mmhip
