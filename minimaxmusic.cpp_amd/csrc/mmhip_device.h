// mmhip_device.h - device-side helpers shared by the gfx950 kernels.
//
// Weight layout on the device ("row-grouped layout"): a quantized row keeps
// exactly its GGUF byte size (ggml_row_size), so row strides, views and
// ggml_nbytes are unchanged, but inside each row the fields of all blocks are
// grouped so that every field streams with aligned 16-byte loads:
//   Q8_0 : qs[K] (int8)        | d[K/32] (f16)
//   Q4_K : qs[K/2] (nibbles)   | scales[12*K/256] | dm[2*K/256] (f16 d, dmin)
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
constexpr int TYPE_Q6_K = 14;
constexpr int TYPE_Q8_K = 15;
constexpr int TYPE_BF16 = 30;

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

// Sum over all 64 lanes; every lane receives the total.// Sum over all 64 lanes; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        v += __shfl_xor(v, o, WAVE);
    }
    return v;
}

// double-precision wave sum (ggml-CPU accumulates RMS_NORM's squares in double)
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        v += __shfl_xor(v, o, WAVE);
    }
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        v = fmaxf(v, __shfl_xor(v, o, WAVE));
    }
    return v;
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
         : type == TYPE_Q6_K ? (k / 256) * 210
         : type == TYPE_F16 || type == TYPE_BF16 ? k * 2
         : type == TYPE_F32 ? k * 4
         : 0;
}

}  // namespace mmhip
