// k_synth.hip - seeded synthetic GGUF blocks and normal tensors in device
// memory (include/mmhip_synth.h).
#include "mmhip_device.h"
#include "mmhip_internal.h"
#include "mmhip_synth.h"

namespace mmhip {

__device__ __forceinline__ uint64_t smix(uint64_t x) {
    x += 0x9e3779b97f4a7c15ull;
    x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
    x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
    return x ^ (x >> 31);
}

__device__ __forceinline__ uint64_t hash2(uint64_t seed, uint64_t i) {
    return smix(seed ^ smix(i));
}

// 24-bit uniform in (0, 1)
__device__ __forceinline__ float u24(uint64_t h) {
    return ((float) (h >> 40) + 0.5f) * (1.0f / 16777216.0f);
}

__device__ __forceinline__ float normal01(uint64_t seed, uint64_t i) {
    const float u1 = u24(hash2(seed, 2 * i));
    const float u2 = u24(hash2(seed, 2 * i + 1));
    return sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
}

__global__ void k_synth_gguf(int type, uint8_t * __restrict__ dst, int64_t nblocks, uint64_t seed) {
    const int bb = (int) row_bytes(type, type == TYPE_Q8_0 ? 32 : 256);
    for (int64_t b = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; b < nblocks;
         b += (int64_t) gridDim.x * blockDim.x) {
        uint8_t *     p    = dst + b * bb;
        const uint64_t base = (uint64_t) b * 64;
        // random bytes for the whole block, 8 at a time
        for (int j = 0; j < bb; j += 8) {
            const uint64_t h = hash2(seed, base + (uint64_t) (j / 8));
            for (int k = 0; k < 8 && j + k < bb; k++) {
                p[j + k] = (uint8_t) (h >> (8 * k));
            }
        }
        if (type == TYPE_Q8_0) {
            for (int j = 0; j < 32; j++) {
                const uint64_t h = hash2(seed ^ 0x5151ull, base + (uint64_t) j);
                p[2 + j]         = (uint8_t) (int8_t) ((int) (h % 255u) - 127);
            }
            const uint16_t d = f2h(fabsf(normal01(seed ^ 0xd0d0ull, (uint64_t) b)) * 0.02f / 127.0f);
            p[0]             = (uint8_t) (d & 0xff);
            p[1]             = (uint8_t) (d >> 8);
        } else if (type == TYPE_Q4_K || type == TYPE_Q5_K) {
            // Q5_K: blocks centred on zero, |w| ~ 0.01
            const float    dd = type == TYPE_Q5_K ? 512.0f : 1.0f;
            const float    dn = type == TYPE_Q5_K ? 32.0f : 1.0f;
            const uint16_t d  = f2h(fabsf(normal01(seed ^ 0xd0d0ull, (uint64_t) b)) * 0.02f / dd);
            const uint16_t dm = f2h(fabsf(normal01(seed ^ 0xd1d1ull, (uint64_t) b)) * 0.02f / dn);
            p[0]              = (uint8_t) (d & 0xff);
            p[1]              = (uint8_t) (d >> 8);
            p[2]              = (uint8_t) (dm & 0xff);
            p[3]              = (uint8_t) (dm >> 8);
        } else {
            for (int j = 0; j < 16; j++) {
                const uint64_t h = hash2(seed ^ 0x5c5cull, base + (uint64_t) j);
                p[192 + j]       = (uint8_t) (int8_t) ((int) (h % 128u) - 64);
            }
            const uint16_t d = f2h(fabsf(normal01(seed ^ 0xd0d0ull, (uint64_t) b)) * 0.02f / 1024.0f);
            p[208]           = (uint8_t) (d & 0xff);
            p[209]           = (uint8_t) (d >> 8);
        }
    }
}

__global__ void k_synth_normal(int type, void * __restrict__ dst, int64_t n, uint64_t seed, float mean, float stdv) {
    for (int64_t i = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; i < n; i += (int64_t) gridDim.x * blockDim.x) {
        const float v = mean + stdv * normal01(seed, (uint64_t) i);
        if (type == TYPE_F32) {
            ((float *) dst)[i] = v;
        } else if (type == TYPE_BF16) {
            ((uint16_t *) dst)[i] = (uint16_t) (__float_as_uint(round_bf16(v)) >> 16);
        } else {
            ((uint16_t *) dst)[i] = f2h(v);
        }
    }
}

}  // namespace mmhip

using namespace mmhip;

extern "C" int mmhip_synth_gguf(int type, void * dst, int64_t nblocks, uint64_t seed, void * stream) {
    MMHIP_API_BEGIN();
    if (!dst || nblocks < 0 || !is_repacked_type(type)) {
        return set_error(MMHIP_ERR_INVALID, "synth_gguf: bad arguments");
    }
    if (nblocks == 0) {
        return MMHIP_OK;
    }
    const unsigned grid = (unsigned) std::min<int64_t>((nblocks + 255) / 256, 1 << 16);
    hipLaunchKernelGGL(k_synth_gguf, dim3(grid), dim3(256), 0, (hipStream_t) stream, type, (uint8_t *) dst, nblocks,
                       seed);
    return check_launch("synth_gguf");
}

extern "C" int mmhip_synth_normal(int type, void * dst, int64_t n, uint64_t seed, float mean, float stdv,
                                  void * stream) {
    MMHIP_API_BEGIN();
    if (!dst || n < 0 || !(type == TYPE_F32 || type == TYPE_F16 || type == TYPE_BF16)) {
        return set_error(MMHIP_ERR_INVALID, "synth_normal: bad arguments");
    }
    if (n == 0) {
        return MMHIP_OK;
    }
    const unsigned grid = (unsigned) std::min<int64_t>((n + 255) / 256, 1 << 16);
    hipLaunchKernelGGL(k_synth_normal, dim3(grid), dim3(256), 0, (hipStream_t) stream, type, dst, n, seed, mean, stdv);
    return check_launch("synth_normal");
}
