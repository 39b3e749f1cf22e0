/*
 * mmhip_synth.h - seeded synthetic data generated directly in device memory,
 * for benchmarks and tests at full model size (the reference loads real GGUF
 * checkpoints; none is available offline).  No counterpart in the reference.
 *
 * Distributions (counter-based splitmix64 hashing, 24-bit uniforms,
 * Box-Muller normals; element i of stream `seed` is a pure function of
 * (seed, i)):
 *   Q8_0: quants uniform in [-127, 127]; d = f16(|N(0, 0.02)| / 127)
 *   Q4_K: quant and 6-bit scale/min bytes uniform; d, dmin = f16(|N(0, 0.02)|)
 *   Q5_K: quant, fifth-bit and scale/min bytes uniform; d = f16(|N(0, 0.02)| / 512),
 *         dmin = f16(|N(0, 0.02)| / 32) (blocks centred on zero, |w| ~ 0.01)
 *   Q6_K: ql/qh bytes uniform; int8 scales uniform in [-64, 63];
 *         d = f16(|N(0, 0.02)| / 1024)  (|w| ~ 0.01 like real weights)
 */
#ifndef MMHIP_SYNTH_H
#define MMHIP_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* nblocks GGUF blocks of `type` (Q8_0 / Q4_K / Q5_K / Q6_K) written to dst_gguf. */
int mmhip_synth_gguf(int type, void * dst_gguf, int64_t nblocks, uint64_t seed, void * stream);

/* n values of N(mean, std) as f32 (type 0), f16 (type 1) or bf16 (type 30,
 * rounded as ggml rounds f32 to bf16). */
int mmhip_synth_normal(int type, void * dst, int64_t n, uint64_t seed, float mean, float std, void * stream);

#ifdef __cplusplus
}
#endif
#endif
