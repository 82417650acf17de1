/*
 * Seeded synthetic inputs for the MoE block benchmarks and tests (host side, C ABI).
 *
 * This is not part of the reference's operator surface: the reference benchmarks on real
 * checkpoints. The benchmark configurations describe their synthetic tensors by distribution
 * only, so this generator makes them concrete and reproducible:
 *
 *   draw(seed, n)    = mix64(seed + (n + 1) * 0x9E3779B97F4A7C15)     (SplitMix64, counter form)
 *   uniform(seed, n) = (draw(seed, n) >> 11) * 2^-53
 *   normal(seed, i)  = Box-Muller on uniforms 2*(i/2) and 2*(i/2)+1 in float64:
 *                      r = sqrt(-2 ln(1 - u1)), even i -> r cos(2 pi u2), odd i -> r sin(2 pi u2)
 *   4-bit codes      : code j of word w is draw(seed, 8w + j) >> 60, packed LSB first
 *   8-bit codes      : byte j of word w is draw(seed, 4w + j) >> 56, packed LSB first
 *   scales           : bf16(|0.02 * normal| / 7.5); biases: bf16(-8 * scale) (exact)
 *   bf16(v)          : v rounded to float32, then to bfloat16, both to nearest even
 *   tensor seed      : base ^ mix64((config << 48) ^ (layer << 24) ^ tensor)
 *   Zipf router bias : a Fisher-Yates permutation rank: E -> 1..E driven by draw(seed, i), then
 *                      bias[e] = bf16(amp * rank[e]^-s)
 */
#ifndef MRUN_SYNTH_H
#define MRUN_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

uint64_t mrun_synth_mix64(uint64_t z);
uint64_t mrun_synth_tensor_seed(uint64_t base, uint32_t config, uint32_t layer, uint32_t tensor);
uint64_t mrun_synth_draw(uint64_t seed, uint64_t n);
double mrun_synth_normal(uint64_t seed, uint64_t i);

/* Packed affine codes: n_words u32 words of `bits` (4 or 8) bit codes. */
int mrun_synth_codes(uint64_t seed, int32_t bits, uint32_t *words, size_t n_words);
/* bf16(std * normal(i)) for i < n. */
void mrun_synth_normal_bf16(uint64_t seed, float std, uint16_t *out, size_t n);
/* scales[i] = bf16(|0.02 * normal(i)| / 7.5), biases[i] = bf16(-8 * scales[i]). */
void mrun_synth_scales_biases(uint64_t seed, uint16_t *scales, uint16_t *biases, size_t n);
/* The Zipf-skewed router bias; rank_out [experts] optional. */
int mrun_synth_zipf_bias(uint64_t seed, int32_t experts, double s, double amp, uint16_t *bias,
                         int32_t *rank_out);

/* Device variants (libmrun_synth_dev.so), asynchronous on a HIP stream, writing device memory:
 * the same draws, so codes are bit-identical to mrun_synth_codes; normals use the device's float64
 * math. Return 0, or -1 for bad arguments or a launch error. */
int mrun_synth_codes_dev(uint64_t seed, int32_t bits, uint32_t *words, size_t n_words,
                         void *stream);
int mrun_synth_normal_bf16_dev(uint64_t seed, float std, uint16_t *out, size_t n, void *stream);
int mrun_synth_scales_biases_dev(uint64_t seed, uint16_t *scales, uint16_t *biases, size_t n,
                                 void *stream);

#ifdef __cplusplus
}
#endif
#endif
