// Device variants of the seeded synthetic-input generator (include/mrun_synth.h): the same
// SplitMix64 counter-form draws, so codes are bit-identical to the host generator's; normals use
// the same float64 Box-Muller formula with the device's float64 log/sqrt/sin/cos. Benchmark input
// generation for multi-gigabyte weight stacks; not part of the reference's operator surface.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mrun_synth.h"

namespace {

constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t draw(uint64_t seed, uint64_t n) { return mix64(seed + (n + 1) * kGamma); }

__device__ __forceinline__ double uniform(uint64_t seed, uint64_t n) {
    return (double)(draw(seed, n) >> 11) * (1.0 / 9007199254740992.0);
}

__device__ __forceinline__ double normal(uint64_t seed, uint64_t i) {
    const uint64_t b = i & ~1ull;
    const double u1 = uniform(seed, b), u2 = uniform(seed, b + 1);
    const double r = sqrt(-2.0 * log(1.0 - u1));
    const double th = 6.283185307179586476925286766559 * u2;
    return (i & 1) ? r * sin(th) : r * cos(th);
}

__device__ __forceinline__ uint16_t bf16_of(double v) {
    const float f = (float)v;
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__global__ void codes_kernel(uint64_t seed, int bits, uint32_t *words, size_t n) {
    const int per = 32 / bits, shift = 64 - bits;
    for (size_t w = (size_t)blockIdx.x * blockDim.x + threadIdx.x; w < n;
         w += (size_t)gridDim.x * blockDim.x) {
        uint32_t v = 0;
        for (int j = 0; j < per; ++j) v |= (uint32_t)(draw(seed, (uint64_t)w * per + j) >> shift) << (bits * j);
        words[w] = v;
    }
}

__global__ void normal_kernel(uint64_t seed, float std, uint16_t *out, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        out[i] = bf16_of((double)std * normal(seed, i));
}

__global__ void scales_kernel(uint64_t seed, uint16_t *scales, uint16_t *biases, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        const uint16_t s = bf16_of(fabs(0.02 * normal(seed, i)) / 7.5);
        scales[i] = s;
        if (biases) biases[i] = bf16_of(-8.0 * (double)__uint_as_float((uint32_t)s << 16));
    }
}

unsigned grid_for(size_t n) {
    const size_t g = (n + 255) / 256;
    return (unsigned)(g < 65536 ? (g ? g : 1) : 65536);
}

}  // namespace

extern "C" {

int mrun_synth_codes_dev(uint64_t seed, int32_t bits, uint32_t *words, size_t n_words,
                         void *stream) {
    if ((bits != 4 && bits != 8) || !words) return -1;
    codes_kernel<<<grid_for(n_words), 256, 0, (hipStream_t)stream>>>(seed, bits, words, n_words);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int mrun_synth_normal_bf16_dev(uint64_t seed, float std, uint16_t *out, size_t n, void *stream) {
    if (!out) return -1;
    normal_kernel<<<grid_for(n), 256, 0, (hipStream_t)stream>>>(seed, std, out, n);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int mrun_synth_scales_biases_dev(uint64_t seed, uint16_t *scales, uint16_t *biases, size_t n,
                                 void *stream) {
    if (!scales) return -1;
    scales_kernel<<<grid_for(n), 256, 0, (hipStream_t)stream>>>(seed, scales, biases, n);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // extern "C"
