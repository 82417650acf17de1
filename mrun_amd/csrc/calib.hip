// Calibration kernels for the benchmark's roofline denominators: the copy rate this box's HBM
// reaches and the rate of v_mfma_f32_32x32x16_bf16 (the instruction the prefill GEMMs issue),
// each measured beside the published peak. Not part of the MoE block's C ABI: bench.py loads
// this library by itself.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;

// Grid-stride copy of n 16-byte units, four loads in flight per thread before their stores.
__global__ __launch_bounds__(256) void copy_kernel(const uint4 *__restrict__ src,
                                                   uint4 *__restrict__ dst, size_t n) {
    const size_t stride = (size_t)gridDim.x * 256;
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    for (; i + 3 * stride < n; i += 4 * stride) {
        const uint4 a = src[i], b = src[i + stride], c = src[i + 2 * stride],
                    d = src[i + 3 * stride];
        dst[i] = a;
        dst[i + stride] = b;
        dst[i + 2 * stride] = c;
        dst[i + 3 * stride] = d;
    }
    for (; i < n; i += stride) dst[i] = src[i];
}

// Grid-stride read of n 16-byte units (four loads in flight per thread), folded by xor into one
// word per thread, so the loads stay live.
__global__ __launch_bounds__(256) void read_kernel(const uint4 *__restrict__ src, size_t n,
                                                   uint32_t *__restrict__ out) {
    const size_t stride = (size_t)gridDim.x * 256;
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    uint32_t x = 0;
    for (; i + 3 * stride < n; i += 4 * stride) {
        const uint4 a = src[i], b = src[i + stride], c = src[i + 2 * stride],
                    d = src[i + 3 * stride];
        x ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^
             d.z ^ d.w;
    }
    for (; i < n; i += stride) x ^= src[i].x ^ src[i].y ^ src[i].z ^ src[i].w;
    out[(size_t)blockIdx.x * 256 + threadIdx.x] = x;
}

// NCH independent accumulator chains per wave, iters rounds of one MFMA per chain. Every operand
// element is the bf16 pair `pair` (a kernel argument: nothing for the compiler to fold) and every
// accumulator ends in the stored sum, so no MFMA is dead. With pair = (1, 1) each lane stores
// NCH * 16 * 16 * iters exactly (iters <= 2^16).
template <int NCH>
__global__ __launch_bounds__(256) void mfma_kernel(int iters, uint32_t pair,
                                                   float *__restrict__ out) {
    const bf16x8_t a = __builtin_bit_cast(bf16x8_t, make_uint4(pair, pair, pair, pair));
    const bf16x8_t b = a;
    f32x16_t acc[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[c][i] = 0.f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int c = 0; c < NCH; ++c)
            acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
    }
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int i = 0; i < 16; ++i) s += acc[c][i];
    out[(size_t)blockIdx.x * 256 + threadIdx.x] = s;
}

constexpr int kChains = 4;

// One link of a chain of dependent launches: every thread reads one word that the previous launch
// wrote (READ; a different word per workgroup, so the reads spread over the memory channels) and
// stores one word for the next launch. The floor under a forward made of such launches.
template <bool READ>
__global__ __launch_bounds__(256) void chain_kernel(const uint32_t *__restrict__ src, int n_src,
                                                    uint32_t *__restrict__ dst) {
    uint32_t v = blockIdx.x;
    if (READ) v += src[((size_t)blockIdx.x * 256 + threadIdx.x) % (size_t)n_src];
    dst[(size_t)blockIdx.x * 256 + threadIdx.x] = v + 1;
}

}  // namespace

extern "C" {

// Copies `bytes` (a multiple of 16, both pointers 16-byte aligned) from src to dst on `stream`.
// Returns 0, or the HIP error code.
int mrun_calib_copy(const void *src, void *dst, size_t bytes, void *stream) {
    if (bytes % 16 != 0 || ((uintptr_t)src | (uintptr_t)dst) % 16 != 0) return (int)hipErrorInvalidValue;
    const size_t n = bytes / 16;
    if (n == 0) return 0;
    const unsigned blocks = 256 * 16;  // 16 workgroups per CU
    copy_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>((const uint4 *)src, (uint4 *)dst, n);
    return (int)hipGetLastError();
}

// Reads `bytes` (a multiple of 16, src 16-byte aligned) on `stream`; out receives one word per
// thread of mrun_calib_read_threads() threads.
int mrun_calib_read(const void *src, size_t bytes, uint32_t *out, void *stream) {
    if (bytes % 16 != 0 || (uintptr_t)src % 16 != 0 || !out) return (int)hipErrorInvalidValue;
    const size_t n = bytes / 16;
    if (n == 0) return 0;
    read_kernel<<<256 * 16, 256, 0, (hipStream_t)stream>>>((const uint4 *)src, n, out);
    return (int)hipGetLastError();
}

int mrun_calib_read_threads(void) { return 256 * 16 * 256; }

// blocks workgroups of 4 waves, each wave issuing iters * mrun_calib_mfma_chains() MFMAs of
// 32 x 32 x 16 (32,768 flops each) on operands of ones; out receives blocks * 256 floats, each
// mrun_calib_mfma_chains() * 256 * iters (iters <= 65536).
int mrun_calib_mfma(int blocks, int iters, float *out, void *stream) {
    if (blocks <= 0 || iters <= 0 || iters > 65536 || !out) return (int)hipErrorInvalidValue;
    mfma_kernel<kChains><<<blocks, 256, 0, (hipStream_t)stream>>>(iters, 0x3F803F80u, out);
    return (int)hipGetLastError();
}

int mrun_calib_mfma_chains(void) { return kChains; }

// Three dependent launches of g[0], g[1], g[2] workgroups of 256 threads: launch i reads (with
// `read`) buf[i], the words launch i - 1 wrote (buf[0]: g[0] * 256 words the caller provides),
// and writes buf[i + 1]; buf[i + 1] holds g[i] * 256 words.
int mrun_calib_chain(uint32_t *const *buf, const int *g, int read, void *stream) {
    if (!buf || !g) return (int)hipErrorInvalidValue;
    for (int i = 0; i < 3; ++i) {
        if (g[i] <= 0 || !buf[i] || !buf[i + 1]) return (int)hipErrorInvalidValue;
        const int n_src = (i == 0 ? g[0] : g[i - 1]) * 256;
        if (read) chain_kernel<true><<<g[i], 256, 0, (hipStream_t)stream>>>(buf[i], n_src, buf[i + 1]);
        else chain_kernel<false><<<g[i], 256, 0, (hipStream_t)stream>>>(buf[i], n_src, buf[i + 1]);
    }
    return (int)hipGetLastError();
}

}  // extern "C"
