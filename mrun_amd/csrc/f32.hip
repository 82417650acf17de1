// The MoE block for float32 checkpoints (a model whose tensors are all f32, as the reference's
// Hugging Face fixture: gen_tiny.py:235-274 writes it in f32 because MLX runs the dense gather_mm
// only in f32). The reference then computes every op of SparseMoe::forward (moe.rs:149-174) in
// f32: nothing is rounded to bf16, and the SwiGLU's casts (activations.rs:64-66) are identities.
//
// These kernels are the path for such blocks, not a tuned one: each output element is one wave's
// dot product over float4 loads, with a fixed reduction order, so a row's result does not depend
// on the batch. Expert weights are read once per pair (no sort by expert).
#include "common.hpp"
#include "kernels.hpp"

namespace mrun {

namespace {

// f32 sum over the wave by a fixed butterfly (every lane ends with the same value).
__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// lane's part of a . w over K (float4 chunks lane, lane + 64, ...; K a multiple of 4)
__device__ __forceinline__ float dot_part(const float *__restrict__ a, const float *__restrict__ w,
                                          int K, int lane) {
    float acc = 0.f;
    for (int c = lane; c < K / 4; c += 64) {
        const float4 x = ((const float4 *)a)[c], y = ((const float4 *)w)[c];
        acc = __builtin_fmaf(x.x, y.x, acc);
        acc = __builtin_fmaf(x.y, y.y, acc);
        acc = __builtin_fmaf(x.z, y.z, acc);
        acc = __builtin_fmaf(x.w, y.w, acc);
    }
    return acc;
}

__device__ __forceinline__ float sigmoid_f32(float z) { return 1.0f / (1.0f + expf(-z)); }

// out[r][n] = A[r / a_div] . W[e_r][n] (e_r = ids ? ids[r] : 0), or under GLU
// silu(A . W0[e_r][n]) * (A . W1[e_r][n]). One wave per (r, n): 4 columns per workgroup, rows
// strided over grid.y.
template <bool GLU>
__global__ __launch_bounds__(256) void f32_rows_kernel(F32Rows j) {
    const int lane = threadIdx.x & 63;
    const int n = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    if (n >= j.N) return;
    for (int r = blockIdx.y; r < j.R; r += gridDim.y) {
        const int e = j.ids ? (int)j.ids[r] : 0;
        const float *a = j.A + (size_t)(r / j.a_div) * j.K;
        const size_t wr = ((size_t)e * j.N + n) * j.K;
        const float g = wave_sum_f32(dot_part(a, j.W0 + wr, j.K, lane));
        float v = g;
        if (GLU) {
            const float u = wave_sum_f32(dot_part(a, j.W1 + wr, j.K, lane));
            v = (g * sigmoid_f32(g)) * u;
        }
        if (lane == 0) j.out[(size_t)r * j.N + n] = v;
    }
}

// Softmax and top-k of one token per wave: gates = exp(l - max) / sum; the k largest gates, equal
// gates by lower id, in rank order; scores = gates, or gates / (their sum in rank order) with norm.
__global__ __launch_bounds__(64) void f32_topk_kernel(const float *__restrict__ logits, int T,
                                                      int E, int k, int norm,
                                                      uint32_t *__restrict__ ids,
                                                      float *__restrict__ scores) {
    constexpr int NPER = 8;  // E <= 512
    const int t = blockIdx.x, lane = threadIdx.x;
    if (t >= T) return;
    const float *l = logits + (size_t)t * E;
    float v[NPER];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
        const int e = lane + 64 * i;
        v[i] = e < E ? l[e] : -INFINITY;
        m = fmaxf(m, v[i]);
    }
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) m = fmaxf(m, __shfl_xor(m, s, 64));
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
        v[i] = lane + 64 * i < E ? expf(v[i] - m) : 0.f;
        sum += v[i];
    }
    sum = wave_sum_f32(sum);
    // keys: gate bits (non-negative floats order as integers) over 0xffffffff - id
    uint64_t key[NPER];
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
        const int e = lane + 64 * i;
        const float g = v[i] / sum;
        key[i] = e < E ? ((uint64_t)__float_as_uint(g) << 32) | (uint64_t)(0xffffffffu - (uint32_t)e)
                       : 0ull;
    }
    float tot = 0.f;
    uint64_t mine = 0;
    for (int j = 0; j < k; ++j) {
        uint64_t b = key[0];
#pragma unroll
        for (int i = 1; i < NPER; ++i) b = key[i] > b ? key[i] : b;
#pragma unroll
        for (int s = 32; s >= 1; s >>= 1) {
            const uint64_t o = __shfl_xor(b, s, 64);
            b = o > b ? o : b;
        }
#pragma unroll
        for (int i = 0; i < NPER; ++i) key[i] = key[i] == b ? 0ull : key[i];
        tot += __uint_as_float((uint32_t)(b >> 32));  // in rank order
        if (lane == j) mine = b;
    }
    if (lane < k) {
        const float g = __uint_as_float((uint32_t)(mine >> 32));
        ids[(size_t)t * k + lane] = 0xffffffffu - (uint32_t)(mine & 0xffffffffu);
        scores[(size_t)t * k + lane] = norm ? g / tot : g;
    }
}

// out[t][d] = sum_j y[t k + j][d] * scores[t k + j] (j ascending), plus, with a shared expert,
// sigmoid(glogit[t]) * shared[t][d].
__global__ __launch_bounds__(256) void f32_combine_kernel(const float *__restrict__ y,
                                                          const float *__restrict__ scores, int T,
                                                          int k, int D,
                                                          const float *__restrict__ glogit,
                                                          const float *__restrict__ shared,
                                                          float *__restrict__ out) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)T * D) return;
    const size_t t = i / D, d = i % D;
    float acc = 0.f;
    for (int j = 0; j < k; ++j) acc += y[(t * k + j) * D + d] * scores[t * k + j];
    if (shared) acc += sigmoid_f32(glogit[t]) * shared[i];
    out[i] = acc;
}

}  // namespace

hipError_t launch_f32_rows(const F32Rows &j, bool glu, hipStream_t stream) {
    if (j.R <= 0 || j.N <= 0) return hipSuccess;
    if (j.K % 4 != 0 || j.a_div < 1) return hipErrorInvalidValue;
    dim3 grid((j.N + 3) / 4, j.R < 65535 ? j.R : 65535);
    if (glu) f32_rows_kernel<true><<<grid, 256, 0, stream>>>(j);
    else f32_rows_kernel<false><<<grid, 256, 0, stream>>>(j);
    return hipGetLastError();
}

hipError_t launch_f32_topk(const float *logits, int T, int E, int k, bool norm, uint32_t *ids,
                           float *scores, hipStream_t stream) {
    if (T <= 0) return hipSuccess;
    if (E > 512 || k > E || k < 1) return hipErrorInvalidValue;
    f32_topk_kernel<<<T, 64, 0, stream>>>(logits, T, E, k, norm ? 1 : 0, ids, scores);
    return hipGetLastError();
}

hipError_t launch_f32_combine(const float *y, const float *scores, int T, int k, int D,
                              const float *glogit, const float *shared, float *out,
                              hipStream_t stream) {
    const size_t n = (size_t)T * D;
    if (n == 0) return hipSuccess;
    f32_combine_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(y, scores, T, k, D, glogit,
                                                                       shared, out);
    return hipGetLastError();
}

}  // namespace mrun
