// Router of the MoE block (moe.rs:151-159) and the stable expert permute (moe.rs:62-78):
//  - router_gemv: bf16 logits for decode-sized token counts, one workgroup per expert row, the
//    row read once with 128-bit loads; the accumulation order of a token does not depend on T;
//  - topk: one wave per token — f32 softmax, bf16 gates, k rounds of a wave-wide max over
//    (gate, id) keys, norm_topk;
//  - permute: LDS-atomic histogram, block prefix sums, and a stable rank from per-expert token
//    bitmaps (LDS atomicOr + popcount), so sorted rows come out in (expert, token) order.
#include "common.hpp"
#include "kernels.hpp"

namespace mrun {

// ---------------------------------------------------------------------------------------------
// router logits (decode)

template <int MAXT>
__global__ __launch_bounds__(256) void router_gemv_kernel(const bf16_t *__restrict__ x, int T,
                                                          int D, const bf16_t *__restrict__ W,
                                                          const bf16_t *__restrict__ bias, int E,
                                                          bf16_t *__restrict__ logits,
                                                          const bf16_t *__restrict__ xw,
                                                          bf16_t *__restrict__ xout) {
    const int r = blockIdx.x;
    const bf16_t *wr = (r < E) ? W + (size_t)r * D : xw;
    float acc[MAXT];
#pragma unroll
    for (int t = 0; t < MAXT; ++t) acc[t] = 0.f;
    for (int c = threadIdx.x * 8; c < D; c += 256 * 8) {
        float wf[8];
        unpack8(*(const uint4 *)(wr + c), wf);
#pragma unroll
        for (int t = 0; t < MAXT; ++t) {
            if (t < T) {
                float xf[8];
                unpack8(*(const uint4 *)(x + (size_t)t * D + c), xf);
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[t] += xf[i] * wf[i];
            }
        }
    }
    __shared__ float red[4][MAXT];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int t = 0; t < MAXT; ++t) {
        if (t < T) {
            float v = group_sum<64>(acc[t]);
            if (lane == 0) red[wave][t] = v;
        }
    }
    __syncthreads();
    if ((int)threadIdx.x < T) {
        const int t = threadIdx.x;
        float v = ((red[0][t] + red[1][t]) + red[2][t]) + red[3][t];
        float l = rbf(v);
        if (r < E) {
            if (bias) l = rbf(l + bf2f(bias[r]));
            logits[(size_t)t * E + r] = (bf16_t)f2bf(l);
        } else {
            xout[t] = (bf16_t)f2bf(l);
        }
    }
}

hipError_t launch_router_gemv(const bf16_t *x, int T, int D, const bf16_t *W, const bf16_t *bias,
                              int E, bf16_t *logits, const bf16_t *xw, bf16_t *xout,
                              hipStream_t stream) {
    dim3 grid(E + (xw ? 1 : 0));
    if (T <= 4)
        router_gemv_kernel<4><<<grid, 256, 0, stream>>>(x, T, D, W, bias, E, logits, xw, xout);
    else
        router_gemv_kernel<16><<<grid, 256, 0, stream>>>(x, T, D, W, bias, E, logits, xw, xout);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// stable permute (block-wide)

// Exclusive scan of one value per thread over a block of NT threads; returns the prefix and
// writes the total to *total (every thread). tmp: NT/64 + 1 words of LDS.
template <int NT>
__device__ uint32_t block_exclusive_scan(uint32_t v, uint32_t *tmp, uint32_t *total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t inc = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        uint32_t o = (uint32_t)__shfl_up((int)inc, d, 64);
        if (lane >= d) inc += o;
    }
    if (lane == 63) tmp[wave] = inc;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t run = 0;
        for (int w = 0; w < NT / 64; ++w) {
            uint32_t t = tmp[w];
            tmp[w] = run;
            run += t;
        }
        tmp[NT / 64] = run;
    }
    __syncthreads();
    uint32_t ex = tmp[wave] + inc - v;
    *total = tmp[NT / 64];
    __syncthreads();
    return ex;
}

// Tokens ranked per pass (a multiple of 32): its bitmap and word prefixes, 2 * E * chunk/32
// words, stay within 48 KiB of LDS.
__host__ __device__ inline int permute_chunk(int T, int E) {
    int w = (T + 31) / 32;
    int wmax = 6144 / E;
    if (wmax < 1) wmax = 1;
    if (w > wmax) w = wmax;
    if (w > 32) w = 32;
    return 32 * w;
}

__host__ __device__ inline size_t permute_lds_bytes(int T, int E) {
    const int W = permute_chunk(T, E) / 32;
    return sizeof(uint32_t) * ((size_t)E * W /*bitmap*/ + (size_t)E * W /*word prefix*/ +
                               4 * (size_t)(E + 1) /*hist, off, run, rowtot*/ + 32 /*scan*/);
}

// Block of 1024 threads. ids [P = T*k] (values < E).
__device__ void permute_block(const uint32_t *__restrict__ ids, int P, int k, int E,
                              const PermuteOut &o, uint32_t *lds) {
    constexpr int NT = 1024;
    const int T = P / k;
    const int C = permute_chunk(T, E), W = C / 32;
    uint32_t *bm = lds;                       // [E][W]
    uint32_t *wp = bm + (size_t)E * W;        // [E][W]
    uint32_t *hist = wp + (size_t)E * W;      // [E+1]
    uint32_t *off = hist + (E + 1);           // [E+1]
    uint32_t *run = off + (E + 1);            // [E+1]
    uint32_t *rowtot = run + (E + 1);         // [E+1]
    uint32_t *tmp = rowtot + (E + 1);         // [32]
    const int tid = threadIdx.x;

    for (int e = tid; e < E; e += NT) hist[e] = 0, run[e] = 0;
    __syncthreads();
    for (int p = tid; p < P; p += NT) atomicAdd(&hist[ids[p]], 1u);
    __syncthreads();

    // offsets, active list, tiles (E <= 1024: one expert per thread)
    uint32_t cnt = tid < E ? hist[tid] : 0u, total;
    uint32_t ex = block_exclusive_scan<NT>(cnt, tmp, &total);
    if (tid < E) {
        off[tid] = ex;
        o.offsets[tid] = ex;
    }
    if (tid == 0) o.offsets[E] = total;
    if (o.active) {
        uint32_t a = block_exclusive_scan<NT>(cnt > 0 ? 1u : 0u, tmp, &total);
        if (tid < E && cnt > 0) o.active[a] = (uint32_t)tid;
        if (tid == 0) *o.n_active = total;
    }
    if (o.tiles) {
        const uint32_t m = (uint32_t)o.tile_m;
        uint32_t nt = (cnt + m - 1) / m;
        uint32_t base = block_exclusive_scan<NT>(nt, tmp, &total);
        if (tid < E) {
            for (uint32_t i = 0; i < nt; ++i) {
                uint32_t *t3 = o.tiles + 3 * (size_t)(base + i);
                t3[0] = (uint32_t)tid;
                t3[1] = ex + i * m;
                t3[2] = min(m, cnt - i * m);
            }
        }
        if (tid == 0) *o.n_tiles = total;
    }
    __syncthreads();

    // stable ranks: chunk by chunk of C tokens
    for (int c0 = 0; c0 < T; c0 += C) {
        const int c1 = min(T, c0 + C);
        for (int i = tid; i < E * W; i += NT) bm[i] = 0;
        __syncthreads();
        for (int p = c0 * k + tid; p < c1 * k; p += NT) {
            const int tl = p / k - c0;
            atomicOr(&bm[ids[p] * W + (tl >> 5)], 1u << (tl & 31));
        }
        __syncthreads();
        for (int e = tid; e < E; e += NT) {
            uint32_t acc = 0;
            for (int w = 0; w < W; ++w) {
                wp[e * W + w] = acc;
                acc += __popc(bm[e * W + w]);
            }
            rowtot[e] = acc;
        }
        __syncthreads();
        for (int p = c0 * k + tid; p < c1 * k; p += NT) {
            const uint32_t e = ids[p];
            const int tl = p / k - c0;
            const uint32_t word = bm[e * W + (tl >> 5)];
            const uint32_t pos = off[e] + run[e] + wp[e * W + (tl >> 5)] +
                                 __popc(word & ((1u << (tl & 31)) - 1u));
            if (o.order) o.order[pos] = (uint32_t)p;
            if (o.inverse) o.inverse[p] = pos;
            if (o.token) o.token[pos] = (uint32_t)(p / k);
        }
        __syncthreads();
        for (int e = tid; e < E; e += NT) run[e] += rowtot[e];
        __syncthreads();
    }
}

__global__ __launch_bounds__(1024) void permute_kernel(const uint32_t *__restrict__ ids, int P,
                                                       int k, int E, PermuteOut o) {
    extern __shared__ uint32_t lds[];
    permute_block(ids, P, k, E, o, lds);
}

hipError_t launch_permute(const uint32_t *ids, int P, int k, int E, const PermuteOut &out,
                          hipStream_t stream) {
    size_t lds = permute_lds_bytes(P / k, E);
    permute_kernel<<<1, 1024, lds, stream>>>(ids, P, k, E, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// softmax + top-k (+ fused permute for decode)

constexpr int kMaxExpertsPerLane = 8;  // E <= 512
constexpr int kMaxTopK = 16;

__device__ void topk_token(const bf16_t *__restrict__ lrow, int E, int k, bool norm,
                           bf16_t *__restrict__ grow, uint32_t *__restrict__ idrow,
                           bf16_t *__restrict__ srow) {
    const int lane = threadIdx.x & 63;
    float lv[kMaxExpertsPerLane];
    uint32_t key[kMaxExpertsPerLane];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < kMaxExpertsPerLane; ++i) {
        const int e = lane + 64 * i;
        lv[i] = e < E ? bf2f(lrow[e]) : -INFINITY;
        m = fmaxf(m, lv[i]);
    }
    m = wave_max(m);
    float s = 0.f, ex[kMaxExpertsPerLane];
#pragma unroll
    for (int i = 0; i < kMaxExpertsPerLane; ++i) {
        const int e = lane + 64 * i;
        ex[i] = e < E ? expf(lv[i] - m) : 0.f;
        s += ex[i];
    }
    s = group_sum<64>(s);
#pragma unroll
    for (int i = 0; i < kMaxExpertsPerLane; ++i) {
        const int e = lane + 64 * i;
        if (e < E) {
            const uint32_t g = f2bf(ex[i] / s);
            if (grow) grow[e] = (bf16_t)g;
            key[i] = (g << 16) | (uint32_t)(0xffff - e);
        } else {
            key[i] = 0;
        }
    }
    float gsel[kMaxTopK];
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j) {
        if (j < k) {
            uint32_t best = 0;
#pragma unroll
            for (int i = 0; i < kMaxExpertsPerLane; ++i) best = key[i] > best ? key[i] : best;
            best = wave_max_u32(best);
#pragma unroll
            for (int i = 0; i < kMaxExpertsPerLane; ++i)
                if (key[i] == best) key[i] = 0;
            gsel[j] = bf2f(best >> 16);
            if (lane == 0) idrow[j] = 0xffffu - (best & 0xffffu);
        }
    }
    if (lane == 0) {
        float sum = 0.f;
        if (norm) {
#pragma unroll
            for (int j = 0; j < kMaxTopK; ++j)
                if (j < k) sum += gsel[j];
            sum = rbf(sum);
        }
#pragma unroll
        for (int j = 0; j < kMaxTopK; ++j)
            if (j < k) srow[j] = (bf16_t)f2bf(norm ? gsel[j] / sum : gsel[j]);
    }
}

__global__ __launch_bounds__(256) void topk_kernel(const bf16_t *__restrict__ logits, int T, int E,
                                                   int k, int norm, bf16_t *__restrict__ gates,
                                                   uint32_t *__restrict__ ids,
                                                   bf16_t *__restrict__ scores) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;
    topk_token(logits + (size_t)t * E, E, k, norm != 0, gates ? gates + (size_t)t * E : nullptr,
               ids + (size_t)t * k, scores + (size_t)t * k);
}

// Decode: one block of 1024 threads; wave w handles tokens w, w+16, ...; then the permute.
__global__ __launch_bounds__(1024) void topk_permute_kernel(const bf16_t *__restrict__ logits,
                                                            int T, int E, int k, int norm,
                                                            bf16_t *__restrict__ gates,
                                                            uint32_t *__restrict__ ids,
                                                            bf16_t *__restrict__ scores,
                                                            PermuteOut o) {
    extern __shared__ uint32_t lds[];
    for (int t = threadIdx.x >> 6; t < T; t += 16)
        topk_token(logits + (size_t)t * E, E, k, norm != 0,
                   gates ? gates + (size_t)t * E : nullptr, ids + (size_t)t * k,
                   scores + (size_t)t * k);
    __threadfence_block();
    __syncthreads();
    permute_block(ids, T * k, k, E, o, lds);
}

hipError_t launch_topk(const bf16_t *logits, int T, int E, int k, bool norm, bf16_t *gates,
                       uint32_t *ids, bf16_t *scores, const PermuteOut *fused,
                       hipStream_t stream) {
    if (fused) {
        size_t lds = permute_lds_bytes(T, E);
        topk_permute_kernel<<<1, 1024, lds, stream>>>(logits, T, E, k, norm ? 1 : 0, gates, ids,
                                                      scores, *fused);
    } else {
        topk_kernel<<<(T + 3) / 4, 256, 0, stream>>>(logits, T, E, k, norm ? 1 : 0, gates, ids,
                                                     scores);
    }
    return hipGetLastError();
}

}  // namespace mrun
