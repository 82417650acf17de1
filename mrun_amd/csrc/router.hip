// Router of the MoE block (moe.rs:151-159) and the stable expert permute (moe.rs:62-78):
//  - topk: one wave per token — f32 softmax, bf16 gates, k rounds of a wave-wide max over
//    (gate, id) keys, norm_topk;
//  - permute: LDS-atomic histogram, block prefix sums, and a stable rank from per-expert token
//    bitmaps (LDS atomicOr + popcount), so sorted rows come out in (expert, token) order.
#include "common.hpp"
#include "kernels.hpp"
#include "topk.hpp"

namespace mrun {

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

__global__ __launch_bounds__(256) void topk_kernel(const bf16_t *__restrict__ logits, int T, int E,
                                                   int k, int norm, bf16_t *__restrict__ gates,
                                                   uint32_t *__restrict__ ids,
                                                   bf16_t *__restrict__ scores) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;
    topk_token(logits + (size_t)t * E, E, k, norm != 0, gates ? gates + (size_t)t * E : nullptr,
               ids + (size_t)t * k, scores + (size_t)t * k);
}

hipError_t launch_topk(const bf16_t *logits, int T, int E, int k, bool norm, bf16_t *gates,
                       uint32_t *ids, bf16_t *scores, hipStream_t stream) {
    topk_kernel<<<(T + 3) / 4, 256, 0, stream>>>(logits, T, E, k, norm ? 1 : 0, gates, ids, scores);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// prefill routing: top-k + ranks, then scatter

constexpr int kRankTokensPerWave = 1;

__global__ __launch_bounds__(256) void topk_rank_kernel(const bf16_t *__restrict__ logits, int T,
                                                        int E, int k, int norm,
                                                        uint32_t *__restrict__ ids,
                                                        bf16_t *__restrict__ scores,
                                                        uint32_t *__restrict__ counts,
                                                        uint32_t *__restrict__ rank) {
    constexpr int TPB = 4 * kRankTokensPerWave;
    __shared__ uint32_t hist[512], base[512], lr[TPB * kMaxTopK];
    const int wave = threadIdx.x >> 6;
    const int t0 = blockIdx.x * TPB;
    for (int e = threadIdx.x; e < E; e += 256) hist[e] = 0;
    for (int i = 0; i < kRankTokensPerWave; ++i) {
        const int t = t0 + wave * kRankTokensPerWave + i;
        if (t < T)
            topk_token(logits + (size_t)t * E, E, k, norm != 0, nullptr, ids + (size_t)t * k,
                       scores + (size_t)t * k);
    }
    __syncthreads();  // ids of this block are written (block-visible) and hist is clear
    const int np = min(TPB, T - t0) * k;
    const size_t p0 = (size_t)t0 * k;
    if ((int)threadIdx.x < np) lr[threadIdx.x] = atomicAdd(&hist[ids[p0 + threadIdx.x]], 1u);
    __syncthreads();
    uint32_t *slot_counts = counts + (size_t)(blockIdx.x % kRankSlots) * E;
    for (int e = threadIdx.x; e < E; e += 256)
        if (hist[e]) base[e] = atomicAdd(&slot_counts[e], hist[e]);
    __syncthreads();
    if ((int)threadIdx.x < np) rank[p0 + threadIdx.x] = base[ids[p0 + threadIdx.x]] + lr[threadIdx.x];
}

hipError_t launch_topk_rank(const bf16_t *logits, int T, int E, int k, bool norm, uint32_t *ids,
                            bf16_t *scores, uint32_t *counts, uint32_t *rank,
                            hipStream_t stream) {
    const int tpb = 4 * kRankTokensPerWave;
    topk_rank_kernel<<<(T + tpb - 1) / tpb, 256, 0, stream>>>(logits, T, E, k, norm ? 1 : 0, ids,
                                                               scores, counts, rank);
    return hipGetLastError();
}

// Every block scans the E counts (kRankSlots x E words) itself; block 0 also writes offsets, the
// active list and the tile list.
__global__ __launch_bounds__(1024) void scatter_kernel(const uint32_t *__restrict__ ids,
                                                       const uint32_t *__restrict__ rank,
                                                       const uint32_t *__restrict__ counts, int P,
                                                       int k, int E, PermuteOut o) {
    __shared__ uint32_t off[kRankSlots][1025], tmp[32];
    const int tid = threadIdx.x;
    // expert e's slot ranges follow each other in slot order
    uint32_t cnt = 0;
    if (tid < E) {
#pragma unroll
        for (int sl = 0; sl < kRankSlots; ++sl) {
            off[sl][tid] = cnt;
            cnt += counts[(size_t)sl * E + tid];
        }
    }
    uint32_t total;
    const uint32_t ex = block_exclusive_scan<1024>(cnt, tmp, &total);
    if (tid < E) {
#pragma unroll
        for (int sl = 0; sl < kRankSlots; ++sl) off[sl][tid] += ex;
    }
    __syncthreads();
    const int p = blockIdx.x * 1024 + tid;
    if (p < P) {
        // pair p came from top-k workgroup p / (4 k): slot (p / (4 k)) % kRankSlots
        const int sl = (p / (4 * kRankTokensPerWave * k)) % kRankSlots;
        const uint32_t pos = off[sl][ids[p]] + rank[p];
        if (o.order) o.order[pos] = (uint32_t)p;
        if (o.inverse) o.inverse[p] = pos;
        if (o.token) o.token[pos] = (uint32_t)(p / k);
    }
    if (blockIdx.x != 0) return;
    if (tid < E) o.offsets[tid] = ex;
    if (tid == 0) o.offsets[E] = total;
    if (o.active) {
        uint32_t a = block_exclusive_scan<1024>(cnt > 0 ? 1u : 0u, tmp, &total);
        if (tid < E && cnt > 0) o.active[a] = (uint32_t)tid;
        if (tid == 0) *o.n_active = total;
    }
    if (o.tiles) {
        const uint32_t m = (uint32_t)o.tile_m;
        const uint32_t nt = (cnt + m - 1) / m;
        const uint32_t b0 = block_exclusive_scan<1024>(nt, tmp, &total);
        if (tid < E)
            for (uint32_t i = 0; i < nt; ++i) {
                uint32_t *t3 = o.tiles + 3 * (size_t)(b0 + i);
                t3[0] = (uint32_t)tid;
                t3[1] = ex + i * m;
                t3[2] = min(m, cnt - i * m);
            }
        if (tid == 0) *o.n_tiles = total;
    }
}

hipError_t launch_scatter(const uint32_t *ids, const uint32_t *rank, const uint32_t *counts,
                          int P, int k, int E, const PermuteOut &out, hipStream_t stream) {
    scatter_kernel<<<(P + 1023) / 1024, 1024, 0, stream>>>(ids, rank, counts, P, k, E, out);
    return hipGetLastError();
}

}  // namespace mrun
