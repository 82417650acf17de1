// Router of the MoE block (moe.rs:151-159) and the stable expert permute (moe.rs:62-78):
//  - topk: one wave per token — f32 softmax, bf16 gates, k rounds of a wave-wide max over
//    (gate, id) keys, norm_topk;
//  - permute: per-block expert counts, an exclusive scan over experts and blocks, and a stable
//    rank inside each block from per-expert pair bitmaps (LDS atomicOr + popcount), so sorted rows
//    come out in (expert, pair) order: the stable argsort of the flat ids.
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
    if (wave == 0) {  // the wave totals' exclusive scan, lane w holding wave w
        constexpr int NWV = NT / 64;
        const uint32_t t = lane < NWV ? tmp[lane] : 0u;
        uint32_t s = t;
#pragma unroll
        for (int d = 1; d < NWV; d <<= 1) {
            const uint32_t o = (uint32_t)__shfl_up((int)s, d, 64);
            if (lane >= d) s += o;
        }
        if (lane < NWV) tmp[lane] = s - t;
        if (lane == NWV - 1) tmp[NWV] = s;
    }
    __syncthreads();
    uint32_t ex = tmp[wave] + inc - v;
    *total = tmp[NT / 64];
    __syncthreads();
    return ex;
}

// Counting blocks. Pairs are ranked inside fixed blocks of consecutive pair indices; a block's
// per-expert bitmap (E x BP/32 words) stays within 32 KiB of LDS. Blocks of at most 512 pairs
// keep many workgroups in the scatter and a pair's rank within 16 bitmap words.
__host__ __device__ inline int permute_block_pairs(int E) {
    int words = 8192 / (E > 0 ? E : 1);
    if (words > 16) words = 16;
    if (words < 1) words = 1;
    return 32 * words;
}

int route_block_tokens(int k, int E) {
    // a multiple of the top-k launch's tokens per workgroup, so none of its workgroups straddles
    // two blocks (k <= 16 and E <= 1024 give at least 16 tokens)
    const int bt = permute_block_pairs(E) / (4 * k) * 4;
    return bt > 0 ? bt : 4;
}

// counts[b][e] = number of pairs of block b (pairs [b BP, (b+1) BP)) routed to expert e. One
// workgroup per block; every count is written, so the array needs no clearing. Ids >= E are
// skipped.
__global__ __launch_bounds__(1024) void route_count_kernel(const uint32_t *__restrict__ ids, int P,
                                                           int E, int BP,
                                                           uint32_t *__restrict__ counts) {
    __shared__ uint32_t hist[1024];
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += 1024) hist[e] = 0;
    __syncthreads();
    const int p = blockIdx.x * BP + tid;
    if (tid < BP && p < P) {
        const uint32_t e = ids[p];
        if (e < (uint32_t)E) atomicAdd(&hist[e], 1u);
    }
    __syncthreads();
    for (int e = tid; e < E; e += 1024) counts[(size_t)blockIdx.x * E + e] = hist[e];
}

// The stable sort by expert (argsort of the flat ids, moe.rs:69-75). Workgroup b places the pairs
// of block b: a pair's sorted position is its expert's offset (exclusive scan of the totals over
// experts), plus the expert's pairs in blocks before b (the counts), plus the expert's pairs
// before it inside the block (popcounts of the block's bitmap of that expert). Positions follow
// pair order within every expert, so `order` is the stable argsort: the same result however the
// counts were accumulated. Workgroup 0 also writes the offsets, the active list and the tiles.
__global__ __launch_bounds__(1024) void route_scatter_kernel(const uint32_t *__restrict__ ids,
                                                             const uint32_t *__restrict__ counts,
                                                             int P, int k, int E, int BP, int nb,
                                                             PermuteOut o) {
    __shared__ uint32_t bm[8192];        // [E][W] pair bitmaps of this block
    __shared__ uint32_t part[2][1024];   // per (split, expert): pairs before this block, all pairs
    __shared__ uint32_t base[1024], tbase[1024], eoff[1024], ecnt[1024], tmp[32];
    const int tid = threadIdx.x, b = blockIdx.x;
    const int W = (BP + 31) / 32;
    // this block's ids are loaded first, then every block's counts, summed by ns threads per
    // expert in batches of 8 loads issued before any is added, so the kernel waits for about one
    // round trip instead of one per block
    const int p0 = b * BP;
    const int np = min(BP, P - p0);
    uint32_t my_e = tid < np ? ids[p0 + tid] : 0xffffffffu;
    for (int i = tid; i < E * W; i += 1024) bm[i] = 0;
    const int ns = E <= 1024 ? 1024 / E : 1;
    {
        const int e = tid % E, s = tid / E;
        if (s < ns) {
            uint32_t bef = 0, tot = 0;
            for (int bb0 = s; bb0 < nb; bb0 += 8 * ns) {
                uint32_t c[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int bb = bb0 + u * ns;
                    c[u] = counts[(size_t)min(bb, nb - 1) * E + e];
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int bb = bb0 + u * ns;
                    tot += bb < nb ? c[u] : 0u;
                    bef += bb < b ? c[u] : 0u;
                }
            }
            part[0][s * E + e] = bef;
            part[1][s * E + e] = tot;
        }
    }
    __syncthreads();  // bitmaps clear, partial sums in
    if (my_e < (uint32_t)E) atomicOr(&bm[my_e * W + (tid >> 5)], 1u << (tid & 31));
    uint32_t cnt = 0, bef = 0;
    if (tid < E)
        for (int s = 0; s < ns; ++s) cnt += part[1][s * E + tid], bef += part[0][s * E + tid];
    uint32_t total;
    const uint32_t ex = block_exclusive_scan<1024>(cnt, tmp, &total);  // (barriers inside)
    if (tid < E) base[tid] = ex + bef;
    // first tile of each expert (tiles of tile_m rows), for the tile row lists
    const uint32_t m = (uint32_t)o.tile_m;
    const uint32_t nt = m ? (cnt + m - 1) / m : 0u;
    uint32_t n_tiles = 0;
    const uint32_t b0 = block_exclusive_scan<1024>(nt, tmp, &n_tiles);
    if (tid < E) tbase[tid] = b0, eoff[tid] = ex, ecnt[tid] = cnt;
    __syncthreads();
    if (my_e < (uint32_t)E) {
        const uint32_t *row = bm + my_e * W;
        uint32_t r = __popc(row[tid >> 5] & ((1u << (tid & 31)) - 1u));
        for (int w = 0; w < (tid >> 5); ++w) r += __popc(row[w]);
        const uint32_t pos = base[my_e] + r;
        const uint32_t p = (uint32_t)(p0 + tid);
        if (o.order) o.order[pos] = p;
        if (o.inverse) o.inverse[p] = pos;
        if (o.token) o.token[pos] = p / (uint32_t)k;
        if (o.tile_rows) {  // the token of each tile row (rows past a partial tile's are not written)
            const uint32_t in_e = pos - eoff[my_e];
            o.tile_rows[(size_t)(tbase[my_e] + in_e / m) * m + in_e % m] = p / (uint32_t)k;
        }
    }
    if (b != 0) return;
    if (tid < E) o.offsets[tid] = ex;
    if (tid == 0) o.offsets[E] = total;
    if (o.active) {
        const uint32_t a = block_exclusive_scan<1024>(cnt > 0 ? 1u : 0u, tmp, &total);
        if (tid < E && cnt > 0) o.active[a] = (uint32_t)tid;
        if (tid == 0) *o.n_active = total;
    }
    if (o.tiles) {
        if (tid < E)
            for (uint32_t i = 0; i < nt; ++i) {
                uint32_t *t3 = o.tiles + 3 * (size_t)(b0 + i);
                t3[0] = (uint32_t)tid;
                t3[1] = ex + i * m;
                t3[2] = min(m, cnt - i * m);
            }
        if (tid == 0) *o.n_tiles = n_tiles;
    }
}

size_t permute_counts_words(int P, int E) {
    const int bp = permute_block_pairs(E);
    return (size_t)((P + bp - 1) / bp) * (size_t)E;
}

hipError_t launch_permute(const uint32_t *ids, int P, int k, int E, uint32_t *counts,
                          const PermuteOut &out, hipStream_t stream) {
    const int bp = permute_block_pairs(E);
    const int nb = (P + bp - 1) / bp;
    route_count_kernel<<<nb, 1024, 0, stream>>>(ids, P, E, bp, counts);
    route_scatter_kernel<<<nb, 1024, 0, stream>>>(ids, counts, P, k, E, bp, nb, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// softmax + top-k (+ fused permute for decode)

__global__ __launch_bounds__(256) void topk_kernel(const bf16_t *__restrict__ logits, int T, int E,
                                                   int k, int norm, bf16_t *__restrict__ gates,
                                                   uint32_t *__restrict__ ids,
                                                   bf16_t *__restrict__ scores) {
    const int t = blockIdx.x * (int)(blockDim.x >> 6) + (int)(threadIdx.x >> 6);
    if (t >= T) return;
    topk_token(logits + (size_t)t * E, E, k, norm != 0, gates ? gates + (size_t)t * E : nullptr,
               ids + (size_t)t * k, scores + (size_t)t * k);
}

hipError_t launch_topk(const bf16_t *logits, int T, int E, int k, bool norm, bf16_t *gates,
                       uint32_t *ids, bf16_t *scores, hipStream_t stream) {
    // one token (one wave) per workgroup, so the tokens spread over CUs (T = 16 58.07 -> 57.87 us
    // per block against four per workgroup)
    topk_kernel<<<T, 64, 0, stream>>>(logits, T, E, k, norm ? 1 : 0, gates, ids, scores);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// prefill routing: top-k + block counts, then the stable scatter

// Four tokens per workgroup (one wave each): softmax + top-k, then the workgroup's expert
// histogram added into its block's counts (counts [blocks][E], zero on entry; a block is bt
// tokens). Sums do not depend on the order the atomics arrive in, so the counts, and the scatter
// that reads them, are deterministic.
__global__ __launch_bounds__(256) void topk_count_kernel(const bf16_t *__restrict__ logits, int T,
                                                         int E, int k, int norm, int bt,
                                                         uint32_t *__restrict__ ids,
                                                         bf16_t *__restrict__ scores,
                                                         uint32_t *__restrict__ counts) {
    __shared__ uint32_t hist[512];
    const int wave = threadIdx.x >> 6;
    const int t0 = blockIdx.x * 4;
    for (int e = threadIdx.x; e < E; e += 256) hist[e] = 0;
    const int t = t0 + wave;
    if (t < T)
        topk_token(logits + (size_t)t * E, E, k, norm != 0, nullptr, ids + (size_t)t * k,
                   scores + (size_t)t * k);
    __syncthreads();  // ids of this workgroup are written (workgroup-visible) and hist is clear
    const int np = min(4, T - t0) * k;
    const size_t p0 = (size_t)t0 * k;
    if ((int)threadIdx.x < np) atomicAdd(&hist[ids[p0 + threadIdx.x]], 1u);
    __syncthreads();
    uint32_t *bc = counts + (size_t)(t0 / bt) * E;
    for (int e = threadIdx.x; e < E; e += 256)
        if (hist[e]) atomicAdd(&bc[e], hist[e]);
}

hipError_t launch_topk_count(const bf16_t *logits, int T, int E, int k, bool norm, uint32_t *ids,
                             bf16_t *scores, uint32_t *counts, hipStream_t stream) {
    topk_count_kernel<<<(T + 3) / 4, 256, 0, stream>>>(logits, T, E, k, norm ? 1 : 0,
                                                       route_block_tokens(k, E), ids, scores,
                                                       counts);
    return hipGetLastError();
}

hipError_t launch_route_scatter(const uint32_t *ids, const uint32_t *counts, int T, int k, int E,
                                const PermuteOut &out, hipStream_t stream) {
    const int bp = route_block_tokens(k, E) * k;
    const int P = T * k;
    const int nb = (P + bp - 1) / bp;
    route_scatter_kernel<<<nb, 1024, 0, stream>>>(ids, counts, P, k, E, bp, nb, out);
    return hipGetLastError();
}

}  // namespace mrun
