// Internal launch interface between the host layer (moe.cpp) and the HIP kernels.
// Every launcher enqueues on `stream` and returns hipGetLastError() of its launches.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint16_t bf16_t;

namespace mrun {

// One affine-quantized stacked weight on the device: codes [experts, out, in*bits/32] (LSB-first),
// scales/biases [experts, out, in/group] bf16 (biases may be null = zeros).
struct QW {
    const uint32_t *codes;
    const bf16_t *scales;
    const bf16_t *biases;
    int experts, out, in, group, bits;
};

// Routing state produced by the permute: expert e's rows sit at sorted positions
// [offsets[e], offsets[e+1]); active[0..*n_active) lists the experts with rows, ascending;
// tiles[3*i .. 3*i+2] = (expert, first position, rows <= tile_m) for i < *n_tiles.
struct Routing {
    const uint32_t *offsets;
    const uint32_t *active;
    const uint32_t *n_active;
    const uint32_t *tiles;
    const uint32_t *n_tiles;
};

// Benchmark instrumentation: an event recorded on the stream after each stage of a forward.
struct StageMarks {
    hipEvent_t *events = nullptr;
    int n_events = 0;
    int count = 0;
    // optional: 64 (start, end) pairs; the decode gate/up kernel lowers start to its workgroups'
    // starts and raises end to their waves' ends (workgroup i in pair i % 64), in ticks of the
    // device wall clock (s_memrealtime)
    unsigned long long *k2_clock = nullptr;
    void mark(hipStream_t s) {
        if (events && count + 1 < n_events) (void)hipEventRecord(events[count + 1], s);
        ++count;
    }
};

// ---- router ----

// Dense Linear for T <= 16 rows: out[t][r] = R(x[t] . W[r]) then, with bias, R(. + bias[r]); one
// wave per output row, a token's accumulation order independent of T.
hipError_t launch_rows(const bf16_t *x, int T, int D, const bf16_t *W, const bf16_t *bias, int N,
                       bf16_t *out, hipStream_t stream);

// Softmax (f32, one rounding), top-k (equal gates: lower id first; ids in rank order) and
// scores (normalised when norm) for T tokens; gates optional.
struct PermuteOut {
    uint32_t *offsets;   // [E+1]
    uint32_t *order;     // [P] or null
    uint32_t *inverse;   // [P] or null
    uint32_t *token;     // [P] or null
    uint32_t *active;    // [E] or null
    uint32_t *n_active;  // [1] or null
    uint32_t *tiles;     // [3 * max_tiles] or null
    uint32_t *n_tiles;   // [1] or null
    int tile_m;          // rows per tile
    uint32_t *tile_rows; // [max tiles][tile_m] token (pair / k) of each tile row, or null; the
                         // entries past a partial tile's rows are left unwritten
};
hipError_t launch_topk(const bf16_t *logits, int T, int E, int k, bool norm, bf16_t *gates,
                       uint32_t *ids, bf16_t *scores, hipStream_t stream);

// The stable sort of ids [P] (values < E) by expert: order = argsort(ids) (stable), inverse,
// token = order / k, offsets, and the active list and tiles when asked for (moe.rs:69-75). Two
// launches: per-block expert counts into counts [permute_counts_words(P, E)], then the scatter.
size_t permute_counts_words(int P, int E);
hipError_t launch_permute(const uint32_t *ids, int P, int k, int E, uint32_t *counts,
                          const PermuteOut &out, hipStream_t stream);

// The forward's prefill routing in two launches: softmax + top-k of four tokens per workgroup,
// whose expert histograms are added into counts [ceil(T / bt)][E] (zero on entry; bt =
// route_block_tokens(k, E) tokens per block), then the same stable scatter as launch_permute.
// Atomics only ever sum counts, so every output is deterministic and equals the stable argsort.
int route_block_tokens(int k, int E);
hipError_t launch_topk_count(const bf16_t *logits, int T, int E, int k, bool norm, uint32_t *ids,
                             bf16_t *scores, uint32_t *counts, hipStream_t stream);
hipError_t launch_route_scatter(const uint32_t *ids, const uint32_t *counts, int T, int k, int E,
                                const PermuteOut &out, hipStream_t stream);

// ---- products ----

// Decode-shaped gathered product (GEMV; every row's accumulation order is independent of how
// many rows there are). Routed slots: slot s < max_slots serves expert active[s] over its sorted
// positions (routing given) or, without routing, expert 0 over positions [0, rows). Position pos
// reads A row (a_map ? a_map[pos] / a_div : pos) and writes output row (o_map ? o_map[pos] : pos).
// glu: out = R(silu(R(A.w0)) * R(A.w1)); else out = R(A.w0).
// Extra slots (shared expert): x_rows rows of xA through expert 0 of xw0 (and xw1), into xout.
struct GemvJob {
    const bf16_t *A;
    int lda;
    const uint32_t *a_map;
    int a_div;
    QW w0, w1;
    Routing routing;
    int has_routing;
    int max_slots;
    int rows;
    const uint32_t *o_map;
    bf16_t *out;
    int ldo;
    int glu;
    // extra slots
    const bf16_t *xA;
    int x_lda;
    QW xw0, xw1;
    int x_rows;
    bf16_t *xout;
    int x_ldo;
};
hipError_t launch_gemv(const GemvJob &job, hipStream_t stream);

// The decode schedule (decode.hip): router + shared expert gate/up, routed gate/up, down +
// combine, for T <= 32 tokens and T*k <= 256 pairs.
struct DecodeJob {
    const bf16_t *x;
    int T, D, E, k, I, S, norm, max_slots;
    const bf16_t *router, *router_bias, *sh_gate_w, *sh_gate_b;
    // a quantized router or shared gate (4 or 8 bits; router null / sh_gate_w null): K1 dequantizes
    // its rows itself (mlx-community conversions store both in 8 bits)
    QW router_q, sh_gate_q;
    QW wg, wu, wd, sg, su, sd;
    bf16_t *logits;   // [T, E]
    uint32_t *ids;    // [T, k] and
    bf16_t *scores;   // [T, k]: the routing, computed once by a top-k launch when T > 4
    int topk_in_kernel;  // T <= 4: each workgroup re-derives the top-k from the logits instead
    int router_done;     // logits and sh_logit already computed (quantized router or gate)
    int gu_loop;         // row blocks per K2 workgroup (set by the launcher)
    int down_tokens;     // tokens per K3 workgroup (set by the launcher)
    bf16_t *sh_logit; // [T]
    bf16_t *sh_act;   // [T, S]
    bf16_t *act;      // [T*k, I], pair p = t*k + j
    bf16_t *out;      // [T, D]
    // Decoder-layer fusion (the layer stack): with norm_src set, K1 forms the block input
    // x = R(R(norm_src * rsqrt(mean(norm_src^2) + eps)) * norm_w) itself into LDS (norm_w null:
    // weight 1; 2*T*D bytes <= 64 KiB) and its workgroup 0 writes it to `x` for K2; with residual
    // set, K3 writes
    // out = R(residual + block output) (out may alias residual).
    const bf16_t *norm_src, *norm_w, *residual;
    float eps;
    unsigned long long *clock;  // benchmark instrumentation (StageMarks::k2_clock), or null
};
bool decode_supported(int D, int I, int S, int T, int k, int E);
bool decode_supported_bits(int D, int I, int S, int bits);
hipError_t launch_decode(const DecodeJob &job, hipStream_t stream, StageMarks *marks);

// MFMA bf16 grouped GEMM (prefill): rows at sorted positions grouped in tiles (routing.tiles) or,
// without routing, M rows of expert 0. B is quantized (w0, and w1 with glu) or dense bf16 bd
// [N, K]. Epilogue: glu -> R(silu(R(.w0)) * R(.w1)); else R(.), then with bias R(. + bias[n]).
struct GemmJob {
    const bf16_t *A;
    int lda;
    const uint32_t *a_map;
    int a_div;
    int M;
    int N, K;
    QW w0, w1;
    const bf16_t *bd;
    const bf16_t *bias;
    Routing routing;
    int has_routing;
    int max_tiles;
    const uint32_t *o_map;
    bf16_t *out;
    int ldo;
    int glu;
    uint32_t *zero;  // block (0, 0) clears zero[0..n_zero) (routing counters of the next launch)
    int n_zero;
    // a non-routed product with the same N run in the same launch (the shared expert)
    struct {
        const bf16_t *A;
        int lda, M, K;
        QW w0, w1;
        bf16_t *out;
        int ldo;
    } sh;
    int has_shared;
};
hipError_t launch_gemm(const GemmJob &job, hipStream_t stream);
// whether launch_gemm runs the tuned kernel (4-bit, group 64), which also takes `sh`
bool qgemm_supported(const GemmJob &job);
constexpr int kGemmTileM = 64;  // rows per routed tile

constexpr int kGemmTileN = 64;

// The prefill forward's grouped expert GEMM (moe_gemm.hip): 4-bit group-64 weights (biases may be
// null), K % 512 == 0, N a multiple of 128 (glu) or 256. A is packed (launch_apack) with its X
// splits AX [rows][3][ax_e] (ax_e = K / 64: one entry per group).
// Routed tiles come from routing.tiles (64 rows); their A rows from tile_rows [tile][64] (token
// of each tile row; only the tile's rows are read, rows past them repeat its last one) or,
// without tile_rows, the sorted positions themselves. glu: out = packed R(silu(R(A.w0)) * R(A.w1)) and OX [rows][3][N / 64]
// the X splits of each output row's groups; else out = R(A.w0). The shared product (sh)
// has the same K and N and comes first.
struct MoeGemmJob {
    const bf16_t *A;
    int lda;
    int a_rows;  // rows of A (its byte offsets are 32-bit: a_rows * lda * 2 < 2^32)
    const bf16_t *AX;
    int ax_e;
    const uint32_t *tile_rows;
    int K, N, glu;
    QW w0, w1;
    Routing routing;
    int has_routing, max_tiles;
    int tile_m;  // rows per tile: 64, or 32 (the routed tiles cut to 32 rows by the permute)
    int M;
    bf16_t *out;
    int ldo;
    bf16_t *OX;
    struct {
        const bf16_t *A;
        int lda;
        const bf16_t *AX;
        int ax_e;
        int M;
        QW w0, w1;
        bf16_t *out;
        int ldo;
        bf16_t *OX;
    } sh;
    int has_shared;
};
bool moe_gemm_supported(const MoeGemmJob &j);
hipError_t launch_moe_gemm(const MoeGemmJob &j, hipStream_t stream);
// x [rows][K] (row stride lda) -> packed rows (stride ldp) and X splits [rows][3][K / 64]
hipError_t launch_apack(const bf16_t *x, int lda, int rows, int K, bf16_t *xp, int ldp,
                        bf16_t *xs, hipStream_t stream);

// Dense bf16 Linear for more than 16 rows on the MFMAs (dense.hip): out0 = R(A W0^T) then
// R(. + bias0), and optionally out1 from W1 in the same launch (the shared expert's gate beside the
// router). K % 64 == 0. Workgroup (0, 0) clears zero[0..n_zero) first.
struct DenseJob {
    const bf16_t *A;
    int lda, M, K;
    const bf16_t *W0, *bias0;
    int N0;
    bf16_t *out0;
    int ldo0;
    const bf16_t *W1, *bias1;  // W1 null: none
    int N1;
    bf16_t *out1;
    int ldo1;
    uint32_t *zero;
    int n_zero;
    // optional: A packed for the grouped GEMM (launch_apack's layout and bits: pack_a [M][K],
    // pack_x [M][3][K / 64]) by extra workgroups of the same launch
    bf16_t *pack_a, *pack_x;
};
bool dense_gemm_supported(int M, int K);
hipError_t launch_dense_gemm(const DenseJob &job, hipStream_t stream);

// ---- elementwise ----

hipError_t launch_swiglu(const bf16_t *g, const bf16_t *u, int64_t n, bf16_t *out,
                         hipStream_t stream);
// The layer stack's step after a block (rows of at most 2048): resid = R(resid + block output),
// then the next layer's input h = R(R(resid * rsqrt(mean(resid^2) + eps)) * w) (w null: ones),
// with the bits of launch_rms_norm(resid, block output, w, ...).
struct PostNorm {
    bf16_t *resid;
    const bf16_t *w;
    float eps;
    bf16_t *h;
};
// post: the combine also takes that step for its rows (then `out` is not written).
hipError_t launch_combine(const bf16_t *y, const uint32_t *inverse, const bf16_t *scores, int T,
                          int k, int D, const bf16_t *sh_y, const bf16_t *sh_logit, bf16_t *out,
                          hipStream_t stream, const PostNorm *post = nullptr);
hipError_t launch_rms_norm(const bf16_t *x, const bf16_t *res, const bf16_t *w, int rows, int D,
                           float eps, bf16_t *h, bf16_t *y, hipStream_t stream);
hipError_t launch_rowdot(const bf16_t *x, int T, int D, const bf16_t *W, int N,
                         const bf16_t *bias, bf16_t *y, hipStream_t stream);
hipError_t launch_add_bias(bf16_t *y, const bf16_t *bias, int rows, int n, hipStream_t stream);
// dst[0..n) = v (a kernel, not a memset node, so that captured graphs replay it faithfully)
hipError_t launch_fill_u32(uint32_t *dst, uint32_t v, int n, hipStream_t stream);
// dst[r] = src[map[r]], r < rows, rows of `width` bf16 (width % 8 == 0; 16-byte aligned rows)
hipError_t launch_rows_gather(const bf16_t *src, const uint32_t *map, int rows, int width,
                              bf16_t *dst, hipStream_t stream);

// ---- float32 blocks (f32.hip): every op in f32, nothing rounded to bf16 ----

// out[r][n] = A[r / a_div] . W0[e_r][n] (e_r = ids ? ids[r] : 0), r < R, n < N, over K (a multiple
// of 4, 16-byte aligned rows); with glu, silu(A . W0[e_r][n]) * (A . W1[e_r][n]). W [experts][N][K].
struct F32Rows {
    const float *A;
    int a_div, K;
    const float *W0, *W1;
    const uint32_t *ids;
    int R, N;
    float *out;
};
hipError_t launch_f32_rows(const F32Rows &j, bool glu, hipStream_t stream);
// softmax (f32) and top-k of T tokens (E <= 512; equal gates: lower id first; rank order); scores
// are the gates, divided by their sum (in rank order) with norm
hipError_t launch_f32_topk(const float *logits, int T, int E, int k, bool norm, uint32_t *ids,
                           float *scores, hipStream_t stream);
// out = sum_j y[t k + j] * scores[t k + j] (+ sigmoid(glogit[t]) * shared[t] when shared is set)
hipError_t launch_f32_combine(const float *y, const float *scores, int T, int k, int D,
                              const float *glogit, const float *shared, float *out,
                              hipStream_t stream);

}  // namespace mrun
