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

// ---- router ----

// logits[t][r] = R(x[t] . W[r]) then, with bias, R(logit + bias[r]) for r < E, t < T <= 16.
// With xw (one extra weight row [D]) the extra block writes xout[t] = R(x[t] . xw).
hipError_t launch_router_gemv(const bf16_t *x, int T, int D, const bf16_t *W, const bf16_t *bias,
                              int E, bf16_t *logits, const bf16_t *xw, bf16_t *xout,
                              hipStream_t stream);

// Softmax (f32, one rounding), top-k (equal gates: lower id first; ids in rank order) and
// scores (normalised when norm) for T tokens; gates optional. With permute outputs given
// (decode: T*k <= 1024), the same launch also runs the stable permute.
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
};
hipError_t launch_topk(const bf16_t *logits, int T, int E, int k, bool norm, bf16_t *gates,
                       uint32_t *ids, bf16_t *scores, const PermuteOut *fused_permute,
                       hipStream_t stream);

// Stable counting sort of ids [P] (values < E) by expert (one workgroup).
hipError_t launch_permute(const uint32_t *ids, int P, int k, int E, const PermuteOut &out,
                          hipStream_t stream);

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

// Decode down projection fused with the combine (moe.rs:84-93, 161-171): for each output row d,
// every active expert's pairs (act rows at sorted positions) and the shared expert's rows, then
// out[t][d] = R(R(sum_j R(y[inverse[t*k+j]][d] * scores[t][j])) + R(R(sigmoid(sh_logit[t])) *
// ysh[t][d])). T*k <= 128.
struct DownCombineJob {
    const bf16_t *act;   // [P, I] sorted positions
    QW wd;               // [E, D, I]
    Routing routing;
    int max_slots;
    const uint32_t *inverse;
    const bf16_t *scores;
    int T, k;
    int has_shared;
    const bf16_t *sh_act; // [T, I_s]
    QW swd;               // [1, D, I_s]
    const bf16_t *sh_logit;
    bf16_t *out;          // [T, D]
};
hipError_t launch_down_combine(const DownCombineJob &job, hipStream_t stream);

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
};
hipError_t launch_gemm(const GemmJob &job, hipStream_t stream);
constexpr int kGemmTileM = 64;
constexpr int kGemmTileN = 64;

// ---- elementwise ----

hipError_t launch_swiglu(const bf16_t *g, const bf16_t *u, int64_t n, bf16_t *out,
                         hipStream_t stream);
hipError_t launch_combine(const bf16_t *y, const uint32_t *inverse, const bf16_t *scores, int T,
                          int k, int D, const bf16_t *sh_y, const bf16_t *sh_logit, bf16_t *out,
                          hipStream_t stream);
hipError_t launch_rms_norm(const bf16_t *x, const bf16_t *res, const bf16_t *w, int rows, int D,
                           float eps, bf16_t *h, bf16_t *y, hipStream_t stream);
hipError_t launch_rowdot(const bf16_t *x, int T, int D, const bf16_t *W, int N,
                         const bf16_t *bias, bf16_t *y, hipStream_t stream);
hipError_t launch_add_bias(bf16_t *y, const bf16_t *bias, int rows, int n, hipStream_t stream);

}  // namespace mrun
