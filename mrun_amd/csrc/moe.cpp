// Host layer of the MoE block: the C++ counterpart of the reference's operator surface and
// layers, and the C ABI of include/mrun_moe.h over it.
//
//   mrun::tensor   — the facade ops the MoE path uses (crates/mrun-engine/src/tensor/nuvec.rs):
//                    gather_qmm, quantized_matmul, linear, softmax/top-k (router), argsort-based
//                    permute, swiglu, combine, rms_norm; each returns a Status carrying the
//                    message, as the facade returns Result<_, Error(String)>.
//   mrun::models   — SparseMoe::forward (models/moe.rs:149-174) composed from those ops, with the
//                    decode (GEMV) or prefill (MFMA) schedule chosen from the token count.
//
// Nothing here allocates device memory: scratch comes from the caller's workspace.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <mutex>
#include <string>

#include "kernels.hpp"
#include "mrun_moe.h"
#include "status.hpp"

namespace mrun {

// ---------------------------------------------------------------------------------------------
// the thread's last error (status.hpp)

static thread_local std::string g_last_error;

int report(const Status &s) {
    g_last_error = s.ok() ? std::string() : s.msg;
    return s.code;
}

static bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

static QW qw_of(const mrun_quantized &q) {
    return QW{q.weight, q.scales, q.biases, q.experts, q.out, q.in, q.group_size, q.bits};
}

// ---------------------------------------------------------------------------------------------
// validation: Quantized::new / QParams::checked / infer (nuvec.rs:609-626, load.rs:14-42, 131-156)

static Status check_quantized(const mrun_quantized *q, const std::string &path, int experts,
                              int out, int in) {
    if (q && q->bits == 32)
        return Err(MRUN_ERR_UNSUPPORTED,
                   path + ": f32 weights (bits 32) run through mrun_moe_forward_f32, whose block "
                          "is f32 throughout");
    if (q && q->bits == 16) {  // dense bf16 experts (SwitchLinear::Dense, moe.rs:43-46)
        if (!q->weight) return Err(MRUN_ERR_INVALID, path + ": missing tensors");
        if (q->scales || q->biases)
            return Err(MRUN_ERR_INVALID, path + ": dense (16-bit) weights carry no scales or biases");
        if (q->experts != experts || q->out != out || q->in != in)
            return Err(MRUN_ERR_INVALID, path + ": shape [" + std::to_string(q->experts) + ", " +
                                             std::to_string(q->out) + ", " + std::to_string(q->in) +
                                             "], expected [" + std::to_string(experts) + ", " +
                                             std::to_string(out) + ", " + std::to_string(in) + "]");
        if (in % 8 != 0 || in > 4096)
            return Err(MRUN_ERR_UNSUPPORTED,
                       path + ": dense experts need an input width that is a multiple of 8, at "
                              "most 4096");
        if (!aligned16(q->weight)) return Err(MRUN_ERR_INVALID, path + ": weights must be 16-byte aligned");
        return Ok();
    }
    if (!q || !q->weight || !q->scales) return Err(MRUN_ERR_INVALID, path + ": missing tensors");
    if (q->experts != experts || q->out != out || q->in != in)
        return Err(MRUN_ERR_INVALID,
                   path + ": shape [" + std::to_string(q->experts) + ", " +
                       std::to_string(q->out) + ", " + std::to_string(q->in) + "], expected [" +
                       std::to_string(experts) + ", " + std::to_string(out) + ", " +
                       std::to_string(in) + "]");
    const bool bits_ok = q->bits == 4 || q->bits == 8;
    const bool group_ok = q->group_size == 32 || q->group_size == 64 || q->group_size == 128;
    if (!bits_ok || !group_ok)
        return Err(MRUN_ERR_INVALID, path + ": bits = " + std::to_string(q->bits) +
                                         ", group_size = " + std::to_string(q->group_size) +
                                         "; a quantized weight has 4 or 8 bits and groups of "
                                         "32, 64 or 128 (16 bits: dense bf16)");
    if (q->in % q->group_size != 0)
        return Err(MRUN_ERR_INVALID, path + ": input width " + std::to_string(q->in) +
                                         " is not a multiple of group_size " +
                                         std::to_string(q->group_size));
    if (q->in % (128 / q->bits) != 0)
        return Err(MRUN_ERR_UNSUPPORTED, path + ": input width " + std::to_string(q->in) +
                                             " must be a multiple of " +
                                             std::to_string(128 / q->bits));
    if (!aligned16(q->weight)) return Err(MRUN_ERR_INVALID, path + ": codes must be 16-byte aligned");
    return Ok();
}

static bool same_quant(const mrun_quantized &a, const mrun_quantized &b) {
    return a.bits == b.bits && (a.bits == 16 || a.group_size == b.group_size);
}

// A Linear's weight as a stacked weight of one expert: quantized as is, dense bf16 as bits 16.
static mrun_quantized as_quantized(const mrun_linear &l) {
    if (!l.weight) return l.q;
    mrun_quantized q{};
    q.weight = (const uint32_t *)l.weight, q.experts = 1, q.out = l.out, q.in = l.in, q.bits = 16;
    return q;
}

static Status check_ptr(const void *p, const char *what) {
    if (!p) return Err(MRUN_ERR_INVALID, std::string(what) + " is null");
    if (!aligned16(p)) return Err(MRUN_ERR_INVALID, std::string(what) + " must be 16-byte aligned");
    return Ok();
}

static Status check_config(const mrun_moe_config &c) {
    if (c.hidden <= 0 || c.experts <= 0 || c.intermediate <= 0)
        return Err(MRUN_ERR_INVALID, "config: hidden, experts and intermediate must be positive");
    if (c.top_k < 1 || c.top_k > c.experts)  // qwen3_5_moe.rs:508-513
        return Err(MRUN_ERR_INVALID, "config: num_experts_per_tok " + std::to_string(c.top_k) +
                                         " must be in 1..=" + std::to_string(c.experts));
    if (c.shared_intermediate < 0) return Err(MRUN_ERR_INVALID, "config: shared width < 0");
    if (c.experts > 512) return Err(MRUN_ERR_UNSUPPORTED, "config: more than 512 experts");
    if (c.top_k > 16) return Err(MRUN_ERR_UNSUPPORTED, "config: top_k above 16");
    if (c.hidden % 32 != 0 || c.intermediate % 32 != 0 || c.shared_intermediate % 32 != 0)
        return Err(MRUN_ERR_UNSUPPORTED, "config: widths must be multiples of 32");
    return Ok();
}

static Status check_block(const mrun_sparse_moe *m) {
    if (!m) return Err(MRUN_ERR_INVALID, "moe is null");
    const mrun_moe_config &c = m->cfg;
    TRY(check_config(c));
    const int D = c.hidden, E = c.experts, I = c.intermediate, S = c.shared_intermediate;
    // router: dense bf16 or quantized [E, D] (+ bias [E])
    if (m->gate.out != E || m->gate.in != D)
        return Err(MRUN_ERR_INVALID, "gate: shape must be [experts, hidden]");
    if (m->gate.weight) TRY(check_ptr(m->gate.weight, "gate.weight"));
    else TRY(check_quantized(&m->gate.q, "gate", 1, E, D));
    TRY(check_quantized(&m->switch_gate_proj, "switch_mlp.gate_proj", E, I, D));
    TRY(check_quantized(&m->switch_up_proj, "switch_mlp.up_proj", E, I, D));
    TRY(check_quantized(&m->switch_down_proj, "switch_mlp.down_proj", E, D, I));
    if (!same_quant(m->switch_gate_proj, m->switch_up_proj))
        return Err(MRUN_ERR_UNSUPPORTED,
                   "switch_mlp.gate_proj and up_proj must share bits and group size");
    if (S > 0) {
        const mrun_linear *mlp[3] = {&m->shared_gate_proj, &m->shared_up_proj,
                                     &m->shared_down_proj};
        const char *names[3] = {"shared_expert.gate_proj", "shared_expert.up_proj",
                                "shared_expert.down_proj"};
        for (int i = 0; i < 3; ++i)
            if (mlp[i]->bias)
                return Err(MRUN_ERR_INVALID, std::string(names[i]) + ".bias is not supported");
        // dense shared experts (a bf16 Linear) run as one 16-bit expert
        const mrun_quantized sgq = as_quantized(m->shared_gate_proj),
                             suq = as_quantized(m->shared_up_proj),
                             sdq = as_quantized(m->shared_down_proj);
        TRY(check_quantized(&sgq, names[0], 1, S, D));
        TRY(check_quantized(&suq, names[1], 1, S, D));
        TRY(check_quantized(&sdq, names[2], 1, D, S));
        if (!same_quant(sgq, suq))
            return Err(MRUN_ERR_UNSUPPORTED,
                       "shared_expert.gate_proj and up_proj must share bits and group size");
        if (m->shared_expert_gate.out != 1 || m->shared_expert_gate.in != D)
            return Err(MRUN_ERR_INVALID, "shared_expert_gate: shape must be [1, hidden]");
        if (m->shared_expert_gate.weight)
            TRY(check_ptr(m->shared_expert_gate.weight, "shared_expert_gate.weight"));
        else TRY(check_quantized(&m->shared_expert_gate.q, "shared_expert_gate", 1, 1, D));
    }
    return Ok();
}

namespace models {
static Status check_block_f32(const mrun_sparse_moe *m);  // float32 blocks, below
}

// ---------------------------------------------------------------------------------------------
// workspace plan (the counterpart of SparseMoe::scratch_per_token, moe.rs:176-187)

struct Plan {
    size_t logits, ids, scores, offsets, order, inverse, token, active, n_active, tiles, n_tiles;
    size_t counts;
    int n_counts;
    size_t xp, xs, act_x, sh_act_x, tile_rows;  // the packed operands of the prefill GEMMs
    size_t act, y, sh_logit, sh_act, sh_y, total;
    int max_tiles;
};

static size_t a256(size_t v) { return (v + 255) & ~(size_t)255; }

static Plan make_plan(const mrun_moe_config &c, int T) {
    Plan p{};
    size_t at = 0;
    auto take = [&](size_t bytes) {
        size_t o = at;
        at += a256(bytes);
        return o;
    };
    const size_t E = c.experts, D = c.hidden, I = c.intermediate, S = c.shared_intermediate;
    const size_t P = (size_t)T * c.top_k;
    // tiles of 64 rows, or of 32 (mid-size batches on the grouped GEMM): room for the smaller
    p.max_tiles = (int)((P + 31) / 32 + E);
    p.logits = take(2 * (size_t)T * E);
    p.ids = take(4 * P);
    p.scores = take(2 * P);
    p.offsets = take(4 * (E + 1));
    p.order = take(4 * P);
    p.inverse = take(4 * P);
    p.token = take(4 * P);
    p.active = take(4 * E);
    p.n_active = take(4);
    p.tiles = take(12 * (size_t)p.max_tiles);
    p.n_tiles = take(4);
    // per-block expert counts of the prefill routing (route_block_tokens tokens per block)
    const int bt = route_block_tokens(c.top_k, c.experts);
    p.n_counts = (int)(((size_t)T + bt - 1) / bt * E);
    p.counts = take(4 * (size_t)p.n_counts);
    p.act = take(2 * P * I);
    p.y = take(2 * P * D);
    if (S > 0) {
        p.sh_logit = take(2 * (size_t)T);
        p.sh_act = take(2 * (size_t)T * S);
        p.sh_y = take(2 * (size_t)T * D);
    }
    // prefill GEMM operands (moe_gemm.hip): packed x and its group-sum splits, the group-sum
    // splits of act (and of the shared expert's act), the token rows of each routed tile
    if (T > 16) {
        p.xp = take(2 * (size_t)T * D);
        p.xs = take(2 * 3 * (size_t)T * (D / 64));
        p.act_x = take(2 * 3 * P * (I / 64));
        if (S > 0) p.sh_act_x = take(2 * 3 * (size_t)T * (S / 64));
        p.tile_rows = take(4 * (size_t)p.max_tiles * kGemmTileM);
    }
    p.total = at;
    return p;
}

namespace tensor {

// ---------------------------------------------------------------------------------------------
// facade ops

// Linear::forward with a dense bf16 weight (load.rs:294-306): y = R(x W^T), then R(y + bias).
static Status linear_dense(const bf16_t *x, int rows, const mrun_linear &l, bf16_t *y,
                           hipStream_t s, uint32_t *zero = nullptr, int n_zero = 0) {
    const int N = l.out, K = l.in;
    if (K % 8 != 0) return Err(MRUN_ERR_UNSUPPORTED, "linear: input width must be a multiple of 8");
    if (dense_gemm_supported(rows, K)) {
        DenseJob j{};
        j.A = x, j.lda = K, j.M = rows, j.K = K;
        j.W0 = l.weight, j.bias0 = l.bias, j.N0 = N, j.out0 = y, j.ldo0 = N;
        j.zero = zero, j.n_zero = n_zero;
        TRY_HIP(launch_dense_gemm(j, s), "linear (mfma)");
        return Ok();
    }
    if (rows > 16 && N < 16) {
        TRY_HIP(launch_rowdot(x, rows, K, l.weight, N, l.bias, y, s), "linear (rowdot)");
        return Ok();
    }
    if (rows > 16 && K % 64 == 0) {
        GemmJob j{};
        j.A = x, j.lda = K, j.a_div = 1, j.M = rows, j.N = N, j.K = K;
        j.bd = l.weight, j.bias = l.bias, j.out = y, j.ldo = N;
        j.zero = zero, j.n_zero = n_zero;
        TRY_HIP(launch_gemm(j, s), "linear (mfma)");
        return Ok();
    }
    for (int r0 = 0; r0 < rows; r0 += 16) {
        const int n = rows - r0 < 16 ? rows - r0 : 16;
        TRY_HIP(launch_rows(x + (size_t)r0 * K, n, K, l.weight, l.bias, N, y + (size_t)r0 * N, s),
                "linear (rows)");
    }
    return Ok();
}

// quantized_matmul (nuvec.rs:660-663) over expert 0 of w: y [rows, w.out].
static Status quantized_matmul(const bf16_t *x, int rows, const mrun_quantized &w, bf16_t *y,
                               hipStream_t s) {
    if (rows > 16 && w.in % 64 == 0) {
        GemmJob j{};
        j.A = x, j.lda = w.in, j.a_div = 1, j.M = rows, j.N = w.out, j.K = w.in;
        j.w0 = qw_of(w), j.out = y, j.ldo = w.out;
        TRY_HIP(launch_gemm(j, s), "quantized_matmul (mfma)");
        return Ok();
    }
    GemvJob j{};
    j.A = x, j.lda = w.in, j.a_div = 1, j.w0 = qw_of(w), j.max_slots = 1, j.rows = rows;
    j.out = y, j.ldo = w.out;
    TRY_HIP(launch_gemv(j, s), "quantized_matmul (gemv)");
    return Ok();
}

// Linear::forward (load.rs:294-306), dense or quantized. `zero` [n_zero] is cleared before the
// product's results are visible to later launches (the prefill routing counters).
static Status linear(const bf16_t *x, int rows, const mrun_linear &l, bf16_t *y, hipStream_t s,
                     uint32_t *zero = nullptr, int n_zero = 0) {
    if (l.weight) {
        // the MFMA branches clear `zero` themselves
        const bool mfma = dense_gemm_supported(rows, l.in) || (rows > 16 && !(l.out < 16) && l.in % 64 == 0);
        if (zero && !mfma) TRY_HIP(launch_fill_u32(zero, 0u, n_zero, s), "clear");
        return linear_dense(x, rows, l, y, s, mfma ? zero : nullptr, n_zero);
    }
    if (zero) TRY_HIP(launch_fill_u32(zero, 0u, n_zero, s), "clear");
    TRY(quantized_matmul(x, rows, l.q, y, s));
    if (l.bias) TRY_HIP(launch_add_bias(y, l.bias, rows, l.out, s), "linear bias");
    return Ok();
}

// Router: logits = gate(x); gates = softmax; ids = top-k; scores (moe.rs:151-159).
static Status router(const mrun_sparse_moe &m, const bf16_t *x, int T, bf16_t *logits,
                     bf16_t *gates, uint32_t *ids, bf16_t *scores, hipStream_t s) {
    const mrun_moe_config &c = m.cfg;
    TRY(linear(x, T, m.gate, logits, s));
    TRY_HIP(launch_topk(logits, T, c.experts, c.top_k, c.norm_topk_prob != 0, gates, ids, scores,
                        s),
            "router top-k");
    return Ok();
}

}  // namespace tensor

namespace models {

using Stages = StageMarks;

static const char *kDecodeStages = "router,gate_up,down_combine";
static const char *kPrefillStages =
    "router,shared_gate,topk,permute,gate_up,down,shared_gate_up,shared_down,combine";

// whether the decode router launch takes this Linear: dense bf16, or 4/8-bit quantized
static bool k1_router_ok(const mrun_linear &l) {
    return l.weight || l.q.bits == 4 || l.q.bits == 8;
}

static bool is_decode(const mrun_moe_config &c, int T) {
    return decode_supported(c.hidden, c.intermediate, c.shared_intermediate, T, c.top_k,
                            c.experts);
}

// The decode kernels stream 4-bit experts, and 8-bit ones of the shapes decode_supported_bits
// takes; every routed and shared expert projection has the same width of codes.
static bool is_decode(const mrun_sparse_moe &m, int T) {
    const mrun_moe_config &c = m.cfg;
    const int bits = m.switch_gate_proj.bits;
    bool same = (bits == 4 || bits == 8) && m.switch_up_proj.bits == bits &&
                m.switch_down_proj.bits == bits;
    if (c.shared_intermediate > 0)
        same = same && !m.shared_gate_proj.weight && !m.shared_up_proj.weight &&
               !m.shared_down_proj.weight && m.shared_gate_proj.q.bits == bits &&
               m.shared_up_proj.q.bits == bits && m.shared_down_proj.q.bits == bits;
    return same && decode_supported_bits(c.hidden, c.intermediate, c.shared_intermediate, bits) &&
           is_decode(c, T);
}

// ---------------------------------------------------------------------------------------------
// SparseMoe::forward (moe.rs:149-174)

// The decoder layer around a decode-schedule block (the layer stack): the block's input x is
// written by its first launch as the RMSNorm of `src` (weight w or ones), and its last launch
// writes out = R(src + block output).
struct FusedNorm {
    const bf16_t *src;
    const bf16_t *w;
    float eps;
};

// post (the layer stack): when the forward ends in the combine launch and its rows are at most
// 2048 wide, that launch also takes the stack's residual add and next RMSNorm (post_done set, and
// `out` is not written).
// Prefill batches whose experts average at most this many rows have their routed tiles cut to 32
// rows for the grouped GEMM. On the configs[1] block (per block, 32- against 64-row tiles):
// T = 33 131 -> 111 us, 64 154 -> 132, 128 164 -> 144, 256 180 -> 159, 512 190 -> 165, 768 199 ->
// 179; T = 1024 (32 rows on average) the same; T = 2048 281 -> 308 (Zipf router: 268 -> 311).
constexpr int kHalfTileMaxRows = 28;

// the largest batch that runs as decode-schedule chunks of at most 16 tokens, when the decode
// kernels do not take it whole (more than 256 pairs: k above 8)
constexpr int kChunkedDecodeMax = 32;

// Workspace of a batch that runs as decode chunks: the whole batch's ids and scores where the
// batch's own plan keeps them (mrun_moe_workspace_routing), then one chunk's workspace.
static size_t chunk_ws_offset(const mrun_moe_config &c, int T) {
    const Plan p = make_plan(c, T);
    return p.scores + a256(2 * (size_t)T * c.top_k);
}
static bool runs_chunked(const mrun_moe_config &c, int T) {
    return T > 16 && T <= kChunkedDecodeMax && !is_decode(c, T);
}
// the batch runs the decode schedule (whole, or in chunks of at most 16 tokens)
static bool decode_schedule(const mrun_sparse_moe &m, int T) {
    if (runs_chunked(m.cfg, T)) return is_decode(m, 16) && is_decode(m, T % 16 ? T % 16 : 16);
    return is_decode(m, T);
}
// tokens per decode launch of a batch on the decode schedule
static int decode_launch_tokens(const mrun_moe_config &c, int T) {
    return runs_chunked(c, T) ? 16 : T;
}
static size_t forward_ws_bytes(const mrun_moe_config &c, int T) {
    const size_t plain = make_plan(c, T).total;
    if (!runs_chunked(c, T)) return plain;
    const size_t chunked = chunk_ws_offset(c, T) + make_plan(c, 16).total;
    return plain > chunked ? plain : chunked;
}

// ids_at / scores_at (decode schedule only): where the routing goes instead of the plan's arrays.
static Status sparse_moe_forward(const mrun_sparse_moe &m, const bf16_t *x, int T, bf16_t *out,
                                 char *ws, size_t ws_bytes, hipStream_t s, Stages *stg = nullptr,
                                 const FusedNorm *fn = nullptr, const PostNorm *post = nullptr,
                                 bool *post_done = nullptr, uint32_t *ids_at = nullptr,
                                 bf16_t *scores_at = nullptr) {
    // 17 to kChunkedDecodeMax tokens with more pairs than the decode kernels take (k above 8):
    // the decode schedule on chunks of at most 16 tokens (the tokens of a chunk, then the rest),
    // which streams each chunk's expert rows once, against the prefill schedule's 64-row tiles
    // that are mostly padding at these sizes. Every token's row is computed alone as in any
    // decode batch. Instrumented calls (stg) keep one schedule.
    if (!stg && runs_chunked(m.cfg, T) && decode_schedule(m, T)) {
        const mrun_moe_config &c = m.cfg;
        const int D = c.hidden, k = c.top_k;
        if (ws_bytes < forward_ws_bytes(c, T))
            return Err(MRUN_ERR_WORKSPACE, "workspace of " + std::to_string(ws_bytes) +
                                               " bytes, need " + std::to_string(forward_ws_bytes(c, T)));
        const Plan p = make_plan(c, T);
        const size_t off = chunk_ws_offset(c, T);
        if (post_done) *post_done = false;
        for (int t0 = 0; t0 < T; t0 += 16) {
            const int tc = T - t0 < 16 ? T - t0 : 16;
            FusedNorm f{};
            if (fn) f = FusedNorm{fn->src + (size_t)t0 * D, fn->w, fn->eps};
            TRY(sparse_moe_forward(m, x + (size_t)t0 * D, tc, out + (size_t)t0 * D, ws + off,
                                   ws_bytes - off, s, nullptr, fn ? &f : nullptr, nullptr, nullptr,
                                   (uint32_t *)(ws + p.ids) + (size_t)t0 * k,
                                   (bf16_t *)(ws + p.scores) + (size_t)t0 * k));
        }
        return Ok();
    }
    Stages none;
    Stages &st = stg ? *stg : none;
    if (st.events && st.n_events > 0) (void)hipEventRecord(st.events[0], s);
    const mrun_moe_config &c = m.cfg;
    const int D = c.hidden, E = c.experts, k = c.top_k, I = c.intermediate;
    const int S = c.shared_intermediate;
    const int P = T * k;
    const Plan p = make_plan(c, T);
    if (ws_bytes < p.total)
        return Err(MRUN_ERR_WORKSPACE, "workspace of " + std::to_string(ws_bytes) +
                                           " bytes, need " + std::to_string(p.total));
    auto at = [&](size_t off) { return (void *)(ws + off); };
    bf16_t *logits = (bf16_t *)at(p.logits);
    uint32_t *ids = (uint32_t *)at(p.ids);
    bf16_t *scores = (bf16_t *)at(p.scores);
    PermuteOut po{};
    po.offsets = (uint32_t *)at(p.offsets);
    po.order = (uint32_t *)at(p.order);
    po.inverse = (uint32_t *)at(p.inverse);
    po.token = (uint32_t *)at(p.token);
    po.active = (uint32_t *)at(p.active);
    po.n_active = (uint32_t *)at(p.n_active);
    po.tile_m = kGemmTileM;
    Routing rt{po.offsets, po.active, po.n_active, (const uint32_t *)at(p.tiles),
               (const uint32_t *)at(p.n_tiles)};
    bf16_t *act = (bf16_t *)at(p.act);
    bf16_t *y = (bf16_t *)at(p.y);
    bf16_t *sh_logit = S ? (bf16_t *)at(p.sh_logit) : nullptr;
    bf16_t *sh_act = S ? (bf16_t *)at(p.sh_act) : nullptr;
    bf16_t *sh_y = S ? (bf16_t *)at(p.sh_y) : nullptr;
    const int max_slots = E < P ? E : P;

    const bool decode = is_decode(m, T);
    const bool mfma = D % 64 == 0 && I % 64 == 0 && (S == 0 || S % 64 == 0);  // K of each product

    if (decode) {
        DecodeJob j{};
        j.x = x, j.T = T, j.D = D, j.E = E, j.k = k, j.I = I, j.S = S;
        j.norm = c.norm_topk_prob != 0, j.max_slots = max_slots;
        j.router = m.gate.weight, j.router_bias = m.gate.bias;
        j.wg = qw_of(m.switch_gate_proj), j.wu = qw_of(m.switch_up_proj);
        j.wd = qw_of(m.switch_down_proj);
        if (S) {
            j.sh_gate_w = m.shared_expert_gate.weight, j.sh_gate_b = m.shared_expert_gate.bias;
            j.sg = qw_of(as_quantized(m.shared_gate_proj)), j.su = qw_of(as_quantized(m.shared_up_proj));
            j.sd = qw_of(as_quantized(m.shared_down_proj));
        }
        j.logits = logits, j.sh_logit = sh_logit, j.sh_act = sh_act, j.act = act, j.out = out;
        j.ids = ids_at ? ids_at : ids, j.scores = scores_at ? scores_at : scores;
        j.topk_in_kernel = T <= 4;
        // a quantized router or shared gate (8-bit in mlx-community conversions): K1 dequantizes
        // its rows (4 or 8 bits; the checked group sizes keep a lane's 8-element chunks in one
        // group)
        const bool r_ok = k1_router_ok(m.gate);
        const bool g_ok = !S || k1_router_ok(m.shared_expert_gate);
        if (!m.gate.weight && r_ok) j.router_q = qw_of(m.gate.q);
        if (S && !m.shared_expert_gate.weight && g_ok) j.sh_gate_q = qw_of(m.shared_expert_gate.q);
        if (fn) {  // K1 normalises fn->src into x; K3 adds the residual
            if (!r_ok || !g_ok)
                return Err(MRUN_ERR_UNSUPPORTED,
                           "fused norm needs a dense or 4/8-bit router and shared gate");
            j.norm_src = fn->src, j.norm_w = fn->w, j.eps = fn->eps, j.residual = fn->src;
        }
        if (!r_ok || !g_ok) {
            TRY(tensor::linear(x, T, m.gate, logits, s));
            if (S) TRY(tensor::linear(x, T, m.shared_expert_gate, sh_logit, s));
            j.router_done = 1;
        }
        j.clock = st.k2_clock;
        TRY_HIP(launch_decode(j, s, &st), "decode");
        return Ok();
    }

    // prefill
    uint32_t *counts = (uint32_t *)at(p.counts);
    // the grouped GEMM's packed x: written by the router launch when the router is dense, else
    // by its own launch after the routing
    const bool packs = mfma && T > 16 && D % 512 == 0 && I % 512 == 0;
    bool packed = false;
    if (m.gate.weight && (!S || m.shared_expert_gate.weight) && dense_gemm_supported(T, D)) {
        // router and shared gate: one launch over x
        DenseJob dj{};
        dj.A = x, dj.lda = D, dj.M = T, dj.K = D;
        dj.W0 = m.gate.weight, dj.bias0 = m.gate.bias, dj.N0 = E, dj.out0 = logits, dj.ldo0 = E;
        if (S) {
            dj.W1 = m.shared_expert_gate.weight, dj.bias1 = m.shared_expert_gate.bias;
            dj.N1 = 1, dj.out1 = sh_logit, dj.ldo1 = 1;
        }
        dj.zero = counts, dj.n_zero = p.n_counts;
        if (packs) dj.pack_a = (bf16_t *)at(p.xp), dj.pack_x = (bf16_t *)at(p.xs), packed = true;
        TRY_HIP(launch_dense_gemm(dj, s), "router (mfma)");
        st.mark(s);  // (the shared gate's stage below stays empty: it ran in this launch)
    } else {
        TRY(tensor::linear(x, T, m.gate, logits, s, counts, p.n_counts));
        st.mark(s);
        if (S) TRY(tensor::linear(x, T, m.shared_expert_gate, sh_logit, s));
    }
    st.mark(s);
    TRY_HIP(launch_topk_count(logits, T, E, k, c.norm_topk_prob != 0, ids, scores, counts, s),
            "top-k");
    st.mark(s);
    // the grouped GEMM of moe_gemm.hip: 4-bit group-64 experts, K a multiple of 512, the shared
    // expert in the same launches when its width equals the routed one
    MoeGemmJob mg{}, md{};
    bool new_path = false, fuse_new = false;
    if (mfma && T > 16) {
        mg.A = (const bf16_t *)at(p.xp), mg.lda = D, mg.a_rows = T, mg.AX = (const bf16_t *)at(p.xs);
        mg.ax_e = D / 64, mg.tile_rows = (const uint32_t *)at(p.tile_rows);
        mg.K = D, mg.N = I, mg.glu = 1;
        mg.w0 = qw_of(m.switch_gate_proj), mg.w1 = qw_of(m.switch_up_proj);
        mg.routing = rt, mg.has_routing = 1, mg.max_tiles = p.max_tiles;
        mg.out = act, mg.ldo = I, mg.OX = (bf16_t *)at(p.act_x);
        md.A = act, md.lda = I, md.a_rows = P, md.AX = (const bf16_t *)at(p.act_x), md.ax_e = I / 64;
        md.K = I, md.N = D, md.glu = 0, md.w0 = qw_of(m.switch_down_proj);
        md.routing = rt, md.has_routing = 1, md.max_tiles = p.max_tiles, md.out = y, md.ldo = D;
        new_path = moe_gemm_supported(mg) && moe_gemm_supported(md);
        if (new_path && S == I && !m.shared_gate_proj.weight && !m.shared_up_proj.weight &&
            !m.shared_down_proj.weight) {
            MoeGemmJob tg = mg, td = md;
            tg.sh = {mg.A, D, mg.AX, D / 64, T, qw_of(m.shared_gate_proj.q),
                     qw_of(m.shared_up_proj.q), sh_act, S, (bf16_t *)at(p.sh_act_x)};
            tg.has_shared = 1;
            td.sh = {sh_act, S, (const bf16_t *)at(p.sh_act_x), S / 64, T,
                     qw_of(m.shared_down_proj.q), QW{}, sh_y, D, nullptr};
            td.has_shared = 1;
            if (moe_gemm_supported(tg) && moe_gemm_supported(td)) mg = tg, md = td, fuse_new = true;
        }
    }
    // mid-size batches: the routed tiles cut to 32 rows (most experts hold a few rows, so a 64-row
    // tile is mostly padding), on the grouped GEMM's one-row-fragment instantiation
    const bool half = new_path && (long long)P <= (long long)kHalfTileMaxRows * E;
    mg.tile_m = md.tile_m = half ? 32 : kGemmTileM;
    PermuteOut pt = po;
    pt.tile_m = half ? 32 : kGemmTileM;
    pt.tiles = (uint32_t *)at(p.tiles);
    pt.n_tiles = (uint32_t *)at(p.n_tiles);
    if (packs) pt.tile_rows = (uint32_t *)at(p.tile_rows);
    TRY_HIP(launch_route_scatter(ids, counts, T, k, E, pt, s), "scatter");
    if (packs && !packed)
        TRY_HIP(launch_apack(x, D, T, D, (bf16_t *)at(p.xp), D, (bf16_t *)at(p.xs), s), "pack x");
    st.mark(s);
    if (new_path) {
        TRY_HIP(launch_moe_gemm(mg, s), "gate/up (moe gemm)");
        st.mark(s);
        TRY_HIP(launch_moe_gemm(md, s), "down (moe gemm)");
        st.mark(s);
        if (S && !fuse_new) {  // a shared expert of another width or format: the generic GEMMs
            GemmJob sg{}, sd{};
            sg.A = x, sg.lda = D, sg.a_div = 1, sg.M = T, sg.N = S, sg.K = D;
            sg.w0 = qw_of(as_quantized(m.shared_gate_proj));
            sg.w1 = qw_of(as_quantized(m.shared_up_proj));
            sg.out = sh_act, sg.ldo = S, sg.glu = 1;
            sd.A = sh_act, sd.lda = S, sd.a_div = 1, sd.M = T, sd.N = D, sd.K = S;
            sd.w0 = qw_of(as_quantized(m.shared_down_proj)), sd.out = sh_y, sd.ldo = D;
            TRY_HIP(launch_gemm(sg, s), "shared gate/up (mfma)");
            st.mark(s);
            TRY_HIP(launch_gemm(sd, s), "shared down (mfma)");
            st.mark(s);
        } else {
            st.mark(s);
            st.mark(s);
        }
    } else if (mfma && T > 16) {  // at decode sizes the gathered GEMV streams the rows once
        GemmJob g{};
        g.A = x, g.lda = D, g.a_map = po.order, g.a_div = k, g.N = I, g.K = D;
        g.w0 = qw_of(m.switch_gate_proj), g.w1 = qw_of(m.switch_up_proj);
        g.routing = rt, g.has_routing = 1, g.max_tiles = p.max_tiles;
        g.out = act, g.ldo = I, g.glu = 1;
        GemmJob dn{};
        dn.A = act, dn.lda = I, dn.a_div = 1, dn.N = D, dn.K = I;
        dn.w0 = qw_of(m.switch_down_proj), dn.routing = rt, dn.has_routing = 1;
        dn.max_tiles = p.max_tiles, dn.out = y, dn.ldo = D;
        GemmJob sg{}, sd{};
        if (S) {
            sg.A = x, sg.lda = D, sg.a_div = 1, sg.M = T, sg.N = S, sg.K = D;
            sg.w0 = qw_of(as_quantized(m.shared_gate_proj));
            sg.w1 = qw_of(as_quantized(m.shared_up_proj));
            sg.out = sh_act, sg.ldo = S, sg.glu = 1;
            sd.A = sh_act, sd.lda = S, sd.a_div = 1, sd.M = T, sd.N = D, sd.K = S;
            sd.w0 = qw_of(as_quantized(m.shared_down_proj)), sd.out = sh_y, sd.ldo = D;
        }
        // the shared expert rides in the routed launches when its products have the same N
        bool fuse = S == I && qgemm_supported(g) && qgemm_supported(dn) && qgemm_supported(sg) &&
                    qgemm_supported(sd);
        if (fuse) {
            g.sh = {x, D, T, D, sg.w0, sg.w1, sh_act, S}, g.has_shared = 1;
            dn.sh = {sh_act, S, T, S, sd.w0, QW{}, sh_y, D}, dn.has_shared = 1;
        }
        TRY_HIP(launch_gemm(g, s), "gate/up (mfma)");
        st.mark(s);
        TRY_HIP(launch_gemm(dn, s), "down (mfma)");
        st.mark(s);
        if (S && !fuse) {
            TRY_HIP(launch_gemm(sg, s), "shared gate/up (mfma)");
            st.mark(s);
            TRY_HIP(launch_gemm(sd, s), "shared down (mfma)");
            st.mark(s);
        } else {
            st.mark(s);
            st.mark(s);
        }
    } else {
        GemvJob g{};
        g.A = x, g.lda = D, g.a_map = po.order, g.a_div = k;
        g.w0 = qw_of(m.switch_gate_proj), g.w1 = qw_of(m.switch_up_proj);
        g.routing = rt, g.has_routing = 1, g.max_slots = max_slots;
        g.out = act, g.ldo = I, g.glu = 1;
        if (S) {
            g.xA = x, g.x_lda = D, g.xw0 = qw_of(as_quantized(m.shared_gate_proj));
            g.xw1 = qw_of(as_quantized(m.shared_up_proj)), g.x_rows = T, g.xout = sh_act, g.x_ldo = S;
        }
        TRY_HIP(launch_gemv(g, s), "gate/up (gemv)");
        st.mark(s);
        GemvJob dn{};
        dn.A = act, dn.lda = I, dn.a_div = 1, dn.w0 = qw_of(m.switch_down_proj);
        dn.routing = rt, dn.has_routing = 1, dn.max_slots = max_slots, dn.out = y, dn.ldo = D;
        if (S) {
            dn.xA = sh_act, dn.x_lda = S, dn.xw0 = qw_of(as_quantized(m.shared_down_proj));
            dn.x_rows = T, dn.xout = sh_y, dn.x_ldo = D;
        }
        TRY_HIP(launch_gemv(dn, s), "down (gemv)");
        st.mark(s);
        st.mark(s);
        st.mark(s);
    }
    const bool fuse_post = post && D <= 2048 && k <= 16;
    TRY_HIP(launch_combine(y, po.inverse, scores, T, k, D, sh_y, sh_logit, out, s,
                           fuse_post ? post : nullptr),
            "combine");
    if (post_done) *post_done = fuse_post;
    st.mark(s);
    return Ok();
}

}  // namespace models
}  // namespace mrun

// ---------------------------------------------------------------------------------------------
// C ABI

using namespace mrun;

extern "C" {

const char *mrun_last_error(void) { return g_last_error.c_str(); }

const char *mrun_version(void) { return "mrun-moe 0.1.0 (gfx950)"; }

int mrun_moe_check(const mrun_sparse_moe *moe) {
    // a block of f32 experts is an f32 block (mrun_moe_forward_f32) and is checked as one
    if (moe && moe->switch_gate_proj.bits == 32) return report(models::check_block_f32(moe));
    return report(check_block(moe));
}

size_t mrun_moe_workspace_bytes(const mrun_moe_config *cfg, int32_t tokens) {
    if (!cfg || tokens <= 0 || !check_config(*cfg).ok()) return 0;
    return models::forward_ws_bytes(*cfg, tokens);
}

int mrun_moe_forward(const mrun_sparse_moe *moe, const mrun_bf16 *x, int32_t tokens,
                     mrun_bf16 *out, void *workspace, size_t workspace_bytes,
                     mrun_stream_t stream) {
    Status st = check_block(moe);
    if (st.ok() && tokens < 0) st = Err(MRUN_ERR_INVALID, "tokens must not be negative");
    if (st.ok() && tokens == 0) return report(st);  // an empty batch: nothing to do
    if (st.ok()) st = check_ptr(x, "x");
    if (st.ok()) st = check_ptr(out, "out");
    if (st.ok()) st = check_ptr(workspace, "workspace");
    if (st.ok() && x == out) st = Err(MRUN_ERR_INVALID, "out must not alias x");
    if (st.ok())
        st = models::sparse_moe_forward(*moe, x, tokens, out, (char *)workspace, workspace_bytes,
                                        (hipStream_t)stream);
    return report(st);
}

}  // extern "C"

// ---------------------------------------------------------------------------------------------
// float32 blocks: SparseMoe::forward (moe.rs:149-174) with every tensor f32, as the reference runs
// an f32 checkpoint (its dense gather_mm, nuvec.rs:688-697, and every other op then compute and
// keep f32). The weights are dense f32 stacked weights (bits 32); the op sequence is the bf16
// forward's without its bf16 roundings.

namespace mrun {
namespace models {

static Status check_f32(const mrun_quantized &q, const std::string &path, int experts, int out,
                        int in) {
    if (q.bits != 32 || !q.weight)
        return Err(MRUN_ERR_INVALID, path + ": an f32 block takes dense f32 weights (bits 32)");
    if (q.scales || q.biases)
        return Err(MRUN_ERR_INVALID, path + ": dense f32 weights carry no scales or biases");
    if (q.experts != experts || q.out != out || q.in != in)
        return Err(MRUN_ERR_INVALID, path + ": shape [" + std::to_string(q.experts) + ", " +
                                         std::to_string(q.out) + ", " + std::to_string(q.in) +
                                         "], expected [" + std::to_string(experts) + ", " +
                                         std::to_string(out) + ", " + std::to_string(in) + "]");
    return check_ptr(q.weight, path.c_str());
}

static Status check_f32_linear(const mrun_linear &l, const std::string &path, int out, int in) {
    if (l.weight)
        return Err(MRUN_ERR_INVALID,
                   path + ": an f32 block's Linear carries its weight in q (bits 32)");
    if (l.bias) return Err(MRUN_ERR_UNSUPPORTED, path + ": f32 Linear biases are not run");
    return check_f32(l.q, path, 1, out, in);
}

static Status check_block_f32(const mrun_sparse_moe *m) {
    if (!m) return Err(MRUN_ERR_INVALID, "moe is null");
    const mrun_moe_config &c = m->cfg;
    TRY(check_config(c));
    const int D = c.hidden, E = c.experts, I = c.intermediate, S = c.shared_intermediate;
    TRY(check_f32_linear(m->gate, "gate", E, D));
    TRY(check_f32(m->switch_gate_proj, "switch_mlp.gate_proj", E, I, D));
    TRY(check_f32(m->switch_up_proj, "switch_mlp.up_proj", E, I, D));
    TRY(check_f32(m->switch_down_proj, "switch_mlp.down_proj", E, D, I));
    if (S > 0) {
        TRY(check_f32_linear(m->shared_gate_proj, "shared_expert.gate_proj", S, D));
        TRY(check_f32_linear(m->shared_up_proj, "shared_expert.up_proj", S, D));
        TRY(check_f32_linear(m->shared_down_proj, "shared_expert.down_proj", D, S));
        TRY(check_f32_linear(m->shared_expert_gate, "shared_expert_gate", 1, D));
    }
    return Ok();
}

// logits [T, E], ids [T, k], scores [T, k], act [P, I], y [P, D]; with a shared expert its gate
// logit [T], act [T, S] and output [T, D] (all f32 but the ids)
struct PlanF32 {
    size_t logits, ids, scores, act, y, sh_logit, sh_act, sh_y, total;
};

static PlanF32 plan_f32(const mrun_moe_config &c, int T) {
    PlanF32 p{};
    size_t at = 0;
    auto take = [&](size_t bytes) {
        const size_t o = at;
        at += a256(bytes);
        return o;
    };
    const size_t P = (size_t)T * c.top_k, S = (size_t)c.shared_intermediate;
    p.logits = take(4 * (size_t)T * c.experts);
    p.ids = take(4 * P);
    p.scores = take(4 * P);
    p.act = take(4 * P * c.intermediate);
    p.y = take(4 * P * c.hidden);
    if (S) {
        p.sh_logit = take(4 * (size_t)T);
        p.sh_act = take(4 * (size_t)T * S);
        p.sh_y = take(4 * (size_t)T * c.hidden);
    }
    p.total = at;
    return p;
}

static Status sparse_moe_forward_f32(const mrun_sparse_moe &m, const float *x, int T, float *out,
                                     char *ws, size_t ws_bytes, hipStream_t s) {
    const mrun_moe_config &c = m.cfg;
    const PlanF32 p = plan_f32(c, T);
    if (ws_bytes < p.total)
        return Err(MRUN_ERR_WORKSPACE, "workspace of " + std::to_string(ws_bytes) +
                                           " bytes, need " + std::to_string(p.total));
    const int D = c.hidden, E = c.experts, k = c.top_k, I = c.intermediate,
              S = c.shared_intermediate, P = T * k;
    float *logits = (float *)(ws + p.logits), *scores = (float *)(ws + p.scores);
    uint32_t *ids = (uint32_t *)(ws + p.ids);
    float *act = (float *)(ws + p.act), *y = (float *)(ws + p.y);
    auto W = [](const mrun_quantized &q) { return (const float *)q.weight; };
    // router: gates = softmax(gate(x)), top-k, scores (moe.rs:151-159)
    TRY_HIP(launch_f32_rows(F32Rows{x, 1, D, W(m.gate.q), nullptr, nullptr, T, E, logits}, false, s),
            "f32 router");
    TRY_HIP(launch_f32_topk(logits, T, E, k, c.norm_topk_prob != 0, ids, scores, s), "f32 top-k");
    // SwitchGlu (moe.rs:61-94): pair p = t k + j reads token t's row and expert ids[p]
    TRY_HIP(launch_f32_rows(F32Rows{x, k, D, W(m.switch_gate_proj), W(m.switch_up_proj), ids, P, I,
                                    act},
                            true, s),
            "f32 experts gate/up");
    TRY_HIP(launch_f32_rows(F32Rows{act, 1, I, W(m.switch_down_proj), nullptr, ids, P, D, y}, false,
                            s),
            "f32 experts down");
    // the shared expert under its sigmoid gate (moe.rs:166-171)
    const float *gl = nullptr, *sy = nullptr;
    if (S > 0) {
        float *sh_logit = (float *)(ws + p.sh_logit), *sh_act = (float *)(ws + p.sh_act),
              *sh_y = (float *)(ws + p.sh_y);
        TRY_HIP(launch_f32_rows(F32Rows{x, 1, D, W(m.shared_expert_gate.q), nullptr, nullptr, T, 1,
                                        sh_logit},
                                false, s),
                "f32 shared gate");
        TRY_HIP(launch_f32_rows(F32Rows{x, 1, D, W(m.shared_gate_proj.q), W(m.shared_up_proj.q),
                                        nullptr, T, S, sh_act},
                                true, s),
                "f32 shared gate/up");
        TRY_HIP(launch_f32_rows(F32Rows{sh_act, 1, S, W(m.shared_down_proj.q), nullptr, nullptr, T,
                                        D, sh_y},
                                false, s),
                "f32 shared down");
        gl = sh_logit, sy = sh_y;
    }
    TRY_HIP(launch_f32_combine(y, scores, T, k, D, gl, sy, out, s), "f32 combine");
    return Ok();
}

}  // namespace models
}  // namespace mrun

extern "C" {

size_t mrun_moe_workspace_bytes_f32(const mrun_moe_config *cfg, int32_t tokens) {
    if (!cfg || tokens <= 0 || !check_config(*cfg).ok()) return 0;
    return models::plan_f32(*cfg, tokens).total;
}

int mrun_moe_forward_f32(const mrun_sparse_moe *moe, const float *x, int32_t tokens, float *out,
                         void *workspace, size_t workspace_bytes, mrun_stream_t stream) {
    Status st = models::check_block_f32(moe);
    if (st.ok() && tokens < 0) st = Err(MRUN_ERR_INVALID, "tokens must not be negative");
    if (st.ok() && tokens == 0) return report(st);  // an empty batch: nothing to do
    if (st.ok()) st = check_ptr(x, "x");
    if (st.ok()) st = check_ptr(out, "out");
    if (st.ok()) st = check_ptr(workspace, "workspace");
    if (st.ok() && (const void *)x == (const void *)out) st = Err(MRUN_ERR_INVALID, "out must not alias x");
    if (st.ok())
        st = models::sparse_moe_forward_f32(*moe, x, tokens, out, (char *)workspace,
                                            workspace_bytes, (hipStream_t)stream);
    return report(st);
}

}  // extern "C"

// ---------------------------------------------------------------------------------------------
// The forward that allocates nothing: its workspace is a file-scope device array.

namespace mrun {

constexpr size_t kScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// `scratch` names a host-side stand-in in host code; its device address (one per GPU, each GPU
// holding its own copy) comes from hipGetSymbolAddress, once per device, kept here.
constexpr int kMaxDevices = 64;
static void *g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

static Status scratch_of_current_device(void **ptr) {
    int dev = -1;
    TRY_HIP(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices)
        return Err(MRUN_ERR_UNSUPPORTED, "device index " + std::to_string(dev) + " out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        TRY_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        if (!p) return Err(MRUN_ERR_HIP, "hipGetSymbolAddress(scratch) returned null");
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    return Ok();
}

}  // namespace mrun

extern "C" {

size_t mrun_moe_forward_noalloc_max_bytes(void) {
    void *p = nullptr;
    (void)scratch_of_current_device(&p);  // the address lookup, outside any capture (errors: the
                                          // forward reports them)
    return kScratchBytes;
}

int mrun_moe_forward_noalloc(const mrun_sparse_moe *moe, const mrun_bf16 *x, int32_t tokens,
                             mrun_bf16 *out, mrun_stream_t stream) {
    Status st = check_block(moe);
    if (st.ok() && tokens < 0) st = Err(MRUN_ERR_INVALID, "tokens must not be negative");
    if (st.ok() && tokens == 0) return report(st);  // an empty batch: nothing to do
    if (st.ok()) st = check_ptr(x, "x");
    if (st.ok()) st = check_ptr(out, "out");
    if (st.ok() && x == out) st = Err(MRUN_ERR_INVALID, "out must not alias x");
    if (st.ok()) {
        const size_t need = models::forward_ws_bytes(moe->cfg, tokens);
        if (need > kScratchBytes)
            st = Err(MRUN_ERR_WORKSPACE,
                     "forward_noalloc: " + std::to_string(tokens) + " tokens need " +
                         std::to_string(need) + " bytes of scratch, above its fixed " +
                         std::to_string(kScratchBytes) + " bytes (use mrun_moe_forward with a "
                                                         "workspace)");
    }
    void *ws = nullptr;
    if (st.ok()) st = scratch_of_current_device(&ws);
    if (st.ok())
        st = models::sparse_moe_forward(*moe, x, tokens, out, (char *)ws, kScratchBytes,
                                        (hipStream_t)stream);
    return report(st);
}

int mrun_moe_forward_profiled(const mrun_sparse_moe *moe, const mrun_bf16 *x, int32_t tokens,
                              mrun_bf16 *out, void *workspace, size_t workspace_bytes,
                              mrun_stream_t stream, void **events, int32_t n_events,
                              int32_t *n_stages) {
    Status st = check_block(moe);
    if (st.ok() && tokens < 0) st = Err(MRUN_ERR_INVALID, "tokens must not be negative");
    if (st.ok() && tokens == 0) {  // an empty batch: nothing to do, no stage
        if (n_stages) *n_stages = 0;
        return report(st);
    }
    if (st.ok()) st = check_ptr(x, "x");
    if (st.ok()) st = check_ptr(out, "out");
    if (st.ok()) st = check_ptr(workspace, "workspace");
    if (st.ok() && x == out) st = Err(MRUN_ERR_INVALID, "out must not alias x");
    StageMarks stages;
    stages.events = (hipEvent_t *)events;
    stages.n_events = events ? n_events : 0;
    if (st.ok())
        st = models::sparse_moe_forward(*moe, x, tokens, out, (char *)workspace, workspace_bytes,
                                        (hipStream_t)stream, &stages);
    if (n_stages) *n_stages = stages.count;
    return report(st);
}

int mrun_moe_forward_timed(const mrun_sparse_moe *moe, const mrun_bf16 *x, int32_t tokens,
                           mrun_bf16 *out, void *workspace, size_t workspace_bytes,
                           mrun_stream_t stream, uint64_t *clock) {
    Status st = check_block(moe);
    if (st.ok() && tokens < 0) st = Err(MRUN_ERR_INVALID, "tokens must not be negative");
    if (st.ok() && tokens == 0) return report(st);  // an empty batch: nothing to do
    if (st.ok()) st = check_ptr(x, "x");
    if (st.ok()) st = check_ptr(out, "out");
    if (st.ok()) st = check_ptr(workspace, "workspace");
    if (st.ok() && x == out) st = Err(MRUN_ERR_INVALID, "out must not alias x");
    if (st.ok()) st = check_ptr(clock, "clock");
    if (st.ok() && !models::is_decode(*moe, tokens))
        st = Err(MRUN_ERR_UNSUPPORTED,
                 "forward_timed: this batch runs the prefill schedule, which has no decode "
                 "gate/up launch to time");
    StageMarks marks;
    marks.k2_clock = (unsigned long long *)clock;
    if (st.ok())
        st = models::sparse_moe_forward(*moe, x, tokens, out, (char *)workspace, workspace_bytes,
                                        (hipStream_t)stream, &marks);
    return report(st);
}

int64_t mrun_wall_clock_hz(void) {
    int dev = 0, khz = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess || khz <= 0)
        return -1;
    return (int64_t)khz * 1000;
}

const char *mrun_moe_stage_names(const mrun_moe_config *cfg, int32_t tokens) {
    if (!cfg || tokens <= 0) return "";
    // for 4-bit experts (8-bit ones run the prefill stages at every token count)
    return models::is_decode(*cfg, tokens) ? models::kDecodeStages : models::kPrefillStages;
}

int mrun_moe_router(const mrun_sparse_moe *moe, const mrun_bf16 *x, int32_t tokens,
                    mrun_bf16 *logits, mrun_bf16 *gates, uint32_t *ids, mrun_bf16 *scores,
                    void *workspace, size_t workspace_bytes, mrun_stream_t stream) {
    Status st = check_block(moe);
    if (st.ok() && tokens < 0) st = Err(MRUN_ERR_INVALID, "tokens must not be negative");
    if (st.ok() && tokens == 0) return report(st);  // an empty batch: nothing to do
    if (st.ok()) st = check_ptr(x, "x");
    if (st.ok() && (!ids || !scores)) st = Err(MRUN_ERR_INVALID, "ids and scores are required");
    bf16_t *lg = logits;
    if (st.ok() && !lg) {
        const size_t need = 2 * (size_t)tokens * moe->cfg.experts;
        if (!workspace || workspace_bytes < need)
            st = Err(MRUN_ERR_WORKSPACE, "router needs " + std::to_string(need) +
                                             " workspace bytes for the logits");
        lg = (bf16_t *)workspace;
    }
    if (st.ok() && lg) st = check_ptr(lg, "logits");
    if (st.ok())
        st = tensor::router(*moe, x, tokens, lg, gates, ids, scores, (hipStream_t)stream);
    return report(st);
}

size_t mrun_moe_permute_workspace_bytes(int32_t pairs, int32_t experts) {
    if (pairs <= 0 || experts <= 0 || experts > 1024) return 0;
    return a256(4 * permute_counts_words(pairs, experts));
}

int mrun_moe_permute(const uint32_t *ids, int32_t pairs, int32_t top_k, int32_t experts,
                     uint32_t *offsets, uint32_t *order, uint32_t *inverse, uint32_t *token,
                     void *workspace, size_t workspace_bytes, mrun_stream_t stream) {
    Status st;
    if (!ids || !offsets) st = Err(MRUN_ERR_INVALID, "ids and offsets are required");
    else if (pairs <= 0 || top_k <= 0 || pairs % top_k != 0)
        st = Err(MRUN_ERR_INVALID, "pairs must be a positive multiple of top_k");
    else if (experts <= 0 || experts > 1024)
        st = Err(MRUN_ERR_UNSUPPORTED, "permute runs 1..=1024 experts");
    const size_t need = st.ok() ? mrun_moe_permute_workspace_bytes(pairs, experts) : 0;
    if (st.ok() && (!workspace || workspace_bytes < need))
        st = Err(MRUN_ERR_WORKSPACE, "permute needs " + std::to_string(need) + " workspace bytes");
    if (st.ok()) {
        PermuteOut po{};
        po.offsets = offsets, po.order = order, po.inverse = inverse, po.token = token;
        st = hip_status(launch_permute(ids, pairs, top_k, experts, (uint32_t *)workspace, po,
                                       (hipStream_t)stream),
                        "permute");
    }
    return report(st);
}

int mrun_moe_workspace_routing(const mrun_moe_config *cfg, int32_t tokens, size_t *at) {
    Status st;
    if (!cfg || !at) st = Err(MRUN_ERR_INVALID, "cfg and at are required");
    else if (tokens <= 0) st = Err(MRUN_ERR_INVALID, "tokens must be positive");
    if (st.ok()) st = check_config(*cfg);
    if (st.ok()) {
        const Plan p = make_plan(*cfg, tokens);
        at[0] = p.ids, at[1] = p.scores, at[2] = p.offsets, at[3] = p.order, at[4] = p.inverse;
        at[5] = p.token;
    }
    return report(st);
}

// gather_qmm's workspace: the routing of its indices and, above 16 indices, the grouped GEMM's
// operands (x packed with its group sums, each tile's x rows) and its output in expert order.
struct GqPlan {
    size_t offsets, order, inverse, active, n_active, tiles, n_tiles, counts, xp, xs, tile_rows, ys;
    size_t total;
    size_t max_tiles;
};

static GqPlan gq_plan(int n, int experts, int x_rows, int in, int out) {
    GqPlan p{};
    size_t at = 0;
    auto take = [&](size_t bytes) {
        const size_t o = at;
        at += a256(bytes);
        return o;
    };
    p.max_tiles = (size_t)(n + kGemmTileM - 1) / kGemmTileM + experts;
    p.offsets = take(4 * ((size_t)experts + 1));
    p.order = take(4 * (size_t)n);
    p.active = take(4 * (size_t)experts);
    p.n_active = take(4);
    p.tiles = take(12 * p.max_tiles);
    p.n_tiles = take(4);
    p.counts = take(4 * permute_counts_words(n, experts));
    if (n > 16) {
        p.inverse = take(4 * (size_t)n);
        p.xp = take(2 * (size_t)x_rows * in);
        p.xs = take(2 * 3 * (size_t)x_rows * (in / 64));
        p.tile_rows = take(4 * p.max_tiles * kGemmTileM);
        p.ys = take(2 * (size_t)n * out);
    }
    p.total = at;
    return p;
}

size_t mrun_gather_qmm_workspace_bytes(int32_t n, int32_t experts, int32_t x_rows, int32_t in,
                                       int32_t out) {
    if (n <= 0 || experts <= 0 || experts > 1024 || x_rows <= 0 || in <= 0 || out <= 0) return 0;
    return gq_plan(n, experts, x_rows, in, out).total;
}

int mrun_gather_qmm(const mrun_bf16 *x, int32_t x_rows, const mrun_quantized *w,
                    const uint32_t *indices, int32_t n, int32_t sorted_indices, mrun_bf16 *out,
                    void *workspace, size_t workspace_bytes, mrun_stream_t stream) {
    (void)sorted_indices;  // the permute below orders any index list; sorted input stays put
    Status st;
    if (w && n == 0 && x_rows >= 0) {  // no index: an empty result, nothing to do
        st = check_quantized(w, "gather_qmm weight", w->experts, w->out, w->in);
        return report(st);
    }
    if (!w || !indices || x_rows <= 0 || n <= 0 || n % x_rows != 0)
        st = Err(MRUN_ERR_INVALID, "gather_qmm: n must be a positive multiple of x_rows");
    if (st.ok()) st = check_quantized(w, "gather_qmm weight", w->experts, w->out, w->in);
    if (st.ok()) st = check_ptr(x, "x");
    if (st.ok()) st = check_ptr(out, "out");
    if (st.ok() && w->experts > 1024) st = Err(MRUN_ERR_UNSUPPORTED, "more than 1024 experts");
    const size_t need =
        st.ok() ? mrun_gather_qmm_workspace_bytes(n, w->experts, x_rows, w->in, w->out) : 0;
    if (st.ok() && (!workspace || workspace_bytes < need))
        st = Err(MRUN_ERR_WORKSPACE, "gather_qmm needs " + std::to_string(need) + " bytes");
    if (st.ok()) {
        hipStream_t s = (hipStream_t)stream;
        char *ws = (char *)workspace;
        const int E = w->experts, per_x = n / x_rows;
        const GqPlan p = gq_plan(n, E, x_rows, w->in, w->out);
        auto u32 = [&](size_t off) { return (uint32_t *)(ws + off); };
        PermuteOut po{};
        po.offsets = u32(p.offsets), po.order = u32(p.order), po.active = u32(p.active);
        po.n_active = u32(p.n_active), po.tiles = u32(p.tiles), po.n_tiles = u32(p.n_tiles);
        po.tile_m = kGemmTileM;
        Routing rt{po.offsets, po.active, po.n_active, po.tiles, po.n_tiles};
        // the tuned grouped GEMM (4-bit group 64, in % 512, out % 256): x packed, the tiles' x
        // rows from the permute, the product in expert order, then each index's row in place
        MoeGemmJob mj{};
        if (n > 16) {
            mj.A = (const bf16_t *)(ws + p.xp), mj.lda = w->in, mj.a_rows = x_rows;
            mj.AX = (const bf16_t *)(ws + p.xs);
            mj.ax_e = w->in / 64, mj.tile_rows = u32(p.tile_rows), mj.K = w->in, mj.N = w->out;
            mj.glu = 0, mj.w0 = qw_of(*w), mj.routing = rt, mj.has_routing = 1;
            mj.max_tiles = (int)p.max_tiles, mj.out = (bf16_t *)(ws + p.ys), mj.ldo = w->out;
        }
        const bool tuned = n > 16 && moe_gemm_supported(mj);
        if (tuned) po.inverse = u32(p.inverse), po.tile_rows = u32(p.tile_rows);
        st = hip_status(launch_permute(indices, n, tuned ? per_x : 1, E, u32(p.counts), po, s),
                        "gather_qmm permute");
        if (st.ok() && tuned) {
            st = hip_status(launch_apack(x, w->in, x_rows, w->in, (bf16_t *)(ws + p.xp), w->in,
                                         (bf16_t *)(ws + p.xs), s),
                            "gather_qmm pack x");
            if (st.ok()) st = hip_status(launch_moe_gemm(mj, s), "gather_qmm (moe gemm)");
            if (st.ok())
                st = hip_status(launch_rows_gather((const bf16_t *)(ws + p.ys), po.inverse, n, w->out,
                                                   out, s),
                                "gather_qmm rows");
        } else if (st.ok() && n > 16 && w->in % 64 == 0) {
            GemmJob j{};
            j.A = x, j.lda = w->in, j.a_map = po.order, j.a_div = per_x, j.N = w->out, j.K = w->in;
            j.w0 = qw_of(*w), j.routing = rt, j.has_routing = 1, j.max_tiles = (int)p.max_tiles;
            j.o_map = po.order, j.out = out, j.ldo = w->out;
            st = hip_status(launch_gemm(j, s), "gather_qmm (mfma)");
        } else if (st.ok()) {
            GemvJob j{};
            j.A = x, j.lda = w->in, j.a_map = po.order, j.a_div = per_x, j.w0 = qw_of(*w);
            j.routing = rt, j.has_routing = 1, j.max_slots = E < n ? E : n;
            j.o_map = po.order, j.out = out, j.ldo = w->out;
            st = hip_status(launch_gemv(j, s), "gather_qmm (gemv)");
        }
    }
    return report(st);
}

int mrun_quantized_matmul(const mrun_bf16 *x, int32_t rows, const mrun_quantized *w,
                          mrun_bf16 *out, mrun_stream_t stream) {
    Status st;
    if (!w || rows < 0) st = Err(MRUN_ERR_INVALID, "quantized_matmul: bad arguments");
    if (st.ok()) st = check_quantized(w, "quantized_matmul weight", 1, w->out, w->in);
    if (st.ok() && rows == 0) return report(st);  // an empty batch: nothing to do
    if (st.ok()) st = check_ptr(x, "x");
    if (st.ok()) st = check_ptr(out, "out");
    if (st.ok()) st = tensor::quantized_matmul(x, rows, *w, out, (hipStream_t)stream);
    return report(st);
}

int mrun_linear_forward(const mrun_linear *l, const mrun_bf16 *x, int32_t rows, mrun_bf16 *out,
                        mrun_stream_t stream) {
    Status st;
    if (!l || rows < 0) st = Err(MRUN_ERR_INVALID, "linear: bad arguments");
    if (st.ok() && l->weight) st = check_ptr(l->weight, "weight");
    if (st.ok() && !l->weight) st = check_quantized(&l->q, "linear weight", 1, l->out, l->in);
    if (st.ok() && l->weight && (l->out <= 0 || l->in <= 0))
        st = Err(MRUN_ERR_INVALID, "linear: bad shape");
    if (st.ok() && rows == 0) return report(st);  // an empty batch: nothing to do
    if (st.ok()) st = check_ptr(x, "x");
    if (st.ok()) st = check_ptr(out, "out");
    if (st.ok()) st = tensor::linear(x, rows, *l, out, (hipStream_t)stream);
    return report(st);
}

int mrun_swiglu(const mrun_bf16 *gate, const mrun_bf16 *up, int64_t n, mrun_bf16 *out,
                mrun_stream_t stream) {
    Status st;
    if (n < 0) st = Err(MRUN_ERR_INVALID, "swiglu: n < 0");
    if (st.ok()) st = check_ptr(gate, "gate");
    if (st.ok()) st = check_ptr(up, "up");
    if (st.ok()) st = check_ptr(out, "out");
    if (st.ok()) st = hip_status(launch_swiglu(gate, up, n, out, (hipStream_t)stream), "swiglu");
    return report(st);
}

int mrun_moe_combine(const mrun_bf16 *y, const uint32_t *inverse, const mrun_bf16 *scores,
                     int32_t tokens, int32_t top_k, int32_t hidden, const mrun_bf16 *shared_y,
                     const mrun_bf16 *shared_logit, mrun_bf16 *out, mrun_stream_t stream) {
    Status st;
    if (tokens < 0 || top_k <= 0 || hidden <= 0 || hidden % 8 != 0)
        st = Err(MRUN_ERR_INVALID, "combine: bad shape (hidden must be a multiple of 8)");
    else if (top_k > 16)
        st = Err(MRUN_ERR_UNSUPPORTED, "combine: top_k above 16");
    if (st.ok() && tokens == 0) return report(st);  // an empty batch: nothing to do
    if (st.ok()) st = check_ptr(y, "y");
    if (st.ok() && !scores) st = Err(MRUN_ERR_INVALID, "scores is null");
    if (st.ok() && shared_y) st = check_ptr(shared_y, "shared_y");
    if (st.ok() && shared_y && !shared_logit)
        st = Err(MRUN_ERR_INVALID, "shared_y needs shared_logit");
    if (st.ok()) st = check_ptr(out, "out");
    if (st.ok())
        st = hip_status(launch_combine(y, inverse, scores, tokens, top_k, hidden, shared_y,
                                       shared_logit, out, (hipStream_t)stream),
                        "combine");
    return report(st);
}

size_t mrun_moe_stack_workspace_bytes(const mrun_moe_config *cfg, int32_t tokens) {
    const size_t block = mrun_moe_workspace_bytes(cfg, tokens);
    if (block == 0) return 0;
    return block + 2 * a256(2 * (size_t)tokens * cfg->hidden);  // h and the block output
}

int mrun_moe_stack_forward(const mrun_sparse_moe *layers, int32_t n_layers,
                           const mrun_bf16 *const *norm_w, float eps, mrun_bf16 *x, int32_t tokens,
                           void *workspace, size_t workspace_bytes, mrun_stream_t stream) {
    Status st;
    if (!layers || n_layers <= 0) st = Err(MRUN_ERR_INVALID, "stack: no layers");
    for (int32_t l = 0; st.ok() && l < n_layers; ++l) {
        st = check_block(&layers[l]);
        if (st.ok() && std::memcmp(&layers[l].cfg, &layers[0].cfg, sizeof(mrun_moe_config)) != 0)
            st = Err(MRUN_ERR_INVALID, "stack: layers must share one config");
    }
    if (st.ok() && tokens < 0) st = Err(MRUN_ERR_INVALID, "tokens must not be negative");
    if (st.ok() && tokens == 0) return report(st);  // an empty batch: nothing to do
    if (st.ok()) st = check_ptr(x, "x");
    if (st.ok()) st = check_ptr(workspace, "workspace");
    const mrun_moe_config &c = layers[0].cfg;
    const size_t need = st.ok() ? mrun_moe_stack_workspace_bytes(&c, tokens) : 0;
    if (st.ok() && workspace_bytes < need)
        st = Err(MRUN_ERR_WORKSPACE, "workspace of " + std::to_string(workspace_bytes) +
                                         " bytes, need " + std::to_string(need));
    if (st.ok()) {
        const int D = c.hidden;
        const size_t blk = mrun_moe_workspace_bytes(&c, tokens);
        char *ws = (char *)workspace;
        bf16_t *h = (bf16_t *)(ws + blk);
        bf16_t *o = (bf16_t *)(ws + blk + a256(2 * (size_t)tokens * D));
        hipStream_t s = (hipStream_t)stream;
        auto wl = [&](int l) { return norm_w ? norm_w[l] : nullptr; };
        // decode-sized chunks with dense or 4/8-bit routers: the norm runs inside each block's
        // router launch and the residual add inside its last launch (three launches per layer,
        // no norm kernel)
        const int chunk = models::decode_launch_tokens(c, tokens);  // tokens per decode launch
        bool fused = models::decode_schedule(layers[0], tokens) &&
                     2 * (size_t)chunk * D <= 65536;  // the normalised rows fit the router's LDS
        for (int32_t l = 0; fused && l < n_layers; ++l)
            fused = models::k1_router_ok(layers[l].gate) &&
                    (c.shared_intermediate == 0 || models::k1_router_ok(layers[l].shared_expert_gate));
        for (int32_t l = 0; fused && st.ok() && l < n_layers; ++l) {
            const models::FusedNorm fn{x, wl(l), eps};
            st = models::sparse_moe_forward(layers[l], h, tokens, x, ws, blk, s, nullptr, &fn);
        }
        if (!fused)
            st = hip_status(launch_rms_norm(x, nullptr, wl(0), tokens, D, eps, nullptr, h, s), "stack norm");
        for (int32_t l = 0; !fused && st.ok() && l < n_layers; ++l) {
            // x = R(x + o), and the next layer's input h = rms_norm(x) (the last h is unused):
            // inside the block's combine launch when it has one, else a launch of its own
            const bf16_t *w = wl(l + 1 < n_layers ? l + 1 : l);
            const PostNorm pn{x, w, eps, h};
            bool done = false;
            st = models::sparse_moe_forward(layers[l], h, tokens, o, ws, blk, s, nullptr, nullptr,
                                            &pn, &done);
            if (!st.ok()) break;
            if (!done)
                st = hip_status(launch_rms_norm(x, o, w, tokens, D, eps, x, h, s),
                                "stack add_rms_norm");
        }
    }
    return report(st);
}

int mrun_rms_norm(const mrun_bf16 *x, const mrun_bf16 *w, int32_t rows, int32_t hidden, float eps,
                  mrun_bf16 *out, mrun_stream_t stream) {
    Status st;
    if (rows < 0 || hidden <= 0 || hidden % 8 != 0)
        st = Err(MRUN_ERR_INVALID, "rms_norm: bad shape (hidden must be a multiple of 8)");
    if (st.ok() && rows == 0) return report(st);  // an empty batch: nothing to do
    if (st.ok()) st = check_ptr(x, "x");
    if (st.ok()) st = check_ptr(out, "out");
    if (st.ok() && x == out) st = Err(MRUN_ERR_INVALID, "rms_norm: out must not alias x");
    if (st.ok())
        st = hip_status(launch_rms_norm(x, nullptr, w, rows, hidden, eps, nullptr, out,
                                        (hipStream_t)stream),
                        "rms_norm");
    return report(st);
}

int mrun_add_rms_norm(const mrun_bf16 *x, const mrun_bf16 *residual, const mrun_bf16 *w,
                      int32_t rows, int32_t hidden, float eps, mrun_bf16 *h, mrun_bf16 *y,
                      mrun_stream_t stream) {
    Status st;
    if (rows < 0 || hidden <= 0 || hidden % 8 != 0)
        st = Err(MRUN_ERR_INVALID, "add_rms_norm: bad shape (hidden must be a multiple of 8)");
    if (st.ok() && rows == 0) return report(st);  // an empty batch: nothing to do
    if (st.ok()) st = check_ptr(x, "x");
    if (st.ok()) st = check_ptr(residual, "residual");
    if (st.ok()) st = check_ptr(h, "h");
    if (st.ok()) st = check_ptr(y, "y");
    if (st.ok() && (y == x || y == residual || y == h))
        st = Err(MRUN_ERR_INVALID, "add_rms_norm: y must not alias its inputs");
    if (st.ok())
        st = hip_status(launch_rms_norm(x, residual, w, rows, hidden, eps, h, y,
                                        (hipStream_t)stream),
                        "add_rms_norm");
    return report(st);
}

}  // extern "C"
