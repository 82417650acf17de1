/*
 * mrun_moe.h — C ABI of the MI355X-native MoE sparse block.
 *
 * This is the drop-in boundary for the MoE path of hupe1980/mrun's mrun-engine. In the reference
 * every op of that path goes through the Rust tensor facade crates/mrun-engine/src/tensor/nuvec.rs
 * (the only module that touches the backend, tensor/mod.rs:1-4); the entry points below are what a
 * Rust `-sys` crate behind that facade binds, one per facade op or layer the path uses. Paths in
 * citations are relative to the reference checkout.
 *
 * Conventions (mirroring the facade):
 *  - Tensors are caller-owned DEVICE memory (hipMalloc'd), row-major, bf16 passed as uint16_t bits.
 *  - Every call is asynchronous on the caller's HIP stream (NULL = the null stream), as the facade's
 *    ops are lazy until async_eval (nuvec.rs:4-8, 267-275). Nothing allocates device memory on the
 *    hot path: scratch comes from a caller workspace sized by the *_workspace_bytes functions.
 *  - Every call returns 0 on success or a nonzero MRUN_ERR_* status, with a message readable from
 *    mrun_last_error() on the same thread — the facade's Result<_, tensor::Error(String)>
 *    (nuvec.rs:18-38). A failed call enqueues no work.
 *  - One stream per caller thread; the library starts no threads (engine.rs:647-648).
 *  - A token or row count of 0 is an empty batch, as the facade's ops take empty arrays: the call
 *    checks its weights and configuration, enqueues no work and returns 0 (no pointer or
 *    workspace is read). Negative counts are MRUN_ERR_INVALID. mrun_moe_permute needs at least one
 *    pair (the reference sorts only when T*k >= 64, moe.rs:17, 64).
 *  - Numerics follow the reference's bf16 semantics: each op computes in f32 and rounds its output
 *    once to bf16 (round to nearest even); contractions accumulate in f32.
 */
#ifndef MRUN_MOE_H
#define MRUN_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t mrun_bf16;   /* bfloat16 bits */
typedef void *mrun_stream_t;  /* hipStream_t */

enum {
    MRUN_OK = 0,
    MRUN_ERR_INVALID = 1,      /* bad shape, pointer or argument */
    MRUN_ERR_UNSUPPORTED = 2,  /* a valid reference configuration this build does not run */
    MRUN_ERR_WORKSPACE = 3,    /* workspace too small */
    MRUN_ERR_HIP = 4,          /* the HIP runtime reported an error */
};

/* tensor::Quantized (nuvec.rs:602-638): affine codes, scales and biases with their group size and
 * bits. weight [experts, out, in*bits/32] u32, LSB-first codes (nuvec.rs:1199-1203); scales and
 * biases [experts, out, in/group_size] bf16; biases NULL means zeros (nuvec.rs:604, 616-619).
 * A non-stacked weight (quantized_matmul) has experts = 1.
 * bits = 16 carries unquantized experts (SwitchLinear::Dense, moe.rs:43-46, run by gather_mm,
 * nuvec.rs:688-697): weight points to bf16 [experts, out, in], scales and biases are NULL and
 * group_size is ignored. bits = 32 carries dense f32 weights the same way (weight -> float
 * [experts, out, in]); only mrun_moe_forward_f32 runs them. */
typedef struct mrun_quantized {
    const uint32_t *weight;
    const mrun_bf16 *scales;
    const mrun_bf16 *biases;
    int32_t experts, out, in, group_size, bits;
} mrun_quantized;

/* load::Linear (load.rs:246-306): y = x W^T (+ bias). Dense when `weight` is not NULL ([out, in]
 * bf16), else quantized by `q`. bias [out] bf16 or NULL. */
typedef struct mrun_linear {
    const mrun_bf16 *weight;
    mrun_quantized q;
    const mrun_bf16 *bias;
    int32_t out, in;
} mrun_linear;

/* MoeConfig (moe.rs:97-107); shared_intermediate 0 = no shared expert (Qwen3-MoE). */
typedef struct mrun_moe_config {
    int32_t hidden, experts, top_k, intermediate, norm_topk_prob, shared_intermediate;
} mrun_moe_config;

/* SparseMoe (moe.rs:109-147): the router `gate`, the SwitchGlu projections and, with a shared
 * expert, its Mlp (common.rs:311-339) and `shared_expert_gate`. */
typedef struct mrun_sparse_moe {
    mrun_moe_config cfg;
    mrun_linear gate;
    mrun_quantized switch_gate_proj, switch_up_proj, switch_down_proj;
    mrun_linear shared_gate_proj, shared_up_proj, shared_down_proj, shared_expert_gate;
} mrun_sparse_moe;

/* The message of this thread's last failed call ("" when none). */
const char *mrun_last_error(void);

/* Library version string. */
const char *mrun_version(void);

/* Validates a block's configuration and weight shapes as SparseMoe::load does
 * (moe.rs:120-147, load.rs:14-156, qwen3_5_moe.rs:508-513); a block with f32 (bits 32) experts
 * as mrun_moe_forward_f32 takes it. No device work. */
int mrun_moe_check(const mrun_sparse_moe *moe);

/* Workspace bytes mrun_moe_forward needs for `tokens` rows (the counterpart of
 * SparseMoe::scratch_per_token, moe.rs:176-187). Returns 0 for an invalid config. */
size_t mrun_moe_workspace_bytes(const mrun_moe_config *cfg, int32_t tokens);

/* SparseMoe::forward (moe.rs:149-174), also Ffn::forward's Moe arm (moe.rs:202-207):
 * x [tokens, hidden] -> out [tokens, hidden]. out must not alias x. */
int mrun_moe_forward(const mrun_sparse_moe *moe, const mrun_bf16 *x, int32_t tokens,
                     mrun_bf16 *out, void *workspace, size_t workspace_bytes,
                     mrun_stream_t stream);

/* SparseMoe::forward (moe.rs:149-174) for a block whose tensors are all float32, as the reference
 * runs an f32 checkpoint: its Hugging Face fixture is f32 (gen_tiny.py:235-274) because MLX runs
 * the dense gather_mm (nuvec.rs:688-697) only in f32, and every op of the block then computes and
 * keeps f32. Every weight is dense f32 with bits = 32: the experts as mrun_quantized (weight ->
 * float [experts, out, in], scales and biases NULL), each Linear in its `q` (experts 1, `weight`
 * and `bias` NULL). x, out [tokens, hidden] float; out must not alias x. The op sequence is
 * mrun_moe_forward's without its bf16 roundings: f32 softmax, top-k with equal gates ranked by
 * lower id, SwiGLU, the weighted combine (pairs in rank order) and the sigmoid-gated shared
 * expert. mrun_moe_forward refuses bits-32 weights with MRUN_ERR_UNSUPPORTED. */
size_t mrun_moe_workspace_bytes_f32(const mrun_moe_config *cfg, int32_t tokens);
int mrun_moe_forward_f32(const mrun_sparse_moe *moe, const float *x, int32_t tokens, float *out,
                         void *workspace, size_t workspace_bytes, mrun_stream_t stream);

/* mrun_moe_forward for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). It has no counterpart in the reference.
 * The workspace is a fixed scratch array inside the library, one per GPU, held until the process
 * ends: mrun_moe_forward_noalloc_max_bytes() bytes (32 MiB: every decode batch, and prefill
 * chunks whose mrun_moe_workspace_bytes fits, e.g. up to 649 tokens of the Qwen3.6-like
 * block). A batch that needs more returns MRUN_ERR_WORKSPACE. The call allocates nothing; the
 * caller still passes x and out. Every call on one GPU shares that GPU's array, so calls that
 * overlap in time on one GPU (two streams, two threads) race: serialise them.
 * mrun_moe_forward_noalloc_max_bytes() also resolves the current GPU's scratch address; call it
 * once on each GPU before capturing a graph, so that no call under capture looks up a symbol. */
int mrun_moe_forward_noalloc(const mrun_sparse_moe *moe, const mrun_bf16 *x, int32_t tokens,
                             mrun_bf16 *out, mrun_stream_t stream);
size_t mrun_moe_forward_noalloc_max_bytes(void);

/* mrun_moe_forward with benchmark instrumentation; it has no counterpart in the reference and is
 * for profilers and benchmarks that time each stage on the device. events are hipEvent_t handles
 * created by the caller: events[0] is recorded on the stream before the first launch and
 * events[i + 1] after stage i, while i + 1 < n_events. *n_stages receives the stage count; the
 * stage names, comma-separated, are mrun_moe_stage_names(cfg, tokens). */
int mrun_moe_forward_profiled(const mrun_sparse_moe *moe, const mrun_bf16 *x, int32_t tokens,
                              mrun_bf16 *out, void *workspace, size_t workspace_bytes,
                              mrun_stream_t stream, void **events, int32_t n_events,
                              int32_t *n_stages);
const char *mrun_moe_stage_names(const mrun_moe_config *cfg, int32_t tokens);

/* mrun_moe_forward with the decode gate/up kernel timed from inside (benchmark instrumentation;
 * no counterpart in the reference): clock is a device buffer of 64 u64 pairs that the caller sets
 * to (UINT64_MAX, 0) beforehand; workgroup i of the kernel lowers pair i % 64's first value to
 * its start and raises its second to its waves' ends, in ticks of the device's constant wall
 * clock (mrun_wall_clock_hz). The largest second value minus the smallest first one is the
 * kernel's duration without launch gaps or dispatch latency. A batch that runs the prefill
 * schedule has no such kernel: the call returns MRUN_ERR_UNSUPPORTED and enqueues nothing. */
int mrun_moe_forward_timed(const mrun_sparse_moe *moe, const mrun_bf16 *x, int32_t tokens,
                           mrun_bf16 *out, void *workspace, size_t workspace_bytes,
                           mrun_stream_t stream, uint64_t *clock);

/* Ticks per second of the wall clock mrun_moe_forward_timed reads, on the current device; -1 if
 * the runtime does not report it. */
int64_t mrun_wall_clock_hz(void);

/* Where a forward leaves its routing inside the caller's workspace (instrumentation for tests and
 * profilers; no counterpart in the reference, whose intermediate arrays are not observable). For
 * `tokens` rows, at[0..6) receive byte offsets into the workspace of: ids [tokens, k] u32 and
 * scores [tokens, k] bf16 (the router's choice, moe.rs:151-159), and, for a batch that runs the
 * prefill schedule (more than 32 tokens; more than 16 with experts the decode kernels do not
 * take), the sorted dispatch of SwitchGlu::forward (moe.rs:65-75): offsets [experts + 1], order,
 * inverse and token [tokens*k]. They hold the last forward's values until the workspace is
 * reused. */
int mrun_moe_workspace_routing(const mrun_moe_config *cfg, int32_t tokens, size_t *at);

/* The router of SparseMoe::forward (moe.rs:151-159): logits = gate.forward(x) (load.rs:294-306),
 * gates = softmax(logits, precise) (nuvec.rs:593-598), ids = the top-k of argpartition + slice
 * (nuvec.rs:558-562, 313-316; equal gates rank the lower id first, ids listed by rank), scores =
 * take_along_axis(gates, ids) normalised by sum when norm_topk_prob (nuvec.rs:538-540, 585, 503).
 * logits and gates [tokens, experts] are optional outputs (NULL to skip); ids [tokens, k] u32,
 * scores [tokens, k] bf16. */
int mrun_moe_router(const mrun_sparse_moe *moe, const mrun_bf16 *x, int32_t tokens,
                    mrun_bf16 *logits, mrun_bf16 *gates, uint32_t *ids, mrun_bf16 *scores,
                    void *workspace, size_t workspace_bytes, mrun_stream_t stream);

/* The sorted dispatch of SwitchGlu::forward (moe.rs:65-75): order = argsort(flat ids) (stable,
 * nuvec.rs:554-556), inverse = argsort(order), token = floor_divide(order, k) (nuvec.rs:523-526).
 * ids [pairs] u32 with pairs = tokens*k; offsets [experts + 1] (expert e's sorted rows are
 * [offsets[e], offsets[e+1])), order, inverse, token [pairs]. Any output may be NULL except
 * offsets. Ids must be below `experts` (others are skipped and leave their entries unwritten).
 * The workspace holds per-block expert counts: mrun_moe_permute_workspace_bytes(pairs, experts)
 * bytes. */
int mrun_moe_permute(const uint32_t *ids, int32_t pairs, int32_t top_k, int32_t experts,
                     uint32_t *offsets, uint32_t *order, uint32_t *inverse, uint32_t *token,
                     void *workspace, size_t workspace_bytes, mrun_stream_t stream);
size_t mrun_moe_permute_workspace_bytes(int32_t pairs, int32_t experts);

/* tensor::gather_qmm (nuvec.rs:670-686, transpose = true): out[p] = x[p / (n / x_rows)] .
 * dequant(w[indices[p]])^T for p < n, i.e. x [x_rows, in] broadcast over the n / x_rows indices of
 * each row (SwitchGlu's unsorted case, moe.rs:62, 79-83) or one row per index (its sorted case).
 * sorted_indices promises ascending indices, as in the reference. out [n, w->out]. */
int mrun_gather_qmm(const mrun_bf16 *x, int32_t x_rows, const mrun_quantized *w,
                    const uint32_t *indices, int32_t n, int32_t sorted_indices, mrun_bf16 *out,
                    void *workspace, size_t workspace_bytes, mrun_stream_t stream);
/* Workspace of mrun_gather_qmm for n indices over `experts` experts, x [x_rows, in], out width
 * `out` (the routing of the indices and, above 16 indices, the grouped GEMM's packed x and its
 * output in expert order). */
size_t mrun_gather_qmm_workspace_bytes(int32_t n, int32_t experts, int32_t x_rows, int32_t in,
                                       int32_t out);

/* tensor::quantized_matmul (nuvec.rs:660-663): out [rows, w->out] = x . dequant(w)^T, w with
 * experts = 1. */
int mrun_quantized_matmul(const mrun_bf16 *x, int32_t rows, const mrun_quantized *w,
                          mrun_bf16 *out, mrun_stream_t stream);

/* Linear::forward (load.rs:294-306): out = R(x W^T) and, with a bias, R(out + bias). */
int mrun_linear_forward(const mrun_linear *l, const mrun_bf16 *x, int32_t rows, mrun_bf16 *out,
                        mrun_stream_t stream);

/* activations::swiglu (activations.rs:55-59): out = R(silu(gate) * up), f32 inside. n elements. */
int mrun_swiglu(const mrun_bf16 *gate, const mrun_bf16 *up, int64_t n, mrun_bf16 *out,
                mrun_stream_t stream);

/* The combine of SparseMoe::forward (moe.rs:84-93, 161-171): for token t,
 * routed = R(sum_j R(y[row(t, j)] * scores[t, j])) where row(t, j) = inverse[t*k + j] when
 * inverse is given (y in sorted order) else t*k + j; then, when shared_y is given,
 * out = R(routed + R(R(sigmoid(shared_logit[t])) * shared_y[t])). y [tokens*k, hidden],
 * shared_y [tokens, hidden], shared_logit [tokens]. */
int mrun_moe_combine(const mrun_bf16 *y, const uint32_t *inverse, const mrun_bf16 *scores,
                     int32_t tokens, int32_t top_k, int32_t hidden, const mrun_bf16 *shared_y,
                     const mrun_bf16 *shared_logit, mrun_bf16 *out, mrun_stream_t stream);

/* fast::rms_norm (nuvec.rs:796-798) as RmsNorm::forward (load.rs:361-363): out = R(R(x *
 * rsqrt(mean(x^2) + eps)) * w), f32 inside; w [hidden] or NULL (ones). */
int mrun_rms_norm(const mrun_bf16 *x, const mrun_bf16 *w, int32_t rows, int32_t hidden, float eps,
                  mrun_bf16 *out, mrun_stream_t stream);

/* fast::add_rms_norm (nuvec.rs:800-811): h = R(x + residual); y = rms_norm(h). h and y
 * [rows, hidden]; h may alias x or residual. */
int mrun_add_rms_norm(const mrun_bf16 *x, const mrun_bf16 *residual, const mrun_bf16 *w,
                      int32_t rows, int32_t hidden, float eps, mrun_bf16 *h, mrun_bf16 *y,
                      mrun_stream_t stream);

/* The decoder-layer loop around the MoE block for a stack of MoE layers (qwen3_5_moe.rs:622-624,
 * 664-666): for each layer l, h = rms_norm(x) * norm_w[l] (eps; load.rs:361-363), then
 * x = R(x + SparseMoe_l(h)). The residual add of layer l and the norm of layer l + 1 run as one
 * add_rms_norm (nuvec.rs:800-811). x [tokens, hidden] is updated in place. norm_w holds n_layers
 * pointers to [hidden] bf16 weights (NULL, or a NULL entry, means weight 1). All layers share one
 * config. */
int mrun_moe_stack_forward(const mrun_sparse_moe *layers, int32_t n_layers,
                           const mrun_bf16 *const *norm_w, float eps, mrun_bf16 *x, int32_t tokens,
                           void *workspace, size_t workspace_bytes, mrun_stream_t stream);
size_t mrun_moe_stack_workspace_bytes(const mrun_moe_config *cfg, int32_t tokens);

#ifdef __cplusplus
}
#endif
#endif
