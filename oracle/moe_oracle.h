/*
 * CPU restatement of the reference's MoE sparse block: TEST INFRASTRUCTURE ONLY.
 *
 * This is the parity oracle and the CPU baseline. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it, and only as the checker. The product path
 * (mrun_amd/, libmrun_moe.so) never links, loads or calls it.
 *
 * What it restates (reference paths relative to the hupe1980/mrun checkout):
 *   crates/mrun-engine/src/models/moe.rs:16-17, 40-95, 149-174   op order, SORT_AT, dispatch
 *   crates/mrun-engine/src/models/activations.rs:45-59            swiglu = silu(g)*u, one rounding
 *   crates/mrun-engine/src/models/common.rs:336-339                shared Mlp
 *   crates/mrun-engine/src/load.rs:294-306                         Linear: x*W^T, then +bias
 *   crates/mrun-engine/src/tensor/nuvec.rs:593-598 (softmax, f32, one rounding),
 *     602-626 (absent affine biases are zeros), 670-686 (gather_qmm), 523-526 (floor_divide),
 *     1173-1204 (affine dequant, LSB-first nibbles), 796-811 (rms_norm, add_rms_norm)
 *   crates/mrun-engine/src/models/qwen3_5_moe.rs:622-624           residual add around the block
 *
 * Numerics: every tensor is stored as bf16; each op computes in f32 and rounds once to bf16
 * with round-to-nearest-even. Contractions accumulate in f32 in ascending index order.
 * Choices the reference leaves implementation-defined, fixed here:
 *   - top-k: the k largest bf16 gates; equal gates rank the lower expert id first; the k ids of a
 *     token are listed in that rank order (nuvec.rs:558-562 leaves the order open);
 *   - argsort is stable (pairs of one expert stay in token order).
 *
 * How each function is pinned (tests/test_oracle_*.py):
 *   orc_bf16_from_f32      torch's float32->bfloat16 conversion (RNE) on random and edge values
 *   orc_dequant_row        nuvec.rs:1173-1204 known answers (LSB-first nibbles, code*scale+bias,
 *                          zero biases); brute force on tiny shapes; dense bf16 rows (bits 16)
 *                          equal the stored weights
 *   orc_qmatmul / orc_gather_qmm   numpy float64 dequant+matmul (within f32 accumulation error),
 *                          the expert-selection closed form of nuvec.rs:1331-1357
 *   orc_linear             numpy float64 matmul + bias with the two roundings
 *   orc_softmax            scipy.special.softmax in float64 (within one bf16 ulp), nuvec.rs:1311-1319
 *   orc_topk               brute-force lexsort over (gate desc, id asc)
 *   orc_norm_scores        closed form
 *   orc_permute            numpy.argsort(kind="stable") (the reference's argsort), order/inverse
 *                          invariants, floor_divide known answers (nuvec.rs:1264-1309)
 *   orc_swiglu             the closed form of activations.rs:92-123
 *   orc_combine            numpy restatement
 *   orc_rms_norm           torch.nn.functional.rms_norm in float32
 *   orc_moe_forward        an independent numpy float64 restatement of the whole block with the
 *                          same rounding points, on tiny and small shapes
 *   orc_moe_forward_f32    the same numpy restatement without roundings (float64, within f32
 *                          accumulation error); closed forms of one-expert and zero-weight blocks
 * Functions whose arithmetic only nuvec could pin (its accumulation order, its exp, its
 * argpartition tie order) are pinned by the checks above to within those freedoms.
 */
#ifndef MRUN_MOE_ORACLE_H
#define MRUN_MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t orc_bf16;

/* tensor::Quantized (nuvec.rs:602-626): codes [experts, out, in*bits/32], scales and biases
 * [experts, out, in/group]; biases NULL means zeros. bits == 16 holds dense bf16 weights
 * [experts, out, in] in `codes` (SwitchLinear::Dense, moe.rs:43-46, run by gather_mm,
 * nuvec.rs:688-697), with no scales. */
typedef struct {
    const uint32_t *codes;
    const orc_bf16 *scales;
    const orc_bf16 *biases;
    int32_t experts, out, in, group, bits;
} orc_qweight;

/* load::Linear (load.rs:246-306): dense bf16 [out, in] or quantized; optional bias [out]. */
typedef struct {
    const orc_bf16 *dense;
    orc_qweight q;
    const orc_bf16 *bias;
    int32_t out, in;
} orc_linear;

/* MoeConfig (moe.rs:97-107); shared_intermediate 0 means no shared expert. */
typedef struct {
    int32_t hidden, experts, top_k, intermediate, norm_topk_prob, shared_intermediate;
} orc_config;

/* SparseMoe (moe.rs:109-115). */
typedef struct {
    orc_config cfg;
    orc_linear gate;
    orc_qweight sw_gate, sw_up, sw_down;
    orc_linear sh_gate, sh_up, sh_down, sh_expert_gate;
} orc_block;

/* Intermediates of one forward; every pointer may be NULL. */
typedef struct {
    orc_bf16 *logits;   /* [T, E] router output (after the optional bias) */
    orc_bf16 *gates;    /* [T, E] softmax */
    uint32_t *ids;      /* [T, k] */
    orc_bf16 *scores;   /* [T, k] (normalised when norm_topk_prob) */
    uint32_t *order;    /* [T*k] sorted path only: argsort of the flat ids */
    uint32_t *inverse;  /* [T*k] argsort(order) */
    orc_bf16 *act;      /* [T*k, I] swiglu output, in pair order p = t*k + j */
    orc_bf16 *y;        /* [T*k, D] expert outputs, in pair order */
    orc_bf16 *routed;   /* [T, D] */
    orc_bf16 *shared_gate; /* [T] sigmoid gate */
    orc_bf16 *shared_y; /* [T, D] shared Mlp output */
} orc_trace;

/* bf16 <-> f32 (round to nearest even; NaN stays NaN). */
orc_bf16 orc_bf16_from_f32(float f);
float orc_f32_from_bf16(orc_bf16 h);
void orc_round_bf16_array(const float *in, size_t n, orc_bf16 *out);

/* One dequantized row of expert `e`, output row `o`: code*scale + bias in f32. */
void orc_dequant_row(const orc_qweight *w, int32_t e, int32_t o, float *row);

/* y[r] = R(x[r] . W^T (+ bias, rounded again)) for a Linear; x [rows, in]. */
int orc_linear_forward(const orc_linear *l, const orc_bf16 *x, int32_t rows, orc_bf16 *y);

/* quantized_matmul (nuvec.rs:660-663): y [rows, out] = R(x . dequant(W[0])^T). */
int orc_qmatmul(const orc_qweight *w, const orc_bf16 *x, int32_t rows, orc_bf16 *y);

/* gather_qmm (nuvec.rs:670-686): pair p uses x row p / (n_idx / x_rows) and expert idx[p];
 * y [n_idx, out]. */
int orc_gather_qmm(const orc_qweight *w, const orc_bf16 *x, int32_t x_rows,
                   const uint32_t *idx, int32_t n_idx, orc_bf16 *y);

/* softmax over the last axis, f32 inside, one rounding (nuvec.rs:593-598). */
void orc_softmax(const orc_bf16 *logits, int32_t rows, int32_t n, orc_bf16 *out);

/* top-k of bf16 gates with the tie rule above: ids [rows, k]. */
int orc_topk(const orc_bf16 *gates, int32_t rows, int32_t n, int32_t k, uint32_t *ids);

/* scores = take(gates, ids); if norm: R(scores / R(sum(scores))) (moe.rs:156-159). */
void orc_scores(const orc_bf16 *gates, int32_t rows, int32_t n, const uint32_t *ids, int32_t k,
                int32_t norm, orc_bf16 *scores);

/* The sorted dispatch of SwitchGlu::forward (moe.rs:65-75): order = argsort(flat) (stable),
 * inverse = argsort(order), token = order // k. counts [E] optional. */
int orc_permute(const uint32_t *ids, int32_t pairs, int32_t k, int32_t experts, uint32_t *order,
                uint32_t *inverse, uint32_t *token, uint32_t *counts);

/* floor_divide for u32 operands (nuvec.rs:523-526). */
void orc_floor_divide_u32(const uint32_t *a, size_t n, uint32_t b, uint32_t *out);

/* swiglu(g, u) = R(silu(g) * u), silu(z) = z * sigmoid(z), f32 inside (activations.rs:45-59). */
void orc_swiglu(const orc_bf16 *g, const orc_bf16 *u, size_t n, orc_bf16 *out);
/* The same formula without the final rounding (the f32 case of activations.rs:92-123). */
void orc_swiglu_f32(const float *g, const float *u, size_t n, float *out);

/* routed[t] = R(sum_j R(y[t, j] * scores[t, j])) (moe.rs:161-165); y [T, k, D]. */
void orc_combine(const orc_bf16 *y, const orc_bf16 *scores, int32_t T, int32_t k, int32_t D,
                 orc_bf16 *routed);

/* out = R(routed + R(R(sigmoid(glogit)) * shared)) (moe.rs:166-171); glogit [T] already rounded. */
void orc_shared_add(const orc_bf16 *routed, const orc_bf16 *glogit, const orc_bf16 *shared,
                    int32_t T, int32_t D, orc_bf16 *out, orc_bf16 *gate_out);

/* fast::rms_norm (nuvec.rs:796-798): R(R(x * rsqrt(mean(x^2) + eps)) * w), f32 inside. */
void orc_rms_norm(const orc_bf16 *x, const orc_bf16 *w, int32_t rows, int32_t D, float eps,
                  orc_bf16 *y);

/* Whole SparseMoe::forward (moe.rs:149-174) on x [T, D] -> out [T, D].
 * forced_ids, when not NULL, replaces the computed top-k: each token's forced set must then be a
 * valid top-k under ties (see orc_topk_valid), else the call fails with -2.
 * Returns 0 on success, -1 on invalid arguments. */
int orc_moe_forward(const orc_block *b, const orc_bf16 *x, int32_t T, orc_bf16 *out,
                    const uint32_t *forced_ids, orc_trace *trace);

/* Whether `ids` [k] is a valid top-k of gates [n] for one token when exact ties may be broken
 * either way, and entries whose logit lies within `ulps` bf16 ulps of the k-th boundary may be
 * swapped. Returns 1 when valid. */
int orc_topk_valid(const orc_bf16 *gates, const orc_bf16 *logits, int32_t n, int32_t k,
                   const uint32_t *ids, int32_t ulps);

/* The layer stack of configs[3] (qwen3_5_moe.rs:622-624): x <- R(x + moe(rms_norm(x))).
 * blocks: n_layers blocks; x [T, D] is updated in place. */
int orc_moe_stack(const orc_block *blocks, int32_t n_layers, const orc_bf16 *norm_w, float eps,
                  orc_bf16 *x, int32_t T);

/* A SparseMoe whose tensors are all float32 (an f32 checkpoint: the reference's Hugging Face
 * fixture, gen_tiny.py:235-274). Dense weights, row-major: router [E, D], gate/up [E, I, D],
 * down [E, D, I]; with shared_intermediate S > 0: shared gate/up [S, D], down [D, S] and the
 * shared expert's gate [D]. */
typedef struct {
    orc_config cfg;
    const float *router, *sw_gate, *sw_up, *sw_down;
    const float *sh_gate, *sh_up, *sh_down, *sh_expert_gate;
} orc_block_f32;

/* SparseMoe::forward (moe.rs:149-174) of an f32 block on x [T, D] -> out [T, D]: the op sequence
 * of orc_moe_forward with every tensor kept in f32 (no bf16 rounding). Contractions accumulate in
 * f32 in ascending index order; softmax max, exp(l - max), sum in ascending expert order; top-k
 * with equal gates ranked by the lower id; scores = gates, or gates / (their sum in rank order);
 * routed = sum over the token's pairs in rank order of y * score; out = routed +
 * sigmoid(gate logit) * shared. ids_out [T, k] optional. Returns 0, or -1 on invalid arguments. */
int orc_moe_forward_f32(const orc_block_f32 *b, const float *x, int32_t T, float *out,
                        uint32_t *ids_out);

/* Threads the oracle's parallel loops use (OpenMP); 0 = leave the default. Returns the count. */
int orc_set_threads(int32_t n);

#ifdef __cplusplus
}
#endif
#endif
