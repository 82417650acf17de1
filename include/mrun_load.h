/*
 * Checkpoint loading for the MoE block (libmrun_moe.so): MLX / Hugging Face safetensors
 * checkpoints into the device views of include/mrun_moe.h.
 *
 * The counterpart of crates/mrun-engine/src/load.rs (Weights, Quantization, Linear::load) and
 * SparseMoe::load (models/moe.rs:120-147). Loading allocates device memory (it is not on the hot
 * path); everything a loaded block points into is owned by its mrun_weights and freed by
 * mrun_weights_close. Functions return 0 or an MRUN_ERR_* code with mrun_last_error() set.
 */
#ifndef MRUN_LOAD_H
#define MRUN_LOAD_H

#include <stddef.h>
#include <stdint.h>

#include "mrun_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mrun_weights mrun_weights;

/* Weights::load (load.rs:179-196) and Quantization::from_config (load.rs:52-103): the tensor
 * headers of every *.safetensors file in `dir` (sorted by name; later files do not replace
 * earlier names), except the names no family reads (unused_tensor, load.rs:164-173: vision
 * towers, MTP heads, rotary tables), and config.json when present. Quantization modes other than
 * affine and per-path settings other than 4/8 bits with groups 32/64/128 are refused here, before
 * any tensor data is read. Tensor data is read when a layer takes it. */
int mrun_weights_open(const char *dir, mrun_weights **out);
void mrun_weights_close(mrun_weights *w);

/* The MoE config of config.json (text_config when nested): hidden_size, num_experts,
 * num_experts_per_tok (1..=num_experts, qwen3_5_moe.rs:508-513), moe_intermediate_size,
 * norm_topk_prob (default true), shared_expert_intermediate_size (absent: 0, qwen3_moe.rs:65-80),
 * rms_norm_eps (default 1e-6). */
int mrun_weights_moe_config(const mrun_weights *w, mrun_moe_config *cfg, float *rms_norm_eps);

/* Header of tensor `name` not taken yet: dtype ("BF16", "U32", "F32", ...; 8 bytes with the
 * terminator) and shape (up to 8 dims). MRUN_ERR_INVALID "missing tensor" when absent. */
int mrun_weights_tensor_info(const mrun_weights *w, const char *name, char *dtype,
                             int64_t *shape, int32_t *ndim);

/* Tensors not taken by a layer yet (Weights::remaining, load.rs:250-255). */
int32_t mrun_weights_remaining(const mrun_weights *w);

/* Quantization::resolve (load.rs:105-126) for the quantized layer at `path` (without `.weight`)
 * whose unquantized input width is `in_dims`: a path named in the config wins, any other is
 * inferred from the packed shapes (infer, load.rs:128-156). Reads headers only. */
int mrun_weights_resolve_quant(const mrun_weights *w, const char *path, int32_t in_dims,
                               int32_t *group_size, int32_t *bits);

/* SparseMoe::load (moe.rs:120-147): takes `<prefix>.gate`, `<prefix>.switch_mlp.*` and, when
 * cfg->shared_intermediate > 0, `<prefix>.shared_expert.*` and `<prefix>.shared_expert_gate`,
 * copies them to the device and fills `out`. Hugging Face layouts at `prefix` are restated first:
 * per-expert `experts.<e>.<proj>.weight` are stacked (qwen3_moe.rs:39-58) and a fused
 * `experts.gate_up_proj` is split into gate and up (qwen3_5_moe.rs:391-405). Dense bf16 experts
 * become 16-bit stacked weights (gather_mm); dense weights other than bf16 (f32 checkpoints) are
 * refused with MRUN_ERR_UNSUPPORTED. */
int mrun_weights_load_moe(mrun_weights *w, const char *prefix, const mrun_moe_config *cfg,
                          mrun_sparse_moe *out);

/* A bf16 tensor of `n` elements (an RMSNorm weight, RmsNorm::load load.rs:352-357) copied to the
 * device; *out points into memory owned by `w`. */
int mrun_weights_load_bf16(mrun_weights *w, const char *name, int64_t n, const mrun_bf16 **out);

#ifdef __cplusplus
}
#endif
#endif
