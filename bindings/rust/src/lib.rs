//! Raw declarations of libmrun_moe's C ABI (`include/mrun_moe.h`, `include/mrun_load.h`), one
//! item per C declaration, for a `-sys` crate behind mrun-engine's tensor facade
//! (crates/mrun-engine/src/tensor/nuvec.rs, the only module that touches the backend,
//! tensor/mod.rs:1-4).
//!
//! Every function is asynchronous on the given HIP stream and returns 0 or an `MRUN_ERR_*`
//! status whose message `mrun_last_error()` gives on the same thread (the facade's
//! `Result<_, tensor::Error(String)>`, nuvec.rs:18-38). Tensors are caller-owned device memory;
//! bf16 travels as `u16` bits. The safe layer (status to `tensor::Error`, `Array` to device
//! pointers, the thread's stream and scratch) belongs to the engine, around `gather_qmm` and
//! `SparseMoe::forward`.
//!
//! This file is checked against the C headers by tests/test_rust_binding.py (names, argument
//! order and types, struct layouts); this image has no Rust toolchain to compile it.
#![allow(non_camel_case_types)]
#![no_std]

use core::ffi::{c_char, c_int, c_void};

/// bfloat16 bits.
pub type mrun_bf16 = u16;
/// A `hipStream_t` (null: the null stream).
pub type mrun_stream_t = *mut c_void;

pub const MRUN_OK: c_int = 0;
/// Bad shape, pointer or argument.
pub const MRUN_ERR_INVALID: c_int = 1;
/// A valid reference configuration this build does not run.
pub const MRUN_ERR_UNSUPPORTED: c_int = 2;
/// Workspace too small.
pub const MRUN_ERR_WORKSPACE: c_int = 3;
/// The HIP runtime reported an error.
pub const MRUN_ERR_HIP: c_int = 4;

/// `tensor::Quantized` (nuvec.rs:602-638): codes `[experts, out, in*bits/32]` u32 (LSB first,
/// nuvec.rs:1199-1203), scales and biases `[experts, out, in/group_size]` bf16, biases null for
/// zeros (nuvec.rs:609-626). bits 16: dense bf16 `[experts, out, in]` in `weight`
/// (`SwitchLinear::Dense`, moe.rs:43-46); bits 32: dense f32 the same way (an f32 block, run by
/// `mrun_moe_forward_f32`).
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct mrun_quantized {
    pub weight: *const u32,
    pub scales: *const mrun_bf16,
    pub biases: *const mrun_bf16,
    pub experts: i32,
    pub out: i32,
    pub in_: i32,
    pub group_size: i32,
    pub bits: i32,
}

/// `load::Linear` (load.rs:246-306): dense when `weight` is not null, else quantized by `q`;
/// optional bias `[out]`.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct mrun_linear {
    pub weight: *const mrun_bf16,
    pub q: mrun_quantized,
    pub bias: *const mrun_bf16,
    pub out: i32,
    pub in_: i32,
}

/// `MoeConfig` (moe.rs:97-107); `shared_intermediate` 0: no shared expert.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct mrun_moe_config {
    pub hidden: i32,
    pub experts: i32,
    pub top_k: i32,
    pub intermediate: i32,
    pub norm_topk_prob: i32,
    pub shared_intermediate: i32,
}

/// `SparseMoe` (moe.rs:109-147): router, SwitchGlu projections, shared expert and its gate.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct mrun_sparse_moe {
    pub cfg: mrun_moe_config,
    pub gate: mrun_linear,
    pub switch_gate_proj: mrun_quantized,
    pub switch_up_proj: mrun_quantized,
    pub switch_down_proj: mrun_quantized,
    pub shared_gate_proj: mrun_linear,
    pub shared_up_proj: mrun_linear,
    pub shared_down_proj: mrun_linear,
    pub shared_expert_gate: mrun_linear,
}

/// An open safetensors checkpoint (`Weights`, load.rs:179-196); opaque.
#[repr(C)]
pub struct mrun_weights {
    _private: [u8; 0],
}

#[link(name = "mrun_moe")]
extern "C" {
    // ---- include/mrun_moe.h ----

    /// The message of this thread's last failed call ("" when none).
    pub fn mrun_last_error() -> *const c_char;
    pub fn mrun_version() -> *const c_char;
    /// `SparseMoe::load`'s shape rules (moe.rs:120-147, load.rs:14-156).
    pub fn mrun_moe_check(moe: *const mrun_sparse_moe) -> c_int;
    /// `SparseMoe::scratch_per_token` (moe.rs:176-187) as bytes for `tokens` rows.
    pub fn mrun_moe_workspace_bytes(cfg: *const mrun_moe_config, tokens: i32) -> usize;
    /// `SparseMoe::forward` (moe.rs:149-174) and `Ffn::forward`'s Moe arm (moe.rs:202-207).
    pub fn mrun_moe_forward(
        moe: *const mrun_sparse_moe,
        x: *const mrun_bf16,
        tokens: i32,
        out: *mut mrun_bf16,
        workspace: *mut c_void,
        workspace_bytes: usize,
        stream: mrun_stream_t,
    ) -> c_int;
    /// `SparseMoe::forward` of an f32 checkpoint's block: every weight dense f32 (bits 32),
    /// x and out f32 (nuvec.rs:688-697 runs the dense gather_mm in f32).
    pub fn mrun_moe_workspace_bytes_f32(cfg: *const mrun_moe_config, tokens: i32) -> usize;
    pub fn mrun_moe_forward_f32(
        moe: *const mrun_sparse_moe,
        x: *const f32,
        tokens: i32,
        out: *mut f32,
        workspace: *mut c_void,
        workspace_bytes: usize,
        stream: mrun_stream_t,
    ) -> c_int;
    /// `mrun_moe_forward` on the library's per-GPU scratch array, for callers that cannot
    /// allocate; no counterpart in the reference.
    pub fn mrun_moe_forward_noalloc(
        moe: *const mrun_sparse_moe,
        x: *const mrun_bf16,
        tokens: i32,
        out: *mut mrun_bf16,
        stream: mrun_stream_t,
    ) -> c_int;
    pub fn mrun_moe_forward_noalloc_max_bytes() -> usize;
    /// Benchmark instrumentation (no counterpart in the reference).
    pub fn mrun_moe_forward_profiled(
        moe: *const mrun_sparse_moe,
        x: *const mrun_bf16,
        tokens: i32,
        out: *mut mrun_bf16,
        workspace: *mut c_void,
        workspace_bytes: usize,
        stream: mrun_stream_t,
        events: *mut *mut c_void,
        n_events: i32,
        n_stages: *mut i32,
    ) -> c_int;
    pub fn mrun_moe_stage_names(cfg: *const mrun_moe_config, tokens: i32) -> *const c_char;
    /// Benchmark instrumentation (no counterpart in the reference).
    pub fn mrun_moe_forward_timed(
        moe: *const mrun_sparse_moe,
        x: *const mrun_bf16,
        tokens: i32,
        out: *mut mrun_bf16,
        workspace: *mut c_void,
        workspace_bytes: usize,
        stream: mrun_stream_t,
        clock: *mut u64,
    ) -> c_int;
    /// Ticks per second of the clock `mrun_moe_forward_timed` reads (instrumentation).
    pub fn mrun_wall_clock_hz() -> i64;
    /// Byte offsets of the last forward's routing inside its workspace (instrumentation).
    pub fn mrun_moe_workspace_routing(cfg: *const mrun_moe_config, tokens: i32, at: *mut usize)
        -> c_int;
    /// The router (moe.rs:151-159): `Linear::forward`, softmax, argpartition, norm_topk.
    pub fn mrun_moe_router(
        moe: *const mrun_sparse_moe,
        x: *const mrun_bf16,
        tokens: i32,
        logits: *mut mrun_bf16,
        gates: *mut mrun_bf16,
        ids: *mut u32,
        scores: *mut mrun_bf16,
        workspace: *mut c_void,
        workspace_bytes: usize,
        stream: mrun_stream_t,
    ) -> c_int;
    /// The sorted dispatch (moe.rs:65-75): argsort (nuvec.rs:554-556), inverse, floor_divide
    /// (nuvec.rs:523-526).
    pub fn mrun_moe_permute(
        ids: *const u32,
        pairs: i32,
        top_k: i32,
        experts: i32,
        offsets: *mut u32,
        order: *mut u32,
        inverse: *mut u32,
        token: *mut u32,
        workspace: *mut c_void,
        workspace_bytes: usize,
        stream: mrun_stream_t,
    ) -> c_int;
    pub fn mrun_moe_permute_workspace_bytes(pairs: i32, experts: i32) -> usize;
    /// `tensor::gather_qmm` (nuvec.rs:670-686).
    pub fn mrun_gather_qmm(
        x: *const mrun_bf16,
        x_rows: i32,
        w: *const mrun_quantized,
        indices: *const u32,
        n: i32,
        sorted_indices: i32,
        out: *mut mrun_bf16,
        workspace: *mut c_void,
        workspace_bytes: usize,
        stream: mrun_stream_t,
    ) -> c_int;
    pub fn mrun_gather_qmm_workspace_bytes(n: i32, experts: i32, x_rows: i32, in_: i32, out: i32)
        -> usize;
    /// `tensor::quantized_matmul` (nuvec.rs:660-663).
    pub fn mrun_quantized_matmul(
        x: *const mrun_bf16,
        rows: i32,
        w: *const mrun_quantized,
        out: *mut mrun_bf16,
        stream: mrun_stream_t,
    ) -> c_int;
    /// `Linear::forward` (load.rs:294-306).
    pub fn mrun_linear_forward(
        l: *const mrun_linear,
        x: *const mrun_bf16,
        rows: i32,
        out: *mut mrun_bf16,
        stream: mrun_stream_t,
    ) -> c_int;
    /// `activations::swiglu` (activations.rs:55-59).
    pub fn mrun_swiglu(
        gate: *const mrun_bf16,
        up: *const mrun_bf16,
        n: i64,
        out: *mut mrun_bf16,
        stream: mrun_stream_t,
    ) -> c_int;
    /// Unsort, weighted sum over k and the sigmoid-gated shared expert (moe.rs:84-93, 161-171).
    pub fn mrun_moe_combine(
        y: *const mrun_bf16,
        inverse: *const u32,
        scores: *const mrun_bf16,
        tokens: i32,
        top_k: i32,
        hidden: i32,
        shared_y: *const mrun_bf16,
        shared_logit: *const mrun_bf16,
        out: *mut mrun_bf16,
        stream: mrun_stream_t,
    ) -> c_int;
    /// `fast::rms_norm` (nuvec.rs:796-798) as `RmsNorm::forward` (load.rs:361-363).
    pub fn mrun_rms_norm(
        x: *const mrun_bf16,
        w: *const mrun_bf16,
        rows: i32,
        hidden: i32,
        eps: f32,
        out: *mut mrun_bf16,
        stream: mrun_stream_t,
    ) -> c_int;
    /// `fast::add_rms_norm` (nuvec.rs:800-811).
    pub fn mrun_add_rms_norm(
        x: *const mrun_bf16,
        residual: *const mrun_bf16,
        w: *const mrun_bf16,
        rows: i32,
        hidden: i32,
        eps: f32,
        h: *mut mrun_bf16,
        y: *mut mrun_bf16,
        stream: mrun_stream_t,
    ) -> c_int;
    /// The decoder-layer loop around the block (qwen3_5_moe.rs:622-624, 664-666).
    pub fn mrun_moe_stack_forward(
        layers: *const mrun_sparse_moe,
        n_layers: i32,
        norm_w: *const *const mrun_bf16,
        eps: f32,
        x: *mut mrun_bf16,
        tokens: i32,
        workspace: *mut c_void,
        workspace_bytes: usize,
        stream: mrun_stream_t,
    ) -> c_int;
    pub fn mrun_moe_stack_workspace_bytes(cfg: *const mrun_moe_config, tokens: i32) -> usize;

    // ---- include/mrun_load.h ----

    /// `Weights::load` (load.rs:179-196) of a checkpoint directory.
    pub fn mrun_weights_open(dir: *const c_char, out: *mut *mut mrun_weights) -> c_int;
    pub fn mrun_weights_close(w: *mut mrun_weights);
    pub fn mrun_weights_moe_config(
        w: *const mrun_weights,
        cfg: *mut mrun_moe_config,
        rms_norm_eps: *mut f32,
    ) -> c_int;
    pub fn mrun_weights_tensor_info(
        w: *const mrun_weights,
        name: *const c_char,
        dtype: *mut c_char,
        shape: *mut i64,
        ndim: *mut i32,
    ) -> c_int;
    pub fn mrun_weights_remaining(w: *const mrun_weights) -> i32;
    /// `Quantization::resolve` (load.rs:105-126).
    pub fn mrun_weights_resolve_quant(
        w: *const mrun_weights,
        path: *const c_char,
        in_dims: i32,
        group_size: *mut i32,
        bits: *mut i32,
    ) -> c_int;
    /// `SparseMoe::load` (moe.rs:120-147) into device memory the checkpoint owns.
    pub fn mrun_weights_load_moe(
        w: *mut mrun_weights,
        prefix: *const c_char,
        cfg: *const mrun_moe_config,
        out: *mut mrun_sparse_moe,
    ) -> c_int;
    pub fn mrun_weights_load_bf16(
        w: *mut mrun_weights,
        name: *const c_char,
        n: i64,
        out: *mut *const mrun_bf16,
    ) -> c_int;
}
