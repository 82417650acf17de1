"""Blocks loaded from the reference's tiny checkpoints (tests/golden/) by the library's loader,
run on the GPU against the oracle over the same tensors read independently."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from mrun_amd import moe as M
from mrun_amd import synth
from mrun_amd.load import Weights
from oracle import oracle as O
from tests import checkpoint as C
from tests.helpers import bf16_ulp, stats
from tests.test_gpu_parity import run_block

pytestmark = pytest.mark.gpu

MOE35 = "tiny_qwen3_5_moe"
MOE3 = "tiny_qwen3_moe"


@pytest.mark.parametrize("fixture,prefix", [
    (MOE35, f"language_model.model.layers.{l}.mlp") for l in range(4)
] + [(MOE3, "model.layers.0.mlp"), (MOE3, "model.layers.2.mlp")])
@pytest.mark.parametrize("T", [1, 4, 40])
def test_loaded_block_matches_oracle(fixture, prefix, T):
    """8-bit group-64 router (and shared gate), 4-bit group-32 experts, as mlx-lm wrote them."""
    with Weights(C.GOLDEN / fixture) as w:
        dev = w.load_moe(prefix)
        hb = C.host_block(fixture, prefix)
        x = synth.make_x(hb.shape, T, config=13, layer=T)
        run_block(hb, dev, x, f"{fixture} {prefix} T={T}")
        torch.cuda.synchronize()


@pytest.mark.parametrize("T", [3, 33])
def test_loaded_stack_with_norm_weights(T):
    """The four MoE layers of the Qwen3.5 fixture as a stack, each behind its own RMSNorm weight
    (post_attention_layernorm, RmsNorm::load load.rs:352-357; eps from config.json). The stack
    entry point equals the loop of single GPU ops bit for bit; against the oracle, layer by layer
    on the GPU's expert choices (each validated as a top-k within ties), within the block bar plus
    one bf16 ulp of the residual stream."""
    pre = [f"language_model.model.layers.{l}" for l in range(4)]
    t = C.read(C.GOLDEN / MOE35 / "model.safetensors")
    norms = [t[p + ".post_attention_layernorm.weight"][2] for p in pre]
    with Weights(C.GOLDEN / MOE35) as w:
        cfg, eps = w.moe_config()
        layers = [w.load_moe(p + ".mlp", cfg) for p in pre]
        nw = [w.load_bf16(p + ".post_attention_layernorm.weight", cfg.hidden) for p in pre]
        st = M.MoeStack(layers, nw, eps)
        x_np = synth.make_x(layers[0].shape, T, config=14, layer=T)
        got = M.bf16_bits(st.forward_(M.bf16_tensor(x_np)))
        # the loop of single ops, keeping each layer's expert choice
        nd = [M.bf16_tensor(n) for n in norms]
        x = M.bf16_tensor(x_np)
        h = M.rms_norm(x, nd[0], eps)
        ids = []
        for l, layer in enumerate(layers):
            ids.append(M.u32_array(layer.router_forward(h)[2]).reshape(T, -1))
            o = layer.forward(h)
            x, h = M.add_rms_norm(x, o, nd[min(l + 1, 3)], eps)
        torch.cuda.synchronize()
        assert np.array_equal(got, M.bf16_bits(x)), "stack entry point differs from the op loop"
    ref = x_np.copy()
    for p, n, gi in zip(pre, norms, ids):
        hb = C.host_block(MOE35, p + ".mlp")
        o = O.moe_forward(hb, O.rms_norm(ref, n, eps), forced_ids=gi)
        ref = O.bf16_from_f32(synth.bf16_to_f32(ref) + synth.bf16_to_f32(o))
    g, r = synth.bf16_to_f32(got).astype(np.float64), synth.bf16_to_f32(ref).astype(np.float64)
    s = stats(got, ref)
    assert np.all(np.abs(g - r) <= 2e-2 + bf16_ulp(np.maximum(np.abs(g), np.abs(r)))), s
    assert s["l1_rel"] <= 1e-3, s
    print(f"loaded stack T={T}: {s}", flush=True)


@pytest.mark.parametrize("T", [2, 40])
def test_hugging_face_layout_in_bf16(tmp_path, T):
    """The Hugging Face fixture (fused gate_up_proj, dense experts, the model.language_model
    prefix) with its f32 tensors rounded to bf16: the loader splits gate_up (qwen3_5_moe.rs:391-405)
    and runs the dense experts; the oracle reads the same bf16 tensors split in numpy."""
    src = C.read(C.GOLDEN / "tiny_qwen3_5_moe_hf" / "model.safetensors")
    bf = {n: synth.f32_to_bf16(a.astype(np.float32)) for n, (dt, shp, a) in src.items() if dt == "F32"}
    C.write(tmp_path / "model.safetensors", bf, {"format": "pt"})
    (tmp_path / "config.json").write_text((C.GOLDEN / "tiny_qwen3_5_moe_hf" / "config.json").read_text())
    p = "model.language_model.layers.0.mlp"
    c = C.config("tiny_qwen3_5_moe_hf")
    D, E, I, S = c["hidden_size"], c["num_experts"], c["moe_intermediate_size"], c["shared_expert_intermediate_size"]
    gu = bf[p + ".experts.gate_up_proj"]                   # [E, 2I, D]
    dense = lambda w: synth.QTensor(codes=np.ascontiguousarray(w).view(np.uint32), scales=None,
                                    biases=None, experts=w.shape[0], out=w.shape[1], in_=w.shape[2],
                                    group=0, bits=16)
    shape = synth.Shape(hidden=D, experts=E, top_k=c["num_experts_per_tok"], intermediate=I, shared=S)
    hb = synth.HostBlock(shape=shape, router=bf[p + ".gate.weight"], router_bias=None,
                         gate_proj=dense(gu[:, :I, :]), up_proj=dense(gu[:, I:, :]),
                         down_proj=dense(bf[p + ".experts.down_proj"]))
    hb.sh_gate_proj = dense(bf[p + ".shared_expert.gate_proj.weight"][None])
    hb.sh_up_proj = dense(bf[p + ".shared_expert.up_proj.weight"][None])
    hb.sh_down_proj = dense(bf[p + ".shared_expert.down_proj.weight"][None])
    hb.sh_expert_gate = bf[p + ".shared_expert_gate.weight"]
    with Weights(tmp_path) as w:
        dev = w.load_moe(p)
        run_block(hb, dev, synth.make_x(shape, T, config=15, layer=T), f"HF bf16 T={T}")
        torch.cuda.synchronize()
