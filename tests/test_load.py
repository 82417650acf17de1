"""The checkpoint loader (include/mrun_load.h) on the reference's own tiny checkpoints (MLX 4-bit
with 8-bit routers, and the Hugging Face f32 layout), and the oracle on their real packed data.
Host-side only: nothing here touches a GPU (device copies are in test_gpu_load.py)."""
from __future__ import annotations

import numpy as np
import pytest

from mrun_amd import _lib, synth
from mrun_amd.load import Weights
from oracle import oracle as O
from tests import checkpoint as C
from tests import np_reference as NP
from tests.helpers import assert_close, beyond_rounding

MOE35 = "tiny_qwen3_5_moe"
MOE3 = "tiny_qwen3_moe"
HF = "tiny_qwen3_5_moe_hf"


def test_headers_match_an_independent_reader():
    for fx in (MOE35, MOE3):
        ref = C.read(C.GOLDEN / fx / "model.safetensors")
        with Weights(C.GOLDEN / fx) as w:
            assert w.remaining() == len(ref)
            for name, (dtype, shape, _) in ref.items():
                assert w.tensor_info(name) == (dtype, shape), name


def test_moe_config_from_config_json():
    with Weights(C.GOLDEN / MOE35) as w:      # nested text_config (qwen3_5_moe.rs:497-517)
        cfg, eps = w.moe_config()
        assert (cfg.hidden, cfg.experts, cfg.top_k, cfg.intermediate, cfg.norm_topk_prob,
                cfg.shared_intermediate) == (64, 8, 4, 32, 1, 32)
        assert eps == pytest.approx(1e-6)
    with Weights(C.GOLDEN / MOE3) as w:       # flat, no shared expert (qwen3_moe.rs:65-80)
        cfg, _ = w.moe_config()
        assert (cfg.hidden, cfg.experts, cfg.top_k, cfg.intermediate,
                cfg.shared_intermediate) == (64, 8, 4, 32, 0)


def test_quantization_resolution():
    """Quantization::resolve (load.rs:105-156): the Qwen3.5 fixture lists its 8-bit routers only
    under quantization_config, which is ignored while `quantization` exists, so they are inferred
    from the packed shapes; the Qwen3 fixture names them in `quantization`."""
    with Weights(C.GOLDEN / MOE35) as w:
        p = "language_model.model.layers.0.mlp"
        assert w.resolve_quant(p + ".gate", 64) == (64, 8)
        assert w.resolve_quant(p + ".shared_expert_gate", 64) == (64, 8)
        assert w.resolve_quant(p + ".switch_mlp.gate_proj", 64) == (32, 4)
        assert w.resolve_quant(p + ".switch_mlp.down_proj", 32) == (32, 4)
        with pytest.raises(_lib.MrunError, match="no whole number of bits per code for an input width of 48"):
            w.resolve_quant(p + ".switch_mlp.gate_proj", 48)
    with Weights(C.GOLDEN / MOE3) as w:
        assert w.resolve_quant("model.layers.0.mlp.gate", 64) == (64, 8)
        assert w.resolve_quant("model.layers.2.mlp.switch_mlp.up_proj", 64) == (32, 4)


@pytest.mark.parametrize("fixture,says", [("refuse_quant_mode", "mode mxfp4 cannot be loaded"),
                                          ("refuse_quant_bits", "down_proj")])
def test_unsupported_quantization_is_refused_from_the_config(fixture, says):
    """The reference's load_refusal.rs:70-90 cases, from config.json alone."""
    with pytest.raises(_lib.MrunError) as e:
        Weights(C.GOLDEN / fixture)
    assert e.value.code == _lib.MRUN_ERR_INVALID
    assert e.value.message.startswith("quantization: ") and says in e.value.message


def test_hugging_face_layout():
    """Vision and MTP tensors are never loaded (load.rs:164-173); the fused gate_up_proj is split
    (qwen3_5_moe.rs:391-405) and the f32 block passes every check: without a GPU the load stops
    at its first device allocation (the f32 block runs in tests/test_gpu_f32.py)."""
    with Weights(C.GOLDEN / HF) as w:
        with pytest.raises(_lib.MrunError, match="missing tensor"):
            w.tensor_info("mtp.fc.weight")
        with pytest.raises(_lib.MrunError, match="missing tensor"):
            w.tensor_info("model.visual.blocks.0.attn.proj.weight")
        assert w.tensor_info("model.language_model.layers.0.mlp.experts.gate_up_proj") == (
            "F32", (8, 64, 64))
        cfg, _ = w.moe_config()
        try:
            blk = w.load_moe("model.language_model.layers.0.mlp", cfg)
        except _lib.MrunError as e:
            assert e.code == _lib.MRUN_ERR_HIP and "hipMalloc" in e.message, e
        else:  # a GPU: the block is on the device
            assert blk.shape.experts == 8 and blk.workspace_bytes(1) > 0


def test_missing_tensor_is_named():
    with Weights(C.GOLDEN / MOE3) as w:
        cfg, _ = w.moe_config()
        with pytest.raises(_lib.MrunError, match="missing tensor model.layers.1.mlp.gate.weight"):
            w.load_moe("model.layers.1.mlp", cfg)   # layer 1 is a dense MLP (mlp_only_layers)


# ---- the oracle on real MLX-packed tensors ----------------------------------------------------

@pytest.mark.parametrize("fixture,prefix", [
    (MOE35, "language_model.model.layers.0.mlp"),
    (MOE35, "language_model.model.layers.3.mlp"),
    (MOE3, "model.layers.2.mlp"),
])
def test_oracle_on_checkpoint_blocks(fixture, prefix):
    """Dequant rows of the real checkpoint equal the float64 closed form exactly, and the oracle's
    block (8-bit routers, 4-bit group-32 experts) agrees with the numpy restatement."""
    hb = C.host_block(fixture, prefix)
    for q in (hb.gate_proj, hb.down_proj, hb.router):
        Wd = NP.dequant(q)
        for e, o in [(0, 0), (q.experts - 1, q.out - 1)]:
            assert np.array_equal(O.dequant_row(q, e, o), Wd[e, o].astype(np.float32))
    x = synth.make_x(hb.shape, 9, config=12)
    out, tr = O.moe_forward(hb, x, trace=True)
    ref, rtr = NP.forward(hb, x, ids=tr["ids"])
    assert beyond_rounding(tr["logits"], rtr["logits"]) == 0
    assert_close(out, ref, l1_rel=2e-4, what=f"{fixture} {prefix}")
