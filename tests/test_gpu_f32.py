"""The block of a float32 checkpoint (mrun_moe_forward_f32) on the GPU against the oracle's f32
restatement (orc_moe_forward_f32, pinned in tests/test_oracle.py), on seeded blocks and on the
reference's own f32 Hugging Face fixture loaded by the library's loader.

Bar: every output within F32_TOL of the largest |output| (f32 accumulation in another order: the
device sums each dot product over float4 lanes and a butterfly, the oracle in ascending index
order); another expert choice for a token would move its output far beyond that."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from mrun_amd import moe as M
from mrun_amd import synth
from mrun_amd.load import Weights
from oracle import oracle as O
from tests import checkpoint as C

pytestmark = pytest.mark.gpu

F32_TOL = 4e-6

SMALL = synth.Shape(hidden=64, experts=8, top_k=2, intermediate=32, shared=32)
MID = synth.Shape(hidden=256, experts=64, top_k=8, intermediate=128, shared=128)
NOSHARED = synth.Shape(hidden=512, experts=32, top_k=4, intermediate=256, shared=0,
                       norm_topk=False)


def f32_dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to("cuda")


def check(fb, dev, x: np.ndarray, what: str):
    print(f"f32 block {what}", flush=True)
    got = dev.forward(f32_dev(x)).cpu().numpy()
    ref, ids = O.moe_forward_f32(fb, x)
    err = float(np.max(np.abs(got.astype(np.float64) - ref)))
    scale = float(np.max(np.abs(ref)))
    assert np.all(np.isfinite(got)), what
    assert err <= F32_TOL * scale, f"{what}: max |err| {err:.3g}, max |ref| {scale:.3g}"
    return got


@pytest.mark.parametrize("shape,Ts", [(SMALL, (1, 4, 17)), (MID, (1, 16, 300)),
                                      (NOSHARED, (3, 40))])
def test_f32_block_matches_oracle(shape, Ts):
    fb = synth.make_block_f32(shape, config=23)
    dev = M.SparseMoeF32(fb)
    for T in Ts:
        check(fb, dev, synth.make_x_f32(shape, T, config=23, layer=T), f"{shape.name} T={T}")


@pytest.mark.parametrize("shape,T", [
    # 512 experts (eight keys per lane in the top-k) and k = 16, the largest the build takes
    (synth.Shape(hidden=128, experts=512, top_k=16, intermediate=64, shared=64), 5),
    # k = 1: scores are the gates themselves, or 1 with norm
    (synth.Shape(hidden=128, experts=16, top_k=1, intermediate=64, shared=0), 9),
    (synth.Shape(hidden=128, experts=16, top_k=1, intermediate=64, shared=0, norm_topk=False), 9),
    # more pairs than one grid dimension holds (T k > 65535): the rows kernel strides over them
    (synth.Shape(hidden=64, experts=8, top_k=8, intermediate=32, shared=32), 8300),
])
def test_f32_config_edges(shape, T):
    fb = synth.make_block_f32(shape, config=26)
    check(fb, M.SparseMoeF32(fb), synth.make_x_f32(shape, T, config=26, layer=T),
          f"{shape.name} T={T}")


def test_f32_rows_keep_their_bits():
    """A token's output does not depend on the batch around it (every dot product has a fixed
    order): rows of a 33-token batch equal the same rows run alone, bit for bit."""
    fb = synth.make_block_f32(MID, config=24)
    dev = M.SparseMoeF32(fb)
    x = synth.make_x_f32(MID, 33, config=24)
    full = dev.forward(f32_dev(x)).cpu().numpy()
    for t in (0, 17, 32):
        one = dev.forward(f32_dev(x[t:t + 1])).cpu().numpy()
        assert np.array_equal(one[0].view(np.uint32), full[t].view(np.uint32)), t


@pytest.mark.parametrize("T", [1, 5, 40])
def test_hugging_face_fixture_in_f32(T):
    """The reference's f32 Hugging Face fixture (fused gate_up_proj, dense f32 experts, the
    model.language_model prefix), loaded as stored: the loader splits gate_up
    (qwen3_5_moe.rs:391-405) and hands out an f32 block; the oracle reads the same f32 tensors
    split in numpy."""
    src = C.read(C.GOLDEN / "tiny_qwen3_5_moe_hf" / "model.safetensors")
    p = "model.language_model.layers.0.mlp"
    f = lambda n: np.asarray(src[n][2], np.float32)
    c = C.config("tiny_qwen3_5_moe_hf")
    D, E, I, S = (c["hidden_size"], c["num_experts"], c["moe_intermediate_size"],
                  c["shared_expert_intermediate_size"])
    shape = synth.Shape(hidden=D, experts=E, top_k=c["num_experts_per_tok"], intermediate=I,
                        shared=S, norm_topk=bool(c.get("norm_topk_prob", True)))
    gu = f(p + ".experts.gate_up_proj")  # [E, 2I, D]
    fb = synth.F32Block(shape=shape, router=f(p + ".gate.weight"), gate_proj=gu[:, :I],
                        up_proj=gu[:, I:], down_proj=f(p + ".experts.down_proj"),
                        sh_gate_proj=f(p + ".shared_expert.gate_proj.weight"),
                        sh_up_proj=f(p + ".shared_expert.up_proj.weight"),
                        sh_down_proj=f(p + ".shared_expert.down_proj.weight"),
                        sh_expert_gate=f(p + ".shared_expert_gate.weight"))
    with Weights(C.GOLDEN / "tiny_qwen3_5_moe_hf") as w:
        dev = w.load_moe(p)
        assert isinstance(dev, M.SparseMoeF32)
        check(fb, dev, synth.make_x_f32(shape, T, config=25, layer=T), f"HF f32 T={T}")
        torch.cuda.synchronize()
