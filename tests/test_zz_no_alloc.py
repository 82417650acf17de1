"""mrun_moe_forward_noalloc, the forward whose workspace is the library's own scratch array,
against mrun_moe_forward (the same kernels on a caller workspace): bit-identical outputs, over
calls in a row whose later inputs are smaller than the earlier ones (the scratch array keeps the
last call's contents), and a clear refusal above the array's size."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from mrun_amd import _lib
from mrun_amd import moe as M
from mrun_amd import synth

pytestmark = pytest.mark.gpu

SMALL = synth.Shape(hidden=256, experts=16, top_k=4, intermediate=128, shared=128)


def _noalloc(dev, x):
    out = torch.empty_like(x)
    rc = _lib.load().mrun_moe_forward_noalloc(
        ctypes.byref(dev.c), ctypes.c_void_p(x.data_ptr()), x.shape[0],
        ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check(rc)
    return out


@pytest.mark.parametrize("shape,Ts", [(synth.QWEN36, (300, 24, 4, 1)), (SMALL, (40, 3))])
def test_noalloc_matches_forward(shape, Ts):
    hb = synth.make_block(shape, config=synth.CFG_DECODE, layer=900)
    dev = M.SparseMoe(hb)
    cap = int(_lib.load().mrun_moe_forward_noalloc_max_bytes())
    for T in Ts:  # prefill first, then smaller decode batches over stale scratch contents
        assert dev.workspace_bytes(T) <= cap
        x = M.bf16_tensor(synth.make_x(shape, T, config=synth.CFG_DECODE, layer=900 + T))
        want = M.bf16_bits(dev.forward(x))
        got = M.bf16_bits(_noalloc(dev, x))
        torch.cuda.synchronize()
        assert np.array_equal(got, want), f"{shape.name} T={T}"
        print(f"noalloc {shape.name} T={T}: bit-identical to mrun_moe_forward", flush=True)


def test_noalloc_refuses_above_its_scratch():
    dev = M.SparseMoe(synth.make_block(synth.QWEN36, config=synth.CFG_DECODE, layer=901))
    cap = int(_lib.load().mrun_moe_forward_noalloc_max_bytes())
    T = 4096
    assert dev.workspace_bytes(T) > cap
    x = torch.zeros(T, synth.QWEN36.hidden, dtype=torch.bfloat16, device="cuda")
    out = torch.empty_like(x)
    rc = _lib.load().mrun_moe_forward_noalloc(
        ctypes.byref(dev.c), ctypes.c_void_p(x.data_ptr()), T, ctypes.c_void_p(out.data_ptr()),
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == _lib.MRUN_ERR_WORKSPACE
    assert b"scratch" in _lib.load().mrun_last_error()


def test_noalloc_forwards_captured_in_a_graph():
    """Noalloc forwards (decode T = 1, prefill T = 300) captured in a HIP graph: every replay, with
    eager noalloc calls of another size in between (they overwrite the scratch array), equals
    mrun_moe_forward bit for bit. The scratch address is resolved before the capture."""
    hb = synth.make_block(synth.QWEN36, config=synth.CFG_DECODE, layer=902)
    dev = M.SparseMoe(hb)
    lib = _lib.load()
    lib.mrun_moe_forward_noalloc_max_bytes()  # resolves this GPU's scratch address
    for T, other in ((1, 300), (300, 1)):
        x = M.bf16_tensor(synth.make_x(synth.QWEN36, T, config=synth.CFG_DECODE, layer=950 + T))
        xo = M.bf16_tensor(synth.make_x(synth.QWEN36, other, config=synth.CFG_DECODE, layer=960))
        want = M.bf16_bits(dev.forward(x))
        out = torch.empty_like(x)

        def call(stream):
            _lib.check(lib.mrun_moe_forward_noalloc(
                ctypes.byref(dev.c), ctypes.c_void_p(x.data_ptr()), T,
                ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(stream.cuda_stream)))

        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            call(s)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            call(torch.cuda.current_stream())
        for rep in range(3):
            out.zero_()
            _noalloc(dev, xo)  # another size through the same scratch array
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(M.bf16_bits(out), want), f"T={T} replay {rep}"
        print(f"noalloc T={T}: 3 graph replays bit-identical to mrun_moe_forward", flush=True)
