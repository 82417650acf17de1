"""The C-ABI library (include/*.h) loads and exports every declared entry point, and its host-side
validation reports errors the way the facade does (status + message). No GPU: no call here
reaches device work."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from mrun_amd import _lib
from mrun_amd._lib import Linear, MoeConfig, Quantized, SparseMoe

ROOT = Path(__file__).resolve().parent.parent


def declared(header: Path) -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(mrun_\w+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    lib = _lib.load()
    names = declared(ROOT / "include" / "mrun_moe.h") + declared(ROOT / "include" / "mrun_load.h")
    assert len(names) >= 15
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.SIGNATURES), "the ctypes view must cover the header"
    syn = ctypes.CDLL(str(ROOT / "mrun_amd" / "lib" / "libmrun_synth.so"))
    syn_dev = ctypes.CDLL(str(ROOT / "mrun_amd" / "lib" / "libmrun_synth_dev.so"))
    for n in declared(ROOT / "include" / "mrun_synth.h"):
        assert hasattr(syn_dev if n.endswith("_dev") else syn, n), n
    assert b"gfx950" in lib.mrun_version()


def test_calibration_library():
    """bench.py's copy and MFMA-rate kernels: exported, and their argument checks answer before
    any device work."""
    cal = ctypes.CDLL(str(ROOT / "mrun_amd" / "lib" / "libmrun_calib.so"))
    for n in ("mrun_calib_copy", "mrun_calib_read", "mrun_calib_read_threads", "mrun_calib_mfma",
              "mrun_calib_mfma_chains"):
        assert hasattr(cal, n), n
    assert cal.mrun_calib_mfma_chains() == 4
    cal.mrun_calib_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                    ctypes.c_void_p]
    cal.mrun_calib_mfma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    assert cal.mrun_calib_copy(FAKE + 8, FAKE, 64, None) != 0    # misaligned
    assert cal.mrun_calib_copy(FAKE, FAKE, 24, None) != 0        # not whole 16-byte units
    assert cal.mrun_calib_copy(FAKE, FAKE, 0, None) == 0         # nothing to copy
    cal.mrun_calib_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                    ctypes.c_void_p]
    assert cal.mrun_calib_read(FAKE + 4, 64, FAKE, None) != 0   # misaligned
    assert cal.mrun_calib_read_threads() == 256 * 16 * 256
    assert cal.mrun_calib_mfma(0, 8, FAKE, None) != 0
    assert cal.mrun_calib_mfma(8, 1 << 17, FAKE, None) != 0


FAKE = 1 << 20  # a 16-byte aligned address no check dereferences


def q(experts, out, in_, group=64, bits=4, ptr=FAKE):
    return Quantized(ptr, ptr, ptr, experts, out, in_, group, bits)


def block(D=2048, E=256, k=8, I=512, S=512, **over):
    m = SparseMoe()
    m.cfg = MoeConfig(D, E, k, I, 1, S)
    m.gate = Linear(FAKE, Quantized(), None, E, D)
    m.switch_gate_proj = q(E, I, D)
    m.switch_up_proj = q(E, I, D)
    m.switch_down_proj = q(E, D, I)
    if S:
        m.shared_gate_proj = Linear(None, q(1, S, D), None, S, D)
        m.shared_up_proj = Linear(None, q(1, S, D), None, S, D)
        m.shared_down_proj = Linear(None, q(1, D, S), None, D, S)
        m.shared_expert_gate = Linear(FAKE, Quantized(), None, 1, D)
    for k_, v in over.items():
        setattr(m, k_, v)
    return m


def status(m):
    lib = _lib.load()
    rc = lib.mrun_moe_check(ctypes.byref(m))
    return rc, lib.mrun_last_error().decode()


def test_valid_blocks_pass():
    assert status(block()) == (0, "")
    assert status(block(D=6144, E=160, I=2560, S=0)) == (0, "")
    # 8-bit experts, groups 32 and 128, and the 8-bit group-64 router and shared gate of
    # mlx-community conversions (load.rs:14-17)
    E, D, I, S = 256, 2048, 512, 512
    m8 = block(switch_gate_proj=q(E, I, D, bits=8, group=32), switch_up_proj=q(E, I, D, bits=8, group=32),
               switch_down_proj=q(E, D, I, bits=8, group=128),
               gate=Linear(None, q(1, E, D, bits=8), None, E, D),
               shared_expert_gate=Linear(None, q(1, 1, D, bits=8), None, 1, D))
    assert status(m8) == (0, "")
    # dense bf16 experts (bits 16: SwitchLinear::Dense) and a dense bf16 shared expert
    dn = lambda e, o, i: Quantized(FAKE, None, None, e, o, i, 0, 16)
    md = block(switch_gate_proj=dn(E, I, D), switch_up_proj=dn(E, I, D), switch_down_proj=dn(E, D, I),
               shared_gate_proj=Linear(FAKE, Quantized(), None, S, D),
               shared_up_proj=Linear(FAKE, Quantized(), None, S, D),
               shared_down_proj=Linear(FAKE, Quantized(), None, D, S))
    assert status(md) == (0, "")
    bad = block(switch_gate_proj=Quantized(FAKE, FAKE, None, E, I, D, 0, 16))
    rc, msg = status(bad)
    assert rc == _lib.MRUN_ERR_INVALID and "carry no scales" in msg, msg


@pytest.mark.parametrize("over,code,text", [
    ({"switch_gate_proj": q(256, 512, 2048, group=16)}, _lib.MRUN_ERR_INVALID, "group_size = 16"),
    ({"switch_gate_proj": q(256, 512, 2048, bits=3)}, _lib.MRUN_ERR_INVALID, "bits = 3"),
    ({"switch_gate_proj": q(256, 512, 2048, bits=8)}, _lib.MRUN_ERR_UNSUPPORTED,
     "gate_proj and up_proj must share"),
    ({"switch_down_proj": q(256, 512, 2048)}, _lib.MRUN_ERR_INVALID, "down_proj: shape"),
    ({"switch_up_proj": q(256, 512, 2048, ptr=FAKE + 4)}, _lib.MRUN_ERR_INVALID, "aligned"),
    ({"gate": Linear(None, q(1, 256, 2048, bits=8), None, 128, 2048)}, _lib.MRUN_ERR_INVALID,
     "gate: shape"),
    ({"gate": Linear(None, q(1, 128, 2048, bits=8), None, 256, 2048)}, _lib.MRUN_ERR_INVALID,
     "gate: shape [1, 128, 2048], expected [1, 256, 2048]"),
    ({"shared_expert_gate": Linear(None, q(1, 1, 2048, bits=8, group=48), None, 1, 2048)},
     _lib.MRUN_ERR_INVALID, "group_size = 48"),
])
def test_invalid_blocks_are_refused(over, code, text):
    rc, msg = status(block(**over))
    assert rc == code and text in msg, (rc, msg)


def f32_block(D=256, E=64, k=8, I=128, S=128, **over):
    """A block of dense f32 weights (bits 32), as mrun_moe_forward_f32 takes it."""
    d = lambda e, o, i: Quantized(FAKE, None, None, e, o, i, 0, 32)
    lin = lambda o, i: Linear(None, d(1, o, i), None, o, i)
    m = SparseMoe()
    m.cfg = MoeConfig(D, E, k, I, 1, S)
    m.gate = lin(E, D)
    m.switch_gate_proj, m.switch_up_proj, m.switch_down_proj = d(E, I, D), d(E, I, D), d(E, D, I)
    if S:
        m.shared_gate_proj, m.shared_up_proj = lin(S, D), lin(S, D)
        m.shared_down_proj, m.shared_expert_gate = lin(D, S), lin(1, D)
    for k_, v in over.items():
        setattr(m, k_, v)
    return m


def test_f32_blocks():
    """f32 blocks (bits 32 everywhere) pass the check; a bf16 or quantized weight among them, a
    Linear bias or scales are refused; the bf16 forward refuses them before any device work, and
    the f32 forward's workspace is sized from the config alone."""
    lib = _lib.load()
    assert status(f32_block()) == (0, "")
    assert status(f32_block(S=0)) == (0, "")
    d = lambda e, o, i: Quantized(FAKE, None, None, e, o, i, 0, 32)
    cases = [
        ({"gate": Linear(FAKE, Quantized(), None, 64, 256)}, _lib.MRUN_ERR_INVALID,
         "gate: an f32 block's Linear carries its weight in q"),
        ({"shared_up_proj": Linear(None, q(1, 128, 256), None, 128, 256)}, _lib.MRUN_ERR_INVALID,
         "shared_expert.up_proj: an f32 block takes dense f32 weights"),
        ({"switch_down_proj": Quantized(FAKE, FAKE, None, 64, 256, 128, 0, 32)},
         _lib.MRUN_ERR_INVALID, "carry no scales"),
        ({"switch_up_proj": d(64, 128, 255)}, _lib.MRUN_ERR_INVALID, "switch_mlp.up_proj: shape"),
        ({"shared_expert_gate": Linear(None, d(1, 1, 256), FAKE, 1, 256)},
         _lib.MRUN_ERR_UNSUPPORTED, "f32 Linear biases"),
    ]
    for over, code, text in cases:
        rc, msg = status(f32_block(**over))
        assert rc == code and text in msg, (over, rc, msg)
    m = f32_block()
    rc = lib.mrun_moe_forward(ctypes.byref(m), FAKE, 4, FAKE * 2, FAKE * 3, 1 << 30, None)
    msg = lib.mrun_last_error().decode()
    assert rc == _lib.MRUN_ERR_UNSUPPORTED and "run through mrun_moe_forward_f32" in msg, msg
    # a bf16 block is not an f32 one
    rc = lib.mrun_moe_forward_f32(ctypes.byref(block()), FAKE, 4, FAKE * 2, FAKE * 3, 1 << 30, None)
    assert rc == _lib.MRUN_ERR_INVALID, lib.mrun_last_error()
    cfg = MoeConfig(256, 64, 8, 128, 1, 128)
    T, P = 5, 40
    a = lambda n: (n + 255) // 256 * 256
    want = a(4 * T * 64) + 2 * a(4 * P) + a(4 * P * 128) + a(4 * P * 256) + a(4 * T) \
        + a(4 * T * 128) + a(4 * T * 256)
    assert lib.mrun_moe_workspace_bytes_f32(ctypes.byref(cfg), T) == want
    assert lib.mrun_moe_workspace_bytes_f32(ctypes.byref(cfg), 0) == 0
    rc = lib.mrun_moe_forward_f32(ctypes.byref(m), FAKE, 4, FAKE * 2, FAKE * 3, 64, None)
    assert rc == _lib.MRUN_ERR_WORKSPACE, lib.mrun_last_error()
    assert lib.mrun_moe_forward_f32(ctypes.byref(m), FAKE, 0, None, None, 0, None) == 0


def test_top_k_must_fit_the_experts():
    m = block()
    m.cfg = MoeConfig(2048, 256, 257, 512, 1, 512)
    rc, msg = status(m)
    assert rc == _lib.MRUN_ERR_INVALID and "num_experts_per_tok" in msg


def test_workspace_contract():
    lib = _lib.load()
    cfg = MoeConfig(2048, 256, 8, 512, 1, 512)
    sizes = [lib.mrun_moe_workspace_bytes(ctypes.byref(cfg), t) for t in (1, 16, 2048)]
    assert 0 < sizes[0] < sizes[1] < sizes[2]
    # below SparseMoe::scratch_per_token (moe.rs:176-187: 188,416 B per token here)
    assert sizes[2] < 2048 * 188416
    assert lib.mrun_moe_workspace_bytes(ctypes.byref(MoeConfig(0, 0, 0, 0, 0, 0)), 4) == 0
    # a workspace one byte short is refused before any device work
    m = block()
    rc = lib.mrun_moe_forward(ctypes.byref(m), FAKE, 1, FAKE * 2, FAKE * 4, sizes[0] - 1, None)
    assert rc == _lib.MRUN_ERR_WORKSPACE and "workspace" in lib.mrun_last_error().decode()
    rc = lib.mrun_moe_forward(ctypes.byref(m), FAKE, 1, FAKE, FAKE * 4, sizes[0], None)
    assert rc == _lib.MRUN_ERR_INVALID and "alias" in lib.mrun_last_error().decode()
    rc = lib.mrun_moe_forward(ctypes.byref(m), FAKE, -1, FAKE * 2, FAKE * 4, sizes[0], None)
    assert rc == _lib.MRUN_ERR_INVALID


def test_every_decode_batch_fits_the_noalloc_scratch():
    """mrun_moe_forward_noalloc takes every decode batch (T <= 32): the workspace of the widest
    configuration the decode kernels accept (hidden, FFN and shared widths 8192, 512 experts,
    k = 16, 32 tokens) fits its scratch array, and so does a Qwen3.6-like prefill chunk of 512."""
    lib = _lib.load()
    lim = lib.mrun_moe_forward_noalloc_max_bytes()
    assert lim == 32 << 20
    for cfg, T in ((MoeConfig(8192, 512, 16, 8192, 1, 8192), 32),
                   (MoeConfig(6144, 160, 8, 2560, 1, 0), 32),
                   (MoeConfig(2048, 256, 8, 512, 1, 512), 512)):
        assert 0 < lib.mrun_moe_workspace_bytes(ctypes.byref(cfg), T) <= lim, (cfg.hidden, T)


def test_op_argument_errors():
    lib = _lib.load()
    rc = lib.mrun_moe_permute(FAKE, 10, 3, 16, FAKE, None, None, None, None, 0, None)
    assert rc == _lib.MRUN_ERR_INVALID and "multiple of top_k" in lib.mrun_last_error().decode()
    rc = lib.mrun_moe_combine(FAKE, None, FAKE, 2, 8, 2050, None, None, FAKE, None)
    assert rc == _lib.MRUN_ERR_INVALID
    w = q(4, 64, 100)
    rc = lib.mrun_gather_qmm(FAKE, 2, ctypes.byref(w), FAKE, 4, 0, FAKE, FAKE, 1 << 20, None)
    assert rc == _lib.MRUN_ERR_INVALID and "not a multiple of group_size" in lib.mrun_last_error().decode()


def test_empty_batches_are_no_ops():
    """A token or row count of 0 is an empty batch (the facade's ops take empty arrays): the call
    checks its weights and returns 0 without reading a pointer; negative counts are refused."""
    lib = _lib.load()
    m = block()
    assert lib.mrun_moe_forward(ctypes.byref(m), None, 0, None, None, 0, None) == 0
    assert lib.mrun_moe_forward(ctypes.byref(m), FAKE, -1, FAKE * 2, FAKE * 4, 1 << 30,
                                None) == _lib.MRUN_ERR_INVALID
    n_stages = ctypes.c_int32(7)
    assert lib.mrun_moe_forward_profiled(ctypes.byref(m), None, 0, None, None, 0, None, None, 0,
                                         ctypes.byref(n_stages)) == 0
    assert n_stages.value == 0
    assert lib.mrun_moe_router(ctypes.byref(m), None, 0, None, None, None, None, None, 0,
                               None) == 0
    # the weights are still checked
    bad = block(E=4, k=8)
    assert lib.mrun_moe_forward(ctypes.byref(bad), None, 0, None, None, 0,
                                None) == _lib.MRUN_ERR_INVALID
    w = q(4, 64, 128)
    assert lib.mrun_gather_qmm(None, 0, ctypes.byref(w), None, 0, 0, None, None, 0, None) == 0
    assert lib.mrun_gather_qmm(None, 0, ctypes.byref(q(4, 64, 100)), None, 0, 0, None, None, 0,
                               None) == _lib.MRUN_ERR_INVALID
    assert lib.mrun_quantized_matmul(None, 0, ctypes.byref(q(1, 64, 128)), None, None) == 0
    assert lib.mrun_quantized_matmul(None, -2, ctypes.byref(q(1, 64, 128)), None,
                                     None) == _lib.MRUN_ERR_INVALID
    lin = Linear(FAKE, Quantized(), None, 64, 128)
    assert lib.mrun_linear_forward(ctypes.byref(lin), None, 0, None, None) == 0
    assert lib.mrun_moe_combine(None, None, None, 0, 8, 2048, None, None, None, None) == 0
    assert lib.mrun_rms_norm(None, None, 0, 2048, 1e-6, None, None) == 0
    assert lib.mrun_add_rms_norm(None, None, None, 0, 2048, 1e-6, None, None, None) == 0
    assert lib.mrun_rms_norm(None, None, -1, 2048, 1e-6, None, None) == _lib.MRUN_ERR_INVALID
    layers = (SparseMoe * 2)(m, m)
    assert lib.mrun_moe_stack_forward(layers, 2, None, 1e-6, None, 0, None, 0, None) == 0
    assert lib.mrun_moe_workspace_bytes(ctypes.byref(m.cfg), 0) == 0
