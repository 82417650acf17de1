"""ctypes view of the C ABI in include/mrun_moe.h (libmrun_moe.so, built in-tree by mrun_amd/build.py).

Loading fails loudly: there is no fallback path, so a missing or stale library is an error.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_float, c_int32, c_int64, c_size_t, c_uint32, c_void_p
from pathlib import Path

LIB_DIR = Path(__file__).resolve().parent / "lib"
LIB_PATH = LIB_DIR / "libmrun_moe.so"

MRUN_OK = 0
MRUN_ERR_INVALID = 1
MRUN_ERR_UNSUPPORTED = 2
MRUN_ERR_WORKSPACE = 3
MRUN_ERR_HIP = 4


class Quantized(ctypes.Structure):
    _fields_ = [
        ("weight", c_void_p),
        ("scales", c_void_p),
        ("biases", c_void_p),
        ("experts", c_int32),
        ("out", c_int32),
        ("in_", c_int32),
        ("group_size", c_int32),
        ("bits", c_int32),
    ]


class Linear(ctypes.Structure):
    _fields_ = [
        ("weight", c_void_p),
        ("q", Quantized),
        ("bias", c_void_p),
        ("out", c_int32),
        ("in_", c_int32),
    ]


class MoeConfig(ctypes.Structure):
    _fields_ = [
        ("hidden", c_int32),
        ("experts", c_int32),
        ("top_k", c_int32),
        ("intermediate", c_int32),
        ("norm_topk_prob", c_int32),
        ("shared_intermediate", c_int32),
    ]


class SparseMoe(ctypes.Structure):
    _fields_ = [
        ("cfg", MoeConfig),
        ("gate", Linear),
        ("switch_gate_proj", Quantized),
        ("switch_up_proj", Quantized),
        ("switch_down_proj", Quantized),
        ("shared_gate_proj", Linear),
        ("shared_up_proj", Linear),
        ("shared_down_proj", Linear),
        ("shared_expert_gate", Linear),
    ]


# name -> (restype, argtypes)
SIGNATURES = {
    "mrun_last_error": (c_char_p, []),
    "mrun_version": (c_char_p, []),
    "mrun_moe_check": (c_int32, [POINTER(SparseMoe)]),
    "mrun_moe_workspace_bytes": (c_size_t, [POINTER(MoeConfig), c_int32]),
    "mrun_moe_forward": (
        c_int32,
        [POINTER(SparseMoe), c_void_p, c_int32, c_void_p, c_void_p, c_size_t, c_void_p],
    ),
    "mrun_moe_workspace_bytes_f32": (c_size_t, [POINTER(MoeConfig), c_int32]),
    "mrun_moe_forward_f32": (
        c_int32,
        [POINTER(SparseMoe), c_void_p, c_int32, c_void_p, c_void_p, c_size_t, c_void_p],
    ),
    "mrun_moe_forward_noalloc": (
        c_int32, [POINTER(SparseMoe), c_void_p, c_int32, c_void_p, c_void_p],
    ),
    "mrun_moe_forward_noalloc_max_bytes": (c_size_t, []),
    "mrun_moe_forward_profiled": (
        c_int32,
        [POINTER(SparseMoe), c_void_p, c_int32, c_void_p, c_void_p, c_size_t, c_void_p,
         POINTER(c_void_p), c_int32, POINTER(c_int32)],
    ),
    "mrun_moe_stage_names": (c_char_p, [POINTER(MoeConfig), c_int32]),
    "mrun_moe_forward_timed": (
        c_int32,
        [POINTER(SparseMoe), c_void_p, c_int32, c_void_p, c_void_p, c_size_t, c_void_p,
         c_void_p],
    ),
    "mrun_wall_clock_hz": (c_int64, []),
    "mrun_moe_router": (
        c_int32,
        [POINTER(SparseMoe), c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p, c_size_t, c_void_p],
    ),
    "mrun_moe_permute": (
        c_int32,
        [c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
         c_size_t, c_void_p],
    ),
    "mrun_moe_permute_workspace_bytes": (c_size_t, [c_int32, c_int32]),
    "mrun_moe_workspace_routing": (c_int32, [POINTER(MoeConfig), c_int32, POINTER(c_size_t)]),
    "mrun_gather_qmm": (
        c_int32,
        [c_void_p, c_int32, POINTER(Quantized), c_void_p, c_int32, c_int32, c_void_p, c_void_p,
         c_size_t, c_void_p],
    ),
    "mrun_gather_qmm_workspace_bytes": (c_size_t, [c_int32, c_int32, c_int32, c_int32, c_int32]),
    "mrun_quantized_matmul": (c_int32, [c_void_p, c_int32, POINTER(Quantized), c_void_p, c_void_p]),
    "mrun_linear_forward": (c_int32, [POINTER(Linear), c_void_p, c_int32, c_void_p, c_void_p]),
    "mrun_swiglu": (c_int32, [c_void_p, c_void_p, c_int64, c_void_p, c_void_p]),
    "mrun_moe_combine": (
        c_int32,
        [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p,
         c_void_p],
    ),
    "mrun_rms_norm": (
        c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_float, c_void_p, c_void_p]
    ),
    "mrun_add_rms_norm": (
        c_int32,
        [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_float, c_void_p, c_void_p, c_void_p],
    ),
    "mrun_moe_stack_forward": (
        c_int32,
        [c_void_p, c_int32, c_void_p, c_float, c_void_p, c_int32, c_void_p, c_size_t, c_void_p],
    ),
    "mrun_moe_stack_workspace_bytes": (c_size_t, [POINTER(MoeConfig), c_int32]),
    # include/mrun_load.h
    "mrun_weights_open": (c_int32, [c_char_p, POINTER(c_void_p)]),
    "mrun_weights_close": (None, [c_void_p]),
    "mrun_weights_moe_config": (c_int32, [c_void_p, POINTER(MoeConfig), POINTER(c_float)]),
    "mrun_weights_tensor_info": (
        c_int32, [c_void_p, c_char_p, c_char_p, POINTER(c_int64), POINTER(c_int32)]
    ),
    "mrun_weights_remaining": (c_int32, [c_void_p]),
    "mrun_weights_resolve_quant": (
        c_int32, [c_void_p, c_char_p, c_int32, POINTER(c_int32), POINTER(c_int32)]
    ),
    "mrun_weights_load_moe": (
        c_int32, [c_void_p, c_char_p, POINTER(MoeConfig), POINTER(SparseMoe)]
    ),
    "mrun_weights_load_bf16": (c_int32, [c_void_p, c_char_p, c_int64, POINTER(c_void_p)]),
}


class MrunError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"mrun error {code}: {message}")
        self.code = code
        self.message = message


_LIB = None


def load(path: Path | None = None) -> ctypes.CDLL:
    """The C-ABI library, loaded once. Raises if it is missing or lacks a declared symbol."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise RuntimeError(
            f"{p} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
        )
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError: a declared entry point is not exported
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _LIB = lib
    return lib


def check(code: int) -> None:
    if code != MRUN_OK:
        msg = load().mrun_last_error()
        raise MrunError(code, msg.decode() if msg else "")
