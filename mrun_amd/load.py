"""Checkpoint loading over include/mrun_load.h: MLX and Hugging Face safetensors checkpoints into
device views of the MoE block.

Mirrors the reference's crates/mrun-engine/src/load.rs (`Weights::load`, `Quantization`,
`Linear::load`) and `SparseMoe::load` (models/moe.rs:120-147): the same tensor names, the same
quantization rules (per-path config overrides, otherwise inferred from the packed shapes) and the
same refusals. Parsing and device copies run in libmrun_moe.so; device memory belongs to the
`Weights` object and lives until it is closed.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

from . import _lib
from ._lib import MoeConfig, SparseMoe as _SparseMoe, check
from .moe import SparseMoe, SparseMoeF32


class Weights:
    """An opened checkpoint directory (`Weights::load`, load.rs:179-196)."""

    def __init__(self, path: str | Path):
        self._lib = _lib.load()
        h = ctypes.c_void_p()
        check(self._lib.mrun_weights_open(str(path).encode(), ctypes.byref(h)))
        self._h = h
        self.path = Path(path)

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            self._lib.mrun_weights_close(self._h)
        self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def moe_config(self) -> tuple[MoeConfig, float]:
        """(MoeConfig, rms_norm_eps) from config.json."""
        cfg, eps = MoeConfig(), ctypes.c_float()
        check(self._lib.mrun_weights_moe_config(self._h, ctypes.byref(cfg), ctypes.byref(eps)))
        return cfg, float(eps.value)

    def tensor_info(self, name: str) -> tuple[str, tuple[int, ...]]:
        dt = ctypes.create_string_buffer(8)
        shape = (ctypes.c_int64 * 8)()
        nd = ctypes.c_int32()
        check(self._lib.mrun_weights_tensor_info(self._h, name.encode(), dt, shape,
                                                 ctypes.byref(nd)))
        return dt.value.decode(), tuple(shape[i] for i in range(nd.value))

    def remaining(self) -> int:
        return int(self._lib.mrun_weights_remaining(self._h))

    def resolve_quant(self, path: str, in_dims: int) -> tuple[int, int]:
        """(group_size, bits) of the quantized layer at `path` (`Quantization::resolve`)."""
        g, b = ctypes.c_int32(), ctypes.c_int32()
        check(self._lib.mrun_weights_resolve_quant(self._h, path.encode(), in_dims,
                                                   ctypes.byref(g), ctypes.byref(b)))
        return g.value, b.value

    def load_moe(self, prefix: str, cfg: MoeConfig | None = None) -> SparseMoe:
        """`SparseMoe::load` at `prefix` (e.g. "language_model.model.layers.0.mlp")."""
        cfg = cfg if cfg is not None else self.moe_config()[0]
        view = _SparseMoe()
        check(self._lib.mrun_weights_load_moe(self._h, prefix.encode(), ctypes.byref(cfg),
                                              ctypes.byref(view)))
        if view.switch_gate_proj.bits == 32:  # an f32 checkpoint's block
            return SparseMoeF32.from_view(view, owner=self)
        return SparseMoe.from_view(view, owner=self)

    def load_bf16(self, name: str, n: int) -> int:
        """Device address of bf16 tensor `name` ([n] elements, e.g. an RMSNorm weight)."""
        p = ctypes.c_void_p()
        check(self._lib.mrun_weights_load_bf16(self._h, name.encode(), n, ctypes.byref(p)))
        return int(p.value)


__all__ = ["Weights"]
