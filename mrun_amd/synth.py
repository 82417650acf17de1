"""Seeded synthetic MoE blocks and activations (the generator spec is in include/mrun_synth.h).

The benchmark configurations give the synthetic tensors by distribution only; this module makes
them concrete: 4-bit affine weights with group 64, codes uniform 0..15, scales |N(0,0.02)|/7.5,
biases -8*scale, a bf16 N(0,0.02) router (optionally Zipf-biased) and shared-expert gate, bf16
N(0,1) activations. Arrays are host numpy arrays; bf16 is carried as uint16 bits.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_double, c_float, c_int32, c_size_t, c_uint16, c_uint32, c_uint64
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libmrun_synth.so"
BASE_SEED = 0x6D72756E2D6D6F65  # "mrun-moe"

# tensor ids of the generator's seed derivation
X, ROUTER_W, ROUTER_BIAS = 0, 1, 2
GATE_CODES, GATE_SCALES, UP_CODES, UP_SCALES, DOWN_CODES, DOWN_SCALES = 3, 4, 5, 6, 7, 8
SH_GATE_CODES, SH_GATE_SCALES, SH_UP_CODES, SH_UP_SCALES = 9, 10, 11, 12
SH_DOWN_CODES, SH_DOWN_SCALES, SH_EXPERT_GATE = 13, 14, 15


@dataclass(frozen=True)
class Shape:
    """MoeConfig (moe.rs:97-107)."""

    hidden: int
    experts: int
    top_k: int
    intermediate: int
    shared: int = 0
    norm_topk: bool = True
    group: int = 64

    @property
    def name(self) -> str:
        return f"D{self.hidden}_E{self.experts}_k{self.top_k}_I{self.intermediate}_S{self.shared}"


# Qwen3.6-35B-A3B-like and Qwen3-Coder-480B-A35B-like blocks.
QWEN36 = Shape(hidden=2048, experts=256, top_k=8, intermediate=512, shared=512)
CODER = Shape(hidden=6144, experts=160, top_k=8, intermediate=2560, shared=0)

# configuration ids of the seed derivation (the benchmark's configs[0..4])
CFG_PLUMBING, CFG_DECODE, CFG_PREFILL_ZIPF, CFG_STACK, CFG_CODER = 0, 1, 2, 3, 4


@dataclass
class QTensor:
    """An affine 4/8-bit stacked weight: codes [E, out, in*bits/32] u32, scales/biases [E, out, in/g];
    bits 16: dense bf16 weights in `codes` (two per word), no scales."""

    codes: np.ndarray
    scales: np.ndarray | None
    biases: np.ndarray | None
    experts: int
    out: int
    in_: int
    group: int
    bits: int = 4

    @property
    def nbytes(self) -> int:
        b = self.codes.nbytes + (self.scales.nbytes if self.scales is not None else 0)
        return b + (self.biases.nbytes if self.biases is not None else 0)


@dataclass
class HostBlock:
    """The tensors of one SparseMoe (moe.rs:109-147) on the host."""

    shape: Shape
    router: "np.ndarray | QTensor"     # [E, D] bf16, or quantized (8-bit in real checkpoints)
    router_bias: np.ndarray | None     # [E] bf16
    gate_proj: QTensor
    up_proj: QTensor
    down_proj: QTensor
    sh_gate_proj: QTensor | None = None
    sh_up_proj: QTensor | None = None
    sh_down_proj: QTensor | None = None
    sh_expert_gate: "np.ndarray | QTensor | None" = None  # [1, D] bf16 or quantized
    zipf_rank: np.ndarray | None = field(default=None, repr=False)

    @property
    def nbytes(self) -> int:
        n = self.router.nbytes + self.gate_proj.nbytes + self.up_proj.nbytes
        n += self.down_proj.nbytes
        for q in (self.sh_gate_proj, self.sh_up_proj, self.sh_down_proj):
            if q is not None:
                n += q.nbytes
        if self.sh_expert_gate is not None:
            n += self.sh_expert_gate.nbytes
        return n


_LIB = None


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build()")
        l = ctypes.CDLL(str(LIB_PATH))
        l.mrun_synth_mix64.restype = c_uint64
        l.mrun_synth_mix64.argtypes = [c_uint64]
        l.mrun_synth_tensor_seed.restype = c_uint64
        l.mrun_synth_tensor_seed.argtypes = [c_uint64, c_uint32, c_uint32, c_uint32]
        l.mrun_synth_draw.restype = c_uint64
        l.mrun_synth_draw.argtypes = [c_uint64, c_uint64]
        l.mrun_synth_normal.restype = c_double
        l.mrun_synth_normal.argtypes = [c_uint64, c_uint64]
        l.mrun_synth_codes.restype = c_int32
        l.mrun_synth_codes.argtypes = [c_uint64, c_int32, POINTER(c_uint32), c_size_t]
        l.mrun_synth_normal_bf16.restype = None
        l.mrun_synth_normal_bf16.argtypes = [c_uint64, c_float, POINTER(c_uint16), c_size_t]
        l.mrun_synth_scales_biases.restype = None
        l.mrun_synth_scales_biases.argtypes = [c_uint64, POINTER(c_uint16), POINTER(c_uint16),
                                              c_size_t]
        l.mrun_synth_zipf_bias.restype = c_int32
        l.mrun_synth_zipf_bias.argtypes = [c_uint64, c_int32, c_double, c_double,
                                          POINTER(c_uint16), POINTER(c_int32)]
        _LIB = l
    return _LIB


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(POINTER(t))


def seed(config: int, layer: int, tensor: int, base: int = BASE_SEED) -> int:
    return int(lib().mrun_synth_tensor_seed(base, config, layer, tensor))


def codes(s: int, n_words: int, bits: int = 4) -> np.ndarray:
    out = np.empty(n_words, dtype=np.uint32)
    if lib().mrun_synth_codes(s, bits, _p(out, c_uint32), n_words) != 0:
        raise ValueError("bits must be 4 or 8")
    return out


def normal_bf16(s: int, n: int, std: float) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    lib().mrun_synth_normal_bf16(s, std, _p(out, c_uint16), n)
    return out


def scales_biases(s: int, n: int) -> tuple[np.ndarray, np.ndarray]:
    sc = np.empty(n, dtype=np.uint16)
    bi = np.empty(n, dtype=np.uint16)
    lib().mrun_synth_scales_biases(s, _p(sc, c_uint16), _p(bi, c_uint16), n)
    return sc, bi


def zipf_bias(s: int, experts: int, exponent: float = 1.1, amp: float = 2.0):
    b = np.empty(experts, dtype=np.uint16)
    r = np.empty(experts, dtype=np.int32)
    lib().mrun_synth_zipf_bias(s, experts, exponent, amp, _p(b, c_uint16), _p(r, c_int32))
    return b, r


def qtensor(config: int, layer: int, codes_id: int, scales_id: int, experts: int, out: int,
            in_: int, group: int = 64) -> QTensor:
    c = codes(seed(config, layer, codes_id), experts * out * in_ // 8)
    sc, bi = scales_biases(seed(config, layer, scales_id), experts * out * in_ // group)
    return QTensor(
        codes=c.reshape(experts, out, in_ // 8),
        scales=sc.reshape(experts, out, in_ // group),
        biases=bi.reshape(experts, out, in_ // group),
        experts=experts, out=out, in_=in_, group=group,
    )


def qtensor8(config: int, layer: int, codes_id: int, scales_id: int, experts: int, out: int,
             in_: int, group: int = 64) -> QTensor:
    """An 8-bit stacked weight: codes uniform 0..255, scales bf16(|bf16(0.02 N)| / 127.5), biases
    -128 * scale (exact), so each weight dequantises to scale * (q - 128)."""
    c = codes(seed(config, layer, codes_id), experts * out * in_ // 4, bits=8)
    n = experts * out * in_ // group
    sc = f32_to_bf16(np.abs(bf16_to_f32(normal_bf16(seed(config, layer, scales_id), n, 0.02)))
                     / np.float32(127.5))
    bi = f32_to_bf16(np.float32(-128.0) * bf16_to_f32(sc))
    return QTensor(codes=c.reshape(experts, out, in_ // 4), scales=sc.reshape(experts, out, -1),
                   biases=bi.reshape(experts, out, -1), experts=experts, out=out, in_=in_,
                   group=group, bits=8)


def dense_experts(config: int, layer: int, codes_id: int, experts: int, out: int, in_: int,
                  std: float = 0.02) -> QTensor:
    """Unquantized bf16 expert weights N(0, std) [E, out, in] (SwitchLinear::Dense, moe.rs:43-46),
    carried as bits 16: two bf16 per u32 word, the first in the low half; no scales."""
    w = normal_bf16(seed(config, layer, codes_id), experts * out * in_, std)
    return QTensor(codes=w.view(np.uint32).reshape(experts, out, in_ // 2), scales=None,
                   biases=None, experts=experts, out=out, in_=in_, group=0, bits=16)


def quantize(w: np.ndarray, bits: int, group: int) -> QTensor:
    """Affine quantization of a bf16 matrix [out, in] (or [E, out, in]) per group: scale =
    bf16((max - min) / (2^bits - 1)), bias = bf16(min), q = clip(round((w - bias) / scale)),
    codes packed LSB first. The format of mlx-community checkpoints' 8-bit routers; the exact
    rounding of the scale does not matter to the block, which reads the stored values."""
    w3 = bf16_to_f32(w).astype(np.float64)
    if w3.ndim == 2:
        w3 = w3[None]
    E, out, in_ = w3.shape
    g = w3.reshape(E, out, in_ // group, group)
    lo, hi = g.min(axis=-1), g.max(axis=-1)
    levels = (1 << bits) - 1
    sc = f32_to_bf16(np.maximum((hi - lo) / levels, 1e-8).astype(np.float32))
    bi = f32_to_bf16(lo.astype(np.float32))
    s64, b64 = bf16_to_f32(sc).astype(np.float64), bf16_to_f32(bi).astype(np.float64)
    q = np.clip(np.rint((g - b64[..., None]) / s64[..., None]), 0, levels).astype(np.uint32)
    q = q.reshape(E, out, in_)
    per = 32 // bits
    words = np.zeros((E, out, in_ // per), np.uint32)
    for i in range(per):
        words |= q[:, :, i::per] << np.uint32(bits * i)
    return QTensor(codes=words, scales=sc, biases=bi, experts=E, out=out, in_=in_, group=group,
                   bits=bits)


def make_block(shape: Shape, config: int = CFG_DECODE, layer: int = 0,
               zipf: bool = False, expert_bits: int = 4, gate_bits: int = 0) -> HostBlock:
    """The seeded block of the BASELINE configs. expert_bits 8 draws 8-bit experts and shared
    expert (qtensor8), 16 dense bf16 ones (dense_experts); gate_bits 8 (or 4) quantizes the router
    and the shared-expert gate with group 64, as mlx-community conversions store them."""
    D, E, I, S, g = shape.hidden, shape.experts, shape.intermediate, shape.shared, shape.group
    router = normal_bf16(seed(config, layer, ROUTER_W), E * D, 0.02).reshape(E, D)
    rb, rank = (None, None)
    if zipf:
        rb, rank = zipf_bias(seed(config, layer, ROUTER_BIAS), E)
    if expert_bits == 16:
        qt = lambda c, l, ci, si, e, o, i_, g_: dense_experts(c, l, ci, e, o, i_)
    else:
        qt = qtensor8 if expert_bits == 8 else qtensor
    blk = HostBlock(
        shape=shape,
        router=quantize(router, gate_bits, 64) if gate_bits else router,
        router_bias=rb,
        gate_proj=qt(config, layer, GATE_CODES, GATE_SCALES, E, I, D, g),
        up_proj=qt(config, layer, UP_CODES, UP_SCALES, E, I, D, g),
        down_proj=qt(config, layer, DOWN_CODES, DOWN_SCALES, E, D, I, g),
        zipf_rank=rank,
    )
    if S:
        blk.sh_gate_proj = qt(config, layer, SH_GATE_CODES, SH_GATE_SCALES, 1, S, D, g)
        blk.sh_up_proj = qt(config, layer, SH_UP_CODES, SH_UP_SCALES, 1, S, D, g)
        blk.sh_down_proj = qt(config, layer, SH_DOWN_CODES, SH_DOWN_SCALES, 1, D, S, g)
        sg = normal_bf16(seed(config, layer, SH_EXPERT_GATE), D, 0.02).reshape(1, D)
        blk.sh_expert_gate = quantize(sg, gate_bits, 64) if gate_bits else sg
    return blk


@dataclass
class F32Block:
    """The tensors of one SparseMoe of a float32 checkpoint, all dense f32 [out, in] rows: router
    [E, D], gate/up [E, I, D], down [E, D, I]; with a shared expert its gate/up [S, D], down [D, S]
    and gate [1, D]."""

    shape: Shape
    router: np.ndarray
    gate_proj: np.ndarray
    up_proj: np.ndarray
    down_proj: np.ndarray
    sh_gate_proj: np.ndarray | None = None
    sh_up_proj: np.ndarray | None = None
    sh_down_proj: np.ndarray | None = None
    sh_expert_gate: np.ndarray | None = None


def normal_f32(s: int, shape: tuple, std: float) -> np.ndarray:
    """f32 N(0, std) from numpy's PCG64 seeded with s (full f32 mantissas, unlike the bf16 draws)."""
    return (np.random.default_rng(s).standard_normal(shape) * std).astype(np.float32)


def make_block_f32(shape: Shape, config: int = CFG_PLUMBING, layer: int = 0) -> F32Block:
    """A seeded f32 block: weights N(0, 1/sqrt(in)), the router N(0, 2/sqrt(D)) so that its
    softmax is far from uniform."""
    D, E, I, S = shape.hidden, shape.experts, shape.intermediate, shape.shared
    w = lambda tid, shp: normal_f32(seed(config, layer, tid), shp, 1.0 / np.sqrt(shp[-1]))
    blk = F32Block(shape=shape,
                   router=normal_f32(seed(config, layer, ROUTER_W), (E, D), 2.0 / np.sqrt(D)),
                   gate_proj=w(GATE_CODES, (E, I, D)), up_proj=w(UP_CODES, (E, I, D)),
                   down_proj=w(DOWN_CODES, (E, D, I)))
    if S:
        blk.sh_gate_proj = w(SH_GATE_CODES, (S, D))
        blk.sh_up_proj = w(SH_UP_CODES, (S, D))
        blk.sh_down_proj = w(SH_DOWN_CODES, (D, S))
        blk.sh_expert_gate = w(SH_EXPERT_GATE, (1, D))
    return blk


def make_x_f32(shape: Shape, tokens: int, config: int = CFG_PLUMBING, layer: int = 0) -> np.ndarray:
    """f32 N(0,1) activations [tokens, hidden]."""
    return normal_f32(seed(config, layer, X), (tokens, shape.hidden), 1.0)


def make_x(shape: Shape, tokens: int, config: int = CFG_DECODE, layer: int = 0) -> np.ndarray:
    """bf16 N(0,1) activations [tokens, hidden]."""
    return normal_bf16(seed(config, layer, X), tokens * shape.hidden, 1.0).reshape(
        tokens, shape.hidden)


def bf16_to_f32(a: np.ndarray) -> np.ndarray:
    return (a.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    """Round to nearest even (NaN kept quiet)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r
