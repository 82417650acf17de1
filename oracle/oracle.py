"""ctypes loader of the CPU restatement (oracle/moe_oracle.c): TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this module, and only as
the checker; the product (mrun_amd/) never imports it. Arrays are numpy host arrays with bf16
carried as uint16 bits. See moe_oracle.h for what each function restates and how it is pinned.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_float, c_int32, c_size_t, c_uint16, c_uint32, c_void_p
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "_build" / "liborc_moe.so"


class OrcQ(ctypes.Structure):
    _fields_ = [("codes", c_void_p), ("scales", c_void_p), ("biases", c_void_p),
                ("experts", c_int32), ("out", c_int32), ("in_", c_int32), ("group", c_int32),
                ("bits", c_int32)]


class OrcLinear(ctypes.Structure):
    _fields_ = [("dense", c_void_p), ("q", OrcQ), ("bias", c_void_p), ("out", c_int32),
                ("in_", c_int32)]


class OrcConfig(ctypes.Structure):
    _fields_ = [("hidden", c_int32), ("experts", c_int32), ("top_k", c_int32),
                ("intermediate", c_int32), ("norm_topk_prob", c_int32),
                ("shared_intermediate", c_int32)]


class OrcBlock(ctypes.Structure):
    _fields_ = [("cfg", OrcConfig), ("gate", OrcLinear), ("sw_gate", OrcQ), ("sw_up", OrcQ),
                ("sw_down", OrcQ), ("sh_gate", OrcLinear), ("sh_up", OrcLinear),
                ("sh_down", OrcLinear), ("sh_expert_gate", OrcLinear)]


class OrcBlockF32(ctypes.Structure):
    _fields_ = [("cfg", OrcConfig)] + [(n, c_void_p) for n in (
        "router", "sw_gate", "sw_up", "sw_down", "sh_gate", "sh_up", "sh_down", "sh_expert_gate")]


class OrcTrace(ctypes.Structure):
    _fields_ = [(n, c_void_p) for n in ("logits", "gates", "ids", "scores", "order", "inverse",
                                        "act", "y", "routed", "shared_gate", "shared_y")]


_LIB = None


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: run `make -C oracle`")
        l = ctypes.CDLL(str(LIB_PATH))
        l.orc_bf16_from_f32.restype = c_uint16
        l.orc_bf16_from_f32.argtypes = [c_float]
        l.orc_f32_from_bf16.restype = c_float
        l.orc_f32_from_bf16.argtypes = [c_uint16]
        l.orc_round_bf16_array.argtypes = [c_void_p, c_size_t, c_void_p]
        l.orc_dequant_row.argtypes = [POINTER(OrcQ), c_int32, c_int32, c_void_p]
        l.orc_linear_forward.argtypes = [POINTER(OrcLinear), c_void_p, c_int32, c_void_p]
        l.orc_qmatmul.argtypes = [POINTER(OrcQ), c_void_p, c_int32, c_void_p]
        l.orc_gather_qmm.argtypes = [POINTER(OrcQ), c_void_p, c_int32, c_void_p, c_int32, c_void_p]
        l.orc_softmax.argtypes = [c_void_p, c_int32, c_int32, c_void_p]
        l.orc_topk.argtypes = [c_void_p, c_int32, c_int32, c_int32, c_void_p]
        l.orc_scores.argtypes = [c_void_p, c_int32, c_int32, c_void_p, c_int32, c_int32, c_void_p]
        l.orc_permute.argtypes = [c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p,
                                  c_void_p, c_void_p]
        l.orc_floor_divide_u32.argtypes = [c_void_p, c_size_t, c_uint32, c_void_p]
        l.orc_swiglu.argtypes = [c_void_p, c_void_p, c_size_t, c_void_p]
        l.orc_swiglu_f32.argtypes = [c_void_p, c_void_p, c_size_t, c_void_p]
        l.orc_combine.argtypes = [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p]
        l.orc_shared_add.argtypes = [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p,
                                     c_void_p]
        l.orc_rms_norm.argtypes = [c_void_p, c_void_p, c_int32, c_int32, c_float, c_void_p]
        l.orc_moe_forward.argtypes = [POINTER(OrcBlock), c_void_p, c_int32, c_void_p, c_void_p,
                                      POINTER(OrcTrace)]
        l.orc_topk_valid.argtypes = [c_void_p, c_void_p, c_int32, c_int32, c_void_p, c_int32]
        l.orc_moe_stack.argtypes = [POINTER(OrcBlock), c_int32, c_void_p, c_float, c_void_p,
                                    c_int32]
        l.orc_set_threads.argtypes = [c_int32]
        l.orc_moe_forward_f32.argtypes = [POINTER(OrcBlockF32), c_void_p, c_int32, c_void_p,
                                          c_void_p]
        for name in ("orc_moe_forward_f32", "orc_linear_forward", "orc_qmatmul", "orc_gather_qmm", "orc_topk",
                     "orc_permute", "orc_moe_forward", "orc_topk_valid", "orc_moe_stack",
                     "orc_set_threads"):
            getattr(l, name).restype = c_int32
        _LIB = l
    return _LIB


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(c_void_p)


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


def set_threads(n: int) -> int:
    return int(lib().orc_set_threads(n))


def bf16_from_f32(a: np.ndarray) -> np.ndarray:
    a = _c(a, np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().orc_round_bf16_array(_p(a), a.size, _p(out))
    return out


class _Keep:
    """Holds the arrays a ctypes struct points into."""

    def __init__(self):
        self.refs = []

    def __call__(self, a, dtype):
        a = _c(a, dtype)
        if a is not None:
            self.refs.append(a)
        return a


def qweight(q, keep: _Keep) -> OrcQ:
    """Any object with codes/scales/biases arrays and experts/out/in_/group/bits."""
    c = keep(q.codes, np.uint32)
    s = keep(q.scales, np.uint16) if q.scales is not None else None
    b = keep(q.biases, np.uint16) if q.biases is not None else None
    return OrcQ(_p(c), _p(s), _p(b), q.experts, q.out, q.in_, q.group, q.bits)


def linear_of(w, bias, out: int, in_: int, keep: _Keep) -> OrcLinear:
    """A Linear over a dense bf16 array or a quantized weight (anything with `codes`)."""
    if hasattr(w, "codes"):
        return OrcLinear(None, qweight(w, keep), _p(bias), out, in_)
    return OrcLinear(_p(keep(w, np.uint16)), OrcQ(), _p(bias), out, in_)


def block(hb, keep: _Keep) -> OrcBlock:
    """An OrcBlock over the arrays of a synthetic HostBlock (duck-typed)."""
    s = hb.shape
    b = OrcBlock()
    b.cfg = OrcConfig(s.hidden, s.experts, s.top_k, s.intermediate, int(s.norm_topk), s.shared)
    rb = keep(hb.router_bias, np.uint16) if hb.router_bias is not None else None
    b.gate = linear_of(hb.router, rb, s.experts, s.hidden, keep)
    b.sw_gate = qweight(hb.gate_proj, keep)
    b.sw_up = qweight(hb.up_proj, keep)
    b.sw_down = qweight(hb.down_proj, keep)
    if s.shared:
        b.sh_gate = OrcLinear(None, qweight(hb.sh_gate_proj, keep), None, s.shared, s.hidden)
        b.sh_up = OrcLinear(None, qweight(hb.sh_up_proj, keep), None, s.shared, s.hidden)
        b.sh_down = OrcLinear(None, qweight(hb.sh_down_proj, keep), None, s.hidden, s.shared)
        b.sh_expert_gate = linear_of(hb.sh_expert_gate, None, 1, s.hidden, keep)
    return b


def moe_forward(hb, x: np.ndarray, forced_ids: np.ndarray | None = None, trace: bool = False):
    """SparseMoe::forward on the CPU. Returns out [T, D] (uint16 bf16) or (out, trace dict)."""
    keep = _Keep()
    b = block(hb, keep)
    x = keep(x, np.uint16)
    s = hb.shape
    T, D, E, k, I = x.shape[0], s.hidden, s.experts, s.top_k, s.intermediate
    out = np.empty((T, D), dtype=np.uint16)
    fi = keep(forced_ids, np.uint32) if forced_ids is not None else None
    tr = None
    t = {}
    if trace:
        t = {
            "logits": np.empty((T, E), np.uint16), "gates": np.empty((T, E), np.uint16),
            "ids": np.empty((T, k), np.uint32), "scores": np.empty((T, k), np.uint16),
            "order": np.empty(T * k, np.uint32), "inverse": np.empty(T * k, np.uint32),
            "act": np.empty((T * k, I), np.uint16), "y": np.empty((T * k, D), np.uint16),
            "routed": np.empty((T, D), np.uint16), "shared_gate": np.empty(T, np.uint16),
            "shared_y": np.empty((T, D), np.uint16),
        }
        tr = OrcTrace(*[_p(t[n]) for n, _ in OrcTrace._fields_])
    rc = lib().orc_moe_forward(ctypes.byref(b), _p(x), T, _p(out), _p(fi),
                               ctypes.byref(tr) if tr is not None else None)
    if rc == -2:
        raise ValueError("forced ids are not a valid top-k within ties")
    if rc != 0:
        raise RuntimeError(f"orc_moe_forward failed ({rc})")
    return (out, t) if trace else out


def moe_forward_f32(fb, x: np.ndarray):
    """SparseMoe::forward of an f32 block (duck-typed synth.F32Block) on the CPU: (out [T, D]
    float32, ids [T, k])."""
    keep = _Keep()
    s = fb.shape
    b = OrcBlockF32()
    b.cfg = OrcConfig(s.hidden, s.experts, s.top_k, s.intermediate, int(s.norm_topk), s.shared)
    names = ["router", "sw_gate", "sw_up", "sw_down"] + (
        ["sh_gate", "sh_up", "sh_down", "sh_expert_gate"] if s.shared else [])
    src = {"router": fb.router, "sw_gate": fb.gate_proj, "sw_up": fb.up_proj,
           "sw_down": fb.down_proj, "sh_gate": fb.sh_gate_proj, "sh_up": fb.sh_up_proj,
           "sh_down": fb.sh_down_proj, "sh_expert_gate": fb.sh_expert_gate}
    for n in names:
        setattr(b, n, _p(keep(src[n], np.float32)))
    x = keep(x, np.float32)
    T = x.shape[0]
    out = np.empty((T, s.hidden), np.float32)
    ids = np.empty((T, s.top_k), np.uint32)
    if lib().orc_moe_forward_f32(ctypes.byref(b), _p(x), T, _p(out), _p(ids)) != 0:
        raise RuntimeError("orc_moe_forward_f32 failed")
    return out, ids


def moe_stack(blocks, x: np.ndarray, norm_w: np.ndarray | None = None, eps: float = 1e-6):
    keep = _Keep()
    arr = (OrcBlock * len(blocks))(*[block(hb, keep) for hb in blocks])
    x = np.array(x, dtype=np.uint16, copy=True)
    nw = keep(norm_w, np.uint16) if norm_w is not None else None
    if lib().orc_moe_stack(arr, len(blocks), _p(nw), eps, _p(x), x.shape[0]) != 0:
        raise RuntimeError("orc_moe_stack failed")
    return x


def dequant_row(q, e: int, o: int) -> np.ndarray:
    keep = _Keep()
    w = qweight(q, keep)
    row = np.empty(q.in_, dtype=np.float32)
    lib().orc_dequant_row(ctypes.byref(w), e, o, _p(row))
    return row


def gather_qmm(q, x: np.ndarray, idx: np.ndarray) -> np.ndarray:
    keep = _Keep()
    w = qweight(q, keep)
    x = keep(x, np.uint16)
    idx = keep(idx, np.uint32)
    y = np.empty((idx.size, q.out), dtype=np.uint16)
    if lib().orc_gather_qmm(ctypes.byref(w), _p(x), x.shape[0], _p(idx), idx.size, _p(y)) != 0:
        raise ValueError("orc_gather_qmm: invalid arguments")
    return y


def qmatmul(q, x: np.ndarray) -> np.ndarray:
    keep = _Keep()
    w = qweight(q, keep)
    x = keep(x, np.uint16)
    y = np.empty((x.shape[0], q.out), dtype=np.uint16)
    if lib().orc_qmatmul(ctypes.byref(w), _p(x), x.shape[0], _p(y)) != 0:
        raise ValueError("orc_qmatmul: invalid arguments")
    return y


def linear(w, x: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
    """Linear::forward over a dense bf16 [out, in] array or a quantized weight (expert 0)."""
    keep = _Keep()
    b = keep(bias, np.uint16) if bias is not None else None
    x = keep(x, np.uint16)
    out, in_ = (w.out, w.in_) if hasattr(w, "codes") else w.shape
    l = linear_of(w, b, out, in_, keep)
    y = np.empty((x.shape[0], out), dtype=np.uint16)
    if lib().orc_linear_forward(ctypes.byref(l), _p(x), x.shape[0], _p(y)) != 0:
        raise ValueError("orc_linear_forward: invalid arguments")
    return y


def softmax(logits: np.ndarray) -> np.ndarray:
    l = _c(logits, np.uint16)
    out = np.empty_like(l)
    lib().orc_softmax(_p(l), l.shape[0], l.shape[1], _p(out))
    return out


def topk(gates: np.ndarray, k: int) -> np.ndarray:
    g = _c(gates, np.uint16)
    ids = np.empty((g.shape[0], k), dtype=np.uint32)
    if lib().orc_topk(_p(g), g.shape[0], g.shape[1], k, _p(ids)) != 0:
        raise ValueError("orc_topk: invalid arguments")
    return ids


def scores(gates: np.ndarray, ids: np.ndarray, norm: bool) -> np.ndarray:
    g = _c(gates, np.uint16)
    i = _c(ids, np.uint32)
    s = np.empty(i.shape, dtype=np.uint16)
    lib().orc_scores(_p(g), g.shape[0], g.shape[1], _p(i), i.shape[1], int(norm), _p(s))
    return s


def topk_valid(gates: np.ndarray, logits: np.ndarray | None, ids: np.ndarray, ulps: int = 1) -> bool:
    g = _c(gates, np.uint16)
    l = _c(logits, np.uint16) if logits is not None else None
    i = _c(ids, np.uint32)
    return bool(lib().orc_topk_valid(_p(g), _p(l), g.size, i.size, _p(i), ulps))


def permute(ids: np.ndarray, k: int, experts: int):
    i = _c(ids, np.uint32).ravel()
    P = i.size
    order = np.empty(P, np.uint32)
    inverse = np.empty(P, np.uint32)
    token = np.empty(P, np.uint32)
    counts = np.empty(experts, np.uint32)
    if lib().orc_permute(_p(i), P, k, experts, _p(order), _p(inverse), _p(token), _p(counts)) != 0:
        raise ValueError("orc_permute: invalid arguments")
    return order, inverse, token, counts


def floor_divide_u32(a: np.ndarray, b: int) -> np.ndarray:
    a = _c(a, np.uint32)
    out = np.empty_like(a)
    lib().orc_floor_divide_u32(_p(a), a.size, b, _p(out))
    return out


def swiglu(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = _c(g, np.uint16)
    u = _c(u, np.uint16)
    out = np.empty_like(g)
    lib().orc_swiglu(_p(g), _p(u), g.size, _p(out))
    return out


def swiglu_f32(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = _c(g, np.float32)
    u = _c(u, np.float32)
    out = np.empty_like(g)
    lib().orc_swiglu_f32(_p(g), _p(u), g.size, _p(out))
    return out


def combine(y: np.ndarray, scores_: np.ndarray) -> np.ndarray:
    T, k = scores_.shape
    D = y.shape[-1]
    y = _c(y, np.uint16)
    s = _c(scores_, np.uint16)
    out = np.empty((T, D), np.uint16)
    lib().orc_combine(_p(y), _p(s), T, k, D, _p(out))
    return out


def shared_add(routed: np.ndarray, glogit: np.ndarray, shared: np.ndarray):
    r = _c(routed, np.uint16)
    g = _c(glogit, np.uint16).ravel()
    s = _c(shared, np.uint16)
    out = np.empty_like(r)
    gate = np.empty(r.shape[0], np.uint16)
    lib().orc_shared_add(_p(r), _p(g), _p(s), r.shape[0], r.shape[1], _p(out), _p(gate))
    return out, gate


def rms_norm(x: np.ndarray, w: np.ndarray | None, eps: float) -> np.ndarray:
    x = _c(x, np.uint16)
    w = _c(w, np.uint16) if w is not None else None
    out = np.empty_like(x)
    lib().orc_rms_norm(_p(x), _p(w), x.shape[0], x.shape[1], eps, _p(out))
    return out
