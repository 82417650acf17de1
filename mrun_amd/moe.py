"""Python view of the MoE block over the C ABI (include/mrun_moe.h), on torch device memory.

Mirrors the reference's interface for this path (crates/mrun-engine/src/models/moe.rs and the
facade ops of crates/mrun-engine/src/tensor/nuvec.rs): `SparseMoe.forward`, `gather_qmm`,
`quantized_matmul`, `linear`, `router`, `permute`, `swiglu`, `combine`, `rms_norm`,
`add_rms_norm`. Failures raise MrunError with the library's message (the facade's
Result<_, Error(String)>). torch supplies device memory and the stream; every computation runs in
libmrun_moe.so.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from ._lib import Linear, MoeConfig, Quantized, SparseMoe as _SparseMoe, check
from .synth import HostBlock, QTensor, Shape


def _stream(stream=None) -> ctypes.c_void_p:
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def bf16_tensor(a: np.ndarray, device="cuda") -> torch.Tensor:
    """uint16 bf16 bits -> torch.bfloat16 on the device (bit-exact)."""
    a = np.ascontiguousarray(a)
    if not a.flags.writeable:  # e.g. a view of a read-only file buffer
        a = a.copy()
    return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(device)


def u32_tensor(a: np.ndarray, device="cuda") -> torch.Tensor:
    a = np.ascontiguousarray(a, dtype=np.uint32)
    if not a.flags.writeable:
        a = a.copy()
    return torch.from_numpy(a.view(np.int32)).to(device)


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    """torch.bfloat16 (any device) -> uint16 bits on the host."""
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def u32_array(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().numpy().view(np.uint32)


class DeviceQTensor:
    """A QTensor resident on the device, with its C view (tensor::Quantized, nuvec.rs:602-638)."""

    def __init__(self, q: QTensor | None, device="cuda"):
        if q is None:  # filled by from_tensors
            return
        self.codes = u32_tensor(q.codes, device)
        self.scales = bf16_tensor(q.scales, device) if q.scales is not None else None  # bits 16
        self.biases = bf16_tensor(q.biases, device) if q.biases is not None else None
        self.experts, self.out, self.in_, self.group, self.bits = q.experts, q.out, q.in_, q.group, q.bits

    @classmethod
    def from_tensors(cls, codes, scales, biases, experts, out, in_, group, bits=4):
        t = cls(None)
        t.codes, t.scales, t.biases = codes, scales, biases
        t.experts, t.out, t.in_, t.group, t.bits = experts, out, in_, group, bits
        return t

    @property
    def c(self) -> Quantized:
        return Quantized(_ptr(self.codes).value, _ptr(self.scales).value,
                         _ptr(self.biases).value, self.experts, self.out, self.in_, self.group,
                         self.bits)


def _dense_linear(w: torch.Tensor, bias: torch.Tensor | None = None) -> Linear:
    out, in_ = w.shape
    return Linear(_ptr(w).value, Quantized(), _ptr(bias).value, out, in_)


def _q_linear(q: DeviceQTensor, bias: torch.Tensor | None = None) -> Linear:
    return Linear(None, q.c, _ptr(bias).value, q.out, q.in_)


def _linear(w, bias: torch.Tensor | None = None) -> Linear:
    """load::Linear (load.rs:246-306): a dense bf16 tensor or a quantized DeviceQTensor."""
    return _q_linear(w, bias) if isinstance(w, DeviceQTensor) else _dense_linear(w, bias)


class SparseMoe:
    """SparseMoe (moe.rs:109-188) with its weights on the device."""

    def __init__(self, hb: HostBlock, device="cuda"):
        """From host arrays (HostBlock), or from a block whose tensors are on the device already
        (torch tensors and DeviceQTensors, as device_block makes)."""
        s = hb.shape
        self.shape = s
        self.device = torch.device(device)
        dev = lambda a: a if isinstance(a, torch.Tensor) else bf16_tensor(a, device)
        qdev = lambda q: q if isinstance(q, DeviceQTensor) else DeviceQTensor(q, device)
        # the router and the shared-expert gate are dense bf16 or quantized (QTensor)
        lin = lambda a: qdev(a) if isinstance(a, (QTensor, DeviceQTensor)) else dev(a)
        self.router = lin(hb.router)
        self.router_bias = dev(hb.router_bias) if hb.router_bias is not None else None
        self.gate_proj = qdev(hb.gate_proj)
        self.up_proj = qdev(hb.up_proj)
        self.down_proj = qdev(hb.down_proj)
        self.shared = s.shared > 0
        if self.shared:
            self.sh_gate_proj = qdev(hb.sh_gate_proj)
            self.sh_up_proj = qdev(hb.sh_up_proj)
            self.sh_down_proj = qdev(hb.sh_down_proj)
            self.sh_expert_gate = lin(hb.sh_expert_gate)
        self.cfg = MoeConfig(s.hidden, s.experts, s.top_k, s.intermediate, int(s.norm_topk),
                             s.shared)
        m = _SparseMoe()
        m.cfg = self.cfg
        m.gate = _linear(self.router, self.router_bias)
        m.switch_gate_proj = self.gate_proj.c
        m.switch_up_proj = self.up_proj.c
        m.switch_down_proj = self.down_proj.c
        if self.shared:
            m.shared_gate_proj = _q_linear(self.sh_gate_proj)
            m.shared_up_proj = _q_linear(self.sh_up_proj)
            m.shared_down_proj = _q_linear(self.sh_down_proj)
            m.shared_expert_gate = _linear(self.sh_expert_gate)
        self.c = m
        check(_lib.load().mrun_moe_check(ctypes.byref(self.c)))
        self._ws = None

    @classmethod
    def from_view(cls, view: "_SparseMoe", owner=None, device="cuda") -> "SparseMoe":
        """A block over device memory someone else owns (a loaded checkpoint: mrun_amd.load),
        kept alive through `owner`."""
        self = cls.__new__(cls)
        c = view.cfg
        self.shape = Shape(hidden=c.hidden, experts=c.experts, top_k=c.top_k,
                           intermediate=c.intermediate, shared=c.shared_intermediate,
                           norm_topk=bool(c.norm_topk_prob))
        self.device = torch.device(device)
        self.cfg = MoeConfig(c.hidden, c.experts, c.top_k, c.intermediate, c.norm_topk_prob,
                             c.shared_intermediate)
        self.c = view
        self.shared = c.shared_intermediate > 0
        self._owner = owner
        self._ws = None
        check(_lib.load().mrun_moe_check(ctypes.byref(self.c)))
        return self

    def tensors(self) -> list:
        """Every device tensor of the block's weights."""
        qs = [self.gate_proj, self.up_proj, self.down_proj]
        ts = [self.router_bias] if self.router_bias is not None else []
        lins = [self.router] + ([self.sh_expert_gate] if self.shared else [])
        if self.shared:
            qs += [self.sh_gate_proj, self.sh_up_proj, self.sh_down_proj]
        for l in lins:
            (qs if isinstance(l, DeviceQTensor) else ts).append(l)
        for q in qs:
            ts += [q.codes, q.scales] + ([q.biases] if q.biases is not None else [])
        return ts

    def workspace_bytes(self, tokens: int) -> int:
        return int(_lib.load().mrun_moe_workspace_bytes(ctypes.byref(self.cfg), tokens))

    def workspace(self, tokens: int) -> torch.Tensor:
        need = self.workspace_bytes(tokens)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.device)
        return self._ws

    def forward(self, x: torch.Tensor, out: torch.Tensor | None = None,
                workspace: torch.Tensor | None = None, stream=None) -> torch.Tensor:
        """x [T, hidden] bf16 -> [T, hidden] bf16 (SparseMoe::forward, moe.rs:149-174)."""
        T = x.shape[0]
        if out is None:
            out = torch.empty_like(x)
        ws = workspace if workspace is not None else self.workspace(T)
        check(_lib.load().mrun_moe_forward(ctypes.byref(self.c), _ptr(x), T, _ptr(out), _ptr(ws),
                                           ws.numel(), _stream(stream)))
        return out

    def routing_of_last_forward(self, tokens: int, workspace: torch.Tensor | None = None):
        """(ids, scores, offsets, order, inverse, token) that the last forward of `tokens` rows
        left in its workspace (mrun_moe_workspace_routing). The sorted dispatch (offsets, order,
        inverse, token) is written by the prefill schedule only."""
        ws = workspace if workspace is not None else self._ws
        at = (ctypes.c_size_t * 6)()
        check(_lib.load().mrun_moe_workspace_routing(ctypes.byref(self.cfg), tokens, at))
        k, E = self.shape.top_k, self.shape.experts
        P = tokens * k

        def view(off, n, dtype):
            nbytes = n * torch.tensor([], dtype=dtype).element_size()
            return ws[off:off + nbytes].view(dtype)

        return (view(at[0], P, torch.int32), view(at[1], P, torch.bfloat16),
                view(at[2], E + 1, torch.int32), view(at[3], P, torch.int32),
                view(at[4], P, torch.int32), view(at[5], P, torch.int32))

    def router_forward(self, x: torch.Tensor, stream=None):
        """(logits, gates, ids, scores) of the router (moe.rs:151-159)."""
        T, E, k = x.shape[0], self.shape.experts, self.shape.top_k
        logits = torch.empty(T, E, dtype=torch.bfloat16, device=x.device)
        gates = torch.empty(T, E, dtype=torch.bfloat16, device=x.device)
        ids = torch.empty(T, k, dtype=torch.int32, device=x.device)
        scores = torch.empty(T, k, dtype=torch.bfloat16, device=x.device)
        check(_lib.load().mrun_moe_router(ctypes.byref(self.c), _ptr(x), T, _ptr(logits),
                                          _ptr(gates), _ptr(ids), _ptr(scores), None, 0,
                                          _stream(stream)))
        return logits, gates, ids, scores


# ---- device-generated blocks and the layer stack ----

_SYNTH_DEV = None


class SparseMoeF32:
    """SparseMoe (moe.rs:109-188) of a float32 checkpoint: every tensor f32 on the device, run by
    mrun_moe_forward_f32 (each weight a dense bits-32 stacked weight)."""

    def __init__(self, fb, device="cuda"):
        """From host f32 arrays (synth.F32Block)."""
        s = fb.shape
        self.shape = s
        self.device = torch.device(device)
        f32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device)
        self._t = {}

        def q(name, a, experts):
            t = self._t[name] = f32(a)
            return Quantized(_ptr(t).value, None, None, experts, a.shape[-2], a.shape[-1], 0, 32)

        lin = lambda name, a: Linear(None, q(name, a, 1), None, a.shape[-2], a.shape[-1])
        self.cfg = MoeConfig(s.hidden, s.experts, s.top_k, s.intermediate, int(s.norm_topk),
                             s.shared)
        m = _SparseMoe()
        m.cfg = self.cfg
        m.gate = lin("router", fb.router)
        m.switch_gate_proj = q("gate_proj", fb.gate_proj, s.experts)
        m.switch_up_proj = q("up_proj", fb.up_proj, s.experts)
        m.switch_down_proj = q("down_proj", fb.down_proj, s.experts)
        if s.shared:
            m.shared_gate_proj = lin("sh_gate_proj", fb.sh_gate_proj)
            m.shared_up_proj = lin("sh_up_proj", fb.sh_up_proj)
            m.shared_down_proj = lin("sh_down_proj", fb.sh_down_proj)
            m.shared_expert_gate = lin("sh_expert_gate", fb.sh_expert_gate)
        self.c = m
        check(_lib.load().mrun_moe_check(ctypes.byref(self.c)))
        self._ws = None

    @classmethod
    def from_view(cls, view: "_SparseMoe", owner=None, device="cuda") -> "SparseMoeF32":
        """An f32 block over device memory someone else owns (a loaded f32 checkpoint)."""
        self = cls.__new__(cls)
        c = view.cfg
        self.shape = Shape(hidden=c.hidden, experts=c.experts, top_k=c.top_k,
                           intermediate=c.intermediate, shared=c.shared_intermediate,
                           norm_topk=bool(c.norm_topk_prob))
        self.device = torch.device(device)
        self.cfg = MoeConfig(c.hidden, c.experts, c.top_k, c.intermediate, c.norm_topk_prob,
                             c.shared_intermediate)
        self.c = view
        self._owner = owner
        self._ws = None
        check(_lib.load().mrun_moe_check(ctypes.byref(self.c)))
        return self

    def workspace_bytes(self, tokens: int) -> int:
        return int(_lib.load().mrun_moe_workspace_bytes_f32(ctypes.byref(self.cfg), tokens))

    def forward(self, x: torch.Tensor, out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
        """x [T, hidden] f32 -> [T, hidden] f32."""
        T = x.shape[0]
        if out is None:
            out = torch.empty_like(x)
        need = max(self.workspace_bytes(T), 1)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.device)
        check(_lib.load().mrun_moe_forward_f32(ctypes.byref(self.c), _ptr(x), T, _ptr(out),
                                               _ptr(self._ws), self._ws.numel(), _stream(stream)))
        return out


def _synth_dev() -> ctypes.CDLL:
    global _SYNTH_DEV
    if _SYNTH_DEV is None:
        p = _lib.LIB_PATH.parent / "libmrun_synth_dev.so"
        if not p.exists():
            raise RuntimeError(f"{p} is missing: build it with `python -m mrun_amd.build`")
        l = ctypes.CDLL(str(p))
        l.mrun_synth_codes_dev.argtypes = [ctypes.c_uint64, ctypes.c_int32, ctypes.c_void_p,
                                           ctypes.c_size_t, ctypes.c_void_p]
        l.mrun_synth_normal_bf16_dev.argtypes = [ctypes.c_uint64, ctypes.c_float, ctypes.c_void_p,
                                                 ctypes.c_size_t, ctypes.c_void_p]
        l.mrun_synth_scales_biases_dev.argtypes = [ctypes.c_uint64, ctypes.c_void_p,
                                                   ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        for f in (l.mrun_synth_codes_dev, l.mrun_synth_normal_bf16_dev,
                  l.mrun_synth_scales_biases_dev):
            f.restype = ctypes.c_int32
        _SYNTH_DEV = l
    return _SYNTH_DEV


def device_normal_bf16(seed: int, n: int, std: float, device="cuda") -> torch.Tensor:
    out = torch.empty(n, dtype=torch.bfloat16, device=device)
    if _synth_dev().mrun_synth_normal_bf16_dev(seed, std, _ptr(out), n, _stream(None)) != 0:
        raise RuntimeError("mrun_synth_normal_bf16_dev failed")
    return out


def device_qtensor(config: int, layer: int, codes_id: int, scales_id: int, experts: int, out: int,
                   in_: int, group: int = 64, device="cuda") -> DeviceQTensor:
    """synth.qtensor generated on the device (bit-identical codes; same scale formula)."""
    from . import synth
    lib = _synth_dev()
    n_words, n_groups = experts * out * in_ // 8, experts * out * in_ // group
    codes = torch.empty(n_words, dtype=torch.int32, device=device)
    scales = torch.empty(n_groups, dtype=torch.bfloat16, device=device)
    biases = torch.empty(n_groups, dtype=torch.bfloat16, device=device)
    if lib.mrun_synth_codes_dev(synth.seed(config, layer, codes_id), 4, _ptr(codes), n_words,
                                _stream(None)) != 0:
        raise RuntimeError("mrun_synth_codes_dev failed")
    if lib.mrun_synth_scales_biases_dev(synth.seed(config, layer, scales_id), _ptr(scales),
                                        _ptr(biases), n_groups, _stream(None)) != 0:
        raise RuntimeError("mrun_synth_scales_biases_dev failed")
    return DeviceQTensor.from_tensors(codes, scales, biases, experts, out, in_, group)


def device_block(shape, config: int, layer: int, device="cuda") -> "SparseMoe":
    """synth.make_block(shape, config, layer) (no Zipf bias) made on the device: for weight stacks
    too large to generate on the host."""
    from types import SimpleNamespace
    from . import synth as S
    D, E, I, Sh, g = shape.hidden, shape.experts, shape.intermediate, shape.shared, shape.group
    hb = SimpleNamespace(
        shape=shape,
        router=device_normal_bf16(S.seed(config, layer, S.ROUTER_W), E * D, 0.02, device).view(E, D),
        router_bias=None,
        gate_proj=device_qtensor(config, layer, S.GATE_CODES, S.GATE_SCALES, E, I, D, g, device),
        up_proj=device_qtensor(config, layer, S.UP_CODES, S.UP_SCALES, E, I, D, g, device),
        down_proj=device_qtensor(config, layer, S.DOWN_CODES, S.DOWN_SCALES, E, D, I, g, device),
    )
    if Sh:
        hb.sh_gate_proj = device_qtensor(config, layer, S.SH_GATE_CODES, S.SH_GATE_SCALES, 1, Sh, D, g, device)
        hb.sh_up_proj = device_qtensor(config, layer, S.SH_UP_CODES, S.SH_UP_SCALES, 1, Sh, D, g, device)
        hb.sh_down_proj = device_qtensor(config, layer, S.SH_DOWN_CODES, S.SH_DOWN_SCALES, 1, D, Sh, g, device)
        hb.sh_expert_gate = device_normal_bf16(S.seed(config, layer, S.SH_EXPERT_GATE), D, 0.02,
                                               device).view(1, D)
    return SparseMoe(hb, device)


class MoeStack:
    """A stack of MoE layers with the RMSNorm + residual around each (qwen3_5_moe.rs:622-624)."""

    def __init__(self, layers: list, norm_w: list | None = None, eps: float = 1e-6):
        """norm_w: per layer a bf16 [hidden] device tensor, a raw device address (int), or None
        (weight 1)."""
        self.layers = layers
        self.eps = eps
        self.norm_w = norm_w
        n = len(layers)
        self._arr = (_SparseMoe * n)(*[l.c for l in layers])
        self._nw = None
        if norm_w is not None:
            ptr = lambda w: w if isinstance(w, int) else (_ptr(w).value if w is not None else None)
            self._nw = (ctypes.c_void_p * n)(*[ptr(w) for w in norm_w])
        self._ws = None

    def workspace(self, tokens: int) -> torch.Tensor:
        need = int(_lib.load().mrun_moe_stack_workspace_bytes(ctypes.byref(self.layers[0].cfg), tokens))
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.layers[0].device)
        return self._ws

    def forward_(self, x: torch.Tensor, workspace: torch.Tensor | None = None, stream=None) -> torch.Tensor:
        """x [T, hidden] bf16, updated in place."""
        ws = workspace if workspace is not None else self.workspace(x.shape[0])
        check(_lib.load().mrun_moe_stack_forward(self._arr, len(self.layers), self._nw, self.eps,
                                                 _ptr(x), x.shape[0], _ptr(ws), ws.numel(),
                                                 _stream(stream)))
        return x


# ---- facade ops ----

def permute(ids: torch.Tensor, top_k: int, experts: int, stream=None):
    """(offsets [E+1], order, inverse, token) of the sorted dispatch (moe.rs:65-75)."""
    P = ids.numel()
    dev = ids.device
    offsets = torch.empty(experts + 1, dtype=torch.int32, device=dev)
    order = torch.empty(P, dtype=torch.int32, device=dev)
    inverse = torch.empty(P, dtype=torch.int32, device=dev)
    token = torch.empty(P, dtype=torch.int32, device=dev)
    l = _lib.load()
    need = int(l.mrun_moe_permute_workspace_bytes(P, experts))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
    check(l.mrun_moe_permute(_ptr(ids), P, top_k, experts, _ptr(offsets), _ptr(order),
                             _ptr(inverse), _ptr(token), _ptr(ws), ws.numel(), _stream(stream)))
    return offsets, order, inverse, token


def gather_qmm(x: torch.Tensor, w: DeviceQTensor, indices: torch.Tensor,
               sorted_indices: bool = False, stream=None) -> torch.Tensor:
    """tensor::gather_qmm (nuvec.rs:670-686): x [R, in] broadcast over n/R indices each."""
    n = indices.numel()
    out = torch.empty(n, w.out, dtype=torch.bfloat16, device=x.device)
    l = _lib.load()
    need = int(l.mrun_gather_qmm_workspace_bytes(n, w.experts, x.shape[0], w.in_, w.out))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
    qc = w.c
    check(l.mrun_gather_qmm(_ptr(x), x.shape[0], ctypes.byref(qc), _ptr(indices), n,
                            int(sorted_indices), _ptr(out), _ptr(ws), ws.numel(), _stream(stream)))
    return out


def quantized_matmul(x: torch.Tensor, w: DeviceQTensor, stream=None) -> torch.Tensor:
    out = torch.empty(x.shape[0], w.out, dtype=torch.bfloat16, device=x.device)
    qc = w.c
    check(_lib.load().mrun_quantized_matmul(_ptr(x), x.shape[0], ctypes.byref(qc), _ptr(out),
                                            _stream(stream)))
    return out


def linear(x: torch.Tensor, weight, bias: torch.Tensor | None = None,
           stream=None) -> torch.Tensor:
    """Linear::forward (load.rs:294-306) with a dense bf16 weight [out, in] or a quantized
    DeviceQTensor (one expert)."""
    lin = _linear(weight, bias)
    out = torch.empty(x.shape[0], lin.out, dtype=torch.bfloat16, device=x.device)
    check(_lib.load().mrun_linear_forward(ctypes.byref(lin), _ptr(x), x.shape[0], _ptr(out),
                                          _stream(stream)))
    return out


def swiglu(gate: torch.Tensor, up: torch.Tensor, stream=None) -> torch.Tensor:
    out = torch.empty_like(gate)
    check(_lib.load().mrun_swiglu(_ptr(gate), _ptr(up), gate.numel(), _ptr(out), _stream(stream)))
    return out


def combine(y: torch.Tensor, scores: torch.Tensor, inverse: torch.Tensor | None = None,
            shared_y: torch.Tensor | None = None, shared_logit: torch.Tensor | None = None,
            stream=None) -> torch.Tensor:
    T, k = scores.shape
    D = y.shape[-1]
    out = torch.empty(T, D, dtype=torch.bfloat16, device=y.device)
    check(_lib.load().mrun_moe_combine(_ptr(y), _ptr(inverse), _ptr(scores), T, k, D,
                                       _ptr(shared_y), _ptr(shared_logit), _ptr(out),
                                       _stream(stream)))
    return out


def rms_norm(x: torch.Tensor, w: torch.Tensor | None, eps: float, stream=None) -> torch.Tensor:
    out = torch.empty_like(x)
    check(_lib.load().mrun_rms_norm(_ptr(x), _ptr(w), x.shape[0], x.shape[1], eps, _ptr(out),
                                    _stream(stream)))
    return out


def add_rms_norm(x: torch.Tensor, residual: torch.Tensor, w: torch.Tensor | None, eps: float,
                 h: torch.Tensor | None = None, stream=None):
    h = torch.empty_like(x) if h is None else h
    y = torch.empty_like(x)
    check(_lib.load().mrun_add_rms_norm(_ptr(x), _ptr(residual), _ptr(w), x.shape[0], x.shape[1],
                                        eps, _ptr(h), _ptr(y), _stream(stream)))
    return h, y


__all__ = [
    "SparseMoe", "DeviceQTensor", "MoeStack", "device_block", "Shape", "permute", "gather_qmm", "quantized_matmul", "linear",
    "swiglu", "combine", "rms_norm", "add_rms_norm", "bf16_tensor", "u32_tensor", "bf16_bits",
    "u32_array",
]
