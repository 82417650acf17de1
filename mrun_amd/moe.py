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
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(device)


def u32_tensor(a: np.ndarray, device="cuda") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to(device)


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    """torch.bfloat16 (any device) -> uint16 bits on the host."""
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def u32_array(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().numpy().view(np.uint32)


class DeviceQTensor:
    """A QTensor resident on the device, with its C view (tensor::Quantized, nuvec.rs:602-638)."""

    def __init__(self, q: QTensor, device="cuda"):
        self.codes = u32_tensor(q.codes, device)
        self.scales = bf16_tensor(q.scales, device)
        self.biases = bf16_tensor(q.biases, device) if q.biases is not None else None
        self.experts, self.out, self.in_, self.group, self.bits = q.experts, q.out, q.in_, q.group, q.bits

    @property
    def c(self) -> Quantized:
        return Quantized(_ptr(self.codes).value, _ptr(self.scales).value,
                         _ptr(self.biases).value, self.experts, self.out, self.in_, self.group,
                         self.bits)


def _dense_linear(w: torch.Tensor, bias: torch.Tensor | None = None) -> Linear:
    out, in_ = w.shape
    return Linear(_ptr(w).value, Quantized(), _ptr(bias).value, out, in_)


def _q_linear(q: DeviceQTensor) -> Linear:
    return Linear(None, q.c, None, q.out, q.in_)


class SparseMoe:
    """SparseMoe (moe.rs:109-188) with its weights on the device."""

    def __init__(self, hb: HostBlock, device="cuda"):
        s = hb.shape
        self.shape = s
        self.router = bf16_tensor(hb.router, device)
        self.router_bias = bf16_tensor(hb.router_bias, device) if hb.router_bias is not None else None
        self.gate_proj = DeviceQTensor(hb.gate_proj, device)
        self.up_proj = DeviceQTensor(hb.up_proj, device)
        self.down_proj = DeviceQTensor(hb.down_proj, device)
        self.shared = s.shared > 0
        if self.shared:
            self.sh_gate_proj = DeviceQTensor(hb.sh_gate_proj, device)
            self.sh_up_proj = DeviceQTensor(hb.sh_up_proj, device)
            self.sh_down_proj = DeviceQTensor(hb.sh_down_proj, device)
            self.sh_expert_gate = bf16_tensor(hb.sh_expert_gate, device)
        self.cfg = MoeConfig(s.hidden, s.experts, s.top_k, s.intermediate, int(s.norm_topk),
                             s.shared)
        m = _SparseMoe()
        m.cfg = self.cfg
        m.gate = _dense_linear(self.router, self.router_bias)
        m.switch_gate_proj = self.gate_proj.c
        m.switch_up_proj = self.up_proj.c
        m.switch_down_proj = self.down_proj.c
        if self.shared:
            m.shared_gate_proj = _q_linear(self.sh_gate_proj)
            m.shared_up_proj = _q_linear(self.sh_up_proj)
            m.shared_down_proj = _q_linear(self.sh_down_proj)
            m.shared_expert_gate = _dense_linear(self.sh_expert_gate)
        self.c = m
        check(_lib.load().mrun_moe_check(ctypes.byref(self.c)))
        self._ws = None

    def workspace_bytes(self, tokens: int) -> int:
        return int(_lib.load().mrun_moe_workspace_bytes(ctypes.byref(self.cfg), tokens))

    def workspace(self, tokens: int) -> torch.Tensor:
        need = self.workspace_bytes(tokens)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.router.device)
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


# ---- facade ops ----

def permute(ids: torch.Tensor, top_k: int, experts: int, stream=None):
    """(offsets [E+1], order, inverse, token) of the sorted dispatch (moe.rs:65-75)."""
    P = ids.numel()
    dev = ids.device
    offsets = torch.empty(experts + 1, dtype=torch.int32, device=dev)
    order = torch.empty(P, dtype=torch.int32, device=dev)
    inverse = torch.empty(P, dtype=torch.int32, device=dev)
    token = torch.empty(P, dtype=torch.int32, device=dev)
    check(_lib.load().mrun_moe_permute(_ptr(ids), P, top_k, experts, _ptr(offsets), _ptr(order),
                                       _ptr(inverse), _ptr(token), None, 0, _stream(stream)))
    return offsets, order, inverse, token


def gather_qmm(x: torch.Tensor, w: DeviceQTensor, indices: torch.Tensor,
               sorted_indices: bool = False, stream=None) -> torch.Tensor:
    """tensor::gather_qmm (nuvec.rs:670-686): x [R, in] broadcast over n/R indices each."""
    n = indices.numel()
    out = torch.empty(n, w.out, dtype=torch.bfloat16, device=x.device)
    l = _lib.load()
    need = int(l.mrun_gather_qmm_workspace_bytes(n, w.experts))
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


def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None,
           stream=None) -> torch.Tensor:
    """Linear::forward with a dense bf16 weight [out, in] (load.rs:294-306)."""
    lin = _dense_linear(weight, bias)
    out = torch.empty(x.shape[0], weight.shape[0], dtype=torch.bfloat16, device=x.device)
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
    "SparseMoe", "DeviceQTensor", "Shape", "permute", "gather_qmm", "quantized_matmul", "linear",
    "swiglu", "combine", "rms_norm", "add_rms_norm", "bf16_tensor", "u32_tensor", "bf16_bits",
    "u32_array",
]
