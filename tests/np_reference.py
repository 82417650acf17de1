"""An independent numpy restatement of SparseMoe::forward (moe.rs:149-174), used only to pin the C
oracle on small shapes. Sums are float64 and each reference op's output is rounded to float32 and
then to bf16, so it differs from the C oracle (float32 sums) only where the two accumulations land
on different sides of a bf16 rounding boundary. Written from the reference's op list, not from
oracle/moe_oracle.c.
"""
from __future__ import annotations

import numpy as np

from mrun_amd.synth import bf16_to_f32, f32_to_bf16


def R(a) -> np.ndarray:
    """float64 -> float32 -> bf16 value (as float64)."""
    return bf16_to_f32(f32_to_bf16(np.asarray(a, dtype=np.float64).astype(np.float32))).astype(
        np.float64)


def F(bits) -> np.ndarray:
    return bf16_to_f32(np.asarray(bits, dtype=np.uint16)).astype(np.float64)


def dequant(q) -> np.ndarray:
    """[E, out, in] float64: code * scale + bias, codes LSB-first in each u32 word; bits 16 holds
    dense bf16 weights (two per word, the first in the low half)."""
    if q.bits == 16:
        return F(np.ascontiguousarray(q.codes).view(np.uint16).reshape(q.experts, q.out, q.in_))
    per = 32 // q.bits
    shifts = (np.arange(per, dtype=np.uint32) * q.bits)
    codes = (q.codes[..., None] >> shifts) & np.uint32((1 << q.bits) - 1)
    codes = codes.reshape(q.experts, q.out, q.in_).astype(np.float64)
    s = np.repeat(F(q.scales), q.group, axis=-1)
    b = np.repeat(F(q.biases), q.group, axis=-1) if q.biases is not None else 0.0
    return codes * s + b


def weight(w) -> np.ndarray:
    """[out, in] float64 of a Linear's weight: dense bf16, or expert 0 of a quantized one."""
    return dequant(w)[0] if hasattr(w, "codes") else F(w)


def sigmoid(z):
    return 1.0 / (1.0 + np.exp(-z))


def topk_ids(gates_bits: np.ndarray, k: int) -> np.ndarray:
    """k largest bf16 gates per row, equal gates by lower id, in rank order (brute force)."""
    T, E = gates_bits.shape
    out = np.empty((T, k), dtype=np.uint32)
    ids = np.arange(E)
    for t in range(T):
        order = np.lexsort((ids, -F(gates_bits[t])))
        out[t] = order[:k]
    return out


def forward(hb, x_bits: np.ndarray, ids: np.ndarray | None = None):
    s = hb.shape
    x = F(x_bits)
    T, k = x.shape[0], s.top_k
    logits = R(x @ weight(hb.router).T)
    if hb.router_bias is not None:
        logits = R(logits + F(hb.router_bias))
    m = logits.max(axis=1, keepdims=True)
    e = np.exp(logits - m)
    gates = R(e / e.sum(axis=1, keepdims=True))
    gates_bits = f32_to_bf16(gates.astype(np.float32))
    if ids is None:
        ids = topk_ids(gates_bits, k)
    sc = np.take_along_axis(gates, ids.astype(np.int64), axis=1)
    if s.norm_topk:
        sc = R(sc / R(sc.sum(axis=1, keepdims=True)))
    Wg, Wu, Wd = dequant(hb.gate_proj), dequant(hb.up_proj), dequant(hb.down_proj)
    y = np.empty((T, k, s.hidden))
    for t in range(T):
        for j in range(k):
            ex = int(ids[t, j])
            g = R(Wg[ex] @ x[t])
            u = R(Wu[ex] @ x[t])
            act = R(g * sigmoid(g) * u)
            y[t, j] = R(Wd[ex] @ act)
    routed = R((R(y * sc[:, :, None])).sum(axis=1))
    if s.shared:
        gl = R(x @ weight(hb.sh_expert_gate).T)[:, 0]
        sg = R(sigmoid(gl))
        g = R(x @ dequant(hb.sh_gate_proj)[0].T)
        u = R(x @ dequant(hb.sh_up_proj)[0].T)
        act = R(g * sigmoid(g) * u)
        ys = R(act @ dequant(hb.sh_down_proj)[0].T)
        out = R(routed + R(sg[:, None] * ys))
    else:
        out = routed
    return f32_to_bf16(out.astype(np.float32)), {
        "logits": f32_to_bf16(logits.astype(np.float32)), "gates": gates_bits, "ids": ids,
        "scores": f32_to_bf16(sc.astype(np.float32)),
    }


def forward_f32(fb, x: np.ndarray):
    """SparseMoe::forward of an f32 block (synth.F32Block) in float64 with no rounding at all:
    (out [T, D], gates [T, E], ids [T, k]); ids by a brute-force lexsort (gate desc, id asc)."""
    s = fb.shape
    x = np.asarray(x, np.float64)
    T, k = x.shape[0], s.top_k
    logits = x @ np.asarray(fb.router, np.float64).T
    e = np.exp(logits - logits.max(axis=1, keepdims=True))
    gates = e / e.sum(axis=1, keepdims=True)
    ids = np.stack([np.lexsort((np.arange(s.experts), -gates[t]))[:k] for t in range(T)])
    sc = np.take_along_axis(gates, ids, axis=1)
    if s.norm_topk:
        sc = sc / sc.sum(axis=1, keepdims=True)
    Wg, Wu, Wd = (np.asarray(a, np.float64) for a in (fb.gate_proj, fb.up_proj, fb.down_proj))
    out = np.zeros((T, s.hidden))
    for t in range(T):
        for j in range(k):
            ex = int(ids[t, j])
            g, u = Wg[ex] @ x[t], Wu[ex] @ x[t]
            out[t] += (Wd[ex] @ (g * sigmoid(g) * u)) * sc[t, j]
    if s.shared:
        sg = sigmoid(x @ np.asarray(fb.sh_expert_gate, np.float64).reshape(-1))
        g = x @ np.asarray(fb.sh_gate_proj, np.float64).T
        u = x @ np.asarray(fb.sh_up_proj, np.float64).T
        out += sg[:, None] * ((g * sigmoid(g) * u) @ np.asarray(fb.sh_down_proj, np.float64).T)
    return out, gates, ids.astype(np.uint32)
