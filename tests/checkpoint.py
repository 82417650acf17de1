"""An independent reader of the safetensors fixtures (plain json + numpy), used to check the
library's loader and to build the oracle's view of the same weights."""
from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np

from mrun_amd import synth

GOLDEN = Path(__file__).resolve().parent / "golden"
_NP = {"BF16": np.uint16, "U32": np.uint32, "F32": np.float32, "U8": np.uint8}


def read(path: Path) -> dict:
    """name -> (dtype, shape, array) for every tensor of one file."""
    raw = Path(path).read_bytes()
    n = struct.unpack("<Q", raw[:8])[0]
    header = json.loads(raw[8:8 + n])
    out = {}
    for name, e in header.items():
        if name == "__metadata__":
            continue
        b, end = e["data_offsets"]
        a = np.frombuffer(raw[8 + n + b:8 + n + end], dtype=_NP[e["dtype"]]).reshape(e["shape"])
        out[name] = (e["dtype"], tuple(e["shape"]), a)
    return out


def config(fixture: str) -> dict:
    c = json.loads((GOLDEN / fixture / "config.json").read_text())
    return c.get("text_config", c)


def _q(t: dict, path: str, in_dims: int) -> synth.QTensor:
    codes = t[path + ".weight"][2]
    scales = t[path + ".scales"][2]
    biases = t.get(path + ".biases", (None, None, None))[2]
    if codes.ndim == 2:
        codes, scales = codes[None], scales[None]
        biases = biases[None] if biases is not None else None
    bits = codes.shape[-1] * 32 // in_dims
    group = in_dims // scales.shape[-1]
    return synth.QTensor(codes=np.ascontiguousarray(codes), scales=np.ascontiguousarray(scales),
                         biases=None if biases is None else np.ascontiguousarray(biases),
                         experts=codes.shape[0], out=codes.shape[1], in_=in_dims, group=group,
                         bits=bits)


def host_block(fixture: str, prefix: str) -> synth.HostBlock:
    """The MoE block at `prefix` as the oracle reads it (group and bits from the packed shapes)."""
    c = config(fixture)
    t = read(GOLDEN / fixture / "model.safetensors")
    D, I = c["hidden_size"], c["moe_intermediate_size"]
    S = c.get("shared_expert_intermediate_size", 0) or 0
    shape = synth.Shape(hidden=D, experts=c["num_experts"], top_k=c["num_experts_per_tok"],
                        intermediate=I, shared=S, norm_topk=c.get("norm_topk_prob", True),
                        group=D // t[prefix + ".switch_mlp.gate_proj.scales"][2].shape[-1])
    hb = synth.HostBlock(
        shape=shape,
        router=_q(t, prefix + ".gate", D),
        router_bias=None,
        gate_proj=_q(t, prefix + ".switch_mlp.gate_proj", D),
        up_proj=_q(t, prefix + ".switch_mlp.up_proj", D),
        down_proj=_q(t, prefix + ".switch_mlp.down_proj", I),
    )
    if S:
        hb.sh_gate_proj = _q(t, prefix + ".shared_expert.gate_proj", D)
        hb.sh_up_proj = _q(t, prefix + ".shared_expert.up_proj", D)
        hb.sh_down_proj = _q(t, prefix + ".shared_expert.down_proj", S)
        hb.sh_expert_gate = _q(t, prefix + ".shared_expert_gate", D)
    return hb


def write(path: Path, tensors: dict, metadata: dict | None = None) -> None:
    """Writes {name: numpy array (uint16 for bf16 bits, uint32 or float32)} as safetensors."""
    dt = {np.dtype(np.uint16): "BF16", np.dtype(np.uint32): "U32", np.dtype(np.float32): "F32"}
    header, chunks, at = {}, [], 0
    if metadata:
        header["__metadata__"] = metadata
    for name in sorted(tensors):
        a = np.ascontiguousarray(tensors[name])
        b = a.tobytes()
        header[name] = {"dtype": dt[a.dtype], "shape": list(a.shape), "data_offsets": [at, at + len(b)]}
        chunks.append(b)
        at += len(b)
    h = json.dumps(header, separators=(",", ":")).encode()
    h += b" " * (-len(h) % 8)
    Path(path).write_bytes(struct.pack("<Q", len(h)) + h + b"".join(chunks))
