"""Writes the checkpoint fixtures under tests/golden/ from the reference's own test fixtures
(crates/mrun-engine/tests/fixtures/, data written by their gen_tiny.py with mlx-lm 0.32.0).

Run in a checkout that has the reference next to it:
    python tests/golden/make_fixtures.py /root/reference/crates/mrun-engine/tests/fixtures

Each fixture keeps the reference file's config.json unchanged and the subset of its
model.safetensors that the MoE path reads (the MoE blocks and the norm in front of each), byte for
byte, with the original names, dtypes, shapes and metadata; the Hugging Face one also keeps one
vision and one MTP tensor, which loading must skip. The config-only refusal fixtures are copied.
"""
from __future__ import annotations

import json
import re
import shutil
import struct
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent

# fixture -> regular expression of the tensor names kept
SUBSETS = {
    "tiny_qwen3_5_moe": r"language_model\.model\.layers\.\d+\.(mlp\..*|post_attention_layernorm\.weight)",
    "tiny_qwen3_moe": r"model\.layers\.(0|2)\.(mlp\..*|post_attention_layernorm\.weight)",
    "tiny_qwen3_5_moe_hf": r"(model\.language_model\.layers\.0\.mlp\..*|model\.visual\.blocks\.0\.attn\.proj\.weight|mtp\.fc\.weight)",
}
CONFIG_ONLY = ["refuse_quant_mode", "refuse_quant_bits"]


def read(path: Path):
    raw = path.read_bytes()
    n = struct.unpack("<Q", raw[:8])[0]
    header = json.loads(raw[8:8 + n])
    return header, raw[8 + n:]


def write(path: Path, header: dict, data: bytes, keep) -> None:
    names = sorted(k for k in header if k != "__metadata__" and keep(k))
    out_header, chunks, at = {}, [], 0
    if "__metadata__" in header:
        out_header["__metadata__"] = header["__metadata__"]
    for name in names:
        e = header[name]
        b, end = e["data_offsets"]
        chunk = data[b:end]
        out_header[name] = {"dtype": e["dtype"], "shape": e["shape"],
                            "data_offsets": [at, at + len(chunk)]}
        chunks.append(chunk)
        at += len(chunk)
    h = json.dumps(out_header, separators=(",", ":")).encode()
    h += b" " * (-len(h) % 8)
    path.write_bytes(struct.pack("<Q", len(h)) + h + b"".join(chunks))


def main(src: str) -> None:
    src = Path(src)
    for name, pattern in SUBSETS.items():
        dst = HERE / name
        dst.mkdir(exist_ok=True)
        shutil.copyfile(src / name / "config.json", dst / "config.json")
        header, data = read(src / name / "model.safetensors")
        rx = re.compile(pattern + r"$")
        write(dst / "model.safetensors", header, data, lambda k: rx.match(k) is not None)
    for name in CONFIG_ONLY:
        dst = HERE / name
        dst.mkdir(exist_ok=True)
        shutil.copyfile(src / name / "config.json", dst / "config.json")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/crates/mrun-engine/tests/fixtures")
