"""Build recipe of the native libraries (run by __graft_entry__.build(), or `python -m mrun_amd.build`).

- mrun_amd/lib/libmrun_moe.so   : the HIP kernels for gfx950 + the C ABI (include/mrun_moe.h)
- mrun_amd/lib/libmrun_synth.so : the seeded input generator (include/mrun_synth.h), host C
- mrun_amd/lib/libmrun_synth_dev.so : its device variant (HIP)
- mrun_amd/lib/libmrun_calib.so : copy and MFMA calibration kernels (HIP), loaded by bench.py only
- oracle/_build/liborc_moe.so   : the CPU restatement used by tests and the CPU baseline

Every HIP translation unit is compiled with packed-FP32 instructions disabled
(-Xclang -target-feature -Xclang -packed-fp32-ops).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "mrun_amd"
CSRC = PKG / "csrc"
LIB = PKG / "lib"
OBJ = PKG / "_build"
INCLUDE = ROOT / "include"

HIP_SOURCES = ["router.hip", "decode.hip", "qgemv.hip", "qgemm.hip", "moe_gemm.hip", "dense.hip", "f32.hip",
               "elementwise.hip", "moe.cpp", "loader.cpp"]
ARCH = os.environ.get("MRUN_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def _compile(src: str) -> Path:
    out = OBJ / (src + ".o")
    cmd = [HIPCC, *HIP_FLAGS, "-c", str(CSRC / src), "-o", str(out)]
    if src.endswith(".cpp"):
        cmd = [HIPCC, *HIP_FLAGS, "-x", "hip", "-c", str(CSRC / src), "-o", str(out)]
    _run(cmd)
    return out


def build_moe(jobs: int = 8) -> Path:
    OBJ.mkdir(parents=True, exist_ok=True)
    LIB.mkdir(parents=True, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, HIP_SOURCES))
    target = LIB / "libmrun_moe.so"
    tmp = LIB / "libmrun_moe.so.tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
          *map(str, objs), "-Wl,--no-undefined"])
    os.replace(tmp, target)
    return target


def build_synth() -> Path:
    LIB.mkdir(parents=True, exist_ok=True)
    target = LIB / "libmrun_synth.so"
    tmp = LIB / "libmrun_synth.so.tmp"
    _run(["gcc", "-O2", "-fPIC", "-shared", "-std=c11", "-fopenmp", "-ffp-contract=off",
          f"-I{INCLUDE}", str(CSRC / "synth.c"), "-o", str(tmp), "-lm"])
    os.replace(tmp, target)
    return target


def build_synth_dev() -> Path:
    """The device variant of the generator (benchmark inputs too large to make on the host)."""
    LIB.mkdir(parents=True, exist_ok=True)
    OBJ.mkdir(parents=True, exist_ok=True)
    target = LIB / "libmrun_synth_dev.so"
    tmp = LIB / "libmrun_synth_dev.so.tmp"
    _run([HIPCC, *HIP_FLAGS, "-shared", str(CSRC / "synth_dev.hip"), "-o", str(tmp)])
    os.replace(tmp, target)
    return target


def build_calib() -> Path:
    """Copy and MFMA-rate kernels that measure this box's roofline denominators (bench.py)."""
    LIB.mkdir(parents=True, exist_ok=True)
    target = LIB / "libmrun_calib.so"
    tmp = LIB / "libmrun_calib.so.tmp"
    _run([HIPCC, *HIP_FLAGS, "-shared", str(CSRC / "calib.hip"), "-o", str(tmp)])
    os.replace(tmp, target)
    return target


def build_oracle() -> Path:
    """The CPU restatement (test infrastructure); built beside the product, never linked into it."""
    _run(["make", "-s", "-C", str(ROOT / "oracle")])
    return ROOT / "oracle" / "_build" / "liborc_moe.so"


def build_all() -> list[Path]:
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    return [build_synth(), build_synth_dev(), build_calib(), build_oracle(), build_moe()]


if __name__ == "__main__":
    for p in build_all():
        print(p)
