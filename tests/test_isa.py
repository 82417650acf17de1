"""Checks of the grouped GEMM's machine code (CPU only: hipcc cross-compiles for gfx950).

The grouped GEMM issues its LDS reads as inline asm and waits for them with separate lgkmcnt
statements, so the compiler takes a destination register as written at issue. A spill, copy or
other use of that register before the wait that covers the read would see a value the load has not
yet filled. These tests compile the kernel the way the library is built and check its assembly:
no VGPR spills or scratch, and no instruction touching a pending destination register.
"""
import re
import shutil
import subprocess

import pytest

from mrun_amd import build as B

pytestmark = pytest.mark.skipif(shutil.which(B.HIPCC) is None and not __import__("os").path.exists(B.HIPCC),
                                reason="hipcc not available")

_REG = re.compile(r"\b([va])(\d+)\b|\b([va])\[(\d+):(\d+)\]")
_LGKM = re.compile(r"^(ds_|s_load|s_buffer_load|s_memtime|s_memrealtime|s_sendmsg)")


def _regs(text):
    out = set()
    for m in _REG.finditer(text):
        if m.group(1):
            out.add((m.group(1), int(m.group(2))))
        else:
            out.update((m.group(3), r) for r in range(int(m.group(4)), int(m.group(5)) + 1))
    return out


@pytest.fixture(scope="module")
def gemm_asm(tmp_path_factory):
    out = tmp_path_factory.mktemp("isa") / "moe_gemm.s"
    flags = [f for f in B.HIP_FLAGS if f != "-fPIC"]
    subprocess.run([B.HIPCC, *flags, "--cuda-device-only", "-S", str(B.CSRC / "moe_gemm.hip"), "-o",
                    str(out)], check=True, capture_output=True)
    return out.read_text()


def _kernel_bodies(asm):
    bodies = {}
    for name in re.findall(r"^(_ZN4mrun15moe_gemm_kernelI\w+):", asm, re.M):
        start = asm.index(f"\n{name}:") + 1
        end = asm.index("s_endpgm", start)
        bodies[name] = asm[start:end].splitlines()
    assert len(bodies) == 4, "the moe_gemm_kernel instantiations (gate/up, down; 64- and 32-row tiles)"
    return bodies


def test_grouped_gemm_has_no_spills(gemm_asm):
    for name, body in _kernel_bodies(gemm_asm).items():
        desc = gemm_asm[gemm_asm.index(f".amdhsa_kernel {name}"):]
        desc = desc[:desc.index(".end_amdhsa_kernel")]
        m = re.search(r"\.amdhsa_private_segment_fixed_size\s+(\d+)", desc)
        assert m is not None and int(m.group(1)) == 0, f"{name} uses scratch"
        assert not any("scratch_" in ln for ln in body), f"{name} spills VGPRs"


def test_asm_lds_reads_are_not_touched_before_their_wait(gemm_asm):
    """Every asm ds_read's destination stays untouched until an lgkmcnt wait covers the read.

    The scan follows the code in layout order (the K steps are straight-line code). An lgkmcnt(N)
    covers an LDS read once at least N LDS operations were issued after it (LDS operations complete
    in order; scalar loads only make a wait stricter)."""
    for name, lines in _kernel_bodies(gemm_asm).items():
        pending = []  # [dest regs, LDS ops issued after it]
        in_asm = False
        checked = 0
        for ln in lines:
            t = ln.split(";")[0].strip()
            if ln.strip().startswith(";;#ASMSTART"):
                in_asm = True
                continue
            if ln.strip().startswith(";;#ASMEND"):
                in_asm = False
                continue
            if not t or t.endswith(":") or t.startswith("."):
                continue
            op = t.split()[0]
            m = re.search(r"lgkmcnt\((\d+)\)", t) if op == "s_waitcnt" else None
            if m:
                n = int(m.group(1))
                pending = [p for p in pending if p[1] < n]
                continue
            if op.startswith("ds_read") and in_asm:
                dest = _regs(t.split(",")[0])
                for p in pending:
                    assert not (p[0] & _regs(t)), f"{name}: {t} touches a pending LDS destination"
                for p in pending:
                    p[1] += 1
                pending.append([dest, 0])
                checked += 1
                continue
            used = _regs(t)
            for p in pending:
                assert not (p[0] & used), f"{name}: '{t}' touches a pending LDS destination"
            if _LGKM.match(op) and op.startswith("ds_"):
                for p in pending:
                    p[1] += 1
        assert checked >= 40, f"{name}: expected the K steps' asm LDS reads"
