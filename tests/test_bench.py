"""bench.py's contract on the CPU: one GPU only (N > 1 exits with a message before any device
work), and the algorithmic byte and flop counts its roofline fractions divide by, against the
closed forms of the measurement plan (Q = the configs[1] block)."""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import bench
from mrun_amd import synth

ROOT = Path(__file__).resolve().parent.parent
Q = synth.QWEN36


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], cwd=ROOT,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_projection_bytes():
    # 4-bit [512, 2048] with group 64: codes 512 KiB, bf16 scales and biases 64 KiB
    assert bench.proj_bytes(512, 2048) == 589_824
    assert bench.proj_bytes(2048, 512) == 589_824


def test_decode_block_bytes_closed_form():
    # n_distinct * 3 * 589,824 + the shared expert's 3 projections + router + shared gate + x in/out
    b = bench.decode_bytes(Q, n_active=8, T=1)
    assert b["block"] == 16_986_112
    # the gate/up launch: 8 routed + 1 shared expert's gate and up rows, activations, act out,
    # and the logits the routed workgroups read
    assert b["gate_up"] == 9 * 2 * 589_824 + 2 * 2048 + 2 * (8 * 512 + 512) + 2 * 256
    # more tokens only add activations on top of the distinct experts' rows
    assert bench.decode_bytes(Q, 8, 4)["block"] - b["block"] == 4 * 2048 * 3


def test_prefill_flops_closed_form():
    f = bench.prefill_flops(Q, 2048)
    assert f["gate_up"] == 2 * 2048 * 8 * 2048 * 2 * 512
    assert f["down"] == 2 * 2048 * 8 * 512 * 2048
    assert f["shared"] == 2 * 2048 * 3 * 2048 * 512
    assert f["router"] == 2 * 2048 * 2048 * 256
    assert round(f["block"] / 1e9, 2) == 118.11  # 118,111,600,640 flop
