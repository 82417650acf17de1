"""Benchmark of the MI355X MoE sparse block (the reference's SparseMoe::forward, moe.rs:149-174).

Default workload: one Qwen3.6-35B-A3B-like block (hidden 2048, 256 experts,
top-8 with norm_topk_prob, expert FFN 512, shared expert 512), 4-bit affine group-64 weights,
synthetic seeded data, decode T = 1. A step is one block forward over the batch. The JSON line
also carries the T = 2, 4, 16 decode sweep, the configs[2] prefill (T = 2048, Zipf-skewed
router), the configs[3] stack of 40 layers (T = 1 and T = 4096) and the configs[4] Coder-shaped
block (T = 1, 8, 8192) measured the same way, the dominant kernel's roofline (HIP events on the
launch stream), this box's measured copy and MFMA rates beside the published peaks, each decode
point also timed with the 256 MB last-level cache flushed before every forward (`cold_*`: the
repeated forward keeps the 17 MB block in that cache), and the CPU restatement timed on a bounded
sample on this host (all cores, and one thread).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--tokens T] [--no-cpu] [--no-prefill]
                    [--no-stack] [--no-coder] [--no-machine] [--stack-only] [--prefill-only]
                    [--coder-only]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

HBM_PEAK = 8.0e12          # B/s, MI355X HBM3E
MFMA_BF16_PEAK = 2.5e15    # dense bf16 flop/s


def hip():
    lib = ctypes.CDLL("libamdhip64.so")
    lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    lib.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    lib.hipEventSynchronize.argtypes = [ctypes.c_void_p]
    lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                        ctypes.c_void_p]
    lib.hipEventDestroy.argtypes = [ctypes.c_void_p]
    return lib


class Events:
    def __init__(self, n: int):
        self.h = hip()
        self.ev = (ctypes.c_void_p * n)()
        for i in range(n):
            p = ctypes.c_void_p()
            assert self.h.hipEventCreate(ctypes.byref(p)) == 0
            self.ev[i] = p.value

    def record(self, i: int, stream) -> None:
        assert self.h.hipEventRecord(self.ev[i], ctypes.c_void_p(stream.cuda_stream)) == 0

    def ms(self, a: int, b: int) -> float:
        self.h.hipEventSynchronize(self.ev[b])
        t = ctypes.c_float()
        assert self.h.hipEventElapsedTime(ctypes.byref(t), self.ev[a], self.ev[b]) == 0
        return float(t.value)


def proj_bytes(out: int, in_: int, group: int = 64) -> int:
    """Codes plus bf16 scales and biases of one [out, in] 4-bit projection."""
    return out * in_ // 2 + 2 * 2 * out * (in_ // group)


def decode_bytes(shape, n_active: int, T: int) -> dict:
    """Algorithmic HBM bytes of each decode launch and of the block.

    router: router rows and the shared gate row; gate_up: the active experts' and the shared
    expert's gate/up rows, activations in, act out; down_combine: the down rows, act in, out."""
    D, E, I, S = shape.hidden, shape.experts, shape.intermediate, shape.shared
    k = shape.top_k
    P = T * k
    router = 2 * E * D + (2 * D if S else 0) + 2 * T * D + 2 * T * (E + 1)
    gu = (n_active * 2 * proj_bytes(I, D) + (2 * proj_bytes(S, D) if S else 0)
          + 2 * T * D + 2 * (P * I + T * S) + 2 * T * E)
    dn = (n_active * proj_bytes(D, I) + (proj_bytes(D, S) if S else 0)
          + 2 * (P * I + T * S) + 2 * T * D + 2 * P + 4 * P + 2 * T)
    block = (n_active * 3 * proj_bytes(I, D) + (3 * proj_bytes(S, D) if S else 0)
             + 2 * E * D + (2 * D if S else 0) + 4 * D * T)
    return {"gate_up": gu, "down_combine": dn, "router": router, "block": block}


def prefill_flops(shape, T: int) -> dict:
    D, E, I, S, k = shape.hidden, shape.experts, shape.intermediate, shape.shared, shape.top_k
    gate_up = 2 * T * k * D * 2 * I
    down = 2 * T * k * I * D
    shared = 2 * T * 3 * D * S
    router = 2 * T * D * E
    return {"gate_up": gate_up, "down": down, "shared": shared, "router": router,
            "block": gate_up + down + shared + router}


def time_forward(dev, x, steps: int, warmup: int, torch):
    """Wall clock and HIP-event time of `steps` forwards (after `warmup`). Each forward is one call
    of the C ABI's mrun_moe_forward with its arguments converted once, as a native host calls it:
    the Python wrapper's per-call work (about 1.5 us) would otherwise set the pace of the T = 1
    forward, whose three launches take the host 9 to 10.5 us against 13.5 us on the device."""
    from mrun_amd import _lib
    stream = torch.cuda.current_stream()
    out = torch.empty_like(x)
    ws = dev.workspace(x.shape[0])
    for _ in range(warmup):
        dev.forward(x, out=out, workspace=ws)
    fwd = _lib.load().mrun_moe_forward
    args = (ctypes.byref(dev.c), ctypes.c_void_p(x.data_ptr()), x.shape[0],
            ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(ws.data_ptr()), ws.numel(),
            ctypes.c_void_p(stream.cuda_stream))
    _lib.check(fwd(*args))
    ev = Events(2)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev.record(0, stream)
    rc = 0
    for _ in range(steps):
        rc |= fwd(*args)
    _lib.check(rc)
    ev.record(1, stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return wall, ev.ms(0, 1) / steps, out


def time_stages(dev, x, reps: int, torch):
    """Mean device time of each stage of the forward (events between launches)."""
    from mrun_amd import _lib
    lib = _lib.load()
    T = x.shape[0]
    names = lib.mrun_moe_stage_names(ctypes.byref(dev.cfg), T).decode().split(",")
    n = len(names) + 1
    ev = Events(n)
    stream = torch.cuda.current_stream()
    out = torch.empty_like(x)
    ws = dev.workspace(T)
    acc = np.zeros(len(names))
    ns = ctypes.c_int32()
    for r in range(reps + 1):
        rc = lib.mrun_moe_forward_profiled(
            ctypes.byref(dev.c), ctypes.c_void_p(x.data_ptr()), T, ctypes.c_void_p(out.data_ptr()),
            ctypes.c_void_p(ws.data_ptr()), ws.numel(), ctypes.c_void_p(stream.cuda_stream),
            ev.ev, n, ctypes.byref(ns))
        _lib.check(rc)
        torch.cuda.synchronize()
        if r == 0:
            continue  # warm
        for i in range(len(names)):
            acc[i] += ev.ms(i, i + 1)
    return {name: float(acc[i] / reps * 1e3) for i, name in enumerate(names)}  # microseconds


def time_gateup_kernel(dev, x, reps: int, torch, cold=None) -> float:
    """Mean duration of the decode gate/up kernel in microseconds, one forward after another on
    the stream: mrun_moe_forward_timed has the kernel stamp the device wall clock at its
    workgroups' starts and its waves' ends (64 folded pairs per forward); the span from the first
    start to the last end has no launch gap and no dispatch latency. With `cold` (a ColdTimer) the last-level cache is flushed before every forward."""
    from mrun_amd import _lib
    lib = _lib.load()
    hz = lib.mrun_wall_clock_hz()
    if hz <= 0:
        raise RuntimeError("the device does not report its wall clock rate")
    T = x.shape[0]
    stream = torch.cuda.current_stream()
    out = torch.empty_like(x)
    ws = dev.workspace(T)
    clock = torch.zeros(reps, 64, 2, dtype=torch.int64, device=x.device)
    clock[:, :, 0] = -1  # 64 pairs (UINT64_MAX, 0) per forward: the kernel lowers and raises them
    for r in range(reps):
        if cold is not None:
            cold.flush(stream)
        _lib.check(lib.mrun_moe_forward_timed(
            ctypes.byref(dev.c), ctypes.c_void_p(x.data_ptr()), T, ctypes.c_void_p(out.data_ptr()),
            ctypes.c_void_p(ws.data_ptr()), ws.numel(), ctypes.c_void_p(stream.cuda_stream),
            ctypes.c_void_p(clock[r].data_ptr())))
    torch.cuda.synchronize()
    c = clock.cpu().numpy().view(np.uint64)
    ticks = (c[1:, :, 1].max(axis=1) - c[1:, :, 0].min(axis=1)).astype(np.float64)  # (the first
    # forward is a warm-up)
    return float(np.mean(ticks) / hz * 1e6)


def time_graph(dev, x, steps: int, torch, per_graph: int = 1):
    """Device time per forward of `per_graph` forwards captured in one HIP graph, replayed
    back to back. With one forward per graph the replays are bound by the host's graph launch
    (hipGraphLaunch takes longer than the three kernels); per_graph > 1 amortises it."""
    out = torch.empty_like(x)
    ws = dev.workspace(x.shape[0])
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            dev.forward(x, out=out, workspace=ws, stream=s)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for _ in range(per_graph):
            dev.forward(x, out=out, workspace=ws, stream=s)
    torch.cuda.synchronize()
    for _ in range(3):
        g.replay()
    ev = Events(2)
    stream = torch.cuda.current_stream()
    reps = max(steps // per_graph, 3)
    torch.cuda.synchronize()
    ev.record(0, stream)
    for _ in range(reps):
        g.replay()
    ev.record(1, stream)
    torch.cuda.synchronize()
    return ev.ms(0, 1) / (reps * per_graph), out


def _cpu_run(fn, budget: float, min_reps: int = 3, max_reps: int = 2000):
    """Median seconds of fn() repeated for about `budget` seconds after one warm-up call."""
    fn()
    times, t0 = [], time.perf_counter()
    while True:
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
        el = time.perf_counter() - t0
        if (el >= budget and len(times) >= min_reps) or len(times) >= max_reps:
            break
    return float(np.median(times)), len(times), el


def cpu_baseline(args, Q, synth, hb, x_np) -> dict:
    """The CPU restatement (oracle/, scalar C with OpenMP over pairs and rows) on this host's
    cores: the headline configs[1] T = 1 point (all cores, then one thread) and one entry per
    config in `per_config`. Large points time a sample of token rows (rows are independent) or
    2 of the 40 stack layers, as each entry's `sample` says."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import oracle as O
    cores = len(os.sched_getaffinity(0))
    threads = O.set_threads(cores)
    sec = args.cpu_seconds
    where = (f"OpenMP over {threads} threads (sched_getaffinity {cores}, hardware "
             f"{os.cpu_count()})")

    def entry(tokens: int, med: float, sample: str) -> dict:
        return {"value": tokens / med, "unit": "tokens/s", "cores": threads, "kind": "port",
                "sample": f"{sample}; {where}; median s/forward {med:.4g}"}

    def block_point(blk, x, label: str, budget: float, min_reps: int = 3) -> dict:
        med, reps, el = _cpu_run(lambda: O.moe_forward(blk, x), budget, min_reps)
        return entry(x.shape[0], med, f"{reps} block forwards at T={x.shape[0]} ({el:.1f} s), "
                                      f"{label}")

    per = {}
    print("[bench] CPU baseline configs[1]", file=sys.stderr, flush=True)
    T = x_np.shape[0]
    med, reps, el = _cpu_run(lambda: O.moe_forward(hb, x_np), sec, 5)
    head = entry(T, med, f"{reps} block forwards at T={T} ({el:.1f} s), the seeded configs[1] block")
    O.set_threads(1)
    med1, reps1, el1 = _cpu_run(lambda: O.moe_forward(hb, x_np), sec / 3, 3)
    O.set_threads(cores)
    head["one_thread"] = {"value": T / med1, "unit": "tokens/s", "cores": 1,
                          "sample": f"{reps1} block forwards ({el1:.1f} s); median s/forward "
                                    f"{med1:.4g}"}
    per[f"configs[1] T={T}"] = {k: v for k, v in head.items() if k != "one_thread"}
    for t in (1, 2, 4, 16):
        if t != T:
            per[f"configs[1] T={t}"] = block_point(
                hb, synth.make_x(Q, t, config=synth.CFG_DECODE, layer=t), "configs[1] block", 2.0)
    print("[bench] CPU baseline configs[0], configs[2]", file=sys.stderr, flush=True)
    h0 = synth.make_block(Q, config=synth.CFG_PLUMBING)
    per["configs[0] T=16"] = block_point(h0, synth.make_x(Q, 16, config=synth.CFG_PLUMBING),
                                         "configs[0] plumbing block", 2.0)
    del h0
    hz = synth.make_block(Q, config=synth.CFG_PREFILL_ZIPF, zipf=True)
    xz = synth.make_x(Q, 2048, config=synth.CFG_PREFILL_ZIPF)[:256]
    pz = block_point(hz, xz, "the first 256 of the 2,048 token rows of the configs[2] input "
                             "(Zipf router; each expert row is dequantised once per forward, so "
                             "fewer rows understate the full-batch rate)", 1.0, 1)
    per["configs[2] T=2048"] = pz
    del hz
    print("[bench] CPU baseline configs[3]", file=sys.stderr, flush=True)
    layers = [synth.make_block(Q, config=synth.CFG_STACK, layer=l) for l in range(2)]
    for t, rows in ((1, 1), (4096, 32)):
        xs = synth.make_x(Q, t, config=synth.CFG_STACK, layer=t)[:rows]
        med, reps, el = _cpu_run(lambda: O.moe_stack(layers, xs, None, 1e-6), 2.0, 1)
        per_layer = med / 2
        per[f"configs[3] T={t}"] = {
            "value": rows / (40 * per_layer), "unit": "tokens/s (40-layer pass)",
            "cores": threads, "kind": "port",
            "sample": f"{reps} passes of {rows} token row(s) through 2 of the 40 seeded layers "
                      f"(pre-RMSNorm and residual add each) ({el:.1f} s), scaled to 40 layers; "
                      f"{where}; median s/layer {per_layer:.4g}"}
    del layers
    if not args.no_coder:
        print("[bench] CPU baseline configs[4] (generating the block on the host)",
              file=sys.stderr, flush=True)
        C = synth.CODER
        hc = synth.make_block(C, config=synth.CFG_CODER)
        for t in (1, 8):
            per[f"configs[4] T={t}"] = block_point(
                hc, synth.make_x(C, t, config=synth.CFG_CODER, layer=t), "configs[4] Coder block",
                2.0, 1)
        xc = synth.make_x(C, 8192, config=synth.CFG_CODER, layer=8192)[:16]
        per["configs[4] T=8192"] = block_point(
            hc, xc, "the first 16 of the 8,192 token rows of the configs[4] prefill input (each "
                    "expert row is dequantised once per forward, so fewer rows understate the "
                    "full-batch rate)", 1.0, 1)
        del hc
    head["per_config"] = per
    return head


def calib_lib():
    root = os.path.dirname(os.path.abspath(__file__))
    lib = ctypes.CDLL(os.path.join(root, "mrun_amd", "lib", "libmrun_calib.so"))
    lib.mrun_calib_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                    ctypes.c_void_p]
    lib.mrun_calib_mfma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.mrun_calib_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                    ctypes.c_void_p]
    lib.mrun_calib_chain.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                     ctypes.c_void_p]
    return lib


def launch_floor(torch, grids=(65, 288, 256), reps: int = 200) -> dict:
    """The floor under the decode forward's three dependent launches: chains of three launches
    with the T = 1 forward's grids (router, gate/up, down), each workgroup storing a word for the
    next launch, timed like the forward (HIP events around `reps` back-to-back chains). `read`:
    every thread of a launch first reads a word the previous launch wrote (one dependent global
    read per launch, as each decode launch starts with one)."""
    lib = calib_lib()
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    bufs = [torch.ones(max(grids) * 256, dtype=torch.int32, device="cuda") for _ in range(4)]
    ptrs = (ctypes.c_void_p * 4)(*[b.data_ptr() for b in bufs])
    g = (ctypes.c_int * 3)(*grids)
    ev = Events(2)
    res = {}
    for read in (0, 1):
        for _ in range(20):
            assert lib.mrun_calib_chain(ptrs, g, read, sp) == 0
        ev.record(0, stream)
        for _ in range(reps):
            assert lib.mrun_calib_chain(ptrs, g, read, sp) == 0
        ev.record(1, stream)
        res["read" if read else "empty"] = ev.ms(0, 1) * 1e3 / reps
    return {"empty_us": res["empty"], "read_us": res["read"], "grids": list(grids),
            "what": f"three dependent launches of {grids[0]}, {grids[1]} and {grids[2]} "
                    f"workgroups x 256 threads (the T = 1 forward's grids), mean of {reps} "
                    "back-to-back chains; read_us: each thread first reads a word the previous "
                    "launch wrote"}


class ColdTimer:
    """HIP-event time of single forwards, each after a 1 GiB read that pushes the block's weights
    out of the 256 MB last-level cache (the repeated-forward loop keeps a 17 MB block in it)."""

    def __init__(self, torch):
        self.torch = torch
        self.lib = calib_lib()
        self.buf = torch.ones((1 << 30) // 4, dtype=torch.int32, device="cuda")
        self.rout = torch.empty(self.lib.mrun_calib_read_threads(), dtype=torch.int32,
                                device="cuda")

    def flush(self, stream) -> None:
        assert self.lib.mrun_calib_read(self.buf.data_ptr(), 1 << 30, self.rout.data_ptr(),
                                        ctypes.c_void_p(stream.cuda_stream)) == 0

    def time(self, dev, x, n: int) -> float:
        stream = self.torch.cuda.current_stream()
        out = self.torch.empty_like(x)
        ws = dev.workspace(x.shape[0])
        ev = Events(2)
        tot = 0.0
        for _ in range(n):
            self.flush(stream)
            ev.record(0, stream)
            dev.forward(x, out=out, workspace=ws)
            ev.record(1, stream)
            tot += ev.ms(0, 1)
        return tot / n


def machine_point(torch) -> dict:
    """This box's roofline denominators beside the published peaks: a 4 GiB read (larger than the
    256 MB last-level cache), a 1 GiB device copy (bytes read + written per second) and
    back-to-back v_mfma_f32_32x32x16_bf16 on every SIMD (flop/s), all with kernels of
    libmrun_calib.so timed by HIP events on the launch stream."""
    lib = calib_lib()
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    ev = Events(2)
    rbytes = 4 << 30
    rsrc = torch.ones(rbytes // 4, dtype=torch.int32, device="cuda")
    rout = torch.empty(lib.mrun_calib_read_threads(), dtype=torch.int32, device="cuda")
    for _ in range(2):
        assert lib.mrun_calib_read(rsrc.data_ptr(), rbytes, rout.data_ptr(), sp) == 0
    rreps = 10
    ev.record(0, stream)
    for _ in range(rreps):
        assert lib.mrun_calib_read(rsrc.data_ptr(), rbytes, rout.data_ptr(), sp) == 0
    ev.record(1, stream)
    read_ms = ev.ms(0, 1) / rreps
    read_bps = rbytes / (read_ms * 1e-3)
    del rsrc, rout
    nbytes = 1 << 30
    src = torch.ones(nbytes // 4, dtype=torch.int32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        assert lib.mrun_calib_copy(src.data_ptr(), dst.data_ptr(), nbytes, sp) == 0
    reps = 20
    ev.record(0, stream)
    for _ in range(reps):
        assert lib.mrun_calib_copy(src.data_ptr(), dst.data_ptr(), nbytes, sp) == 0
    ev.record(1, stream)
    copy_ms = ev.ms(0, 1) / reps
    assert bool(torch.equal(src, dst)), "calibration copy differs"
    copy_bps = 2 * nbytes / (copy_ms * 1e-3)
    del src, dst
    blocks, iters = 256 * 12, 4096  # 12 workgroups of 4 waves per CU: 12 waves per SIMD queued
    chains = lib.mrun_calib_mfma_chains()
    out = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")
    assert lib.mrun_calib_mfma(blocks, 64, out.data_ptr(), sp) == 0
    ev.record(0, stream)
    assert lib.mrun_calib_mfma(blocks, iters, out.data_ptr(), sp) == 0
    ev.record(1, stream)
    mfma_ms = ev.ms(0, 1)
    assert bool((out == float(chains * 256 * iters)).all()), "calibration MFMA sums differ"
    flops = blocks * 4 * iters * chains * 32 * 32 * 16 * 2
    mfma_fps = flops / (mfma_ms * 1e-3)
    return {"read_GBps": read_bps / 1e9, "read_frac_of_peak": read_bps / HBM_PEAK,
            "read": f"4 GiB, 16-byte loads, mean of {rreps}; {read_ms * 1e3:.0f} us per read",
            "copy_GBps": copy_bps / 1e9, "copy_frac_of_peak": copy_bps / HBM_PEAK,
            "copy": f"1 GiB device to device, 16-byte loads/stores, mean of {reps}; "
                    f"{copy_ms * 1e3:.0f} us per copy",
            "mfma_bf16_TFLOPs": mfma_fps / 1e12, "mfma_frac_of_peak": mfma_fps / MFMA_BF16_PEAK,
            "mfma": f"v_mfma_f32_32x32x16_bf16, {blocks} workgroups x 4 waves x {iters} x "
                    f"{chains} chains; {mfma_ms:.2f} ms"}


def prefill_point(args, Q, M, synth, torch) -> dict:
    """T = 2048 with the Zipf-skewed router."""
    print("[bench] prefill configs[2] T=2048 (Zipf router)", file=sys.stderr, flush=True)
    hz = synth.make_block(Q, config=synth.CFG_PREFILL_ZIPF, zipf=True)
    dz = M.SparseMoe(hz)
    T = 2048
    xz = M.bf16_tensor(synth.make_x(Q, T, config=synth.CFG_PREFILL_ZIPF))
    # 30 warm-up forwards: the first few milliseconds of back-to-back prefill run at lower clocks
    wall, dev_ms, _ = time_forward(dz, xz, max(args.steps // 4, 20), 30, torch)
    stages = time_stages(dz, xz, 10, torch)
    fl = prefill_flops(Q, T)
    return {"tokens": T, "ms_per_step": wall, "device_ms": dev_ms,
            "tokens_per_s": T / (wall * 1e-3), "us_per_layer": dev_ms * 1e3,
            "stages_us": stages, "flops": fl,
            "cache": "warm: repeated forwards (the block's 402 MB of expert weights exceed the "
                     "256 MB last-level cache, so most of them come from HBM anyway)",
            "block_mfma_frac_warm": fl["block"] / (dev_ms * 1e-3) / MFMA_BF16_PEAK,
            "gate_up_mfma_frac_warm": (fl["gate_up"] + fl["shared"] * 2 / 3)
            / (stages["gate_up"] * 1e-6) / MFMA_BF16_PEAK,
            "down_mfma_frac_warm": (fl["down"] + fl["shared"] / 3)
            / (stages["down"] * 1e-6) / MFMA_BF16_PEAK}


def time_call(fn, reps: int, torch, warmup: int = 5) -> float:
    """Mean device ms of fn() over reps calls, HIP events on the current stream."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / reps


def facade_point(args, Q, M, synth, torch) -> dict:
    """The facade ops at configs[2]'s prefill size: gather_qmm over the T k = 16,384 pair rows of
    the gate projection in SwitchGlu's sorted case (moe.rs:62-80: rows gathered by token, indices
    ascending, one row per index), and quantized_matmul over T = 2048 rows of the shared expert's
    gate projection. Each call's permute, packing and reordering are inside the timed region."""
    print("[bench] facade gather_qmm / quantized_matmul at configs[2] sizes", file=sys.stderr,
          flush=True)
    hz = synth.make_block(Q, config=synth.CFG_PREFILL_ZIPF, zipf=True)
    dz = M.SparseMoe(hz)
    T, k, D, I, S = 2048, Q.top_k, Q.hidden, Q.intermediate, Q.shared
    xz = M.bf16_tensor(synth.make_x(Q, T, config=synth.CFG_PREFILL_ZIPF))
    _, _, ids, _ = dz.router_forward(xz)
    flat = ids.reshape(-1).to(torch.int64)
    order = torch.sort(flat, stable=True).indices
    idx = flat[order].to(torch.int32).contiguous()
    rows = xz[order // k].contiguous()
    n = idx.numel()
    reps = max(args.steps // 8, 10)
    ms_g = time_call(lambda: M.gather_qmm(rows, dz.gate_proj, idx, sorted_indices=True), reps, torch)
    fl_g = 2.0 * n * I * D
    xs = xz.contiguous()
    ms_q = time_call(lambda: M.quantized_matmul(xs, dz.sh_gate_proj), reps, torch)
    fl_q = 2.0 * T * S * D
    return {"gather_qmm": {"rows": n, "out": I, "in": D, "device_ms": ms_g, "flops": fl_g,
                           "mfma_frac": fl_g / (ms_g * 1e-3) / MFMA_BF16_PEAK,
                           "kernel": "moe_gemm_kernel (packed x, permute and row reorder included)"},
            "quantized_matmul": {"rows": T, "out": S, "in": D, "device_ms": ms_q, "flops": fl_q,
                                 "mfma_frac": fl_q / (ms_q * 1e-3) / MFMA_BF16_PEAK,
                                 "kernel": "qgemm_kernel (no workspace in the facade signature)"}}


def formats_point(args, Q, M, synth, torch) -> dict:
    """The other expert formats the reference loads (load.rs:15-17) on the configs[1]/[2] block:
    8-bit experts (group 64) and 4-bit experts with group 32, decode T = 1 and 16 and prefill
    T = 2048 (Zipf router)."""
    out = {}
    for name, shape, bits in (("experts8_g64", Q, 8),
                              ("experts4_g32", synth.Shape(hidden=Q.hidden, experts=Q.experts,
                                                           top_k=Q.top_k, intermediate=Q.intermediate,
                                                           shared=Q.shared, group=32), 4)):
        print(f"[bench] formats: {name}", file=sys.stderr, flush=True)
        pt = {}
        hb = synth.make_block(shape, config=synth.CFG_DECODE, expert_bits=bits)
        dv = M.SparseMoe(hb)
        for T in (1, 16):
            x = M.bf16_tensor(synth.make_x(shape, T, config=synth.CFG_DECODE, layer=T))
            wall, dev_ms, _ = time_forward(dv, x, max(args.steps // 4, 20), args.warmup, torch)
            pt[f"decode_T{T}"] = {"device_ms": dev_ms, "ms_per_step": wall,
                                  "tokens_per_s": T / (wall * 1e-3)}
        del dv, hb
        hz = synth.make_block(shape, config=synth.CFG_PREFILL_ZIPF, zipf=True, expert_bits=bits)
        dz = M.SparseMoe(hz)
        xz = M.bf16_tensor(synth.make_x(shape, 2048, config=synth.CFG_PREFILL_ZIPF))
        wall, dev_ms, _ = time_forward(dz, xz, max(args.steps // 8, 10), 10, torch)
        fl = prefill_flops(shape, 2048)
        pt["prefill_T2048"] = {"device_ms": dev_ms, "tokens_per_s": 2048 / (wall * 1e-3),
                               "block_mfma_frac": fl["block"] / (dev_ms * 1e-3) / MFMA_BF16_PEAK}
        del dz, hz
        out[name] = pt
    return out


def stack_point(args, Q, M, synth, torch) -> dict:
    """40 MoE layers with their own seeded weights (generated on the device: about
    18 GB), pre-RMSNorm (eps 1e-6, weight 1) and the residual add, at T = 1 decode and T = 4096
    prefill. A step is one pass of x through all layers."""
    n = args.stack_layers
    print(f"[bench] stack configs[3]: generating {n} layers on the device", file=sys.stderr,
          flush=True)
    layers = [M.device_block(Q, synth.CFG_STACK, l) for l in range(n)]
    st = M.MoeStack(layers, None, 1e-6)
    torch.cuda.synchronize()
    wbytes = sum(t.numel() * t.element_size() for l in layers for t in l.tensors())
    out = {"layers": n, "weight_bytes": wbytes}
    for T, steps in ((1, max(args.steps // 10, 10)), (4096, 5)):
        print(f"[bench] stack T={T}", file=sys.stderr, flush=True)
        x0 = M.bf16_tensor(synth.make_x(Q, T, config=synth.CFG_STACK, layer=T))
        x = x0.clone()
        ws = st.workspace(T)
        for _ in range(2):
            st.forward_(x, ws)
        stream = torch.cuda.current_stream()
        ev = Events(2)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev.record(0, stream)
        for _ in range(steps):
            st.forward_(x, ws)
        ev.record(1, stream)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) * 1e3 / steps
        dev_ms = ev.ms(0, 1) / steps
        assert bool(torch.isfinite(x.float()).all()), "stack output not finite"
        pt = {"tokens": T, "steps": steps, "ms_per_step": wall, "device_ms": dev_ms,
              "tokens_per_s": T / (wall * 1e-3), "us_per_layer": dev_ms * 1e3 / n}
        if T == 1:
            # the whole stack captured as one HIP graph (launch overhead amortised)
            s = torch.cuda.Stream()
            s.wait_stream(stream)
            with torch.cuda.stream(s):
                st.forward_(x, ws, stream=s)
            stream.wait_stream(s)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                st.forward_(x, ws, stream=s)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            ev.record(0, stream)
            for _ in range(steps):
                g.replay()
            ev.record(1, stream)
            torch.cuda.synchronize()
            pt["graph_ms"] = ev.ms(0, 1) / steps
            pt["graph_us_per_layer"] = pt["graph_ms"] * 1e3 / n
            del g
        if T == 1:
            # one token picks top_k distinct experts in every layer; plus the norm's x, h traffic
            b = n * (decode_bytes(Q, Q.top_k, 1)["block"] + 4 * Q.hidden)
            # 18 GB of weights, 70x the last-level cache: every layer reads them from HBM
            pt.update(bytes=b, hbm_frac_cold=b / (dev_ms * 1e-3) / HBM_PEAK)
        else:
            f = n * prefill_flops(Q, T)["block"]
            pt.update(flops=f, mfma_frac_cold=f / (dev_ms * 1e-3) / MFMA_BF16_PEAK)
        out[f"T{T}"] = pt
        del x, x0
    del st, layers
    torch.cuda.empty_cache()
    return out


def coder_point(args, M, synth, torch, cold=None) -> dict:
    """the Coder-shaped block (hidden 6144, 160 experts, top-8, FFN 2560, no shared
    expert; 4.2 GB of 4-bit weights, generated on the device) at decode T = 1 and 8, where a block
    streams 8 experts' 26.5 MB each, and at prefill T = 8192."""
    C = synth.CODER
    print("[bench] coder configs[4]: generating the block on the device", file=sys.stderr,
          flush=True)
    dev = M.device_block(C, synth.CFG_CODER, 0)
    torch.cuda.synchronize()
    out = {"workload": "configs[4]: Coder-shaped block (hidden 6144, 160 experts, top-8, "
                       "FFN 2560, no shared expert), 4-bit affine group 64"}
    for T, steps in ((1, max(args.steps // 4, 20)), (8, max(args.steps // 4, 20)), (8192, 3)):
        print(f"[bench] coder T={T}", file=sys.stderr, flush=True)
        x = M.bf16_tensor(synth.make_x(C, T, config=synth.CFG_CODER, layer=T))
        wall, dev_ms, _ = time_forward(dev, x, steps, 2 if T > 16 else 10, torch)
        pt = {"tokens": T, "steps": steps, "ms_per_step": wall, "device_ms": dev_ms,
              "tokens_per_s": T / (wall * 1e-3)}
        if T <= 16:
            _, _, ids, _ = dev.router_forward(x)
            n_active = int(np.unique(M.u32_array(ids)).size)
            b = decode_bytes(C, n_active, T)["block"]
            # warm: the repeated forward reads the same experts' 212 MB (T = 1), which the 256 MB
            # last-level cache holds; cold: that cache flushed before every forward
            pt.update(n_active=n_active, bytes=b, hbm_frac_warm=b / (dev_ms * 1e-3) / HBM_PEAK)
            if cold is not None:
                cms = cold.time(dev, x, 10)
                pt.update(cold_device_ms=cms, hbm_frac_cold=b / (cms * 1e-3) / HBM_PEAK)
        else:
            f = prefill_flops(C, T)["block"]
            # 4.2 GB of weights, read by every forward: past the last-level cache
            pt.update(flops=f, mfma_frac_cold=f / (dev_ms * 1e-3) / MFMA_BF16_PEAK)
        out[f"T{T}"] = pt
        del x
    del dev
    torch.cuda.empty_cache()
    return out


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 byte counters, or None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    k = rec.get("kernels", {}).get(kernel)
    return None if k is None else k.get("bytes_per_launch")


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--tokens", type=int, default=1)
    ap.add_argument("--cpu-seconds", type=float, default=6.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-stack", action="store_true")
    ap.add_argument("--stack-layers", type=int, default=40)
    ap.add_argument("--no-coder", action="store_true")
    ap.add_argument("--no-machine", action="store_true",
                    help="skip the copy, read and MFMA calibration of the box and the decode "
                         "timings with the last-level cache flushed")
    ap.add_argument("--coder-only", action="store_true",
                    help="only the configs[4] Coder-shaped block; prints its own JSON line")
    ap.add_argument("--stack-only", action="store_true",
                    help="only the configs[3] layer stack; prints its own JSON line")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the configs[2] prefill point (for profilers); prints its own JSON line")
    ap.add_argument("--facade-only", action="store_true",
                    help="only the facade-op and expert-format points; prints its own JSON line")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only copy MIB MiB device to device 10 times (the byte counters' reference)")
    args = ap.parse_args(argv)
    if args.calibrate_copy:
        import torch
        src = torch.empty(args.calibrate_copy << 20, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"[bench] copied {args.calibrate_copy} MiB x 10", file=sys.stderr)
        return 0
    if args.gpus != 1:
        print("bench.py measures one GPU: the MoE block runs on a single MI355X in this build "
              "(expert-parallel sharding is designed but not implemented)",
              file=sys.stderr)
        return 2

    import torch
    from mrun_amd import moe as M
    from mrun_amd import synth

    Q = synth.QWEN36
    if args.prefill_only:
        print(json.dumps({"prefill": prefill_point(args, Q, M, synth, torch)}), flush=True)
        return 0
    if args.stack_only:
        print(json.dumps({"stack": stack_point(args, Q, M, synth, torch)}), flush=True)
        return 0
    if args.coder_only:
        print(json.dumps({"coder": coder_point(args, M, synth, torch)}), flush=True)
        return 0
    if args.facade_only:
        print(json.dumps({"facade": facade_point(args, Q, M, synth, torch),
                          "formats": formats_point(args, Q, M, synth, torch)}), flush=True)
        return 0
    print(f"[bench] generating the configs[1] block ({Q.name})", file=sys.stderr, flush=True)
    hb = synth.make_block(Q, config=synth.CFG_DECODE)
    dev = M.SparseMoe(hb)

    cold = None if args.no_machine else ColdTimer(torch)

    def decode_point(T, steps, warmup):
        x_np = synth.make_x(Q, T, config=synth.CFG_DECODE, layer=T)
        x = M.bf16_tensor(x_np)
        _, _, ids, _ = dev.router_forward(x)
        n_active = int(np.unique(M.u32_array(ids)).size)
        wall, dev_ms, _ = time_forward(dev, x, steps, warmup, torch)
        cold_ms = cold.time(dev, x, 30) if cold else None
        stages = time_stages(dev, x, 50, torch)
        try:
            g_ms, _ = time_graph(dev, x, steps, torch)
            g16_ms, _ = time_graph(dev, x, steps, torch, per_graph=16)
        except Exception as e:  # graph capture is reported, never required
            print(f"[bench] graph capture failed: {e}", file=sys.stderr)
            g_ms = g16_ms = None
        b = decode_bytes(Q, n_active, T)
        return {"tokens": T, "n_active": n_active, "ms_per_step": wall, "device_ms": dev_ms,
                "cold_device_ms": cold_ms, "graph_ms": g_ms, "graph16_ms": g16_ms,
                "tokens_per_s": T / (wall * 1e-3), "stages_us": stages, "bytes": b,
                "block_hbm_frac_warm": b["block"] / (dev_ms * 1e-3) / HBM_PEAK,
                "block_hbm_frac_cold": (b["block"] / (cold_ms * 1e-3) / HBM_PEAK
                                        if cold_ms else None)}, x_np

    print(f"[bench] decode T={args.tokens}", file=sys.stderr, flush=True)
    main_pt, x_main = decode_point(args.tokens, args.steps, args.warmup)
    gu_stage_us = main_pt["stages_us"]["gate_up"]
    gu_us = time_gateup_kernel(dev, M.bf16_tensor(x_main), 100, torch)
    gu_us_cold = (time_gateup_kernel(dev, M.bf16_tensor(x_main), 30, torch, cold=cold)
                  if cold else None)
    gbytes = main_pt["bytes"]["gate_up"]
    achieved = gbytes / (gu_us * 1e-6)
    kname = "decode_gateup_kernel"
    roofline = {"kernel": f"{kname} (routed + shared gate/up, SwiGLU fused)", "bound": "hbm",
                "achieved": achieved / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                "frac": achieved / HBM_PEAK, "traffic": measured_traffic(kname),
                "cache": "frac is warm: the repeated forward keeps the 17 MB block in the 256 MB "
                         "last-level cache; frac_cold: that cache flushed (a 1 GiB read) before "
                         "every forward, outside the kernel's events",
                "achieved_cold": gbytes / (gu_us_cold * 1e-6) / 1e9 if gu_us_cold else None,
                "frac_cold": gbytes / (gu_us_cold * 1e-6) / HBM_PEAK if gu_us_cold else None,
                "bytes_per_launch": gbytes, "us_per_launch": gu_us,
                "us_per_launch_cold": gu_us_cold, "us_per_launch_with_gap": gu_stage_us,
                "timing": "the kernel's own device wall-clock stamps (s_memrealtime) at its first "
                          "wave's start and last wave's end (mrun_moe_forward_timed), mean of 99 "
                          "forwards (29 cold); us_per_launch_with_gap: HIP events between launches"}

    sweep = []
    if not args.no_sweep:
        for T in (1, 2, 4, 16):
            if T == args.tokens:
                continue
            print(f"[bench] decode T={T}", file=sys.stderr, flush=True)
            p, _ = decode_point(T, max(args.steps // 2, 20), args.warmup)
            sweep.append(p)

    # mlx-community conversions store the router and the shared-expert gate in 8 bits (group 64):
    # the same block with those two quantized, decode T = 1 and 16
    gates8 = None
    if not args.no_sweep:
        print("[bench] decode with an 8-bit router and shared gate", file=sys.stderr, flush=True)
        h8 = synth.make_block(Q, config=synth.CFG_DECODE, gate_bits=8)
        d8 = M.SparseMoe(h8)
        gates8 = {"weights": "router and shared-expert gate 8-bit affine, group 64; experts as "
                             "configs[1]"}
        for T in (1, 16):
            x8 = M.bf16_tensor(synth.make_x(Q, T, config=synth.CFG_DECODE, layer=T))
            wall, dev_ms, _ = time_forward(d8, x8, max(args.steps // 2, 20), args.warmup, torch)
            gates8[f"T{T}"] = {"tokens": T, "device_ms": dev_ms, "ms_per_step": wall,
                               "tokens_per_s": T / (wall * 1e-3)}
        del d8, h8

    # between the decode sizes and the prefill chunk: block time by batch size on the configs[1]
    # block (unbiased router); the decode kernels take up to 32 tokens (256 pairs)
    batches = None
    if not args.no_sweep:
        print("[bench] batch sizes 17 to 1024", file=sys.stderr, flush=True)
        batches = []
        for T in (17, 24, 32, 33, 64, 128, 256, 512, 1024):
            xb = M.bf16_tensor(synth.make_x(Q, T, config=synth.CFG_DECODE, layer=T))
            wall, dev_ms, _ = time_forward(dev, xb, 50, 10, torch)
            batches.append({"tokens": T, "device_ms": dev_ms, "ms_per_step": wall,
                            "tokens_per_s": T / (wall * 1e-3),
                            "schedule": "decode" if T <= 32 else "prefill"})
            del xb

    prefill = None if args.no_prefill else prefill_point(args, Q, M, synth, torch)
    facade = None if args.no_prefill else facade_point(args, Q, M, synth, torch)
    formats = None if args.no_sweep else formats_point(args, Q, M, synth, torch)
    stack = None if args.no_stack else stack_point(args, Q, M, synth, torch)
    coder = None if args.no_coder else coder_point(args, M, synth, torch, cold)

    machine = None
    if not args.no_machine:
        print("[bench] copy and MFMA calibration", file=sys.stderr, flush=True)
        machine = machine_point(torch)
        machine["launch_floor"] = launch_floor(torch)

    cpu = None
    if not args.no_cpu:
        print("[bench] CPU restatement baseline", file=sys.stderr, flush=True)
        cpu = cpu_baseline(args, Q, synth, hb, x_main)

    line = {
        "metric": "MoE block tokens/s + % HBM/MFMA roofline, decode T=1..16, prefill T=2048",
        "value": main_pt["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": main_pt["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"configs[1]: Qwen3.6-35B-A3B-like MoE block, decode T={args.tokens}",
                   "hidden": Q.hidden, "experts": Q.experts, "top_k": Q.top_k,
                   "intermediate": Q.intermediate, "shared": Q.shared,
                   "weights": "4-bit affine, group 64, bf16 scales/biases",
                   "tokens": args.tokens},
        "us_per_layer": main_pt["device_ms"] * 1e3,
        "cold_us_per_layer": (main_pt["cold_device_ms"] * 1e3 if main_pt["cold_device_ms"]
                              else None),
        "graph_us_per_layer": main_pt["graph_ms"] * 1e3 if main_pt["graph_ms"] else None,
        "graph16_us_per_layer": main_pt["graph16_ms"] * 1e3 if main_pt["graph16_ms"] else None,
        "block_hbm_frac_warm": main_pt["block_hbm_frac_warm"],
        "block_hbm_frac_cold": main_pt["block_hbm_frac_cold"],
        "stages_us": main_pt["stages_us"],
        "roofline": roofline,
        "cpu_baseline": cpu,
        "machine": machine,
        "sweep": sweep,
        "gates8": gates8,
        "batches": batches,
        "prefill": prefill,
        "facade": facade,
        "formats": formats,
        "stack": stack,
        "coder": coder,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
