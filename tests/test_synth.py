"""The seeded generator (include/mrun_synth.h) against a numpy restatement of its spec, and the
distributions the benchmark configurations ask for. No GPU."""
from __future__ import annotations

import numpy as np

from mrun_amd import synth

M64 = np.uint64(0xFFFFFFFFFFFFFFFF)
GAMMA = np.uint64(0x9E3779B97F4A7C15)


def mix64(z: np.ndarray) -> np.ndarray:
    z = z.astype(np.uint64)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def draws(seed: int, n: int) -> np.ndarray:
    with np.errstate(over="ignore"):
        return mix64(np.uint64(seed) + (np.arange(n, dtype=np.uint64) + np.uint64(1)) * GAMMA)


def test_splitmix_reference_values():
    # SplitMix64 from state 0: its first outputs are published with the algorithm
    s = 0
    assert int(synth.lib().mrun_synth_draw(s, 0)) == 0xE220A8397B1DCDAF
    assert int(synth.lib().mrun_synth_draw(s, 1)) == 0x6E789E6AA1B965F4
    assert int(draws(0, 2)[1]) == 0x6E789E6AA1B965F4


def test_codes_follow_the_spec():
    s = synth.seed(1, 2, synth.GATE_CODES)
    got = synth.codes(s, 1000)
    d = draws(s, 8000).reshape(1000, 8) >> np.uint64(60)
    want = np.zeros(1000, np.uint64)
    for j in range(8):
        want |= d[:, j] << np.uint64(4 * j)
    assert np.array_equal(got, want.astype(np.uint32))
    got8 = synth.codes(s, 100, bits=8)
    d8 = draws(s, 400).reshape(100, 4) >> np.uint64(56)
    want8 = sum(d8[:, j] << np.uint64(8 * j) for j in range(4)).astype(np.uint32)
    assert np.array_equal(got8, want8)


def test_normals_follow_box_muller():
    s = synth.seed(0, 0, synth.X)
    d = draws(s, 2000)
    u = (d >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    r = np.sqrt(-2.0 * np.log(1.0 - u[0::2]))
    th = 2 * np.pi * u[1::2]
    n = np.empty(2000)
    n[0::2], n[1::2] = r * np.cos(th), r * np.sin(th)
    got = np.array([synth.lib().mrun_synth_normal(s, i) for i in range(2000)])
    assert np.max(np.abs(got - n)) < 1e-12
    b = synth.normal_bf16(s, 2000, 1.0)
    assert np.array_equal(b, synth.f32_to_bf16(n.astype(np.float32)))


def test_distributions():
    s = synth.seed(1, 0, synth.GATE_SCALES)
    sc, bi = synth.scales_biases(s, 200000)
    scf = synth.bf16_to_f32(sc).astype(np.float64)
    assert np.all(scf >= 0)
    assert abs(scf.mean() - 0.02 * np.sqrt(2 / np.pi) / 7.5) < 2e-5  # E|N(0, .02)| / 7.5
    assert np.array_equal(synth.bf16_to_f32(bi), -8 * synth.bf16_to_f32(sc))  # exact
    c = synth.codes(synth.seed(1, 0, synth.UP_CODES), 100000)
    nib = ((c[:, None] >> (4 * np.arange(8, dtype=np.uint32))) & 15).ravel()
    h = np.bincount(nib, minlength=16)
    assert h.min() > 0.95 * h.mean() and h.max() < 1.05 * h.mean()
    x = synth.bf16_to_f32(synth.make_x(synth.QWEN36, 64)).astype(np.float64)
    assert abs(x.mean()) < 0.02 and abs(x.std() - 1) < 0.02


def test_zipf_bias_is_a_permuted_power_law():
    b, rank = synth.zipf_bias(synth.seed(2, 0, synth.ROUTER_BIAS), 256)
    assert sorted(rank.tolist()) == list(range(1, 257))
    want = synth.f32_to_bf16((2.0 * rank.astype(np.float64) ** -1.1).astype(np.float32))
    assert np.array_equal(b, want)


def test_block_sizes_and_determinism():
    a = synth.make_block(synth.Shape(hidden=256, experts=8, top_k=2, intermediate=64, shared=64))
    b = synth.make_block(synth.Shape(hidden=256, experts=8, top_k=2, intermediate=64, shared=64))
    assert np.array_equal(a.gate_proj.codes, b.gate_proj.codes)
    assert not np.array_equal(a.gate_proj.codes, a.up_proj.codes)
    assert a.gate_proj.codes.shape == (8, 64, 32) and a.down_proj.codes.shape == (8, 256, 8)
    assert a.gate_proj.scales.shape == (8, 64, 4)
    # Qwen3.6-like block: 455,806,976 bytes of routed+shared expert weights and the router
    q = synth.QWEN36
    per_proj = q.intermediate * q.hidden // 2 + 4 * q.intermediate * q.hidden // 64
    assert per_proj == 589824
