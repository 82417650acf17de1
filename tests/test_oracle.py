"""Pins the CPU restatement (oracle/) before it is trusted as the parity oracle.

Each oracle function is checked against what fixes it independently of its own code: the known
answers of the reference's unit tests (crates/mrun-engine/src/tensor/nuvec.rs:1173-1204,
1293-1319, 1331-1357; models/activations.rs:92-123), a library routine (torch's bf16 conversion,
scipy's softmax, numpy's stable argsort, torch's rms_norm), brute force, or the independent numpy
restatement in tests/np_reference.py. No GPU.
"""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch
from scipy.special import softmax as sp_softmax

from mrun_amd import synth
from mrun_amd.synth import bf16_to_f32, f32_to_bf16
from oracle import oracle as O
from tests import np_reference as NP
from tests.helpers import assert_close, beyond_rounding, ulp_distance


def qt(codes, scales, biases, experts, out, in_, group, bits=4):
    return SimpleNamespace(codes=np.asarray(codes, np.uint32).reshape(experts, out, -1),
                           scales=np.asarray(scales, np.uint16).reshape(experts, out, -1),
                           biases=None if biases is None else
                           np.asarray(biases, np.uint16).reshape(experts, out, -1),
                           experts=experts, out=out, in_=in_, group=group, bits=bits)


# ---- bf16 rounding -------------------------------------------------------------------------

def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    v = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 200000),
        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 65519.0, 3.0e38, -3.0e38, 1e-40,
                  0.08838835, 1.0 / 3.0, np.inf, -np.inf], np.float32),
        # exact ties between two bf16 values, both parities of the kept bit
        (np.arange(1, 5000, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
    ])
    want = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.bf16_from_f32(v), want)
    assert np.array_equal(synth.f32_to_bf16(v), want)
    nan = O.bf16_from_f32(np.array([np.nan], np.float32))
    assert (nan[0] & 0x7F80) == 0x7F80 and (nan[0] & 0x7F) != 0


# ---- affine dequant and the quantized products (nuvec.rs:1173-1204, 1331-1357) -------------

def _nuvec_qmm_case(biases):
    # the reference's test data: 0x76543210 rotated left by 4i, scales [0.5, 0.25], biases
    # [-1.0, 0.5], x = i/64 (all exact in bf16)
    def rotl(v, r):
        r %= 32
        return ((v << r) | (v >> (32 - r))) & 0xFFFFFFFF if r else v

    words = np.array([rotl(0x76543210, 4 * i) for i in range(16)], np.uint32)
    sc = f32_to_bf16(np.array([0.5, 0.25], np.float32))
    bi = f32_to_bf16(np.array([-1.0, 0.5], np.float32)) if biases else None
    return qt(words, sc, bi, 1, 2, 64, 64), words


def test_quantized_matmul_matches_dequantized_known_answer():
    q, words = _nuvec_qmm_case(True)
    x = f32_to_bf16((np.arange(64) / 64.0).astype(np.float32)).reshape(1, 64)
    assert np.array_equal(bf16_to_f32(x), (np.arange(64) / 64.0).astype(np.float32).reshape(1, 64))
    y = O.qmatmul(q, x)
    dense = np.stack([O.dequant_row(q, 0, o) for o in range(2)])
    ref = bf16_to_f32(x).astype(np.float64) @ dense.T.astype(np.float64)
    # the reference compares in f32 within 1e-3; in bf16 the product is the rounded exact value
    assert np.array_equal(y, f32_to_bf16(ref.astype(np.float32))), (bf16_to_f32(y), ref)
    # without biases: code * scale, codes LSB first (nuvec.rs:1193-1203)
    plain, _ = _nuvec_qmm_case(False)
    row = O.dequant_row(plain, 0, 0)
    codes = np.array([(w >> (4 * i)) & 0xF for w in words[:8] for i in range(8)], np.float32)
    assert np.array_equal(row, codes * 0.5)
    # a most-significant-nibble-first reading would give 7, 6, 5, ... for the first word
    assert list(row[:8] / 0.5) == [0, 1, 2, 3, 4, 5, 6, 7]


@pytest.mark.parametrize("bits,code", [(4, 8), (8, 128)])
def test_gathered_product_picks_each_rows_expert(bits, code):
    """nuvec.rs:1331-1357: experts (e+1)*I (64 x 64); rows pick experts [2, 0]."""
    E, n = 3, 64
    per = 32 // bits
    q = np.zeros((E, n, n), np.uint32)
    for o in range(n):
        q[:, o, o] = code
    words = np.zeros((E, n, n // per), np.uint32)
    for i in range(per):
        words |= q[:, :, i::per].astype(np.uint32) << np.uint32(bits * i)
    sc = f32_to_bf16(np.array([(e + 1) / code for e in range(E) for _ in range(n)], np.float32))
    w = qt(words, sc, None, E, n, n, 64, bits)
    x = f32_to_bf16((np.arange(2 * n) % 7).astype(np.float32)).reshape(2, n)
    y = bf16_to_f32(O.gather_qmm(w, x, np.array([2, 0], np.uint32)))
    xs = bf16_to_f32(x)
    assert np.array_equal(y[0], 3 * xs[0]) and np.array_equal(y[1], xs[1])
    # broadcast form: one x row against both indices
    y2 = bf16_to_f32(O.gather_qmm(w, x[:1], np.array([2, 0], np.uint32)))
    assert np.array_equal(y2[0], 3 * xs[0]) and np.array_equal(y2[1], xs[0])


@pytest.mark.parametrize("group", [32, 64, 128])
def test_gather_qmm_matches_float64_dequant(group):
    rng = np.random.default_rng(group)
    E, out, in_, n = 5, 24, 256, 40
    codes = rng.integers(0, 2**32, (E, out, in_ // 8), dtype=np.uint64).astype(np.uint32)
    sc = f32_to_bf16(np.abs(rng.standard_normal((E, out, in_ // group))).astype(np.float32) * 0.01)
    bi = f32_to_bf16(rng.standard_normal((E, out, in_ // group)).astype(np.float32) * 0.05)
    w = qt(codes, sc, bi, E, out, in_, group)
    x = f32_to_bf16(rng.standard_normal((n, in_)).astype(np.float32))
    idx = rng.integers(0, E, n).astype(np.uint32)
    got = O.gather_qmm(w, x, idx)
    Wd = NP.dequant(w)
    ref = np.stack([Wd[idx[p]] @ NP.F(x[p]) for p in range(n)])
    assert beyond_rounding(got, f32_to_bf16(ref.astype(np.float32))) == 0
    # dequant rows equal the float64 closed form exactly (q*s is exact, +b rounds once in f32)
    for e, o in [(0, 0), (4, 23), (2, 11)]:
        assert np.array_equal(O.dequant_row(w, e, o), Wd[e, o].astype(np.float32))


def test_linear_two_roundings():
    rng = np.random.default_rng(4)
    w = f32_to_bf16(rng.standard_normal((16, 128)).astype(np.float32) * 0.1)
    b = f32_to_bf16(rng.standard_normal(16).astype(np.float32))
    x = f32_to_bf16(rng.standard_normal((9, 128)).astype(np.float32))
    plain = O.linear(w, x)
    ref = f32_to_bf16((NP.F(x) @ NP.F(w).T).astype(np.float32))
    assert beyond_rounding(plain, ref) == 0
    biased = O.linear(w, x, b)
    assert np.array_equal(biased, f32_to_bf16(bf16_to_f32(plain) + bf16_to_f32(b)[None]))


# ---- router --------------------------------------------------------------------------------

def test_softmax_known_answer_and_scipy():
    a = f32_to_bf16(np.array([[0.5, 1.0, 2.0]], np.float32))
    p = bf16_to_f32(O.softmax(a))
    assert abs(p.sum() - 1.0) < 1e-2  # nuvec.rs:1311-1319
    rng = np.random.default_rng(1)
    l = f32_to_bf16(rng.standard_normal((64, 256)).astype(np.float32) * 2)
    ref = f32_to_bf16(sp_softmax(bf16_to_f32(l).astype(np.float64), axis=1).astype(np.float32))
    assert ulp_distance(O.softmax(l), ref).max() <= 1


def test_topk_brute_force_with_ties():
    rng = np.random.default_rng(2)
    g = f32_to_bf16(rng.random((300, 64)).astype(np.float32) * 0.05)
    g[:, 10] = g[:, 20] = g[:, 30] = f32_to_bf16(np.array([0.2], np.float32))[0]  # forced ties
    for k in (1, 4, 8, 64):
        assert np.array_equal(O.topk(g, k), NP.topk_ids(g, k))


def test_scores_closed_form():
    rng = np.random.default_rng(3)
    g = f32_to_bf16(rng.random((50, 32)).astype(np.float32) / 32)
    ids = NP.topk_ids(g, 8)
    raw = np.take_along_axis(g, ids.astype(np.int64), axis=1)
    assert np.array_equal(O.scores(g, ids, False), raw)
    s = bf16_to_f32(raw)
    tot = f32_to_bf16(s.sum(axis=1, dtype=np.float32))
    want = f32_to_bf16(s / bf16_to_f32(tot)[:, None])
    assert np.array_equal(O.scores(g, ids, True), want)


def test_topk_valid_accepts_ties_only():
    g = f32_to_bf16(np.array([0.1, 0.3, 0.2, 0.2, 0.05], np.float32))
    lg = f32_to_bf16(np.array([0.0, 1.0, 0.5, 0.5, -1.0], np.float32))
    assert O.topk_valid(g, lg, np.array([1, 2], np.uint32), 0)
    assert O.topk_valid(g, lg, np.array([1, 3], np.uint32), 0)   # 2 and 3 tie
    assert not O.topk_valid(g, lg, np.array([1, 0], np.uint32), 1)
    assert not O.topk_valid(g, lg, np.array([1, 1], np.uint32), 1)


# ---- dispatch ------------------------------------------------------------------------------

def test_floor_divide_known_answers():
    assert list(O.floor_divide_u32(np.array([7, 8, 9], np.uint32), 4)) == [1, 2, 2]
    big = np.array([(1 << 23) + i * 8191 for i in range(64)], np.uint32)
    assert np.array_equal(O.floor_divide_u32(big, 8), big // 8)


@pytest.mark.parametrize("T,k,E", [(1, 8, 256), (7, 8, 256), (300, 8, 256), (2048, 8, 256),
                                   (100, 4, 16), (513, 2, 160)])
def test_permute_is_the_stable_argsort(T, k, E):
    rng = np.random.default_rng(T + k + E)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.uint32)
    flat = ids.ravel()
    order, inverse, token, counts = O.permute(ids, k, E)
    want = np.argsort(flat, kind="stable")
    assert np.array_equal(order, want)
    assert np.array_equal(inverse, np.argsort(want, kind="stable"))
    assert np.array_equal(order[inverse], np.arange(flat.size))
    assert np.array_equal(token, want // k)
    assert np.array_equal(counts, np.bincount(flat, minlength=E))
    # sorted by (expert, token): a token picks an expert once
    key = flat[order].astype(np.int64) * (T + 1) + token
    assert np.all(np.diff(key) > 0)


# ---- element-wise --------------------------------------------------------------------------

def test_swiglu_closed_form():
    g = np.array([-2.0, 0.0, 1.5], np.float32)
    x = np.array([1.0, 2.0, -3.0], np.float32)
    sig = lambda v: 1.0 / (1.0 + np.exp(-v))
    want = g * sig(g) * x  # activations.rs:92-123
    assert np.all(np.abs(O.swiglu_f32(g, x) - want) < 1e-5)
    rng = np.random.default_rng(5)
    gb = f32_to_bf16(rng.standard_normal(5000).astype(np.float32) * 4)
    ub = f32_to_bf16(rng.standard_normal(5000).astype(np.float32))
    ref = f32_to_bf16((NP.F(gb) * NP.sigmoid(NP.F(gb)) * NP.F(ub)).astype(np.float32))
    assert ulp_distance(O.swiglu(gb, ub), ref).max() <= 1


def test_combine_and_shared_gate():
    rng = np.random.default_rng(6)
    T, k, D = 6, 8, 64
    y = f32_to_bf16(rng.standard_normal((T * k, D)).astype(np.float32) * 0.02)
    s = f32_to_bf16(rng.random((T, k)).astype(np.float32) / k)
    routed = O.combine(y, s)
    prod = NP.R(NP.F(y).reshape(T, k, D) * NP.F(s)[:, :, None])
    want = f32_to_bf16(prod.sum(axis=1).astype(np.float32))
    assert np.array_equal(routed, want)
    gl = f32_to_bf16(rng.standard_normal(T).astype(np.float32))
    sy = f32_to_bf16(rng.standard_normal((T, D)).astype(np.float32) * 0.02)
    out, gate = O.shared_add(routed, gl, sy)
    sg = NP.R(NP.sigmoid(NP.F(gl)))
    assert ulp_distance(gate, f32_to_bf16(sg.astype(np.float32))).max() <= 1
    want2 = f32_to_bf16((NP.F(routed) + NP.R(NP.F(gate)[:, None] * NP.F(sy))).astype(np.float32))
    assert np.array_equal(out, want2)


def test_rms_norm_matches_torch():
    rng = np.random.default_rng(7)
    x = f32_to_bf16(rng.standard_normal((9, 2048)).astype(np.float32))
    w = f32_to_bf16((1 + 0.1 * rng.standard_normal(2048)).astype(np.float32))
    xt = torch.from_numpy(bf16_to_f32(x))
    n = torch.nn.functional.rms_norm(xt, (2048,), eps=1e-6)
    ref = f32_to_bf16(bf16_to_f32(f32_to_bf16(n.numpy())) * bf16_to_f32(w))
    assert ulp_distance(O.rms_norm(x, w, 1e-6), ref).max() <= 1
    ones = O.rms_norm(x, None, 1e-6)
    assert ulp_distance(ones, f32_to_bf16(n.numpy())).max() <= 1


# ---- the block -----------------------------------------------------------------------------

TINY = synth.Shape(hidden=64, experts=8, top_k=4, intermediate=32, shared=32, group=32)


@pytest.mark.parametrize("shape,T,zipf", [
    (TINY, 1, False), (TINY, 24, False), (TINY, 16, True),
    (synth.Shape(hidden=256, experts=16, top_k=4, intermediate=128, shared=0), 20, False),
    (synth.Shape(hidden=256, experts=32, top_k=8, intermediate=128, shared=128), 9, True),
])
def test_block_matches_numpy_restatement(shape, T, zipf):
    hb = synth.make_block(shape, config=7, zipf=zipf)
    x = synth.make_x(shape, T, config=7)
    out, tr = O.moe_forward(hb, x, trace=True)
    ref, rtr = NP.forward(hb, x, ids=tr["ids"])
    # the router agrees up to one-ulp rounding flips; ids are the top-k of the oracle's own gates
    assert beyond_rounding(tr["logits"], rtr["logits"]) == 0
    assert np.array_equal(tr["ids"], NP.topk_ids(tr["gates"], shape.top_k))
    own_ids = NP.topk_ids(rtr["gates"], shape.top_k)
    for t in range(T):
        if set(own_ids[t]) != set(tr["ids"][t]):
            assert O.topk_valid(tr["gates"][t], tr["logits"][t], own_ids[t], 1)
    s = assert_close(out, ref, l1_rel=2e-4, what="oracle vs numpy")
    assert s["max_abs"] < 2e-3, s


@pytest.mark.parametrize("shape,T,expert_bits,gate_bits", [
    (TINY, 24, 8, 0), (TINY, 3, 4, 8), (TINY, 17, 8, 8), (TINY, 12, 16, 0), (TINY, 20, 16, 8),
    (synth.Shape(hidden=256, experts=16, top_k=4, intermediate=128, shared=128, group=128),
     20, 8, 8),
])
def test_block_8bit_and_quantized_gates_match_numpy(shape, T, expert_bits, gate_bits):
    """8-bit experts (LSB-first bytes, nuvec.rs:1173-1204), dense bf16 experts (bits 16,
    SwitchLinear::Dense moe.rs:43-46) and 8-bit group-64 router and shared gate
    (Linear::Quantized, load.rs:294-306), as mlx-community checkpoints store them."""
    hb = synth.make_block(shape, config=11, expert_bits=expert_bits, gate_bits=gate_bits)
    x = synth.make_x(shape, T, config=11)
    out, tr = O.moe_forward(hb, x, trace=True)
    ref, rtr = NP.forward(hb, x, ids=tr["ids"])
    assert beyond_rounding(tr["logits"], rtr["logits"]) == 0
    s = assert_close(out, ref, l1_rel=2e-4, what="oracle vs numpy (8-bit)")
    assert s["max_abs"] < 2e-3, s


# ---- the f32 block (an f32 checkpoint: every op in f32, no bf16 rounding) -------------------

F32_TOL = 2e-6  # of the largest |output|: f32 accumulation over at most a few thousand terms


@pytest.mark.parametrize("shape,T", [
    (synth.Shape(hidden=64, experts=8, top_k=2, intermediate=32, shared=32), 7),
    (synth.Shape(hidden=64, experts=8, top_k=8, intermediate=32, shared=0, norm_topk=False), 5),
    (synth.Shape(hidden=256, experts=64, top_k=8, intermediate=128, shared=128), 12),
])
def test_block_f32_matches_float64_restatement(shape, T):
    """orc_moe_forward_f32 against tests/np_reference.forward_f32 (float64, no rounding): the
    same expert choice and outputs within f32 accumulation error."""
    fb = synth.make_block_f32(shape, config=21)
    x = synth.make_x_f32(shape, T, config=21)
    out, ids = O.moe_forward_f32(fb, x)
    ref, gates, rids = NP.forward_f32(fb, x)
    assert np.array_equal(ids, rids)
    assert np.max(np.abs(out - ref)) <= F32_TOL * np.max(np.abs(ref)), np.max(np.abs(out - ref))


def test_block_f32_closed_forms():
    """What the mathematics fixes without a restatement. A zero router gives every expert the
    same gate 1/E: the top-k is then experts 0..k-1 (equal gates by lower id), scores 1/E (1/k
    with norm). Zero down weights leave only the shared expert: sigmoid(g . x) * shared. A zero
    shared gate weighs the shared expert by sigmoid(0) = 1/2 exactly."""
    sh = synth.Shape(hidden=64, experts=8, top_k=3, intermediate=32, shared=32)
    x = synth.make_x_f32(sh, 4, config=22)
    for norm in (False, True):
        s = synth.Shape(hidden=64, experts=8, top_k=3, intermediate=32, shared=0, norm_topk=norm)
        fb = synth.make_block_f32(s, config=22)
        fb.router = np.zeros_like(fb.router)
        out, ids = O.moe_forward_f32(fb, x)
        assert np.array_equal(ids, np.tile(np.arange(3, dtype=np.uint32), (4, 1)))
        w = 1.0 / 3 if norm else 1.0 / 8
        X = x.astype(np.float64)
        want = np.zeros((4, 64))
        for e in range(3):
            g = X @ fb.gate_proj[e].T.astype(np.float64)
            u = X @ fb.up_proj[e].T.astype(np.float64)
            want += ((g / (1 + np.exp(-g)) * u) @ fb.down_proj[e].T.astype(np.float64)) * w
        assert np.max(np.abs(out - want)) <= F32_TOL * np.max(np.abs(want))
    fb = synth.make_block_f32(sh, config=22)
    fb.down_proj = np.zeros_like(fb.down_proj)
    fb.sh_expert_gate = np.zeros_like(fb.sh_expert_gate)
    out, _ = O.moe_forward_f32(fb, x)
    X = x.astype(np.float64)
    g, u = X @ fb.sh_gate_proj.T.astype(np.float64), X @ fb.sh_up_proj.T.astype(np.float64)
    want = 0.5 * ((g / (1 + np.exp(-g)) * u) @ fb.sh_down_proj.T.astype(np.float64))
    assert np.max(np.abs(out - want)) <= F32_TOL * np.max(np.abs(want))


def test_quantize_round_trip():
    """synth.quantize: every weight within half a step of its dequantised value."""
    w = synth.normal_bf16(synth.seed(1, 0, synth.ROUTER_W), 16 * 256, 0.02).reshape(16, 256)
    for bits in (4, 8):
        q = synth.quantize(w, bits, 64)
        d = NP.dequant(q)[0]
        step = np.repeat(bf16_to_f32(q.scales[0]).astype(np.float64), 64, axis=-1)
        assert np.all(np.abs(d - bf16_to_f32(w)) <= 0.5 * step + 1e-6)
        # LSB-first packing: the first code of a row is the low bits of its first word
        assert (q.codes[0, 0, 0] & ((1 << bits) - 1)) == np.rint(
            (bf16_to_f32(w[0, 0]) - bf16_to_f32(q.biases[0, 0, 0])) / bf16_to_f32(q.scales[0, 0, 0]))


def test_sorted_and_unsorted_dispatch_agree():
    """The oracle's sorted path (T*k >= 64, moe.rs:63-75) gives each row its unsorted bits."""
    hb = synth.make_block(TINY, config=8)
    x = synth.make_x(TINY, 16, config=8)   # 64 pairs: sorted
    full = O.moe_forward(hb, x)
    for t in range(16):                    # 4 pairs: unsorted
        assert np.array_equal(O.moe_forward(hb, x[t:t + 1])[0], full[t])


def test_forced_ids_must_be_a_topk():
    hb = synth.make_block(TINY, config=9)
    x = synth.make_x(TINY, 3, config=9)
    _, tr = O.moe_forward(hb, x, trace=True)
    bad = tr["ids"].copy()
    g = NP.F(tr["gates"][0])
    bad[0, 0] = int(np.argmin(g))  # the smallest gate is never in a top-4 of 8 unless tied
    if g[bad[0, 0]] < np.sort(g)[-4]:
        with pytest.raises(ValueError):
            O.moe_forward(hb, x, forced_ids=bad)


def test_stack_is_norm_block_residual():
    blocks = [synth.make_block(TINY, config=3, layer=l) for l in range(3)]
    x = synth.make_x(TINY, 5, config=3)
    got = O.moe_stack(blocks, x, None, 1e-6)
    h = x.copy()
    for hb in blocks:
        n = O.rms_norm(h, None, 1e-6)
        h = f32_to_bf16(bf16_to_f32(h) + bf16_to_f32(O.moe_forward(hb, n)))
    assert np.array_equal(got, h)
