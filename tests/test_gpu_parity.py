"""Parity of the HIP path (through the C ABI) with the CPU restatement on identical seeded inputs.

Bars (the north star's): top-k ids and permutation indices bit-exact except where the router's
bf16 values tie (within one ulp of the k-th boundary logit); block outputs within max-abs 2e-2 and
L1-relative 1e-3 of the bf16 restatement, with f32 accumulation. Block outputs are compared with
the oracle run on the GPU's own expert choice (validated as a top-k within ties first), so a tie
broken the other way does not count as a numeric error.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from mrun_amd import moe as M
from mrun_amd import synth
from oracle import oracle as O
from tests.helpers import assert_close, beyond_rounding, bf16_ulp, stats, ulp_distance

pytestmark = pytest.mark.gpu

SMALL = synth.Shape(hidden=256, experts=16, top_k=4, intermediate=128, shared=128)
Q = synth.QWEN36
# configs[3] deep layers: the largest share of a layer's elements that may differ from the oracle
# by more than the north star's 2e-2 (each of them still within two bf16 ulps of its largest term)
STACK_WIDE_SHARE = 1e-2


def _log(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def q_host():
    return synth.make_block(Q, config=synth.CFG_DECODE)


@pytest.fixture(scope="module")
def q_dev(q_host):
    return M.SparseMoe(q_host)


@pytest.fixture(scope="module")
def small_host():
    return synth.make_block(SMALL, config=synth.CFG_PLUMBING)


@pytest.fixture(scope="module")
def small_dev(small_host):
    return M.SparseMoe(small_host)


def run_block(hb, dev, x_np, label, check_rows=None):
    """GPU forward vs oracle forward on the GPU's expert ids; returns (stats, tie-broken tokens)."""
    T, k = x_np.shape[0], hb.shape.top_k
    x = M.bf16_tensor(x_np)
    out = dev.forward(x)
    _, _, ids, _ = dev.router_forward(x)
    torch.cuda.synchronize()
    got = M.bf16_bits(out)
    gids = M.u32_array(ids).reshape(T, k)
    rows = np.arange(T) if check_rows is None else np.asarray(check_rows)
    ref, tr = O.moe_forward(hb, x_np[rows], forced_ids=gids[rows], trace=True)
    own = O.topk(tr["gates"], k)
    ties = int(sum(set(a) != set(b) for a, b in zip(own.tolist(), gids[rows].tolist())))
    s = assert_close(got[rows], ref, what=label)
    _log(f"{label}: {s} tie-broken tokens {ties}/{len(rows)}")
    return s, ties


# ---------------------------------------------------------------------------------------------
# router

@pytest.mark.parametrize("T", [1, 2, 4, 16, 64, 2048])
def test_router_matches_oracle(q_host, q_dev, T):
    x_np = synth.make_x(Q, T, config=synth.CFG_DECODE, layer=T)
    x = M.bf16_tensor(x_np)
    logits, gates, ids, scores = q_dev.router_forward(x)
    torch.cuda.synchronize()
    lg, gg = M.bf16_bits(logits), M.bf16_bits(gates)
    gi, gs = M.u32_array(ids).reshape(T, -1), M.bf16_bits(scores)
    # logits: f32 accumulation in another order, so a rare one-ulp difference
    ref_l = O.linear(q_host.router, x_np)
    ul = ulp_distance(lg, ref_l)
    assert beyond_rounding(lg, ref_l) == 0, f"logits differ by up to {ul.max()} ulps"
    # the rest is checked on the GPU's own logits: softmax within one ulp (exp and sum order),
    # ids exactly the top-k of the GPU's gates under the tie rule, scores bit-exact from them
    ref_g = O.softmax(lg)
    ug = ulp_distance(gg, ref_g)
    assert ug.max() <= 1, f"gates differ by {ug.max()} ulps"
    assert np.array_equal(gi, O.topk(gg, Q.top_k)), "ids are not the top-k of the gates"
    assert np.array_equal(gs, O.scores(gg, gi, Q.norm_topk)), "scores differ"
    # and against the oracle's own chain: ids equal except within-ulp ties
    ref_gates_own = O.softmax(ref_l)
    own = O.topk(ref_gates_own, Q.top_k)
    diff = 0
    for t in range(T):
        if set(own[t]) != set(gi[t]):
            diff += 1
            assert O.topk_valid(ref_gates_own[t], ref_l[t], gi[t], ulps=1), f"token {t}"
    _log(f"router T={T}: logits 1-ulp share {np.mean(ul > 0):.2e}, gates 1-ulp share "
         f"{np.mean(ug > 0):.2e}, id sets differing within ties {diff}/{T}")


# ---------------------------------------------------------------------------------------------
# permute

@pytest.mark.parametrize("T,k,E", [(1, 8, 256), (8, 8, 256), (16, 8, 256), (2048, 8, 256),
                                   (8192, 8, 160), (20, 4, 16), (3000, 2, 512)])
def test_permute_matches_oracle(T, k, E):
    rng = np.random.default_rng(T * 131 + k * 7 + E)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.uint32)
    dids = M.u32_tensor(ids)
    offsets, order, inverse, token = M.permute(dids, k, E)
    torch.cuda.synchronize()
    r_order, r_inverse, r_token, r_counts = O.permute(ids, k, E)
    assert np.array_equal(M.u32_array(order), r_order)
    assert np.array_equal(M.u32_array(inverse), r_inverse)
    assert np.array_equal(M.u32_array(token), r_token)
    off = M.u32_array(offsets)
    assert off[0] == 0 and np.array_equal(np.diff(off), r_counts)


# ---------------------------------------------------------------------------------------------
# products

@pytest.mark.parametrize("n,x_rows,sorted_", [(8, 1, False), (16, 2, False), (64, 64, True),
                                              (600, 600, False), (1024, 128, False)])
def test_gather_qmm_matches_oracle(q_host, q_dev, n, x_rows, sorted_):
    rng = np.random.default_rng(n + x_rows)
    idx = rng.integers(0, Q.experts, n).astype(np.uint32)
    if sorted_:
        idx.sort()
    x_np = synth.make_x(Q, x_rows, config=synth.CFG_DECODE, layer=1000 + n)
    got = M.bf16_bits(M.gather_qmm(M.bf16_tensor(x_np), q_dev.gate_proj, M.u32_tensor(idx),
                                   sorted_))
    torch.cuda.synchronize()
    ref = O.gather_qmm(q_host.gate_proj, x_np, idx)
    s = assert_close(got, ref, max_ulp=1, what=f"gather_qmm n={n}")
    _log(f"gather_qmm n={n} x_rows={x_rows}: {s}")


@pytest.mark.parametrize("rows", [1, 7, 16, 300])
def test_quantized_matmul_matches_oracle(q_host, q_dev, rows):
    x_np = synth.make_x(Q, rows, config=synth.CFG_DECODE, layer=2000 + rows)
    got = M.bf16_bits(M.quantized_matmul(M.bf16_tensor(x_np), q_dev.sh_gate_proj))
    ref = O.qmatmul(q_host.sh_gate_proj, x_np)
    s = assert_close(got, ref, max_ulp=1, what=f"quantized_matmul rows={rows}")
    # down-shaped (K = 512)
    a_np = synth.make_x(synth.Shape(512, 1, 1, 512), rows, config=9, layer=rows)
    got2 = M.bf16_bits(M.quantized_matmul(M.bf16_tensor(a_np), q_dev.sh_down_proj))
    ref2 = O.qmatmul(q_host.sh_down_proj, a_np)
    s2 = assert_close(got2, ref2, max_ulp=1, what=f"quantized_matmul down rows={rows}")
    _log(f"quantized_matmul rows={rows}: {s} / down {s2}")


@pytest.mark.parametrize("rows", [3, 100])
def test_linear_with_bias(rows):
    zb, _ = synth.zipf_bias(5, 256)
    w = synth.normal_bf16(11, 256 * 2048, 0.02).reshape(256, 2048)
    x_np = synth.normal_bf16(12, rows * 2048, 1.0).reshape(rows, 2048)
    got = M.bf16_bits(M.linear(M.bf16_tensor(x_np), M.bf16_tensor(w), M.bf16_tensor(zb)))
    plain = M.bf16_bits(M.linear(M.bf16_tensor(x_np), M.bf16_tensor(w)))
    # x W^T rounded once: within accumulation-order rounding of the oracle's
    assert beyond_rounding(plain, O.linear(w, x_np)) == 0
    # then the bias add, its own rounding (load.rs:302-305): bit-exact from the GPU's x W^T
    want = synth.f32_to_bf16(synth.bf16_to_f32(plain) + synth.bf16_to_f32(zb)[None, :])
    assert np.array_equal(got, want)


def test_swiglu_combine_norm():
    rng = np.random.default_rng(3)
    g = synth.f32_to_bf16(rng.standard_normal(4096 + 5).astype(np.float32) * 3)
    u = synth.f32_to_bf16(rng.standard_normal(4096 + 5).astype(np.float32))
    got = M.bf16_bits(M.swiglu(M.bf16_tensor(g), M.bf16_tensor(u)))
    assert ulp_distance(got, O.swiglu(g, u)).max() <= 1
    T, k, D = 5, 8, 2048
    y = synth.f32_to_bf16(rng.standard_normal((T * k, D)).astype(np.float32) * 0.02)
    sc = synth.f32_to_bf16(rng.random((T, k)).astype(np.float32) / k)
    sy = synth.f32_to_bf16(rng.standard_normal((T, D)).astype(np.float32) * 0.02)
    gl = synth.f32_to_bf16(rng.standard_normal(T).astype(np.float32))
    routed = O.combine(y, sc)
    ref, _ = O.shared_add(routed, gl, sy)
    got = M.bf16_bits(M.combine(M.bf16_tensor(y), M.bf16_tensor(sc), None, M.bf16_tensor(sy),
                                M.bf16_tensor(gl)))
    assert ulp_distance(got, ref).max() <= 1
    got_r = M.bf16_bits(M.combine(M.bf16_tensor(y), M.bf16_tensor(sc)))
    assert ulp_distance(got_r, routed).max() <= 1
    x = synth.f32_to_bf16(rng.standard_normal((7, D)).astype(np.float32))
    r = synth.f32_to_bf16(rng.standard_normal((7, D)).astype(np.float32))
    w = synth.f32_to_bf16((1 + 0.1 * rng.standard_normal(D)).astype(np.float32))
    got_n = M.bf16_bits(M.rms_norm(M.bf16_tensor(x), M.bf16_tensor(w), 1e-6))
    assert ulp_distance(got_n, O.rms_norm(x, w, 1e-6)).max() <= 1
    h, yv = M.add_rms_norm(M.bf16_tensor(x), M.bf16_tensor(r), M.bf16_tensor(w), 1e-6)
    hs = synth.f32_to_bf16(synth.bf16_to_f32(x) + synth.bf16_to_f32(r))
    assert np.array_equal(M.bf16_bits(h), hs)
    assert ulp_distance(M.bf16_bits(yv), O.rms_norm(hs, w, 1e-6)).max() <= 1


# ---------------------------------------------------------------------------------------------
# the block

# T = 3, 5, 9 and 13: the down launch's token groups of unequal size (two groups below T = 8,
# four from T = 8)
@pytest.mark.parametrize("T", [1, 2, 3, 4, 5, 9, 13, 16])
def test_block_decode_matches_oracle(q_host, q_dev, T):
    x_np = synth.make_x(Q, T, config=synth.CFG_DECODE, layer=T)
    run_block(q_host, q_dev, x_np, f"Q decode T={T}")


@pytest.mark.parametrize("T", [1, 3, 20, 100])
def test_block_small_shape(small_host, small_dev, T):
    x_np = synth.make_x(SMALL, T, config=synth.CFG_PLUMBING, layer=T)
    run_block(small_host, small_dev, x_np, f"small T={T}")


def test_block_plumbing_config(q_host, q_dev):
    """T = 16, 128 pairs (the sorted dispatch of the reference)."""
    x_np = synth.make_x(Q, 16, config=synth.CFG_PLUMBING)
    run_block(q_host, q_dev, x_np, "Q configs[0] T=16")


@pytest.mark.parametrize("T", [17, 33, 64, 300])
def test_block_prefill_small(q_host, q_dev, T):
    x_np = synth.make_x(Q, T, config=synth.CFG_PREFILL_ZIPF, layer=T)
    run_block(q_host, q_dev, x_np, f"Q prefill T={T}")


def test_block_prefill_zipf_2048():
    """T = 2048 with the Zipf-biased router; hot expert load >= 10x the mean."""
    hb = synth.make_block(Q, config=synth.CFG_PREFILL_ZIPF, zipf=True)
    dev = M.SparseMoe(hb)
    x_np = synth.make_x(Q, 2048, config=synth.CFG_PREFILL_ZIPF)
    _, _, ids, _ = dev.router_forward(M.bf16_tensor(x_np))
    counts = np.bincount(M.u32_array(ids).ravel(), minlength=Q.experts)
    assert counts.max() >= 10 * counts.mean(), counts.max()
    rows = np.random.default_rng(0).choice(2048, 256, replace=False)
    run_block(hb, dev, x_np, "Q configs[2] T=2048 (256 sampled rows)", check_rows=np.sort(rows))
    _log(f"zipf: hottest expert {counts.max()} pairs = {counts.max() / counts.mean():.1f}x mean")


@pytest.fixture(scope="module")
def zipf_block():
    hb = synth.make_block(Q, config=synth.CFG_PREFILL_ZIPF, zipf=True)
    return hb, M.SparseMoe(hb)


@pytest.mark.parametrize("T", [1, 4, 24, 300])
def test_block_router_bias(zipf_block, T):
    """The configs[2] block (a router bias from the Zipf ranking, so hot experts take many of a
    batch's pairs) at decode sizes, where the router launch adds the bias (T = 24: one decode batch,
    the hottest experts with several pairs each), and at T = 300 on 32-row tiles."""
    hb, dev = zipf_block
    run_block(hb, dev, synth.make_x(Q, T, config=synth.CFG_PREFILL_ZIPF, layer=500 + T),
              f"router bias T={T}")


def test_block_prefill_4096():
    """configs[3]'s prefill chunk, T = 4096 (experts average 128 rows; the shared expert rides in the
    expert launches)."""
    hb = synth.make_block(Q, config=synth.CFG_STACK, layer=0)
    dev = M.SparseMoe(hb)
    x_np = synth.make_x(Q, 4096, config=synth.CFG_STACK, layer=4096)
    rows = np.random.default_rng(1).choice(4096, 192, replace=False)
    run_block(hb, dev, x_np, "Q T=4096 (192 sampled rows)", check_rows=np.sort(rows))


def test_rows_keep_their_one_row_bits(q_dev):
    """A decode batch of up to 32 rows (256 pairs: T = 24 and 32 fill the third and fourth words
    of the kernels' pair sets) gives every row the bits of its one-row product (with_row_exact,
    nuvec.rs:256-265; lanes.rs:68-112)."""
    x_np = synth.make_x(Q, 32, config=synth.CFG_DECODE, layer=77)
    batch = M.bf16_bits(q_dev.forward(M.bf16_tensor(x_np)))
    for T in (8, 16, 17, 24):
        b = M.bf16_bits(q_dev.forward(M.bf16_tensor(x_np[:T])))
        assert np.array_equal(b, batch[:T]), f"T={T}"
    for t in list(range(16)) + [16, 23, 31]:
        one = M.bf16_bits(q_dev.forward(M.bf16_tensor(x_np[t:t + 1])))
        assert np.array_equal(one[0], batch[t]), f"row {t}"


def test_prefill_rows_keep_their_bits(q_dev):
    """On the prefill schedule (T >= 33) a token's output has the same bits whatever batch it is in
    and whichever tile class the grouped GEMM runs: T = 897 (7,176 pairs, 64-row tiles) against its
    first 896 rows (7,168 = 28 E pairs, the last size on 32-row tiles), 300 and 33 rows. Every row's
    sums run in one order (K steps in sequence, the bias term per 8 of them), whatever tile holds
    the row."""
    x_np = synth.make_x(Q, 897, config=synth.CFG_DECODE, layer=897)
    full = M.bf16_bits(q_dev.forward(M.bf16_tensor(x_np)))
    for T in (896, 300, 33):
        b = M.bf16_bits(q_dev.forward(M.bf16_tensor(x_np[:T])))
        assert np.array_equal(b, full[:T]), f"T={T}"


def test_empty_batch(q_dev):
    """T = 0: the block, the router and the stack return empty results and enqueue nothing."""
    x = torch.empty(0, Q.hidden, dtype=torch.bfloat16, device="cuda")
    out = q_dev.forward(x)
    logits, gates, ids, scores = q_dev.router_forward(x)
    st = M.MoeStack([q_dev, q_dev], None, 1e-6)
    st.forward_(x)
    torch.cuda.synchronize()
    assert tuple(out.shape) == (0, Q.hidden)
    assert tuple(ids.shape) == (0, Q.top_k) and tuple(logits.shape) == (0, Q.experts)


def test_timed_forward_matches_forward(q_dev):
    """mrun_moe_forward_timed (the benchmark's kernel-timed forward) gives the plain forward's bits,
    and its wall-clock stamps bracket the decode gate/up kernel: a positive duration, below the
    span of HIP events around the whole forward."""
    import bench
    from mrun_amd import _lib

    lib = _lib.load()
    hz = lib.mrun_wall_clock_hz()
    assert hz > 0
    x = M.bf16_tensor(synth.make_x(Q, 1, config=synth.CFG_DECODE, layer=11))
    ref = M.bf16_bits(q_dev.forward(x))
    out = torch.empty_like(x)
    ws = q_dev.workspace(1)
    clock = torch.zeros(64, 2, dtype=torch.int64, device="cuda")
    clock[:, 0] = -1  # 64 pairs (UINT64_MAX, 0)
    ev = bench.Events(2)
    stream = torch.cuda.current_stream()
    ev.record(0, stream)
    _lib.check(lib.mrun_moe_forward_timed(
        ctypes.byref(q_dev.c), ctypes.c_void_p(x.data_ptr()), 1, ctypes.c_void_p(out.data_ptr()),
        ctypes.c_void_p(ws.data_ptr()), ws.numel(), ctypes.c_void_p(stream.cuda_stream),
        ctypes.c_void_p(clock.data_ptr())))
    ev.record(1, stream)
    torch.cuda.synchronize()
    assert np.array_equal(M.bf16_bits(out), ref)
    c = clock.cpu().numpy().view(np.uint64)
    kernel_ms = float(c[:, 1].max() - c[:, 0].min()) / hz * 1e3
    assert 0.0 < kernel_ms < ev.ms(0, 1) < 1.0, (kernel_ms, ev.ms(0, 1))


def test_forward_is_deterministic(q_dev):
    x = M.bf16_tensor(synth.make_x(Q, 512, config=synth.CFG_DECODE, layer=5))
    a = M.bf16_bits(q_dev.forward(x))
    b = M.bf16_bits(q_dev.forward(x))
    assert np.array_equal(a, b)


@pytest.mark.parametrize("T", [1, 3, 8, 16, 24])
def test_block_coder_decode(T):
    """configs[4] at decode: hidden 6144, 160 experts, FFN 2560, no shared expert (the streaming
    gate/up and down kernels; T = 3 leaves waves of the down kernel with fewer pairs than others;
    T = 24 is one decode batch of 192 pairs). Against the oracle, and every row equal to its
    one-row forward."""
    hb = _coder_host()
    dev = _coder_dev()
    x_np = synth.make_x(synth.CODER, T, config=synth.CFG_CODER, layer=T)
    run_block(hb, dev, x_np, f"Coder decode T={T}")
    if T > 1:
        batch = M.bf16_bits(dev.forward(M.bf16_tensor(x_np)))
        for t in range(T):
            one = M.bf16_bits(dev.forward(M.bf16_tensor(x_np[t:t + 1])))
            assert np.array_equal(one[0], batch[t]), f"row {t}"


@pytest.mark.parametrize("T", [300, 1024])
def test_block_coder_prefill_rows(T):
    """configs[4] at prefill sizes: T = 300 (15 rows per expert on average) on the grouped GEMM's
    32-row tiles, T = 1024 on its 64-row tiles."""
    hb = _coder_host()
    dev = _coder_dev()
    x_np = synth.make_x(synth.CODER, T, config=synth.CFG_CODER, layer=T)
    rows = np.random.default_rng(1).choice(T, 32, replace=False)
    run_block(hb, dev, x_np, f"Coder prefill T={T} (32 sampled rows)", check_rows=np.sort(rows))


WIDE_SHARED = synth.Shape(hidden=4096, experts=64, top_k=8, intermediate=1024, shared=1024)


def test_wide_rows_with_shared_expert_prefill():
    """The same block at T = 40 (five rows per expert on average): the grouped GEMM's 32-row tiles,
    with the shared expert's rows as tiles of 32 in the same launches. Against the oracle."""
    if "wide" not in _CODER:
        hb = synth.make_block(WIDE_SHARED, config=synth.CFG_DECODE, layer=7)
        _CODER["wide"] = (hb, M.SparseMoe(hb))
    hb, dev = _CODER["wide"]
    run_block(hb, dev, synth.make_x(WIDE_SHARED, 40, config=synth.CFG_DECODE, layer=340),
              "wide rows with a shared expert, prefill T=40")


@pytest.mark.parametrize("T", [1, 2, 5, 24])
def test_wide_rows_with_shared_expert(T):
    """Rows wider than 2048 with a shared expert: the decode gate/up streams two row blocks per
    workgroup (routed and shared workgroups; one pair at T = 1, two pairs at a time above), the
    down kernel is the general one. Against the oracle on the GPU's expert choices."""
    if "wide" not in _CODER:
        hb = synth.make_block(WIDE_SHARED, config=synth.CFG_DECODE, layer=7)
        _CODER["wide"] = (hb, M.SparseMoe(hb))
    hb, dev = _CODER["wide"]
    x_np = synth.make_x(WIDE_SHARED, T, config=synth.CFG_DECODE, layer=300 + T)
    run_block(hb, dev, x_np, f"wide rows + shared expert T={T}")
    # row-exactness: every row equals its one-row forward
    if T > 1:
        batch = M.bf16_bits(dev.forward(M.bf16_tensor(x_np)))
        for t in range(T):
            one = M.bf16_bits(dev.forward(M.bf16_tensor(x_np[t:t + 1])))
            assert np.array_equal(one[0], batch[t]), f"row {t}"


def test_coder_stack_matches_layer_loop():
    """Two Coder-shaped layers (configs[4] weights, the second layer's seeds) in the layer stack at
    T = 1: the streaming decode kernels with the fused norm and residual add give the bits of the
    loop of single ops (rms_norm, block forward, add_rms_norm)."""
    layers = [_coder_dev(), M.device_block(synth.CODER, synth.CFG_CODER, 1)]
    st = M.MoeStack(layers, None, 1e-6)
    x_np = synth.make_x(synth.CODER, 1, config=synth.CFG_CODER, layer=77)
    got = M.bf16_bits(st.forward_(M.bf16_tensor(x_np)))
    x = M.bf16_tensor(x_np)
    h = M.rms_norm(x, None, 1e-6)
    for layer in layers:
        o = layer.forward(h)
        x, h = M.add_rms_norm(x, o, None, 1e-6)
    torch.cuda.synchronize()
    assert np.array_equal(got, M.bf16_bits(x)), "Coder stack differs from the op loop"
    assert np.isfinite(synth.bf16_to_f32(got)).all()


_CODER = {}


def _coder_host():
    if "host" not in _CODER:
        _CODER["host"] = synth.make_block(synth.CODER, config=synth.CFG_CODER)
    return _CODER["host"]


def _coder_dev():
    if "dev" not in _CODER:
        _CODER["dev"] = M.SparseMoe(_coder_host())
    return _CODER["dev"]


# ---------------------------------------------------------------------------------------------
# device-side generator (benchmark inputs) and the layer stack around the block

def _near(a, b, max_diff=2, ulps=1):
    """Equal, or (float64 log/sin/cos of device and host libm may differ in the last place) a
    handful of elements one bf16 ulp apart."""
    d = ulp_distance(a, b)
    return int(np.count_nonzero(d)) <= max_diff and int(d.max(initial=0)) <= ulps


def test_device_generator_matches_host():
    """Codes bit-identical to the host generator; scales, biases and normals equal up to libm's
    last place."""
    E, O_, I_ = 1, 1024, 8192
    dev = M.device_qtensor(7, 3, synth.GATE_CODES, synth.GATE_SCALES, E, O_, I_)
    host = synth.qtensor(7, 3, synth.GATE_CODES, synth.GATE_SCALES, E, O_, I_)
    torch.cuda.synchronize()
    assert np.array_equal(M.u32_array(dev.codes), host.codes.ravel())
    assert _near(M.bf16_bits(dev.scales), host.scales.ravel())
    assert _near(M.bf16_bits(dev.biases), host.biases.ravel())
    s = synth.seed(7, 3, synth.ROUTER_W)
    nd = M.bf16_bits(M.device_normal_bf16(s, 1 << 16, 0.02))
    assert _near(nd, synth.normal_bf16(s, 1 << 16, 0.02))


STACK = synth.Shape(hidden=2048, experts=32, top_k=4, intermediate=512, shared=512)


@pytest.fixture(scope="module")
def stack3():
    hosts = [synth.make_block(STACK, config=synth.CFG_STACK, layer=l) for l in range(3)]
    return hosts, M.MoeStack([M.SparseMoe(h) for h in hosts])


@pytest.fixture(scope="module")
def stack3_gates8():
    hosts = [synth.make_block(STACK, config=synth.CFG_STACK, layer=10 + l, gate_bits=8)
             for l in range(3)]
    return hosts, M.MoeStack([M.SparseMoe(h) for h in hosts])


@pytest.mark.parametrize("T", [4, 24, 40])
def test_stack_matches_layer_loop_and_oracle(stack3, T):
    """configs[3]'s decoder-layer loop, x = R(x + MoE_l(rms_norm(x))) per layer, with layer l's
    residual add and layer l+1's norm fused (add_rms_norm). T=4 takes the decode schedule with the
    norm inside its router launch, T=24 the decode schedule with the norm as its own launch (24
    normalised rows exceed the router launch's LDS), T=40 the prefill one. Bit-identical to the
    loop of single ops on the GPU. Against the CPU restatement,
    layer by layer on the GPU's expert choices (each validated as a top-k within ties): within the
    block bar plus one bf16 ulp of the residual stream (a rounding of x + MoE(h) that lands on the
    neighbouring value moves x by one ulp of |x|, which exceeds 2e-2 where |x| >= 4)."""
    _check_stack(stack3, T, "stack")


@pytest.mark.parametrize("T", [1, 4])
def test_stack_8bit_gates(stack3_gates8, T):
    """The same loop with 8-bit group-64 routers and shared gates (mlx-community conversions):
    at decode sizes the router launch dequantizes their rows itself, with the norm fused."""
    _check_stack(stack3_gates8, T, "stack, 8-bit gates")


def _check_stack(stack, T, label):
    hosts, st = stack
    x_np = synth.make_x(STACK, T, config=synth.CFG_STACK, layer=T)
    got = M.bf16_bits(st.forward_(M.bf16_tensor(x_np)))
    x = M.bf16_tensor(x_np)
    h = M.rms_norm(x, None, 1e-6)
    ids = []
    for layer in st.layers:
        ids.append(M.u32_array(layer.router_forward(h)[2]).reshape(T, -1))
        o = layer.forward(h)
        x, h = M.add_rms_norm(x, o, None, 1e-6)
    torch.cuda.synchronize()
    assert np.array_equal(got, M.bf16_bits(x)), "stack entry point differs from the op loop"
    ref = x_np.copy()
    for hb, gi in zip(hosts, ids):
        o = O.moe_forward(hb, O.rms_norm(ref, None, 1e-6), forced_ids=gi)
        ref = O.bf16_from_f32(synth.bf16_to_f32(ref) + synth.bf16_to_f32(o))
    g, r = synth.bf16_to_f32(got).astype(np.float64), synth.bf16_to_f32(ref).astype(np.float64)
    bound = 2e-2 + bf16_ulp(np.maximum(np.abs(g), np.abs(r)))
    s = stats(got, ref)
    assert np.all(np.abs(g - r) <= bound), f"{label} T={T}: {s}"
    assert s["l1_rel"] <= 1e-3, f"{label} T={T}: {s}"
    # the oracle's own stack entry agrees with its layer loop
    if T == 4:
        own = O.moe_stack(hosts, x_np, None, 1e-6)
        _log(f"oracle stack vs GPU: {stats(got, own)}")
    _log(f"{label} of 3, T={T}: {s}")


# ---------------------------------------------------------------------------------------------
# 8-bit weights and quantized routers (mlx-community conversions: 8-bit group-64 router and shared
# gate, load.rs:14-17 and the tiny fixtures' quantization config)

Q8 = synth.Shape(hidden=2048, experts=64, top_k=8, intermediate=512, shared=512)


@pytest.fixture(scope="module")
def q8_blocks():
    out = {}
    for name, kw in {"experts8": dict(expert_bits=8), "gates8": dict(gate_bits=8),
                     "both8": dict(expert_bits=8, gate_bits=8)}.items():
        hb = synth.make_block(Q8, config=synth.CFG_DECODE, layer=5, **kw)
        out[name] = (hb, M.SparseMoe(hb))
    return out


@pytest.mark.parametrize("kind", ["experts8", "gates8", "both8"])
@pytest.mark.parametrize("T", [1, 3, 16, 24, 40, 300])
def test_8bit_weights_match_oracle(q8_blocks, kind, T):
    """8-bit experts run the decode kernels at T <= 32 (each byte's two nibbles dotted as two 4-bit
    codes; T = 24 as one batch of 192 pairs) and the generic MFMA GEMM above; an 8-bit router and
    shared gate are dequantized inside the decode router launch (T <= 32) or run as the prefill's
    first product."""
    hb, dev = q8_blocks[kind]
    x_np = synth.make_x(Q8, T, config=synth.CFG_DECODE, layer=100 + T)
    run_block(hb, dev, x_np, f"{kind} T={T}")


def test_8bit_experts_rows_keep_their_one_row_bits(q8_blocks):
    """8-bit experts at decode: every row of a batch of up to 16 has its one-row bits, as with
    4-bit experts (the same kernels; nuvec.rs:256-265)."""
    hb, dev = q8_blocks["both8"]
    x_np = synth.make_x(Q8, 16, config=synth.CFG_DECODE, layer=88)
    batch = M.bf16_bits(dev.forward(M.bf16_tensor(x_np)))
    for T in (3, 9):
        assert np.array_equal(M.bf16_bits(dev.forward(M.bf16_tensor(x_np[:T]))), batch[:T])
    for t in (0, 5, 15):
        one = M.bf16_bits(dev.forward(M.bf16_tensor(x_np[t:t + 1])))
        assert np.array_equal(one[0], batch[t]), f"row {t}"


@pytest.mark.parametrize("group", [32, 128])
def test_8bit_groups(group):
    shape = synth.Shape(hidden=1024, experts=16, top_k=4, intermediate=256, shared=256, group=group)
    hb = synth.make_block(shape, config=synth.CFG_PLUMBING, layer=group, expert_bits=8, gate_bits=8)
    dev = M.SparseMoe(hb)
    for T in (2, 70):
        run_block(hb, dev, synth.make_x(shape, T, config=synth.CFG_PLUMBING, layer=T),
                  f"8-bit group {group} T={T}")


@pytest.mark.parametrize("group", [32, 128])
def test_groups_on_the_decode_kernels(group):
    """4-bit experts with groups of 32 and 128 on the Qwen3.6-like shape: the decode kernels (a
    lane's 32-code chunk lies in one group, its scale and bias picked by the group shift) at
    T = 1, 4 and 24, and the generic MFMA GEMM at T = 300."""
    shape = synth.Shape(hidden=2048, experts=256, top_k=8, intermediate=512, shared=512,
                        group=group)
    hb = synth.make_block(shape, config=synth.CFG_DECODE, layer=group)
    dev = M.SparseMoe(hb)
    for T in (1, 4, 24, 300):
        run_block(hb, dev, synth.make_x(shape, T, config=synth.CFG_DECODE, layer=600 + T),
                  f"4-bit group {group} T={T}")


def test_quantized_linear_facade():
    """Linear::forward with an 8-bit weight and a bias (load.rs:294-306): R(R(x Wq^T) + b)."""
    w = synth.normal_bf16(synth.seed(9, 0, synth.ROUTER_W), 96 * 512, 0.02).reshape(96, 512)
    q = synth.quantize(w, 8, 64)
    b = synth.normal_bf16(synth.seed(9, 0, synth.ROUTER_BIAS), 96, 0.1)
    dq = M.DeviceQTensor(q)
    for T in (1, 7, 33):
        x_np = synth.make_x(synth.Shape(512, 1, 1, 32), T, config=9, layer=T)
        got = M.bf16_bits(M.linear(M.bf16_tensor(x_np), dq, M.bf16_tensor(b)))
        ref = O.linear(q, x_np, b)
        assert beyond_rounding(got, ref) == 0, stats(got, ref)


@pytest.mark.parametrize("T", [4, 24, 40])
def test_stack_graph_replays_match_eager(stack3, T):
    """The stack captured as one HIP graph (no memset nodes: counters are cleared by kernels):
    every replay, with eager work in between, equals the eager result."""
    _, st = stack3
    x0 = M.bf16_tensor(synth.make_x(STACK, T, config=synth.CFG_STACK, layer=500 + T))
    eager = st.forward_(x0.clone())
    torch.cuda.synchronize()
    x = x0.clone()
    ws = st.workspace(T).clone()  # the graph's own workspace
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        x.copy_(x0)
        st.forward_(x, ws, stream=s)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        x.copy_(x0)
        st.forward_(x, ws, stream=s)
    torch.cuda.synchronize()
    want = M.bf16_bits(eager)
    for r in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(M.bf16_bits(x), want), f"replay {r}"
        other = st.forward_(x0.clone())  # eager work between replays
        torch.cuda.synchronize()
        assert np.array_equal(M.bf16_bits(other), want)


# ---------------------------------------------------------------------------------------------
# dense bf16 experts (SwitchLinear::Dense, moe.rs:43-46 -> gather_mm, nuvec.rs:688-697)

@pytest.fixture(scope="module")
def dense_block():
    hb = synth.make_block(Q8, config=synth.CFG_DECODE, layer=6, expert_bits=16)
    return hb, M.SparseMoe(hb)


@pytest.mark.parametrize("T", [1, 3, 16, 40, 300])
def test_dense_experts_match_oracle(dense_block, T):
    """Unquantized bf16 experts and shared expert (bits 16) on the generic GEMV and MFMA GEMM."""
    hb, dev = dense_block
    run_block(hb, dev, synth.make_x(Q8, T, config=synth.CFG_DECODE, layer=200 + T), f"dense T={T}")


# ---------------------------------------------------------------------------------------------
# edges of the configuration space (qwen3_5_moe.rs:508-513: 1 <= k <= E)

@pytest.mark.parametrize("shape,Ts", [
    # top-1 routing: one pair per token
    (synth.Shape(hidden=2048, experts=64, top_k=1, intermediate=512, shared=512), (1, 16, 100)),
    # 512 experts (eight per lane in the top-k) with k = 16, the widest top-k (FFN width 256:
    # the generic GEMV and GEMM at every size)
    (synth.Shape(hidden=2048, experts=512, top_k=16, intermediate=256, shared=0), (1, 8, 9, 70)),
    # k = 16 on the decode kernels: T = 16 fills their 256 pairs; T = 20 and 32 (more pairs than
    # that) run as decode chunks of 16 tokens, T = 33 on the prefill schedule
    (synth.Shape(hidden=2048, experts=128, top_k=16, intermediate=512, shared=512),
     (16, 20, 32, 33)),
    # k = E: every expert chosen by every token; norm_topk off
    (synth.Shape(hidden=512, experts=8, top_k=8, intermediate=128, shared=128, norm_topk=False),
     (1, 5, 40)),
    # norm_topk off on the tuned kernels (the Qwen3.6-like shape): the top-k inside the decode
    # gate/up launch (T <= 4), the top-k launch (T = 24), the prefill top-k + counts (T = 300)
    (synth.Shape(hidden=2048, experts=256, top_k=8, intermediate=512, shared=512,
                 norm_topk=False), (1, 4, 24, 300)),
    # hidden not a multiple of 64 (the MFMA paths need K % 64 == 0; group 32): GEMV at every size
    (synth.Shape(hidden=2080, experts=32, top_k=4, intermediate=544, shared=0, group=32), (2, 33)),
])
def test_config_edges(shape, Ts):
    hb = synth.make_block(shape, config=synth.CFG_PLUMBING, layer=shape.experts + shape.top_k)
    dev = M.SparseMoe(hb)
    for T in Ts:
        run_block(hb, dev, synth.make_x(shape, T, config=synth.CFG_PLUMBING, layer=300 + T),
                  f"{shape.name} T={T}")
    if shape.top_k == 16 and shape.intermediate == 512:
        # the decode chunks give every row its one-row bits
        x = synth.make_x(shape, 20, config=synth.CFG_PLUMBING, layer=320)
        batch = M.bf16_bits(dev.forward(M.bf16_tensor(x)))
        for t in (0, 15, 16, 19):
            one = M.bf16_bits(dev.forward(M.bf16_tensor(x[t:t + 1])))
            assert np.array_equal(one[0], batch[t]), f"chunked row {t}"



def test_decode_boundary_t33(q_host, q_dev):
    """T = 32 is the last size that runs the decode kernels and T = 33 the first prefill one: the
    same token's output agrees between them within the bar (the two schedules accumulate in
    different orders), and T = 17 gives its rows the T = 16 bits."""
    x33 = synth.make_x(Q, 33, config=synth.CFG_DECODE, layer=17)
    a = M.bf16_bits(q_dev.forward(M.bf16_tensor(x33)))
    b = M.bf16_bits(q_dev.forward(M.bf16_tensor(x33[:32])))
    c = M.bf16_bits(q_dev.forward(M.bf16_tensor(x33[:17])))
    d = M.bf16_bits(q_dev.forward(M.bf16_tensor(x33[:16])))
    torch.cuda.synchronize()
    assert_close(b, a[:32], what="T=32 decode vs T=33 prefill rows")
    assert np.array_equal(c[:16], d), "T=17 rows 0-15 against T=16"
    assert_close(c, a[:17], what="T=17 decode vs T=33 prefill rows")


# ---------------------------------------------------------------------------------------------
# the sorted dispatch the forward itself uses (moe.rs:65-75), read back from its workspace

def _forward_routing(dev, x, ws):
    out = dev.forward(x, workspace=ws)
    ids, sc, off, order, inverse, token = dev.routing_of_last_forward(x.shape[0], ws)
    torch.cuda.synchronize()
    return (M.bf16_bits(out), M.u32_array(ids), M.bf16_bits(sc), M.u32_array(off),
            M.u32_array(order), M.u32_array(inverse), M.u32_array(token))


def check_forward_permutation(hb, dev, x_np, label, check_rows=None):
    """The forward's order / inverse / token are the oracle's stable argsort of the forward's own
    ids, bit for bit; two forwards leave identical routing and outputs; the ids equal the router
    op's. Then the block output against the oracle (on check_rows)."""
    T, k, E = x_np.shape[0], hb.shape.top_k, hb.shape.experts
    x = M.bf16_tensor(x_np)
    ws = dev.workspace(T)
    a = _forward_routing(dev, x, ws)
    ws2 = torch.empty_like(ws).fill_(0x5A)  # another workspace, different stale contents
    b = _forward_routing(dev, x, ws2)
    for name, u, v in zip(("out", "ids", "scores", "offsets", "order", "inverse", "token"), a, b):
        assert np.array_equal(u, v), f"{label}: {name} differs between two forwards"
    out, ids, _, off, order, inverse, token = a
    r_order, r_inverse, r_token, r_counts = O.permute(ids, k, E)
    assert np.array_equal(order, r_order), f"{label}: order is not the stable argsort"
    assert np.array_equal(inverse, r_inverse), f"{label}: inverse"
    assert np.array_equal(token, r_token), f"{label}: token"
    assert off[0] == 0 and np.array_equal(np.diff(off.astype(np.int64)), r_counts), label
    _, _, rids, _ = dev.router_forward(x)
    assert np.array_equal(M.u32_array(rids).ravel(), ids), f"{label}: forward ids differ from the router's"
    rows = np.arange(T) if check_rows is None else np.asarray(check_rows)
    ref = O.moe_forward(hb, x_np[rows], forced_ids=ids.reshape(T, k)[rows])
    s = assert_close(out[rows], ref, what=label)
    _log(f"{label}: permutation bit-exact ({T * k} pairs), {s}")


@pytest.mark.parametrize("T", [33, 300])
def test_forward_permutation_q(q_host, q_dev, T):
    x_np = synth.make_x(Q, T, config=synth.CFG_PREFILL_ZIPF, layer=40 + T)
    check_forward_permutation(q_host, q_dev, x_np, f"Q forward permutation T={T}")


def test_forward_permutation_zipf_2048():
    hb = _zipf_host()
    dev = M.SparseMoe(hb)
    x_np = synth.make_x(Q, 2048, config=synth.CFG_PREFILL_ZIPF, layer=7)
    rows = np.sort(np.random.default_rng(7).choice(2048, 96, replace=False))
    check_forward_permutation(hb, dev, x_np, "Q Zipf forward permutation T=2048", rows)


def test_forward_permutation_8bit_small(q8_blocks):
    """8-bit experts at the first prefill size (T = 33, 264 pairs; up to 32 tokens they take the
    decode schedule, which needs no permutation): the forward's permutation anyway."""
    hb, dev = q8_blocks["experts8"]
    x_np = synth.make_x(Q8, 33, config=synth.CFG_DECODE, layer=41)
    check_forward_permutation(hb, dev, x_np, "8-bit experts forward permutation T=33")


def test_block_coder_prefill_8192():
    """configs[4] prefill, T = 8192 (65,536 pairs): the forward's permutation bit-exact against the
    stable argsort, and 48 sampled rows of the block output against the oracle (rows are
    independent of each other, so sampled rows are exact checks)."""
    hb, dev = _coder_host(), _coder_dev()
    x_np = synth.make_x(synth.CODER, 8192, config=synth.CFG_CODER, layer=8192)
    rows = np.sort(np.random.default_rng(8192).choice(8192, 48, replace=False))
    check_forward_permutation(hb, dev, x_np, "Coder configs[4] T=8192", rows)


_ZIPF = {}


def _zipf_host():
    if "host" not in _ZIPF:
        _ZIPF["host"] = synth.make_block(Q, config=synth.CFG_PREFILL_ZIPF, zipf=True)
    return _ZIPF["host"]


# ---------------------------------------------------------------------------------------------
# quantized weights without biases: zeros (Quantized::new, nuvec.rs:609-626)

def _without_biases(hb, routed=True, shared=True):
    """The block with its quantized experts' biases dropped. Their scales get seeded random signs,
    so that the dequantized weights q*s keep mean zero and the outputs their usual magnitude
    (with q in 0..15 and positive scales every weight would be positive)."""
    import copy
    nb = copy.copy(hb)
    rng = np.random.default_rng(609)

    def strip(q):
        sign = rng.integers(0, 2, q.scales.shape, dtype=np.uint16) << np.uint16(15)
        return synth.QTensor(q.codes, q.scales ^ sign, None, q.experts, q.out, q.in_, q.group,
                             q.bits)

    if routed:
        nb.gate_proj, nb.up_proj, nb.down_proj = map(strip, (hb.gate_proj, hb.up_proj, hb.down_proj))
    if shared and hb.shape.shared:
        nb.sh_gate_proj, nb.sh_up_proj, nb.sh_down_proj = map(
            strip, (hb.sh_gate_proj, hb.sh_up_proj, hb.sh_down_proj))
    return nb


@pytest.fixture(scope="module")
def nobias_blocks(q_host):
    out = {}
    for name, kw in {"all": {}, "routed": dict(shared=False)}.items():
        hb = _without_biases(q_host, **kw)
        out[name] = (hb, M.SparseMoe(hb))
    return out


@pytest.mark.parametrize("kind", ["all", "routed"])
@pytest.mark.parametrize("T", [1, 4, 16, 17, 300])
def test_null_biases_match_oracle(nobias_blocks, kind, T):
    """Q blocks whose quantized experts (and shared expert) carry no biases, at decode (GEMV
    kernels) and prefill (MFMA GEMM) sizes, against the oracle's zero-bias dequant."""
    hb, dev = nobias_blocks[kind]
    assert hb.gate_proj.biases is None
    x_np = synth.make_x(Q, T, config=synth.CFG_DECODE, layer=600 + T)
    run_block(hb, dev, x_np, f"no biases ({kind}) T={T}")


def test_null_biases_gather_qmm(q_host):
    """gather_qmm over a weight without biases, GEMV and MFMA sizes."""
    w = _without_biases(q_host).down_proj
    dw = M.DeviceQTensor(w)
    for n in (8, 600):
        idx = np.random.default_rng(n).integers(0, Q.experts, n).astype(np.uint32)
        a_np = synth.make_x(synth.Shape(512, 1, 1, 512), n, config=9, layer=n)
        got = M.bf16_bits(M.gather_qmm(M.bf16_tensor(a_np), dw, M.u32_tensor(idx)))
        ref = O.gather_qmm(w, a_np, idx)
        assert_close(got, ref, max_ulp=1, what=f"gather_qmm without biases n={n}")


# ---------------------------------------------------------------------------------------------
# prefill with the routed experts on the grouped GEMM and the shared expert on the generic GEMMs

@pytest.mark.parametrize("kind", ["wider_shared", "shared8"])
@pytest.mark.parametrize("T", [64, 300])
def test_shared_expert_on_generic_gemms(kind, T):
    """The routed experts run the grouped GEMM (4-bit, group 64, widths multiples of 512) while the
    shared expert cannot ride in its launches: a width unlike the routed one (1024 against 512),
    or 8-bit shared projections of the routed width."""
    if kind == "wider_shared":
        shape = synth.Shape(hidden=2048, experts=64, top_k=8, intermediate=512, shared=1024)
        hb = synth.make_block(shape, config=synth.CFG_PLUMBING, layer=T)
    else:
        shape = synth.Shape(hidden=2048, experts=64, top_k=8, intermediate=512, shared=512)
        hb = synth.make_block(shape, config=synth.CFG_PLUMBING, layer=T + 1)
        h8 = synth.make_block(shape, config=synth.CFG_PLUMBING, layer=T + 2, expert_bits=8)
        hb.sh_gate_proj, hb.sh_up_proj, hb.sh_down_proj = h8.sh_gate_proj, h8.sh_up_proj, h8.sh_down_proj
    dev = M.SparseMoe(hb)
    run_block(hb, dev, synth.make_x(shape, T, config=synth.CFG_PLUMBING, layer=T), f"{kind} T={T}")


# ---------------------------------------------------------------------------------------------
# the 40-layer Qwen-shaped stack (weights generated on the device, 18 GB)

N_STACK = 40


@pytest.fixture(scope="module")
def stack40():
    layers = [M.device_block(Q, synth.CFG_STACK, l) for l in range(N_STACK)]
    torch.cuda.synchronize()
    return layers


def _host_view(dev, experts=None):
    """The device block's weights copied to the host for the oracle; with `experts`, only those
    experts' slices are copied (the others stay zero pages that the oracle never reads)."""
    def q(dq):
        E = dq.experts
        shp = lambda t: t.view(E, dq.out, -1)
        if experts is None or len(experts) * 4 >= E:
            c, s_, b = (M.u32_array(shp(dq.codes)), M.bf16_bits(shp(dq.scales)),
                        M.bf16_bits(shp(dq.biases)))
        else:
            c = np.zeros((E, dq.out, dq.in_ * dq.bits // 32), np.uint32)
            s_ = np.zeros((E, dq.out, dq.in_ // dq.group), np.uint16)
            b = np.zeros_like(s_)
            for e in sorted(experts):
                c[e] = M.u32_array(shp(dq.codes)[e])
                s_[e] = M.bf16_bits(shp(dq.scales)[e])
                b[e] = M.bf16_bits(shp(dq.biases)[e])
        return synth.QTensor(c, s_, b, E, dq.out, dq.in_, dq.group, dq.bits)

    s = dev.shape
    hb = synth.HostBlock(shape=s, router=M.bf16_bits(dev.router), router_bias=None,
                         gate_proj=q(dev.gate_proj), up_proj=q(dev.up_proj),
                         down_proj=q(dev.down_proj))
    if s.shared:
        hb.sh_gate_proj, hb.sh_up_proj, hb.sh_down_proj = (
            q(dev.sh_gate_proj), q(dev.sh_up_proj), q(dev.sh_down_proj))
        hb.sh_expert_gate = M.bf16_bits(dev.sh_expert_gate)
    return hb


def _stack_op_loop(layers, x_np, rows):
    """rms_norm, then per layer the block forward and add_rms_norm. Returns the final x and, per
    layer, the sampled rows of its input x, its block input h, its block output o, and its ids
    (read from the forward's own workspace)."""
    T = x_np.shape[0]
    x = M.bf16_tensor(x_np)
    h = M.rms_norm(x, None, 1e-6)
    trace = []
    for layer in layers:
        ws = layer.workspace(T)
        o = layer.forward(h, workspace=ws)
        ids = M.u32_array(layer.routing_of_last_forward(T, ws)[0]).reshape(T, -1)[rows].copy()
        trace.append((M.bf16_bits(x)[rows], M.bf16_bits(h)[rows], M.bf16_bits(o)[rows], ids))
        x, h = M.add_rms_norm(x, o, None, 1e-6)
    torch.cuda.synchronize()
    return M.bf16_bits(x), trace


def _stack_bar(got, ref, trace, label):
    """The block bar for deep layers. L1-relative 1e-3, and each element within max(2e-2, two bf16
    ulps of the largest term its sum rounds: the routed experts' outputs y_j for that element, the
    shared expert's output, the result). The synthetic weights s*(q - 8) have mean -s/2, so the
    residual stream gains a steady direction, and deep in the stack the expert outputs reach
    |y_j| ~ 10. There one bf16 ulp (0.0625) exceeds 2e-2, and the rounding points inside the
    block (y_j, y_j * score, the sum over k, the shared add) each move by up to an ulp of their
    own magnitude under another f32 accumulation order."""
    T, D = got.shape
    g, r = synth.bf16_to_f32(got).astype(np.float64), synth.bf16_to_f32(ref).astype(np.float64)
    terms = np.abs(synth.bf16_to_f32(trace["y"])).reshape(T, -1, D).max(axis=1)
    if "shared_y" in trace:
        terms = np.maximum(terms, np.abs(synth.bf16_to_f32(trace["shared_y"])))
    mag = np.maximum(np.maximum(np.abs(g), np.abs(r)), terms)
    bound = np.maximum(2e-2, 2 * bf16_ulp(mag))
    s = stats(got, ref)
    # the widened allowance is for the few elements whose terms are large: bound how many use it
    s["beyond_2e-2"] = float(np.mean(np.abs(g - r) > 2e-2))
    assert np.all(np.abs(g - r) <= bound), f"{label}: {s}"
    assert s["l1_rel"] <= 1e-3, f"{label}: {s}"
    assert s["beyond_2e-2"] <= STACK_WIDE_SHARE, f"{label}: {s}"
    return s


def _check_stack_layers(layers, trace, final, label):
    """Each layer on the GPU's own input for that layer: the norm within one ulp of the oracle's,
    the block output within the block bar of the oracle's on the GPU's h and ids (each validated
    as a top-k within ties), and the residual add bit-exact. A 40-layer chain compounds one-ulp
    roundings (a residual value one ulp off changes the next norm and so the next routing), so
    the per-layer check is the bar."""
    worst, wide = None, 0.0
    for l, layer in enumerate(layers):
        x_l, h_l, o_l, ids = trace[l]
        assert ulp_distance(h_l, O.rms_norm(x_l, None, 1e-6)).max() <= 1, f"{label} layer {l} norm"
        hb = _host_view(layer, set(np.unique(ids).tolist()))
        ref, tr = O.moe_forward(hb, h_l, forced_ids=ids, trace=True)
        if not layer.shared:
            tr.pop("shared_y")
        s = _stack_bar(o_l, ref, tr, f"{label} layer {l}")
        nxt = trace[l + 1][0] if l + 1 < len(layers) else final
        assert np.array_equal(nxt, O.bf16_from_f32(synth.bf16_to_f32(x_l) + synth.bf16_to_f32(o_l))), \
            f"{label} layer {l} residual"
        worst = s if worst is None or s["l1_rel"] > worst["l1_rel"] else worst
        wide = max(wide, s["beyond_2e-2"])
        del hb
    _log(f"{label}: largest share of a layer's elements beyond 2e-2: {wide:.2e}")
    return worst


def test_stack40_decode_t1(stack40):
    """configs[3] at T = 1: the stack entry point (norm fused into each router launch, residual
    into the last launch) equals the loop of single ops bit for bit, and every one of the 40 layers
    matches the oracle on the GPU's input for that layer."""
    x_np = synth.make_x(Q, 1, config=synth.CFG_STACK, layer=1)
    st = M.MoeStack(stack40, None, 1e-6)
    got = M.bf16_bits(st.forward_(M.bf16_tensor(x_np)))
    loop, trace = _stack_op_loop(stack40, x_np, np.arange(1))
    assert np.array_equal(got, loop), "stack entry point differs from the op loop"
    worst = _check_stack_layers(stack40, trace, loop, "stack40 T=1")
    _log(f"stack of {N_STACK}, T=1: every layer within the bar; worst layer {worst}")


def test_stack40_prefill_t4096(stack40):
    """configs[3] at T = 4096: the stack entry point equals the op loop bit for bit; 32 sampled
    rows checked layer by layer against the oracle (rows are independent of each other, so
    sampled rows are exact checks)."""
    T = 4096
    x_np = synth.make_x(Q, T, config=synth.CFG_STACK, layer=T)
    st = M.MoeStack(stack40, None, 1e-6)
    got = M.bf16_bits(st.forward_(M.bf16_tensor(x_np)))
    rows = np.sort(np.random.default_rng(4096).choice(T, 32, replace=False))
    loop, trace = _stack_op_loop(stack40, x_np, rows)
    assert np.array_equal(got, loop), "stack entry point differs from the op loop"
    worst = _check_stack_layers(stack40, trace, loop[rows], "stack40 T=4096")
    _log(f"stack of {N_STACK}, T=4096, 32 rows: every layer within the bar; worst layer {worst}")
