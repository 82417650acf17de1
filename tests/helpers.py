"""Comparison helpers for bf16 results (bits as uint16) and the tie-aware top-k check."""
from __future__ import annotations

import numpy as np

from mrun_amd.synth import bf16_to_f32


def ordered(bits: np.ndarray) -> np.ndarray:
    """bf16 bits -> integers ordered like the values (adjacent values differ by one)."""
    b = bits.astype(np.int32)
    return np.where(b & 0x8000, -(b & 0x7FFF), b)


def ulp_distance(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    return np.abs(ordered(a) - ordered(b))


def stats(got: np.ndarray, ref: np.ndarray) -> dict:
    """max-abs, L1-relative error, mean relative error (floored), share of differing elements."""
    g = bf16_to_f32(got).astype(np.float64)
    r = bf16_to_f32(ref).astype(np.float64)
    d = np.abs(g - r)
    floor = max(np.mean(np.abs(r)) * 1e-3, 1e-30)
    return {
        "max_abs": float(d.max()) if d.size else 0.0,
        "l1_rel": float(d.sum() / max(np.abs(r).sum(), 1e-30)),
        "mean_rel": float(np.mean(d / np.maximum(np.abs(r), floor))),
        "frac_diff": float(np.mean(got != ref)),
        "max_ulp": int(ulp_distance(got, ref).max()) if got.size else 0,
    }


def bf16_ulp(v: np.ndarray) -> np.ndarray:
    """Spacing of bf16 values at |v| (smallest normal spacing below 2^-126)."""
    a = np.maximum(np.abs(v.astype(np.float64)), 2.0 ** -126)
    return 2.0 ** (np.floor(np.log2(a)) - 7)


def beyond_rounding(got: np.ndarray, ref: np.ndarray, ulps: int = 1,
                    rel_floor: float = 2.0 ** -14) -> int:
    """Elements whose difference exceeds `ulps` bf16 ulps at their magnitude plus an absolute
    floor of rel_floor * rms(ref): two f32 accumulations of the same terms in different orders
    differ by a few f32 ulps of the running sum, which after bf16 rounding is at most one bf16 ulp
    away from the value, except where the sum cancels to near zero (the floor)."""
    g = bf16_to_f32(got).astype(np.float64)
    r = bf16_to_f32(ref).astype(np.float64)
    rms = float(np.sqrt(np.mean(r * r))) if r.size else 0.0
    bound = ulps * bf16_ulp(np.maximum(np.abs(g), np.abs(r))) + rel_floor * rms
    return int(np.sum(np.abs(g - r) > bound))


def assert_close(got, ref, max_abs=2e-2, l1_rel=1e-3, max_ulp=None, what=""):
    s = stats(got, ref)
    assert s["max_abs"] <= max_abs, f"{what} max-abs {s}"
    assert s["l1_rel"] <= l1_rel, f"{what} L1-relative {s}"
    if max_ulp is not None:
        bad = beyond_rounding(got, ref, max_ulp)
        assert bad == 0, f"{what}: {bad} elements beyond {max_ulp} ulp {s}"
    return s
