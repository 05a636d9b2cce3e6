"""Comparison helpers for the parity tests.

rel_err(got, ref, floor): max_i |got_i - ref_i| / max(|ref_i|, floor).  The
floor keeps the relative metric meaningful at zero crossings: for elementwise
outputs it is the RMS of the reference tensor, for reduced outputs (channel
sums, dot products) the root of the sum of squared terms.  The bar is 1e-5
for floating-point outputs and bit equality for copies and single products.
"""
from __future__ import annotations

import numpy as np

TOL = 1e-5


def rms(a) -> float:
    a = np.asarray(a, dtype=np.float64)
    return float(np.sqrt(np.mean(a * a))) if a.size else 0.0


def rel_err(got, ref, floor=None) -> float:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    if ref.size == 0:
        return 0.0
    if floor is None:
        floor = rms(ref)
    floor = np.maximum(np.asarray(floor, dtype=np.float64), 1e-30)
    return float(np.max(np.abs(got - ref) / np.maximum(np.abs(ref), floor)))


def ulp_diff(a, b) -> int:
    """Max distance in units in the last place between two float32 arrays."""
    a = np.ascontiguousarray(a, dtype=np.float32).view(np.int32).astype(np.int64)
    b = np.ascontiguousarray(b, dtype=np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, np.int64(-(2**31)) - a, a)
    b = np.where(b < 0, np.int64(-(2**31)) - b, b)
    return int(np.max(np.abs(a - b))) if a.size else 0


def assert_bits_equal(got, ref, what=""):
    got = np.ascontiguousarray(got, dtype=np.float32)
    ref = np.ascontiguousarray(ref, dtype=np.float32)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    diff = got.view(np.uint32) != ref.view(np.uint32)
    if diff.any():
        i = int(np.flatnonzero(diff.ravel())[0])
        raise AssertionError(
            f"{what}: {int(diff.sum())} of {diff.size} elements differ bitwise; first at {i}: "
            f"got {got.ravel()[i]!r} ref {ref.ravel()[i]!r} (max ulp {ulp_diff(got, ref)})"
        )


def channel_floor(terms_sq_sum) -> np.ndarray:
    """Floor for reduced outputs: sqrt(sum of squared terms) per output."""
    return np.sqrt(np.asarray(terms_sq_sum, dtype=np.float64))


def gn_param_floor(dy_eff, xhat, C):
    """sqrt(sum over (b, hw) of (d*xhat)^2) and of d^2, per channel."""
    d = np.asarray(dy_eff, np.float64).reshape(-1, C)
    xh = np.asarray(xhat, np.float64).reshape(-1, C)
    return channel_floor(np.sum((d * xh) ** 2, axis=0)), channel_floor(np.sum(d * d, axis=0))
