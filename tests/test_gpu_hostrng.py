"""The host generator exported for callers that keep the reference's host code
(nn_hip_rt.h: NnHostRng, nnhip_rng_seed, nnhip_fill_normal,
nnhip_fill_uniform), which replaces the cuRAND fill of reference
src/nn.h:117-135 and curandGenerateUniform at src/mp_fourier.c:50.  cuRAND's
own streams are not reproduced (a closed library's internals), so the checks
are the distribution's: same seed gives the same bits, different seeds differ,
N(mean, std) moments within a few standard errors, uniforms in [0, 1)."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


class Rng(C.Structure):
    _fields_ = [("s", C.c_uint64 * 4)]


def _normal(L, seed, n, mean, std):
    g = Rng()
    L.nnhip_rng_seed(C.byref(g), seed)
    d = L.alloc(n)
    assert L.nnhip_fill_normal(C.byref(g), d.p, n, mean, std) == 0
    return d.download()


def test_fill_normal_is_seeded_and_distributed(L):
    print("[case] host generator: normal fill", flush=True)
    n = 1 << 20
    a = _normal(L, 410293, n, 0.5, 2.0)
    b = _normal(L, 410293, n, 0.5, 2.0)
    c = _normal(L, 410294, n, 0.5, 2.0)
    assert np.array_equal(a, b)
    assert not np.array_equal(a, c)
    x = a.astype(np.float64)
    se = 2.0 / np.sqrt(n)
    assert abs(x.mean() - 0.5) < 5 * se
    assert abs(x.std() - 2.0) < 5 * 2.0 / np.sqrt(2 * n)
    z = (x - 0.5) / 2.0
    assert abs((z ** 3).mean()) < 5 * np.sqrt(15 / n)      # skewness 0
    assert abs((z ** 4).mean() - 3.0) < 5 * np.sqrt(96 / n)  # kurtosis 3


def test_fill_uniform_range_and_moments(L):
    print("[case] host generator: uniform fill", flush=True)
    n = 1 << 20
    g = Rng()
    L.nnhip_rng_seed(C.byref(g), 7)
    d = L.alloc(n)
    assert L.nnhip_fill_uniform(C.byref(g), d.p, n) == 0
    u = d.download().astype(np.float64)
    assert u.min() >= 0.0 and u.max() < 1.0
    assert abs(u.mean() - 0.5) < 5 * np.sqrt(1 / 12 / n)
    assert abs(u.var() - 1 / 12) < 5 * np.sqrt(1 / 180 / n)
    # 24-bit grid: every value is a multiple of 2^-24
    assert np.all(np.floor(u * 2 ** 24) == u * 2 ** 24)
