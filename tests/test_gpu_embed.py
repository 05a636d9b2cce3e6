"""Embedding rows: mp_fourier (reference src/kernels.cu:385-394, 416-423) and
the sinusoidal timestep embedding (:444-456, 569-575) with the cfg2 / cfg4
inputs.  The float arguments are formed as the reference forms them; the
transcendental is the correctly rounded value on both sides."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import TOL, rel_err, ulp_diff

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("batch,C", [(128, 256), (3, 5), (1, 1), (1000, 64)])
def test_mp_fourier(L, orc, rng, batch, C):
    sigma = np.exp(-1.2 + 1.2 * rng.standard_normal(batch)).clip(0.002, 80).astype(np.float32)
    x = (np.log(sigma) / 4).astype(np.float32)  # c_noise = ln(sigma)/4 (src/diffusion/edm.c:52)
    f = rng.standard_normal(C).astype(np.float32)
    ph = rng.uniform(0, 1, C).astype(np.float32)
    xd, fd, pd, od = L.to_device(x), L.to_device(f), L.to_device(ph), L.alloc(batch * C)
    L.launch_mp_fourier(od.p, xd.p, fd.p, pd.p, batch, C, None)
    L.sync()
    ref = orc.mp_fourier(x, f, ph)
    got = od.download(shape=ref.shape)
    assert rel_err(got, ref) <= TOL, ulp_diff(got, ref)


@pytest.mark.parametrize("batch,C", [(256, 256), (4, 2), (7, 10), (1, 512)])
def test_sinusoidal(L, orc, rng, batch, C):
    t = rng.integers(0, 1000, batch).astype(np.float32)
    lmp = float(np.float32(np.log(np.float32(10000.0))))  # logf(max_period), src/sinusoidal.c:47
    td, od = L.to_device(t), L.alloc(batch * C)
    L.launch_sinusoidal(od.p, td.p, batch, C, lmp, None)
    L.sync()
    ref = orc.sinusoidal(t, C, lmp)
    got = od.download(shape=ref.shape)
    assert rel_err(got, ref) <= TOL, ulp_diff(got, ref)
    if batch == 256:
        t0 = np.zeros(1, np.float32)
        L.to_device(t0)
        td.upload(t0)
        L.launch_sinusoidal(od.p, td.p, 1, C, lmp, None)
        L.sync()
        row = od.download(C)
        assert np.all(row[: C // 2] == 0) and np.all(row[C // 2:] == 1)
