"""Elementwise rows: activations (reference src/kernels.cu:21-68, 103-117),
weighted_sum / mp_sum (:308-314, 353-366), scale_by_scalar (:300-306),
sgd_step (:163-168), add_bias (:95-101), bias_grad (:148-161).
HIP path through the C-ABI vs the oracle on the same seeded inputs."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import TOL, assert_bits_equal, rel_err, ulp_diff

pytestmark = pytest.mark.gpu

ACTS = {"identity": 0, "relu": 1, "gelu": 2, "silu": 3, "tanh": 4, "mp_silu": 5}
SIZES = [1, 3, 4, 1023, 4097, 1 << 20]  # tails, one-element, cfg1's 1M


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("act", list(ACTS.values()), ids=list(ACTS))
def test_activation_forward_backward(L, orc, rng, act, n):
    print(f"[case] activation act={act} n={n}", flush=True)
    x = (3.0 * rng.standard_normal(n)).astype(np.float32)
    g = rng.standard_normal(n).astype(np.float32)
    xd, yd, gd, gid = L.to_device(x), L.alloc(n), L.to_device(g), L.alloc(n)
    L.launch_activation_forward(yd.p, xd.p, n, act, None)
    L.launch_activation_backward(gid.p, gd.p, xd.p, n, act, None)
    L.sync()
    y_ref = orc.act_forward(x, act)
    gi_ref = orc.act_backward(g, x, act)
    y, gi = yd.download(), gid.download()
    assert rel_err(y, y_ref) <= TOL, ulp_diff(y, y_ref)
    assert rel_err(gi, gi_ref) <= TOL, ulp_diff(gi, gi_ref)


@pytest.mark.parametrize("act", [3, 5], ids=["silu", "mp_silu"])
def test_activation_misaligned_and_saturated(L, orc, rng, act):
    """Pointers off the 16-byte grid take the scalar shape; |v| up to 40 covers
    the Pade clamp (SiLU exactly 0 below about -9.94)."""
    n = 1000
    x = rng.uniform(-40, 40, n).astype(np.float32)
    xd, yd = L.alloc(n + 1), L.alloc(n + 1)
    xd.upload(np.concatenate([[0.0], x]).astype(np.float32))
    L.launch_activation_forward(yd.offset(1), xd.offset(1), n, act, None)
    L.sync()
    y = yd.download()[1:]
    assert rel_err(y, orc.act_forward(x, act)) <= TOL


def test_activation_large_cfg4(L, orc, rng):
    """SiLU over one quarter of the cfg4 activation tensor (67M elements)."""
    n = 256 * 64 * 64 * 256 // 4
    x = rng.standard_normal(n, dtype=np.float32)
    xd, yd = L.to_device(x), L.alloc(n)
    L.launch_activation_forward(yd.p, xd.p, n, 3, None)
    L.sync()
    assert rel_err(yd.download(), orc.act_forward(x, 3)) <= TOL


@pytest.mark.parametrize("n", [5, 4096, 128 * 32 * 32 * 128])  # the last is cfg2's mp_sum size
def test_weighted_sum_and_mp_sum(L, nn, orc, rng, n):
    print(f"[case] mp_sum n={n}", flush=True)
    a = rng.standard_normal(n, dtype=np.float32)
    b = rng.standard_normal(n, dtype=np.float32)
    ad, bd, od = L.to_device(a), L.to_device(b), L.alloc(n)
    L.launch_mp_sum(od.p, ad.p, bd.p, 0.3, n, None)
    L.sync()
    wa, wb = orc.mp_sum_weights(0.3)
    assert (wa, wb) == nn.mp_sum_weights(0.3)
    ref = orc.weighted_sum(a, b, wa, wb)
    assert rel_err(od.download(), ref) <= TOL
    # EMA form: out aliases a (src/ema.c:31-34)
    L.launch_weighted_sum(ad.p, ad.p, bd.p, 0.9999, float(np.float32(1) - np.float32(0.9999)), n, None)
    L.sync()
    assert rel_err(ad.download(), orc.weighted_sum(a, b, 0.9999, float(np.float32(1) - np.float32(0.9999)))) <= TOL


def test_scale_sgd_add_bias(L, orc, rng):
    M, N = 131072 // 8, 128
    x = rng.standard_normal(M * N, dtype=np.float32)
    s = np.array([1.7], np.float32)
    xd, sd = L.to_device(x), L.to_device(s)
    L.launch_scale_by_scalar(xd.p, sd.p, x.size, None)
    L.sync()
    assert_bits_equal(xd.download(), orc.scale_by_scalar(x, float(s[0])), "scale_by_scalar")

    g = rng.standard_normal(M * N, dtype=np.float32)
    pd, gd = L.to_device(x), L.to_device(g)
    L.launch_sgd_step(pd.p, gd.p, 0.01, x.size, None)
    L.sync()
    assert_bits_equal(pd.download(), orc.sgd_step(x, g, 0.01), "sgd_step")

    for n_cols in (N, 3, 12):
        rows = 1000
        Y = rng.standard_normal((rows, n_cols)).astype(np.float32)
        bias = rng.standard_normal(n_cols).astype(np.float32)
        Yd, bd = L.to_device(Y), L.to_device(bias)
        L.launch_add_bias(Yd.p, bd.p, rows, n_cols, None)
        L.sync()
        assert_bits_equal(Yd.download(shape=Y.shape), orc.add_bias(Y, bias), f"add_bias N={n_cols}")


@pytest.mark.parametrize("rows,N", [(1, 7), (300, 4), (131072, 128), (2 * 36, 6)])
def test_bias_grad(L, orc, rng, rows, N):
    g = rng.standard_normal((rows, N)).astype(np.float32)
    gd, out = L.to_device(g), L.alloc(N)
    out.upload(np.full(N, 5.0, np.float32))  # overwritten, not accumulated
    L.launch_bias_grad(out.p, gd.p, rows, N, None)
    L.sync()
    ref = orc.bias_grad(g, N)
    floor = np.sqrt(np.sum(g.astype(np.float64) ** 2, axis=0))
    assert rel_err(out.download(), ref, floor=floor) <= TOL
