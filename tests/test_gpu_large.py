"""Launches that touch at least 512 MB: the streaming kernels then use
nontemporal loads and stores (a cache-policy choice only), so each such
instantiation is checked here against the oracle at the same bar as its small
counterpart: activations (reference src/kernels.cu:21-68, 103-117), weighted
sum (:308-314), scale / sgd / add_bias (:300-306, 163-168, 95-101), mp channel
cat / split (:1251-1290), LayerNorm (:491-567)."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import TOL, assert_bits_equal, rel_err

pytestmark = pytest.mark.gpu

N_BIG = 64 * 1024 * 1024  # 256 MB per tensor: every launch below moves >= 512 MB


def test_large_activation_backward(L, orc, rng):
    print("[case] large silu backward", flush=True)
    z = rng.standard_normal(N_BIG, dtype=np.float32)
    g = rng.standard_normal(N_BIG, dtype=np.float32)
    zd, gd, od = L.to_device(z), L.to_device(g), L.alloc(N_BIG)
    L.launch_activation_backward(od.p, gd.p, zd.p, N_BIG, 3, None)
    L.sync()
    assert rel_err(od.download(), orc.act_backward(g, z, 3)) <= TOL
    L.launch_activation_forward(od.p, zd.p, N_BIG, 5, None)
    L.sync()
    assert rel_err(od.download(), orc.act_forward(z, 5)) <= TOL


def test_large_weighted_sum_scale_sgd(L, orc, rng):
    print("[case] large weighted_sum / scale / sgd", flush=True)
    a = rng.standard_normal(N_BIG, dtype=np.float32)
    b = rng.standard_normal(N_BIG, dtype=np.float32)
    ad, bd, od = L.to_device(a), L.to_device(b), L.alloc(N_BIG)
    L.launch_weighted_sum(od.p, ad.p, bd.p, 0.8, 0.6, N_BIG, None)
    L.sync()
    assert rel_err(od.download(), orc.weighted_sum(a, b, 0.8, 0.6)) <= TOL
    sd = L.to_device(np.array([1.3], np.float32))
    L.launch_scale_by_scalar(ad.p, sd.p, N_BIG, None)
    L.sync()
    assert_bits_equal(ad.download(), orc.scale_by_scalar(a, 1.3), "scale_by_scalar")
    L.launch_sgd_step(bd.p, od.p, 0.01, N_BIG, None)
    L.sync()
    assert_bits_equal(bd.download(), orc.sgd_step(b, od.download(), 0.01), "sgd_step")


def test_large_add_bias_and_channel_cat_split(L, orc, rng):
    print("[case] large add_bias / mp channel cat / split", flush=True)
    rows, Ca, Cb = 262144, 128, 128
    x = rng.standard_normal((rows, Ca + Cb), dtype=np.float32)
    bias = rng.standard_normal(Ca + Cb).astype(np.float32)
    xd, bd = L.to_device(x), L.to_device(bias)
    L.launch_add_bias(xd.p, bd.p, rows, Ca + Cb, None)
    L.sync()
    assert_bits_equal(xd.download(shape=x.shape), orc.add_bias(x, bias), "add_bias")

    a = rng.standard_normal((rows, Ca), dtype=np.float32)
    b = rng.standard_normal((rows, Cb), dtype=np.float32)
    ad, bd2, od = L.to_device(a), L.to_device(b), L.alloc(rows * (Ca + Cb))
    L.launch_mp_channel_cat(od.p, ad.p, bd2.p, 0.3, rows, Ca, Cb, None)
    L.sync()
    cat = orc.mp_cat(a, b, 0.3)
    assert_bits_equal(od.download(shape=cat.shape), cat, "mp_channel_cat")
    gad, gbd = L.alloc(rows * Ca), L.alloc(rows * Cb)
    L.launch_mp_channel_split(gad.p, gbd.p, od.p, 0.3, rows, Ca, Cb, None)
    L.sync()
    ga, gb = orc.mp_split(cat, Ca, Cb, 0.3)
    assert_bits_equal(gad.download(shape=ga.shape), ga, "grad_a")
    assert_bits_equal(gbd.download(shape=gb.shape), gb, "grad_b")


def test_large_layernorm(L, orc, rng):
    print("[case] large layernorm [262144, 256]", flush=True)
    R, C = 262144, 256
    x = (0.5 + rng.standard_normal((R, C))).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(C)).astype(np.float32)
    dy = rng.standard_normal((R, C)).astype(np.float32)
    xd, yd, gd, bd = L.to_device(x), L.alloc(x.size), L.to_device(gamma), L.to_device(beta)
    mu, rs = L.alloc(R), L.alloc(R)
    L.launch_layernorm_forward(yd.p, mu.p, rs.p, xd.p, gd.p, bd.p, R, C, 1e-5, None)
    L.sync()
    y_ref, mu_ref, rs_ref = orc.layernorm_forward(x, gamma, beta, 1e-5)
    assert rel_err(yd.download(shape=x.shape), y_ref) <= TOL
    dyd, dxd, ggd, gbd = L.to_device(dy), L.alloc(x.size), L.alloc(C), L.alloc(C)
    mud, rsd = L.to_device(mu_ref), L.to_device(rs_ref)
    L.launch_layernorm_backward(dxd.p, ggd.p, gbd.p, dyd.p, xd.p, gd.p, mud.p, rsd.p, R, C, None)
    L.sync()
    dx_ref, gg_ref, gb_ref = orc.layernorm_backward(dy, x, gamma, mu_ref, rs_ref)
    xh = (x.astype(np.float64) - mu_ref[:, None]) * rs_ref[:, None]
    fg = np.sqrt(np.sum((dy.astype(np.float64) * xh) ** 2, axis=0))
    fb = np.sqrt(np.sum(dy.astype(np.float64) ** 2, axis=0))
    assert rel_err(dxd.download(shape=x.shape), dx_ref) <= TOL
    assert rel_err(ggd.download(), gg_ref, floor=fg) <= TOL
    assert rel_err(gbd.download(), gb_ref, floor=fb) <= TOL
