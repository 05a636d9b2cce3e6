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


def test_north_star_full_size_groupnorm_silu(L, orc):
    """The bench workload at its full size, GN(32)+SiLU forward and backward on
    [256, 64, 64, 256] (1 GiB per tensor) through the bench's launchers and
    lent workspaces: y and dx of three samples against the oracle, and
    dgamma/dbeta against the oracle's per-sample backward summed over all 256
    samples (the batch sum is linear), at the 1e-5 bar."""
    print("[case] north-star full size GN(32)+SiLU", flush=True)
    B, HW, C, G = 256, 64 * 64, 256, 32
    rng = np.random.default_rng(410293)
    x = rng.standard_normal((B, HW, C), dtype=np.float32)
    dy = rng.standard_normal((B, HW, C), dtype=np.float32)
    gamma = (1.0 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(C)).astype(np.float32)
    xd, dyd = L.to_device(x), L.to_device(dy)
    yd, dxd = L.alloc(x.size), L.alloc(x.size)
    gd, bd, ggd, gbd = L.to_device(gamma), L.to_device(beta), L.alloc(C), L.alloc(C)
    mud, rsd = L.alloc(B * G), L.alloc(B * G)
    fws = L.to_device(np.zeros(max(1, L.nnhip_groupnorm_forward_workspace(B, HW, C, G)), np.float32))
    bws = L.to_device(np.zeros(L.nnhip_groupnorm_backward_workspace(B, HW, C, G), np.float32))
    L.launch_groupnorm_act_forward_ws(yd.p, mud.p, rsd.p, xd.p, gd.p, bd.p, B, HW, C, G, 1e-5, 3, fws.p, None)
    L.launch_groupnorm_act_backward_ws(dxd.p, ggd.p, gbd.p, dyd.p, xd.p, gd.p, bd.p, mud.p, rsd.p, B, HW, C, G, 3,
                                       bws.p, None)
    L.sync()
    assert L.nnhip_groupnorm_workspace_status(fws.p) == 0
    assert L.nnhip_groupnorm_workspace_status(bws.p) == 0
    n = HW * C
    for b in (0, 131, 255):
        y_ref, mu_ref, rs_ref = orc.groupnorm_forward(x[b:b + 1], gamma, beta, G, 1e-5, 3)
        y = np.empty(n, np.float32)
        L.dll.nnhip_memcpy_dtoh(y.ctypes.data, yd.offset(b * n), 4 * n)
        assert rel_err(y.reshape(y_ref.shape), y_ref) <= TOL
        dx_ref, _, _ = orc.groupnorm_backward(dy[b:b + 1], x[b:b + 1], gamma, beta, mu_ref, rs_ref, G, 3)
        dxs = np.empty(n, np.float32)
        L.dll.nnhip_memcpy_dtoh(dxs.ctypes.data, dxd.offset(b * n), 4 * n)
        assert rel_err(dxs.reshape(dx_ref.shape), dx_ref) <= TOL
    gg_ref = np.zeros(C, np.float64)
    gb_ref = np.zeros(C, np.float64)
    sq_g = np.zeros(C, np.float64)
    sq_b = np.zeros(C, np.float64)
    for b in range(B):
        _, mu_b, rs_b = orc.groupnorm_forward(x[b:b + 1], gamma, beta, G, 1e-5, 3)
        _, gg_b, gb_b = orc.groupnorm_backward(dy[b:b + 1], x[b:b + 1], gamma, beta, mu_b, rs_b, G, 3)
        gg_ref += gg_b
        gb_ref += gb_b
        sq_g += gg_b.astype(np.float64) ** 2
        sq_b += gb_b.astype(np.float64) ** 2
    # floor: the root of the summed squared per-sample terms bounds the sums' scale
    assert rel_err(ggd.download(), gg_ref, floor=np.sqrt(sq_g)) <= TOL
    assert rel_err(gbd.download(), gb_ref, floor=np.sqrt(sq_b)) <= TOL
