"""GroupNorm (+ fused activation) parity: HIP launch layer vs the CPU oracle.

Reference maths: src/kernels.cu:622-745 (GroupNorm) and the GN -> SiLU
composition of src/conv_residual.c:28-29, 51-52.  Shapes cover both kernel
paths: register-resident (cpg in {4, 8, 16}, aligned) and generic (cpg = 2,
32, misaligned pointers), masked tails (HW not a multiple of the pixel step),
the cfg1 shape and one full sample of the north-star shape.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import TOL, gn_param_floor, rel_err

pytestmark = pytest.mark.gpu

SHAPES = [
    # B, H, W, C, G
    (8, 32, 32, 128, 32),  # cfg1 (plumbing), cpg 4, register path
    (2, 6, 6, 8, 4),       # reference gradcheck shape, cpg 2, generic path
    (2, 8, 8, 32, 8),      # cpg 4
    (3, 5, 7, 64, 8),      # cpg 8, HW = 35 (masked slots)
    (2, 4, 4, 64, 4),      # cpg 16
    (2, 16, 16, 96, 3),    # cpg 32 -> generic
    (2, 9, 9, 16, 4),      # cpg 4, HW = 81
    (1, 64, 64, 256, 32),  # one sample of the north-star shape (1024 threads x 8 float4)
    (2, 100, 100, 8, 2),   # cpg 4, group of 40000 floats: too big for registers -> generic
    (2, 28, 28, 32, 32),   # cpg 1 (the reference DDPM model's first level) -> generic
]


def make_inputs(rng, B, H, W, C):
    x = rng.standard_normal((B, H * W, C), dtype=np.float32)
    gamma = (1.0 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(C)).astype(np.float32)
    dy = rng.standard_normal((B, H * W, C), dtype=np.float32)
    return x, gamma, beta, dy


def gpu_forward(L, x, gamma, beta, G, act, offset=0):
    B, HW, C = x.shape
    n = x.size
    xd, yd = L.alloc(n + offset), L.alloc(n + offset)
    gd, bd = L.to_device(gamma), L.to_device(beta)
    mu, rs = L.alloc(B * G), L.alloc(B * G)
    xd.upload(np.concatenate([np.zeros(offset, np.float32), x.ravel()]))
    L.launch_groupnorm_act_forward(yd.offset(offset), mu.p, rs.p, xd.offset(offset), gd.p, bd.p, B, HW, C, G,
                                   1e-5, act, None)
    L.sync()
    y = yd.download()[offset:].reshape(x.shape)
    return y, mu.download(), rs.download()


def gpu_backward(L, dy, x, gamma, beta, mu, rs, G, act, offset=0):
    B, HW, C = x.shape
    n = x.size
    pad = np.zeros(offset, np.float32)
    xd, dyd, dxd = L.alloc(n + offset), L.alloc(n + offset), L.alloc(n + offset)
    xd.upload(np.concatenate([pad, x.ravel()]))
    dyd.upload(np.concatenate([pad, dy.ravel()]))
    gd, bd = L.to_device(gamma), L.to_device(beta)
    mud, rsd = L.to_device(mu), L.to_device(rs)
    ggd, gbd = L.alloc(C), L.alloc(C)
    L.launch_groupnorm_act_backward(dxd.offset(offset), ggd.p, gbd.p, dyd.offset(offset), xd.offset(offset), gd.p,
                                    bd.p, mud.p, rsd.p, B, HW, C, G, act, None)
    L.sync()
    return dxd.download()[offset:].reshape(x.shape), ggd.download(), gbd.download()


def effective_terms(orc, x, gamma, beta, mu, rs, dy, G, act):
    """d = dy*act'(h) and xhat, for the floors of the channel sums."""
    B, HW, C = x.shape
    cpg = C // G
    m = np.repeat(mu.reshape(B, G), cpg, axis=1)[:, None, :]
    r = np.repeat(rs.reshape(B, G), cpg, axis=1)[:, None, :]
    xh = ((x - m) * r).astype(np.float32)
    h = (gamma * xh + beta).astype(np.float32)
    d = orc.act_backward(dy, h, act).reshape(x.shape) if act else dy
    return d, xh


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("act", [0, 3], ids=["identity", "silu"])
def test_groupnorm_act_forward_backward(L, orc, rng, shape, act):
    B, H, W, C, G = shape
    print(f"[case] groupnorm act={act} shape={shape}", flush=True)
    x, gamma, beta, dy = make_inputs(rng, B, H, W, C)
    y_ref, mu_ref, rs_ref = orc.groupnorm_forward(x, gamma, beta, G, 1e-5, act)
    y, mu, rs = gpu_forward(L, x, gamma, beta, G, act)
    assert rel_err(y, y_ref) <= TOL
    assert rel_err(mu, mu_ref, floor=1e-3) <= TOL
    assert rel_err(rs, rs_ref) <= TOL

    # backward from the same cached statistics on both sides
    dx_ref, gg_ref, gb_ref = orc.groupnorm_backward(dy, x, gamma, beta, mu_ref, rs_ref, G, act)
    dx, gg, gb = gpu_backward(L, dy, x, gamma, beta, mu_ref, rs_ref, G, act)
    d, xh = effective_terms(orc, x, gamma, beta, mu_ref, rs_ref, dy, G, act)
    fg, fb = gn_param_floor(d, xh, C)
    assert rel_err(dx, dx_ref) <= TOL
    assert rel_err(gg, gg_ref, floor=fg) <= TOL
    assert rel_err(gb, gb_ref, floor=fb) <= TOL


@pytest.mark.parametrize("act", [1, 2, 4, 5], ids=["relu", "gelu", "tanh", "mp_silu"])
def test_groupnorm_other_activations(L, orc, rng, act):
    B, H, W, C, G = 2, 8, 8, 64, 8
    x, gamma, beta, dy = make_inputs(rng, B, H, W, C)
    y_ref, mu_ref, rs_ref = orc.groupnorm_forward(x, gamma, beta, G, 1e-5, act)
    y, _, _ = gpu_forward(L, x, gamma, beta, G, act)
    assert rel_err(y, y_ref) <= TOL
    dx_ref, gg_ref, gb_ref = orc.groupnorm_backward(dy, x, gamma, beta, mu_ref, rs_ref, G, act)
    dx, gg, gb = gpu_backward(L, dy, x, gamma, beta, mu_ref, rs_ref, G, act)
    d, xh = effective_terms(orc, x, gamma, beta, mu_ref, rs_ref, dy, G, act)
    fg, fb = gn_param_floor(d, xh, C)
    assert rel_err(dx, dx_ref) <= TOL
    assert rel_err(gg, gg_ref, floor=fg) <= TOL
    assert rel_err(gb, gb_ref, floor=fb) <= TOL


def test_groupnorm_misaligned_takes_generic_path(L, orc, rng):
    B, H, W, C, G = 2, 8, 8, 32, 8
    x, gamma, beta, dy = make_inputs(rng, B, H, W, C)
    y_ref, mu_ref, rs_ref = orc.groupnorm_forward(x, gamma, beta, G, 1e-5, 3)
    y, _, _ = gpu_forward(L, x, gamma, beta, G, 3, offset=1)
    assert rel_err(y, y_ref) <= TOL
    dx_ref, gg_ref, gb_ref = orc.groupnorm_backward(dy, x, gamma, beta, mu_ref, rs_ref, G, 3)
    dx, gg, gb = gpu_backward(L, dy, x, gamma, beta, mu_ref, rs_ref, G, 3, offset=1)
    assert rel_err(dx, dx_ref) <= TOL


def test_plain_groupnorm_launchers_match_reference_signature(L, orc, rng):
    """launch_groupnorm_forward/backward (reference nn.h:400-407) = act IDENTITY."""
    B, H, W, C, G = 2, 8, 8, 32, 8
    x, gamma, beta, dy = make_inputs(rng, B, H, W, C)
    y_ref, mu_ref, rs_ref = orc.groupnorm_forward(x, gamma, beta, G, 1e-5, 0)
    xd, yd, dyd, dxd = L.to_device(x), L.alloc(x.size), L.to_device(dy), L.alloc(x.size)
    gd, bd = L.to_device(gamma), L.to_device(beta)
    mu, rs, gg, gb = L.alloc(B * G), L.alloc(B * G), L.alloc(C), L.alloc(C)
    L.launch_groupnorm_forward(yd.p, mu.p, rs.p, xd.p, gd.p, bd.p, B, H * W, C, G, 1e-5, None)
    L.launch_groupnorm_backward(dxd.p, gg.p, gb.p, dyd.p, xd.p, gd.p, mu.p, rs.p, B, H * W, C, G, None)
    L.sync()
    assert rel_err(yd.download(shape=x.shape), y_ref) <= TOL
    dx_ref, gg_ref, gb_ref = orc.groupnorm_backward(dy, x, gamma, beta, mu.download(), rs.download(), G, 0)
    assert rel_err(dxd.download(shape=x.shape), dx_ref) <= TOL
    d, xh = effective_terms(orc, x, gamma, beta, mu.download(), rs.download(), dy, G, 0)
    fg, fb = gn_param_floor(d, xh, C)
    assert rel_err(gg.download(), gg_ref, floor=fg) <= TOL
    assert rel_err(gb.download(), gb_ref, floor=fb) <= TOL


def test_groupnorm_empty_batch_and_bad_shapes(L, nn):
    C, G = 16, 4
    gg, gb = L.to_device(np.full(C, 7.0, np.float32)), L.to_device(np.full(C, 7.0, np.float32))
    dummy = L.alloc(16)
    # batch 0: the channel sums are empty, i.e. zero (reference param kernel loop)
    L.launch_groupnorm_backward(dummy.p, gg.p, gb.p, dummy.p, dummy.p, dummy.p, dummy.p, dummy.p, 0, 4, C, G, None)
    L.sync()
    assert np.all(gg.download() == 0) and np.all(gb.download() == 0)
    with pytest.raises(nn.NnHipError):
        L.launch_groupnorm_forward(dummy.p, dummy.p, dummy.p, dummy.p, dummy.p, dummy.p, 1, 4, 10, 4, 1e-5, None)
