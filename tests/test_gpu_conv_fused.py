"""The implicit-GEMM convolutions with a neighbouring pass of the diffusion
blocks folded in (launch_conv2d_*_implicit_fused) against the same work as
separate launches: the plain implicit launcher, then the pass the reference
block runs next (src/cond_conv_residual.c:29-35, 53-54, 61;
src/conv_residual.c:38-39).  Each fused form keeps the operation order of
the pass it replaces, so the comparison is bit for bit:
* forward + residual: launch_weighted_sum(y, res, y, wa, wb);
* forward + modulate + activation: launch_spatial_modulate_act_forward;
* input gradient + activation gradient + residual: launch_activation_backward,
  then launch_weighted_sum(dx, res, dx, wa, 1).
The separate launches themselves are checked against the oracle by
test_gpu_conv_implicit.py, test_gpu_spatial.py and test_gpu_elementwise.py.
Geometries cover a partial row tile, both output-channel tile widths, stride 2
and the EDM block's cfg2 shape."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from helpers import assert_bits_equal

pytestmark = pytest.mark.gpu

ACT_SILU, ACT_MP_SILU = 3, 5

FWD_GEOMS = [
    # B, H, W, C_in, C_out, K, stride, pad
    (3, 5, 7, 32, 128, 3, 1, 1),      # M = 105: one partial row tile
    (2, 8, 8, 64, 64, 3, 1, 1),       # 64-wide output-channel tiles
    (4, 15, 15, 64, 256, 3, 2, 1),    # stride 2, two column tiles
    (16, 32, 32, 128, 128, 3, 1, 1),  # EDM block width (16 samples of cfg2)
]

# input gradient: B, H, W, C_in, C_out, K, pad (stride 1)
DGRAD_GEOMS = [
    (3, 5, 7, 128, 32, 3, 1),
    (2, 8, 8, 64, 64, 3, 1),
    (16, 32, 32, 128, 128, 3, 1),
]


def _out(H, K, s, p):
    return (H + 2 * p - K) // s + 1


def _fusion(nn, **kw):
    f = nn.NnConvFusion()
    for k, v in kw.items():
        setattr(f, k, v)
    return f


def _weights(rng, K, Ci, Co):
    return (rng.standard_normal((K * K * Ci, Co)) / np.sqrt(K * K * Ci)).astype(np.float32)


@pytest.mark.parametrize("epi", ["bias", "gain", "none"])
@pytest.mark.parametrize("geom", FWD_GEOMS, ids=lambda g: "x".join(map(str, g)))
def test_forward_residual_matches_separate_launches(L, nn, rng, geom, epi):
    B, H, W, Ci, Co, K, s, p = geom
    print(f"[case] fused conv forward + residual {geom} {epi}", flush=True)
    Ho, Wo = _out(H, K, s, p), _out(W, K, s, p)
    n = B * Ho * Wo * Co
    xd = L.to_device(rng.standard_normal((B, H, W, Ci)).astype(np.float32))
    Wd = L.to_device(_weights(rng, K, Ci, Co))
    bd = L.to_device((0.1 * rng.standard_normal(Co)).astype(np.float32))
    gd = L.to_device(np.array([1.37], np.float32))
    res = L.to_device(rng.standard_normal(n).astype(np.float32))
    bias, gain = (bd.p if epi == "bias" else None), (gd.p if epi == "gain" else None)
    wa, wb = 0.8320503, 0.5547002  # mp_sum weights at t = 0.4
    want, got = L.alloc(n), L.alloc(n)
    L.launch_conv2d_forward_implicit(want.p, xd.p, Wd.p, bias, gain, B, H, W, Ci, Co, K, s, p, Ho, Wo, None)
    L.launch_weighted_sum(want.p, res.p, want.p, wa, wb, n, None)
    f = _fusion(nn, res=res.p, res_w=wa, out_w=wb)
    L.launch_conv2d_forward_implicit_fused(got.p, xd.p, Wd.p, bias, gain, B, H, W, Ci, Co, K, s, p, Ho, Wo,
                                           C.addressof(f), None)
    L.sync()
    assert_bits_equal(got.download(), want.download(), "y")


@pytest.mark.parametrize("act", [ACT_MP_SILU, ACT_SILU], ids=["mp_silu", "silu"])
@pytest.mark.parametrize("geom", FWD_GEOMS, ids=lambda g: "x".join(map(str, g)))
def test_forward_modulate_act_matches_separate_launches(L, nn, rng, geom, act):
    B, H, W, Ci, Co, K, s, p = geom
    print(f"[case] fused conv forward + modulate act={act} {geom}", flush=True)
    Ho, Wo = _out(H, K, s, p), _out(W, K, s, p)
    n = B * Ho * Wo * Co
    xd = L.to_device(rng.standard_normal((B, H, W, Ci)).astype(np.float32))
    Wd = L.to_device(_weights(rng, K, Ci, Co))
    gd = L.to_device(np.array([0.91], np.float32))
    cd = L.to_device((0.5 * rng.standard_normal((B, Co))).astype(np.float32))
    y_want, y2_want, y_got, y2_got = L.alloc(n), L.alloc(n), L.alloc(n), L.alloc(n)
    L.launch_conv2d_forward_implicit(y_want.p, xd.p, Wd.p, None, gd.p, B, H, W, Ci, Co, K, s, p, Ho, Wo, None)
    L.launch_spatial_modulate_act_forward(y2_want.p, y_want.p, cd.p, B, Ho * Wo, 1, Co, act, None)
    f = _fusion(nn, cond=cd.p, y2=y2_got.p, act=act)
    L.launch_conv2d_forward_implicit_fused(y_got.p, xd.p, Wd.p, None, gd.p, B, H, W, Ci, Co, K, s, p, Ho, Wo,
                                           C.addressof(f), None)
    L.sync()
    assert_bits_equal(y_got.download(), y_want.download(), "y")
    assert_bits_equal(y2_got.download(), y2_want.download(), "y2")


@pytest.mark.parametrize("act", [ACT_MP_SILU, ACT_SILU], ids=["mp_silu", "silu"])
@pytest.mark.parametrize("with_gain", [True, False], ids=["gain", "plain"])
@pytest.mark.parametrize("geom", DGRAD_GEOMS, ids=lambda g: "x".join(map(str, g)))
def test_input_grad_act_residual_matches_separate_launches(L, nn, rng, geom, with_gain, act):
    B, H, W, Ci, Co, K, p = geom
    print(f"[case] fused conv input grad + act' + residual {geom} gain={with_gain} act={act}", flush=True)
    Ho, Wo = _out(H, K, 1, p), _out(W, K, 1, p)
    n_in = B * H * W * Ci
    dyd = L.to_device(rng.standard_normal((B, Ho, Wo, Co)).astype(np.float32))
    Wd = L.to_device(_weights(rng, K, Ci, Co))
    gd = L.to_device(np.array([0.73], np.float32))
    xa = L.to_device((2.0 * rng.standard_normal(n_in)).astype(np.float32))
    res = L.to_device(rng.standard_normal(n_in).astype(np.float32))
    gain = gd.p if with_gain else None
    wa = 0.8320503
    dxr, want, got = L.alloc(n_in), L.alloc(n_in), L.alloc(n_in)
    L.launch_conv2d_input_grad_implicit(dxr.p, dyd.p, Wd.p, gain, B, H, W, Ci, Co, K, p, None)
    L.launch_activation_backward(want.p, dxr.p, xa.p, n_in, act, None)
    L.launch_weighted_sum(want.p, res.p, want.p, wa, 1.0, n_in, None)
    f = _fusion(nn, act_in=xa.p, act=act, res=res.p, res_w=wa, out_w=1.0)
    L.launch_conv2d_input_grad_implicit_fused(got.p, dyd.p, Wd.p, gain, B, H, W, Ci, Co, K, p, C.addressof(f), None)
    L.sync()
    assert_bits_equal(got.download(), want.download(), "dx")


def test_fused_refusals(L, nn):
    """Combinations that are not built are refused before any launch."""
    print("[case] fused conv refusals", flush=True)
    d = L.alloc(64)
    fwd = (d.p, d.p, d.p, None, None, 1, 4, 4, 32, 128, 3, 1, 1, 4, 4)
    dg = (d.p, d.p, d.p, None, 1, 4, 4, 128, 128, 3, 1)
    bad_fwd = [_fusion(nn), _fusion(nn, res=d.p, cond=d.p, y2=d.p, act=ACT_SILU),
               _fusion(nn, cond=d.p, y2=d.p, act=1), _fusion(nn, res=d.p, act_in=d.p)]
    for f in bad_fwd:
        with pytest.raises(nn.NnHipError):
            L.launch_conv2d_forward_implicit_fused(*fwd, C.addressof(f), None)
    bad_dg = [_fusion(nn), _fusion(nn, act_in=d.p, act=ACT_SILU), _fusion(nn, res=d.p),
              _fusion(nn, act_in=d.p, res=d.p, act=2), _fusion(nn, cond=d.p, act_in=d.p, res=d.p, act=ACT_SILU)]
    for f in bad_dg:
        with pytest.raises(nn.NnHipError):
            L.launch_conv2d_input_grad_implicit_fused(*dg, C.addressof(f), None)
