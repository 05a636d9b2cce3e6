"""Convolution forward as an implicit GEMM on the matrix cores
(launch_conv2d_forward_implicit), against the reference's forward
(src/conv2d.c:17-34: im2col, GEMM, then bias add or gain scale) restated on
the CPU: the oracle's im2col (src/kernels.cu:750-781) times the weight in
double, then the bias / gain in float.  Bar 1e-5 relative to
max(|ref|, sqrt(sum of the squared products)) per output (a reduced output
over K*K*C_in terms).  Also launch_transpose (bit-exact) and the refusal of
channel counts the kernel does not take."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import TOL, assert_bits_equal

pytestmark = pytest.mark.gpu

GEOMS = [
    # B, H, W, C_in, C_out, K, stride, pad
    (128, 32, 32, 128, 128, 3, 1, 1),  # cfg3
    (3, 5, 7, 32, 128, 3, 1, 1),       # M = 105: one partial row tile
    (4, 15, 15, 64, 256, 3, 2, 1),     # stride 2, two column tiles
    (2, 8, 8, 32, 256, 1, 1, 0),       # 1x1
    (1, 9, 9, 96, 128, 5, 1, 2),       # 5x5, C_in = 3 slices of 32
    (2, 16, 16, 256, 128, 4, 2, 1),    # even kernel, stride 2
    # 64-wide output-channel tiles (C_out % 128 != 0)
    (2, 8, 8, 64, 64, 3, 1, 1),
    (3, 7, 5, 32, 192, 3, 1, 1),
    (1, 8, 8, 448, 448, 3, 1, 1),      # a DDPM-UNet width
]


def _out(H, K, s, p):
    return (H + 2 * p - K) // s + 1


def _reference(orc, x, Wt, K, s, p, bias=None, gain=None):
    col = orc.im2col(x, K, s, p).astype(np.float64)
    w = Wt.astype(np.float64)
    y = (col @ w).astype(np.float32)
    floor = np.sqrt((col * col) @ (w * w))
    if bias is not None:
        y = (y + bias[None, :]).astype(np.float32)
    if gain is not None:
        y = (y * np.float32(gain)).astype(np.float32)
    return y, floor


# every geometry with the bias epilogue; gain and none on the first two
CASES = [(g, "bias") for g in GEOMS] + [(g, e) for g in GEOMS[:2] for e in ("gain", "none")]


@pytest.mark.parametrize("geom,epi", CASES, ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else v)
def test_conv_forward_implicit(L, orc, rng, geom, epi):
    B, H, W, Ci, Co, K, s, p = geom
    print(f"[case] implicit conv {geom} {epi}", flush=True)
    Ho, Wo = _out(H, K, s, p), _out(W, K, s, p)
    x = rng.standard_normal((B, H, W, Ci)).astype(np.float32)
    Wt = (rng.standard_normal((K * K * Ci, Co)) / np.sqrt(K * K * Ci)).astype(np.float32)
    bias = (0.1 * rng.standard_normal(Co)).astype(np.float32)
    gain = 1.37
    xd, Wd, yd = L.to_device(x), L.to_device(Wt), L.alloc(B * Ho * Wo * Co)
    WTd, bd, gd = L.alloc(Wt.size), L.to_device(bias), L.to_device(np.array([gain], np.float32))
    L.launch_transpose(WTd.p, Wd.p, K * K * Ci, Co, None)
    L.launch_conv2d_forward_implicit(yd.p, xd.p, WTd.p, bd.p if epi == "bias" else None,
                                     gd.p if epi == "gain" else None, B, H, W, Ci, Co, K, s, p, Ho, Wo, None)
    L.sync()
    assert_bits_equal(WTd.download(shape=(Co, K * K * Ci)), np.ascontiguousarray(Wt.T), "transpose")
    y_ref, floor = _reference(orc, x, Wt, K, s, p, bias if epi == "bias" else None, gain if epi == "gain" else None)
    got = yd.download(shape=y_ref.shape).astype(np.float64)
    scale = gain if epi == "gain" else 1.0
    err = np.abs(got - y_ref) / np.maximum(np.abs(y_ref), scale * floor)
    assert float(err.max()) <= TOL


def test_conv_forward_implicit_refuses_unsupported_channels(L, nn):
    print("[case] implicit conv refusals", flush=True)
    assert L.nnhip_conv2d_implicit_supported(128, 128) == 1
    assert L.nnhip_conv2d_implicit_supported(3, 128) == 0
    assert L.nnhip_conv2d_implicit_supported(128, 64) == 1
    assert L.nnhip_conv2d_implicit_supported(128, 96) == 0
    dummy = L.alloc(64)
    with pytest.raises(nn.NnHipError):
        L.launch_conv2d_forward_implicit(dummy.p, dummy.p, dummy.p, None, None, 1, 4, 4, 3, 128, 3, 1, 1, 4, 4, None)
    with pytest.raises(nn.NnHipError):
        L.launch_conv2d_forward_implicit(dummy.p, dummy.p, dummy.p, None, None, 1, 4, 4, 32, 96, 3, 1, 1, 4, 4, None)
    with pytest.raises(nn.NnHipError):
        L.launch_conv2d_forward_implicit(dummy.p, dummy.p, dummy.p, None, None, 1, 4, 4, 32, 128, 3, 1, 1, 5, 4, None)


WGRAD_GEOMS = [
    # B, H, W, C_in, C_out, K, stride, pad
    (128, 32, 32, 128, 128, 3, 1, 1),  # cfg3
    (3, 5, 7, 64, 128, 3, 1, 1),       # K*K*C_in = 576: a partial k tile
    (4, 15, 15, 12, 256, 3, 2, 1),     # stride 2, C_in = 12
    (2, 8, 8, 32, 128, 1, 1, 0),       # 1x1
    (1, 9, 9, 4, 128, 5, 1, 2),        # 5x5, C_in = 4
    (4, 8, 8, 64, 64, 3, 1, 1),        # 64-wide output-channel tiles
    (2, 6, 6, 12, 192, 3, 1, 1),
]


@pytest.mark.parametrize("geom", WGRAD_GEOMS, ids=lambda g: "x".join(map(str, g)))
def test_conv_weight_grad_implicit(L, orc, rng, geom):
    """gW = im2col(x)^T dy (the reference's gemm_dW over launch_im2col,
    src/conv2d.c:44-47) in double, bar 1e-5 relative to
    max(|ref|, sqrt(sum of the squared products)); a lent workspace gives the
    same bits as the library scratch."""
    B, H, W, Ci, Co, K, s, p = geom
    print(f"[case] implicit conv weight grad {geom}", flush=True)
    Ho, Wo = _out(H, K, s, p), _out(W, K, s, p)
    x = rng.standard_normal((B, H, W, Ci)).astype(np.float32)
    dy = rng.standard_normal((B * Ho * Wo, Co)).astype(np.float32)
    xd, dyd, gw = L.to_device(x), L.to_device(dy), L.alloc(K * K * Ci * Co)
    L.launch_conv2d_weight_grad_implicit(gw.p, xd.p, dyd.p, B, H, W, Ci, Co, K, s, p, Ho, Wo, None, None)
    L.sync()
    col = orc.im2col(x, K, s, p).astype(np.float64)
    d = dy.astype(np.float64)
    ref = col.T @ d
    floor = np.sqrt((col * col).T @ (d * d))
    got = gw.download(shape=ref.shape).astype(np.float64)
    assert float((np.abs(got - ref) / np.maximum(np.abs(ref), floor)).max()) <= TOL
    ws = L.alloc(max(1, L.nnhip_conv2d_wgrad_workspace(B, Ci, Co, K, Ho, Wo)))
    gw2 = L.alloc(K * K * Ci * Co)
    L.launch_conv2d_weight_grad_implicit(gw2.p, xd.p, dyd.p, B, H, W, Ci, Co, K, s, p, Ho, Wo, ws.p, None)
    L.sync()
    assert_bits_equal(gw2.download(), gw.download(), "workspace vs scratch")
