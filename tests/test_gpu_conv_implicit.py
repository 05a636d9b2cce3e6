"""Convolution as implicit GEMMs on the matrix cores, against the
reference's sequences restated on the CPU in double:
* forward (launch_conv2d_forward_implicit; src/conv2d.c:17-34: im2col, GEMM,
  then bias add or gain scale): the oracle's im2col (src/kernels.cu:750-781)
  times the weight, then the bias / gain in float;
* weight gradient (launch_conv2d_weight_grad_implicit; src/conv2d.c:44-47):
  im2col(x)^T dy;
* stride-1 input gradient (launch_conv2d_input_grad_implicit;
  src/conv2d.c:48-65: dcol = dy W^T, then col2im): the col2im as the adjoint
  of the oracle's im2col, summed in double.
Bar 1e-5 relative to max(|ref|, sqrt(sum of the squared products)) per
output (each output is a sum of many products), plus the refusal of shapes
the kernels do not take."""
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
    bd, gd = L.to_device(bias), L.to_device(np.array([gain], np.float32))
    L.launch_conv2d_forward_implicit(yd.p, xd.p, Wd.p, bd.p if epi == "bias" else None,
                                     gd.p if epi == "gain" else None, B, H, W, Ci, Co, K, s, p, Ho, Wo, None)
    L.sync()
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


DGRAD_GEOMS = [
    # B, H, W, C_in, C_out, K, pad (stride 1); the layer's shapes: dx is
    # [B, H, W, C_in], dy [B, H + 2 pad - K + 1, ..., C_out]
    (128, 32, 32, 128, 128, 3, 1),  # cfg3 (images 0 and B-1 checked)
    (3, 5, 7, 64, 32, 3, 1),        # M = 105: one partial row tile; one tap per k slice
    (2, 8, 8, 128, 64, 1, 0),       # 1x1
    (1, 9, 9, 192, 96, 5, 2),       # 5x5, 64-wide tiles, 3 slices per tap
    (2, 6, 6, 64, 32, 3, 0),        # no padding: the gradient's padding is K-1
    (2, 7, 7, 256, 128, 4, 2),      # even kernel, padding above K/2
    (1, 8, 8, 448, 448, 3, 1),      # a DDPM-UNet width (64-wide tiles)
]


def _input_grad_reference(orc, dy_b, Wt, shape, K, pad):
    """dx of one image, [H, W, C_in], in double: dcol = dy W^T scattered back
    through im2col's index map (col2im as im2col's adjoint), and the root sum
    of the squared products as the error floor."""
    H, W, Ci = shape
    idx = (np.arange(H * W * Ci, dtype=np.float64) + 1).astype(np.float32).reshape(1, H, W, Ci)
    cidx = orc.im2col(idx, K, 1, pad).astype(np.int64).ravel()  # 0 marks padding
    w = Wt.astype(np.float64)
    d = dy_b.astype(np.float64)
    dcol = (d @ w.T).ravel()
    sq = ((d * d) @ (w * w).T).ravel()
    n = H * W * Ci + 1
    ref = np.bincount(cidx, weights=dcol, minlength=n)[1:].reshape(H, W, Ci)
    floor = np.sqrt(np.bincount(cidx, weights=sq, minlength=n)[1:]).reshape(H, W, Ci)
    return ref, floor


CASES_DG = [(g, False) for g in DGRAD_GEOMS] + [(DGRAD_GEOMS[1], True)]


@pytest.mark.parametrize("geom,with_gain", CASES_DG,
                         ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else ("gain" if v else "plain"))
def test_conv_input_grad_implicit(L, orc, rng, geom, with_gain):
    B, H, W, Ci, Co, K, p = geom
    print(f"[case] implicit conv input grad {geom} gain={with_gain}", flush=True)
    Ho, Wo = _out(H, K, 1, p), _out(W, K, 1, p)
    assert L.nnhip_conv2d_input_grad_implicit_supported(Ci, Co, K, 1, p) == 1
    dy = rng.standard_normal((B, Ho, Wo, Co)).astype(np.float32)
    Wt = (rng.standard_normal((K * K * Ci, Co)) / np.sqrt(K * K * Co)).astype(np.float32)
    gain = 0.73
    dyd, Wd, dxd = L.to_device(dy), L.to_device(Wt), L.alloc(B * H * W * Ci)
    gd = L.to_device(np.array([gain], np.float32))
    L.launch_conv2d_input_grad_implicit(dxd.p, dyd.p, Wd.p, gd.p if with_gain else None, B, H, W, Ci, Co, K, p, None)
    L.sync()
    got = dxd.download(shape=(B, H, W, Ci)).astype(np.float64)
    scale = gain if with_gain else 1.0
    images = range(B) if B <= 4 else (0, B - 1)
    for b in images:
        ref, floor = _input_grad_reference(orc, dy[b].reshape(Ho * Wo, Co), Wt, (H, W, Ci), K, p)
        err = np.abs(got[b] - scale * ref) / np.maximum(np.abs(scale * ref), scale * floor)
        assert float(err.max()) <= TOL, b


def test_conv_input_grad_implicit_refusals(L, nn):
    print("[case] implicit conv input grad refusals", flush=True)
    assert L.nnhip_conv2d_input_grad_implicit_supported(128, 128, 3, 1, 1) == 1
    assert L.nnhip_conv2d_input_grad_implicit_supported(128, 128, 3, 2, 1) == 0  # stride 2
    assert L.nnhip_conv2d_input_grad_implicit_supported(128, 128, 3, 1, 3) == 0  # pad > K - 1
    assert L.nnhip_conv2d_input_grad_implicit_supported(96, 128, 3, 1, 1) == 0   # C_in % 64
    assert L.nnhip_conv2d_input_grad_implicit_supported(128, 48, 3, 1, 1) == 0   # C_out % 32
    dummy = L.alloc(64)
    with pytest.raises(nn.NnHipError):
        L.launch_conv2d_input_grad_implicit(dummy.p, dummy.p, dummy.p, None, 1, 4, 4, 128, 128, 3, 3, None)
    with pytest.raises(nn.NnHipError):
        L.launch_conv2d_input_grad_implicit(dummy.p, dummy.p, dummy.p, None, 1, 4, 4, 96, 128, 3, 1, None)
    with pytest.raises(nn.NnHipError):  # a weight of 2^31 elements or more
        L.launch_conv2d_input_grad_implicit(dummy.p, dummy.p, dummy.p, None, 1, 4, 4, 16384, 16384, 3, 1, None)
