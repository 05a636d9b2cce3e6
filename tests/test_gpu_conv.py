"""Conv helper rows: im2col (reference src/kernels.cu:750-781, 818-827) and
col2im (:785-816, 829-838) in NHWC, bit-exact.  The reference's col2im uses
atomicAdd; parity is against its sequential ascending-index order (for each
im element: ascending (oh, ow)), which the oracle runs and the gather kernel
reproduces.  cfg3 (N=128, 32x32x128, 3x3, s1 p1) at full size."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import assert_bits_equal

pytestmark = pytest.mark.gpu

GEOMS = [
    # B, H, W, C, K, stride, pad
    (128, 32, 32, 128, 3, 1, 1),  # cfg3
    (2, 6, 6, 3, 3, 1, 1),        # reference gradcheck conv3x3 (C not a multiple of 4)
    (2, 5, 5, 4, 1, 1, 0),        # conv1x1_mp
    (1, 7, 5, 4, 3, 2, 1),        # stride 2
    (2, 9, 8, 8, 4, 2, 1),        # even kernel, stride 2
    (1, 4, 4, 12, 5, 1, 2),       # kernel larger than the image's interior
    (3, 8, 8, 6, 3, 3, 0),        # stride 3, no padding
    # row-tiled im2col (C/4 divides 256, C/4 >= 4)
    (2, 9, 7, 16, 3, 1, 1),       # C/4 = 4: 64 rows per tile, ragged last tile
    (3, 10, 6, 64, 4, 2, 1),      # even kernel, stride 2
    (2, 5, 5, 32, 1, 1, 0),       # 1x1 kernel
    (1, 9, 9, 256, 3, 2, 1),      # C/4 = 64
    (1, 6, 5, 1024, 3, 1, 1),     # one row per tile
    (2, 6, 6, 48, 3, 1, 1),       # C/4 = 12 does not divide 256: generic vector path
]


def _conv_out(H, K, s, p):
    return (H + 2 * p - K) // s + 1


@pytest.mark.parametrize("geom", GEOMS, ids=lambda g: "x".join(map(str, g)))
def test_im2col_col2im_bit_exact(L, orc, rng, geom):
    B, H, W, C, K, s, p = geom
    print(f"[case] conv {geom}", flush=True)
    Ho, Wo = _conv_out(H, K, s, p), _conv_out(W, K, s, p)
    im = rng.uniform(-1, 1, (B, H, W, C)).astype(np.float32)
    imd = L.to_device(im)
    n_col = B * Ho * Wo * K * K * C
    cold = L.alloc(n_col)
    L.launch_im2col(cold.p, imd.p, B, H, W, C, K, s, p, Ho, Wo, None)
    L.sync()
    assert_bits_equal(cold.download(shape=(B * Ho * Wo, K * K * C)), orc.im2col(im, K, s, p), "im2col")
    del cold

    gcol = rng.uniform(-1, 1, (B * Ho * Wo, K * K * C)).astype(np.float32)
    gcold = L.to_device(gcol)
    # reference caller sequence: memset(grad_in) then col2im (src/conv2d.c:61-65)
    gim = L.alloc(im.size)
    gim.fill_bytes(0)
    L.launch_col2im(gim.p, gcold.p, B, H, W, C, K, s, p, Ho, Wo, None)
    L.sync()
    ref = orc.col2im(gcol, (B, H, W, C), K, s, p)
    assert_bits_equal(gim.download(shape=im.shape), ref, "col2im")
    # the fused set variant needs no memset: fill with garbage first
    gim.upload(np.full(im.size, np.nan, np.float32))
    L.launch_col2im_set(gim.p, gcold.p, B, H, W, C, K, s, p, Ho, Wo, None)
    L.sync()
    assert_bits_equal(gim.download(shape=im.shape), ref, "col2im_set")


def test_col2im_accumulates_onto_grad_im(L, orc, rng):
    """launch_col2im adds onto what grad_im holds, in the defined order."""
    B, H, W, C, K, s, p = 2, 6, 7, 8, 3, 1, 1
    Ho, Wo = _conv_out(H, K, s, p), _conv_out(W, K, s, p)
    gcol = (1e3 * rng.standard_normal((B * Ho * Wo, K * K * C))).astype(np.float32)
    init = rng.standard_normal((B, H, W, C)).astype(np.float32)
    gim, gcold = L.to_device(init), L.to_device(gcol)
    L.launch_col2im(gim.p, gcold.p, B, H, W, C, K, s, p, Ho, Wo, None)
    L.sync()
    assert_bits_equal(gim.download(shape=init.shape), orc.col2im(gcol, (B, H, W, C), K, s, p, init=init),
                      "col2im accumulate")
