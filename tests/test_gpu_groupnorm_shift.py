"""GroupNorm + activation of x + shift[b, c]
(launch_groupnorm_act_shift_forward_ws / _backward_ws): the DDPM block's
embedding broadcast add folded into GN2, and the embedding gradient's pixel
sum folded into GN2's backward (reference src/conv_residual.c:34-37, 51-55).

Bars:
  * y, mu, rstd, dx, dgamma, dbeta are bit-identical to the plain launchers
    run on xs = x + shift formed in float32 (one rounding per element, as
    launch_spatial_add stores it): the reference's own composition;
  * gshift, summed per 64-pixel tile and then over the tiles, is within TOL of
    the float64 pixel sum of that dx, relative to max(|sum|, sqrt(sum dx^2))
    per channel (the floor of every reduced output in these tests);
  * on one case, y and dx against the oracle's composition.
The shift launchers run fused persistent kernels only: SiLU, the forward at 8
or 16 channels per group and the backward at 4, 8 or 16 with one record per
merging lane (at most 64 pixel tiles per sample and column block), where the
path policy picks the streaming kernels.  Every other case is refused with an
error, writes nothing and allocates nothing (nnhip_groupnorm_shift_supported
says which direction takes a shape); the caller then composes the plain
launchers, which the DDPM block does (tests/test_gpu_blocks.py).  Where the
fused kernels run, the workspaces must hold this launch's tagged records.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import TOL, assert_bits_equal, rel_err
from test_gpu_groupnorm import make_inputs
from test_gpu_groupnorm_stream import BWD_TP, FWD_TP, records_tagged, tiles, zeroed

pytestmark = pytest.mark.gpu

SILU = 3
SENTINEL = np.float32(1234.5)


def shift_case(rng, B, C):
    return (0.5 * rng.standard_normal((B, C))).astype(np.float32)


def refused(L, what):
    """The last call recorded an error naming the fused shift kernels."""
    code, msg = L.last_error()
    assert code != 0 and "fused shift kernels" in msg, (what, code, msg)


def run_shift(L, x, sh, gamma, beta, dy, G, act, fws, bws, fwd=True, bwd=True, stats=None):
    """The fused launchers; returns (y, mu, rstd, dx, gshift, dgamma, dbeta).
    A direction not asked for is called anyway and must be refused, leaving
    its outputs at the sentinel and the library's allocation count as it was;
    its entries are then None.  The backward of a refused forward reads the
    statistics `stats` = (mu, rstd) of the plain forward on x + shift."""
    B, HW, C = x.shape
    xd, shd, dyd = L.to_device(x), L.to_device(sh), L.to_device(dy)
    gd, bd = L.to_device(gamma), L.to_device(beta)
    fill = lambda n: L.to_device(np.full(n, SENTINEL, np.float32))
    yd, dxd, gsd = fill(x.size), fill(x.size), fill(B * C)
    mud, rsd, ggd, gbd = fill(B * G), fill(B * G), fill(C), fill(C)
    L.sync()
    allocs = L.nnhip_launch_allocations()
    args_f = (yd.p, mud.p, rsd.p, xd.p, shd.p, gd.p, bd.p, B, HW, C, G, 1e-5, act, fws.p, None)
    if fwd:
        L.launch_groupnorm_act_shift_forward_ws(*args_f)
    else:
        L.dll.launch_groupnorm_act_shift_forward_ws(*args_f)
        refused(L, "forward")
        mu_s, rs_s = stats
        mud, rsd = L.to_device(mu_s), L.to_device(rs_s)
    args_b = (dxd.p, gsd.p, ggd.p, gbd.p, dyd.p, xd.p, shd.p, gd.p, bd.p, mud.p, rsd.p, B, HW, C, G, act, bws.p,
              None)
    if bwd:
        L.launch_groupnorm_act_shift_backward_ws(*args_b)
    else:
        L.dll.launch_groupnorm_act_shift_backward_ws(*args_b)
        refused(L, "backward")
    L.sync()
    assert L.nnhip_launch_allocations() == allocs, "a shift launcher allocated"
    y, mu, rs = yd.download(shape=x.shape), mud.download(), rsd.download()
    dx, gs, gg, gb = dxd.download(shape=x.shape), gsd.download(shape=(B, C)), ggd.download(), gbd.download()
    if not fwd:
        assert np.all(y == SENTINEL), "a refused forward wrote y"
        y, mu, rs = None, None, None
    if not bwd:
        for a, what in ((dx, "dx"), (gs, "gshift"), (gg, "dgamma"), (gb, "dbeta")):
            assert np.all(a == SENTINEL), f"a refused backward wrote {what}"
        dx, gs, gg, gb = None, None, None, None
    return y, mu, rs, dx, gs, gg, gb


def run_plain(L, xs, gamma, beta, dy, G, act):
    """The plain launchers on xs = x + shift, each with a fresh workspace, and
    launch_spatial_reduce_sum of their dx."""
    B, HW, C = xs.shape
    xd, dyd = L.to_device(xs), L.to_device(dy)
    gd, bd = L.to_device(gamma), L.to_device(beta)
    yd, dxd, gsd = L.alloc(xs.size), L.alloc(xs.size), L.alloc(B * C)
    mud, rsd, ggd, gbd = L.alloc(B * G), L.alloc(B * G), L.alloc(C), L.alloc(C)
    fws = zeroed(L, max(1, L.nnhip_groupnorm_forward_workspace(B, HW, C, G)))
    bws = zeroed(L, L.nnhip_groupnorm_backward_workspace(B, HW, C, G))
    L.launch_groupnorm_act_forward_ws(yd.p, mud.p, rsd.p, xd.p, gd.p, bd.p, B, HW, C, G, 1e-5, act, fws.p, None)
    L.launch_groupnorm_act_backward_ws(dxd.p, ggd.p, gbd.p, dyd.p, xd.p, gd.p, bd.p, mud.p, rsd.p, B, HW, C, G,
                                       act, bws.p, None)
    L.launch_spatial_reduce_sum(gsd.p, dxd.p, B, HW, C, None)
    L.sync()
    return (yd.download(shape=xs.shape), mud.download(), rsd.download(), dxd.download(shape=xs.shape),
            gsd.download(shape=(B, C)), ggd.download(), gbd.download())


def pixel_sum_check(gs, dx, what):
    ref = dx.astype(np.float64).sum(axis=1)
    floor = np.sqrt((dx.astype(np.float64) ** 2).sum(axis=1))
    err = rel_err(gs, ref, floor=floor)
    assert err <= TOL, f"{what}: relative error {err:.3e}"


def check(L, rng, shape, act, stream_fwd, stream_bwd):
    B, H, W, C, G = shape
    HW = H * W
    x, gamma, beta, dy = make_inputs(rng, B, H, W, C)
    sh = shift_case(rng, B, C)
    xs = (x + sh[:, None, :]).astype(np.float32)
    mask = L.nnhip_groupnorm_shift_supported(B, HW, C, G, act)
    assert mask == (1 if stream_fwd else 0) | (2 if stream_bwd else 0), mask
    fws = zeroed(L, max(1, L.nnhip_groupnorm_forward_workspace(B, HW, C, G)))
    bws = zeroed(L, max(1, L.nnhip_groupnorm_shift_backward_workspace(B, HW, C, G)))
    ref = run_plain(L, xs, gamma, beta, dy, G, act)
    got = run_shift(L, x, sh, gamma, beta, dy, G, act, fws, bws, stream_fwd, stream_bwd, stats=ref[1:3])
    if stream_fwd:
        ok, nrec = tiles(L, B, HW, C, G, FWD_TP)
        assert ok and records_tagged(fws, nrec), "forward did not take the streaming path"
    if stream_bwd:
        ok, nrec = tiles(L, B, HW, C, G, BWD_TP)
        assert ok and records_tagged(bws, nrec), "backward did not take the streaming path"
    assert L.nnhip_groupnorm_workspace_status(fws.p) == 0
    assert L.nnhip_groupnorm_workspace_status(bws.p) == 0
    for g, r, what in zip(got, ref, ("y", "mu", "rstd", "dx", None, "dgamma", "dbeta")):
        if what and g is not None:
            assert_bits_equal(g, r, what)
    if stream_bwd:
        pixel_sum_check(got[4], got[3], "gshift vs the pixel sum of dx")
    pixel_sum_check(ref[4], ref[3], "launch_spatial_reduce_sum vs the pixel sum of dx")
    return x, sh, xs, gamma, beta, dy, got


# (B, H, W, C, G), fused shift kernels expected (forward, backward).  On a
# 256-CU device the backward has 128 tiles per 64x64x256 sample, so B = 1, 3,
# 6, 8, 16 give 1, 1-2, 3, 4, 8 rounds per workgroup (the epilogue cases K =
# 1, 2, 3 and both halves of the two-round loop).
STREAM_SHAPES = [
    ((1, 64, 64, 256, 32), True, True),
    ((3, 64, 64, 256, 32), True, True),
    ((6, 64, 64, 256, 32), True, True),
    ((8, 64, 64, 256, 32), True, True),
    ((16, 64, 64, 256, 32), True, True),
    ((16, 32, 32, 256, 32), True, True),   # the DDPM block test's streaming shape
    ((2, 64, 64, 512, 64), True, True),    # cpg 8, four column blocks
    ((2, 16, 16, 256, 16), True, True),    # cpg 16
    ((4, 32, 32, 128, 32), False, True),   # cpg 4: forward refused, backward fused
    ((1, 64, 128, 256, 32), True, False),  # backward merges 2 records per lane: refused
    ((1, 128, 128, 128, 8), True, False),  # forward merges 2 records per lane; backward too large
    ((1, 8, 16, 128, 16), True, True),     # one forward tile, two backward tiles per sample
    ((3, 8, 16, 128, 16), True, True),
]


@pytest.mark.parametrize("shape,sf,sb", STREAM_SHAPES, ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else None)
def test_shift_stream_matches_plain_composition(L, rng, monkeypatch, shape, sf, sb):
    print(f"[case] groupnorm shift stream {shape}", flush=True)
    monkeypatch.setenv("NNHIP_GN_PATH", "stream")
    check(L, rng, shape, SILU, sf, sb)


@pytest.mark.parametrize("shape,act,path", [
    ((2, 64, 64, 256, 32), 0, "stream"),      # identity
    ((2, 64, 64, 256, 32), SILU, "reg"),      # register path forced
    ((2, 8, 8, 32, 8), SILU, ""),             # the small block test's shape, auto policy
    ((4, 32, 32, 64, 32), SILU, "stream"),    # cpg 2 (a reference DDPM width): no streaming plan
], ids=["identity", "reg", "small-auto", "cpg2"])
def test_shift_refuses_what_its_kernels_do_not_take(L, rng, monkeypatch, shape, act, path):
    print(f"[case] groupnorm shift refused {shape} act={act} path={path or 'auto'}", flush=True)
    if path:
        monkeypatch.setenv("NNHIP_GN_PATH", path)
    else:
        monkeypatch.delenv("NNHIP_GN_PATH", raising=False)
    check(L, rng, shape, act, False, False)


def test_shift_against_oracle(L, orc, rng, monkeypatch):
    print("[case] groupnorm shift vs oracle", flush=True)
    monkeypatch.setenv("NNHIP_GN_PATH", "stream")
    B, H, W, C, G = 3, 64, 64, 256, 32
    x, sh, xs, gamma, beta, dy, got = check(L, rng, (B, H, W, C, G), SILU, True, True)
    xs_o = orc.spatial_add(x, sh)
    assert_bits_equal(xs_o, xs, "oracle spatial_add vs float32 x + shift")
    y_ref, mu_ref, rs_ref = orc.groupnorm_forward(xs_o, gamma, beta, G, 1e-5, SILU)
    assert rel_err(got[0], y_ref) <= TOL
    dx_ref, _, _ = orc.groupnorm_backward(dy, xs_o, gamma, beta, mu_ref, rs_ref, G, SILU)
    assert rel_err(got[3], dx_ref) <= TOL
    gs_ref = orc.spatial_reduce_sum(dx_ref)
    floor = np.sqrt((dx_ref.astype(np.float64) ** 2).sum(axis=1))
    assert rel_err(got[4], gs_ref, floor=floor) <= TOL


def test_shift_repeat_is_bit_identical(L, rng, monkeypatch):
    """Two launches on the same lent workspaces give the same bits (fixed
    orders of every sum, the column sums included)."""
    print("[case] groupnorm shift determinism", flush=True)
    monkeypatch.setenv("NNHIP_GN_PATH", "stream")
    B, H, W, C, G = 6, 64, 64, 256, 32
    HW = H * W
    x, gamma, beta, dy = make_inputs(rng, B, H, W, C)
    sh = shift_case(rng, B, C)
    fws = zeroed(L, L.nnhip_groupnorm_forward_workspace(B, HW, C, G))
    bws = zeroed(L, L.nnhip_groupnorm_shift_backward_workspace(B, HW, C, G))
    a = run_shift(L, x, sh, gamma, beta, dy, G, SILU, fws, bws)
    b = run_shift(L, x, sh, gamma, beta, dy, G, SILU, fws, bws)
    for u, v, what in zip(a, b, ("y", "mu", "rstd", "dx", "gshift", "dgamma", "dbeta")):
        assert_bits_equal(u, v, what)
