"""Spatial (per sample and channel) rows of the diffusion blocks through the
C-ABI against the oracle: spatial_add and spatial_modulate (reference
src/kernels.cu:1055-1067, 1132-1142) bit-exact; spatial_reduce_sum and the
modulate backward's grad_cond (:1070-1101, 1145-1158) within 1e-5 of the
double-accumulated sums (floor: root of the summed squared terms); the fused
EDM pairs modulate+activation forward/backward (src/cond_conv_residual.c:30-33,
46-49) bit-exact for the elementwise outputs.  Shapes: BASELINE cfg2's EDM
block [128,32,32,128], the DDPM block's [8,64,64,256], and edge cases (C not
a multiple of 4, misaligned pointers, HW = 1 / 0, batch 0)."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import TOL, assert_bits_equal, rel_err

pytestmark = pytest.mark.gpu

SHAPES = [
    (128, 32 * 32, 128),  # cfg2 EDM block
    (8, 64 * 64, 256),    # DDPM block shape (8 samples)
    (3, 49, 6),           # C % 4 != 0: scalar paths
    (2, 7, 192),          # 48 float4 columns: two column passes
    (5, 1, 64),           # one row per sample
    (1, 5000, 3),         # image channels, many segments
]


def _inputs(rng, B, HW, C):
    x = (1.5 * rng.standard_normal((B, HW, C))).astype(np.float32)
    v = (0.5 * rng.standard_normal((B, C))).astype(np.float32)
    g = rng.standard_normal((B, HW, C)).astype(np.float32)
    return x, v, g


def _sum_floor(terms):
    return np.sqrt(np.sum(np.asarray(terms, np.float64) ** 2, axis=1))


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_spatial_add_and_reduce(L, orc, rng, shape):
    B, HW, C = shape
    print(f"[case] spatial add/reduce {shape}", flush=True)
    x, v, _ = _inputs(rng, B, HW, C)
    xd, vd = L.to_device(x), L.to_device(v)
    L.launch_spatial_add(xd.p, vd.p, B, HW, 1, C, None)
    L.sync()
    assert_bits_equal(xd.download(shape=x.shape), orc.spatial_add(x, v), "spatial_add")
    out = L.alloc(B * C)
    L.launch_spatial_reduce_sum(out.p, xd.p, B, HW, C, None)
    L.sync()
    xa = orc.spatial_add(x, v)
    assert rel_err(out.download(shape=(B, C)), orc.spatial_reduce_sum(xa), floor=_sum_floor(xa)) <= TOL


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_spatial_modulate_forward_backward(L, orc, rng, shape):
    B, HW, C = shape
    print(f"[case] spatial modulate {shape}", flush=True)
    x, c, g = _inputs(rng, B, HW, C)
    xd, cd, gd = L.to_device(x), L.to_device(c), L.to_device(g)
    yd = L.alloc(x.size)
    L.launch_spatial_modulate(yd.p, xd.p, cd.p, B, HW, 1, C, None)
    L.sync()
    assert_bits_equal(yd.download(shape=x.shape), orc.spatial_modulate(x, c), "spatial_modulate")
    gin, gc = L.alloc(x.size), L.alloc(B * C)
    L.launch_spatial_modulate_backward(gin.p, gc.p, gd.p, xd.p, cd.p, B, HW, 1, C, None)
    L.sync()
    gin_ref, gc_ref = orc.spatial_modulate_backward(g, x, c)
    assert_bits_equal(gin.download(shape=x.shape), gin_ref, "grad_in")
    assert rel_err(gc.download(shape=(B, C)), gc_ref, floor=_sum_floor(g * x)) <= TOL


@pytest.mark.parametrize("act", [5, 3, 0], ids=["mp_silu", "silu", "identity"])
@pytest.mark.parametrize("shape", SHAPES[:4], ids=lambda s: "x".join(map(str, s)))
def test_spatial_modulate_act_fused(L, orc, rng, shape, act):
    B, HW, C = shape
    print(f"[case] spatial modulate+act act={act} {shape}", flush=True)
    x, c, g = _inputs(rng, B, HW, C)
    xd, cd, gd = L.to_device(x), L.to_device(c), L.to_device(g)
    yd = L.alloc(x.size)
    L.launch_spatial_modulate_act_forward(yd.p, xd.p, cd.p, B, HW, 1, C, act, None)
    L.sync()
    assert_bits_equal(yd.download(shape=x.shape), orc.spatial_modulate_act_forward(x, c, act), "forward")
    gin, gc = L.alloc(x.size), L.alloc(B * C)
    L.launch_spatial_modulate_act_backward(gin.p, gc.p, gd.p, xd.p, cd.p, B, HW, 1, C, act, None, None)
    L.sync()
    gin_ref, gc_ref = orc.spatial_modulate_act_backward(g, x, c, act)
    assert_bits_equal(gin.download(shape=x.shape), gin_ref, "grad_in")
    g2 = orc.act_backward(g, orc.spatial_modulate(x, c), act)
    assert rel_err(gc.download(shape=(B, C)), gc_ref, floor=_sum_floor(g2 * x)) <= TOL
    # a lent workspace gives the same bits as the library scratch, also reused
    ws = _zeroed(L, L.nnhip_spatial_reduce_workspace(B, HW, C))
    for rep in range(2):
        gin2, gc2 = L.alloc(x.size), L.alloc(B * C)
        L.launch_spatial_modulate_act_backward(gin2.p, gc2.p, gd.p, xd.p, cd.p, B, HW, 1, C, act, ws.p, None)
        L.sync()
        assert_bits_equal(gc2.download(), gc.download(), f"grad_cond ws vs scratch, launch {rep}")
        assert_bits_equal(gin2.download(), gin.download(), f"grad_in ws vs scratch, launch {rep}")


def test_spatial_modulate_act_one_workgroup_per_sample(L, orc, rng):
    """256 samples of 256 K elements each take the plan with one 1024-thread
    workgroup per sample (no segment partials): grad_in bit-exact, grad_cond
    within the bar of the double sums, lent workspace and library scratch
    bit-identical."""
    B, HW, C, act = 256, 1024, 256, 5
    print(f"[case] spatial modulate+act backward, one workgroup per sample {(B, HW, C)}", flush=True)
    x, c, g = _inputs(rng, B, HW, C)
    xd, cd, gd = L.to_device(x), L.to_device(c), L.to_device(g)
    gin, gc = L.alloc(x.size), L.alloc(B * C)
    L.launch_spatial_modulate_act_backward(gin.p, gc.p, gd.p, xd.p, cd.p, B, HW, 1, C, act, None, None)
    L.sync()
    gin_ref, gc_ref = orc.spatial_modulate_act_backward(g, x, c, act)
    assert_bits_equal(gin.download(shape=x.shape), gin_ref, "grad_in")
    g2 = orc.act_backward(g, orc.spatial_modulate(x, c), act)
    assert rel_err(gc.download(shape=(B, C)), gc_ref, floor=_sum_floor(g2 * x)) <= TOL
    ws = _zeroed(L, L.nnhip_spatial_reduce_workspace(B, HW, C))
    gc2 = L.alloc(B * C)
    L.launch_spatial_modulate_act_backward(gin.p, gc2.p, gd.p, xd.p, cd.p, B, HW, 1, C, act, ws.p, None)
    L.sync()
    assert_bits_equal(gc2.download(), gc.download(), "grad_cond ws vs scratch")


def _zeroed(L, n):
    a = L.alloc(max(1, n))
    a.fill_bytes(0)
    return a


@pytest.mark.parametrize("shape", SHAPES + [(1, 64 * 64, 256), (40, 256, 64)], ids=lambda s: "x".join(map(str, s)))
def test_spatial_reduce_sum_lent_workspace(L, orc, rng, shape):
    """launch_spatial_reduce_sum_ws gives the pool path's sums bit for bit,
    launch after launch on one workspace."""
    B, HW, C = shape
    print(f"[case] spatial reduce lent workspace {shape}", flush=True)
    x, _, _ = _inputs(rng, B, HW, C)
    xd, ref = L.to_device(x), L.alloc(B * C)
    L.launch_spatial_reduce_sum(ref.p, xd.p, B, HW, C, None)
    L.sync()
    want = ref.download()
    assert rel_err(want.reshape(B, C), orc.spatial_reduce_sum(x), floor=_sum_floor(x)) <= TOL
    ws = _zeroed(L, L.nnhip_spatial_reduce_workspace(B, HW, C))
    for rep in range(3):
        out = L.alloc(B * C)
        L.launch_spatial_reduce_sum_ws(out.p, xd.p, B, HW, C, ws.p, None)
        L.sync()
        assert_bits_equal(out.download(), want, f"launch {rep}")
    assert L.last_error()[0] == 0


def test_spatial_workspace_serves_smaller_batches(L, rng):
    """A workspace sized for a batch serves every smaller batch: at HW = 2048,
    C = 128 a batch of 102 takes 102 x 21 segment rows, more than 103 x 20 at
    the batch of 103 the workspace was sized for.  Sentinels past the end stay
    untouched and the sums match the pool path bit for bit."""
    print("[case] spatial workspace across batches", flush=True)
    HW, C, Bmax = 2048, 128, 103
    n_ws = L.nnhip_spatial_reduce_workspace(Bmax, HW, C)
    guard = 4096
    ws = L.alloc(n_ws + guard)
    ws.upload(np.concatenate([np.zeros(n_ws, np.float32), np.full(guard, 7.25, np.float32)]))
    x, c, g = _inputs(rng, Bmax, HW, C)
    xd, cd, gd = L.to_device(x), L.to_device(c), L.to_device(g)
    for B in (Bmax, 102, 1, 102):
        gin_r, gc_r, gin_w, gc_w = L.alloc(B * HW * C), L.alloc(B * C), L.alloc(B * HW * C), L.alloc(B * C)
        L.launch_spatial_modulate_act_backward(gin_r.p, gc_r.p, gd.p, xd.p, cd.p, B, HW, 1, C, 5, None, None)
        L.launch_spatial_modulate_act_backward(gin_w.p, gc_w.p, gd.p, xd.p, cd.p, B, HW, 1, C, 5, ws.p, None)
        L.sync()
        assert_bits_equal(gc_w.download(), gc_r.download(), f"grad_cond B={B}")
        assert_bits_equal(gin_w.download(), gin_r.download(), f"grad_in B={B}")
    assert np.all(ws.download()[n_ws:] == np.float32(7.25)), "wrote past the workspace"


def test_spatial_misaligned_pointers_take_the_scalar_path(L, orc, rng):
    print("[case] spatial misaligned", flush=True)
    B, HW, C = 4, 33, 64
    x, c, g = _inputs(rng, B, HW, C)
    xd, gd = L.to_device(np.concatenate([[0.0], x.ravel()])), L.to_device(np.concatenate([[0.0], g.ravel()]))
    cd = L.to_device(np.concatenate([[0.0], c.ravel()]))
    yd, gin, gc = L.alloc(x.size + 1), L.alloc(x.size + 1), L.alloc(B * C + 1)
    L.launch_spatial_modulate_act_forward(yd.offset(1), xd.offset(1), cd.offset(1), B, HW, 1, C, 5, None)
    L.launch_spatial_modulate_act_backward(gin.offset(1), gc.offset(1), gd.offset(1), xd.offset(1), cd.offset(1),
                                           B, HW, 1, C, 5, None, None)
    L.sync()
    assert_bits_equal(yd.download()[1:].reshape(x.shape), orc.spatial_modulate_act_forward(x, c, 5), "forward")
    gin_ref, gc_ref = orc.spatial_modulate_act_backward(g, x, c, 5)
    assert_bits_equal(gin.download()[1:].reshape(x.shape), gin_ref, "grad_in")
    g2 = orc.act_backward(g, orc.spatial_modulate(x, c), 5)
    assert rel_err(gc.download()[1:].reshape(B, C), gc_ref, floor=_sum_floor(g2 * x)) <= TOL


def test_spatial_empty_shapes(L):
    """batch 0 is a no-op; HW = 0 writes zero sums (the reference's empty loop)."""
    print("[case] spatial empty shapes", flush=True)
    null = None
    L.launch_spatial_add(null, null, 0, 4, 4, 8, None)
    L.launch_spatial_reduce_sum(null, null, 0, 16, 8, None)
    gc = L.to_device(np.full(2 * 8, 7.0, np.float32))
    dummy = L.alloc(4)
    L.launch_spatial_modulate_backward(dummy.p, gc.p, dummy.p, dummy.p, dummy.p, 2, 0, 0, 8, None)
    L.sync()
    assert not np.any(gc.download())
    assert L.last_error()[0] == 0
