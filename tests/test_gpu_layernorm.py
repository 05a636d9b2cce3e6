"""LayerNorm row (reference src/kernels.cu:491-567, launchers 594-616; module
src/layernorm.c): HIP path through the C-ABI vs the oracle.  cfg4's
[256*16*16, 256] attention-token shape plus the fast path's edges (C not a
multiple of 4, C above 1024, misaligned pointers, one row)."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import TOL, rel_err

pytestmark = pytest.mark.gpu

# (64 * 70 + 5, 64): 71 partial rows of 64 rows each, a last partial segment.
# (64 * 2048, 16) and (64 * 2048 + 7, 8): 32 and 33 segments of 64 partial
# rows (the column sum takes its segments 16 at a time: two batches, and three
# with a partial last one).  C = 8, 48, 1000 and 1030 end on a partial
# 16-channel chunk of partials.
SHAPES = [(256 * 16 * 16, 256), (2, 16), (37, 48), (5, 1000), (3, 1030), (64, 4), (1, 7), (130, 2048), (1, 1),
          (64 * 70 + 5, 64), (64 * 2048, 16), (64 * 2048 + 7, 8)]


def _inputs(rng, R, C):
    x = (0.5 + rng.standard_normal((R, C))).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(C)).astype(np.float32)
    dy = rng.standard_normal((R, C)).astype(np.float32)
    return x, gamma, beta, dy


def _param_floor(dy, x, mu, rs):
    xh = (x.astype(np.float64) - mu[:, None]) * rs[:, None]
    d = dy.astype(np.float64)
    return np.sqrt(np.sum((d * xh) ** 2, axis=0)), np.sqrt(np.sum(d * d, axis=0))


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_layernorm_forward_backward(L, orc, rng, shape):
    R, C = shape
    print(f"[case] layernorm {shape}", flush=True)
    x, gamma, beta, dy = _inputs(rng, R, C)
    xd, yd, gd, bd = L.to_device(x), L.alloc(x.size), L.to_device(gamma), L.to_device(beta)
    mu, rs = L.alloc(R), L.alloc(R)
    L.launch_layernorm_forward(yd.p, mu.p, rs.p, xd.p, gd.p, bd.p, R, C, 1e-5, None)
    L.sync()
    y_ref, mu_ref, rs_ref = orc.layernorm_forward(x, gamma, beta, 1e-5)
    assert rel_err(yd.download(shape=x.shape), y_ref) <= TOL
    assert rel_err(mu.download(), mu_ref) <= TOL
    assert rel_err(rs.download(), rs_ref) <= TOL

    dyd, dxd, ggd, gbd = L.to_device(dy), L.alloc(x.size), L.alloc(C), L.alloc(C)
    mud, rsd = L.to_device(mu_ref), L.to_device(rs_ref)
    L.launch_layernorm_backward(dxd.p, ggd.p, gbd.p, dyd.p, xd.p, gd.p, mud.p, rsd.p, R, C, None)
    L.sync()
    dx_ref, gg_ref, gb_ref = orc.layernorm_backward(dy, x, gamma, mu_ref, rs_ref)
    fg, fb = _param_floor(dy, x, mu_ref, rs_ref)
    assert rel_err(dxd.download(shape=x.shape), dx_ref) <= TOL
    assert rel_err(ggd.download(), gg_ref, floor=fg) <= TOL
    assert rel_err(gbd.download(), gb_ref, floor=fb) <= TOL

    # workspace variant: identical results, also from a second launch on the
    # same workspace
    ws = L.alloc(max(1, L.nnhip_layernorm_backward_workspace(R, C)))
    ws.fill_bytes(0)
    for rep in range(2):
        dx2, gg2, gb2 = L.alloc(x.size), L.alloc(C), L.alloc(C)
        L.launch_layernorm_backward_ws(dx2.p, gg2.p, gb2.p, dyd.p, xd.p, gd.p, mud.p, rsd.p, R, C, ws.p, None)
        L.sync()
        assert np.array_equal(dx2.download(), dxd.download()), rep
        assert np.array_equal(gg2.download(), ggd.download()), rep
        assert np.array_equal(gb2.download(), gbd.download()), rep


def test_layernorm_misaligned(L, orc, rng):
    R, C = 33, 64
    x, gamma, beta, dy = _inputs(rng, R, C)
    xd, yd = L.alloc(x.size + 1), L.alloc(x.size + 1)
    xd.upload(np.concatenate([[0.0], x.ravel()]).astype(np.float32))
    gd, bd, mu, rs = L.to_device(gamma), L.to_device(beta), L.alloc(R), L.alloc(R)
    L.launch_layernorm_forward(yd.offset(1), mu.p, rs.p, xd.offset(1), gd.p, bd.p, R, C, 1e-5, None)
    L.sync()
    y_ref, _, _ = orc.layernorm_forward(x, gamma, beta, 1e-5)
    assert rel_err(yd.download()[1:].reshape(R, C), y_ref) <= TOL


def test_layernorm_empty_batch_zeroes_param_grads(L):
    C = 16
    gg, gb = L.to_device(np.full(C, 3.0, np.float32)), L.to_device(np.full(C, 3.0, np.float32))
    d = L.alloc(16)
    L.launch_layernorm_backward(d.p, gg.p, gb.p, d.p, d.p, d.p, d.p, d.p, 0, C, None)
    L.sync()
    assert np.all(gg.download() == 0) and np.all(gb.download() == 0)


def test_layernorm_graph_replay(L, orc, rng):
    """Forward + backward with a lent workspace at cfg4's [65536, 256] (the
    backward's 16-wave path and its one-step column sum) captured into a HIP
    graph and replayed on alternating inputs: every replay matches the eager
    launches on the same inputs bit for bit, with eager launches on the same
    workspace between the replays."""
    print("[case] layernorm graph capture and replay [65536, 256]", flush=True)
    from helpers import assert_bits_equal

    R, C = 256 * 16 * 16, 256
    sets = [_inputs(rng, R, C) for _ in range(2)]
    xd, dyd, yd, dxd = L.alloc(R * C), L.alloc(R * C), L.alloc(R * C), L.alloc(R * C)
    gd, bd = L.to_device(sets[0][1]), L.to_device(sets[0][2])
    mud, rsd, ggd, gbd = L.alloc(R), L.alloc(R), L.alloc(C), L.alloc(C)
    ws = L.alloc(L.nnhip_layernorm_backward_workspace(R, C))
    ws.fill_bytes(0)
    s = L.dll.nnhip_stream_create()
    assert s
    outs = (yd, mud, rsd, dxd, ggd, gbd)

    def issue():
        L.launch_layernorm_forward(yd.p, mud.p, rsd.p, xd.p, gd.p, bd.p, R, C, 1e-5, s)
        L.launch_layernorm_backward_ws(dxd.p, ggd.p, gbd.p, dyd.p, xd.p, gd.p, mud.p, rsd.p, R, C, ws.p, s)

    def load(k):
        L.dll.nnhip_stream_synchronize(s)  # the uploads are not ordered with s
        xd.upload(sets[k][0])
        dyd.upload(sets[k][3])

    def results():
        L.dll.nnhip_stream_synchronize(s)
        L.sync()
        return [o.download() for o in outs]

    graph = None
    try:
        refs = []
        for k in range(2):
            load(k)
            issue()
            refs.append(results())
        assert L.dll.nnhip_graph_capture_begin(s) == 0
        issue()
        graph = L.dll.nnhip_graph_capture_end(s)
        assert graph, "graph capture failed"
        names = ("y", "mu", "rstd", "dx", "dgamma", "dbeta")
        for replay in range(4):
            k = replay % 2
            load(k)
            for o in outs:
                o.fill_bytes(0)
            L.sync()
            assert L.dll.nnhip_graph_launch(graph, s) == 0
            for got, ref, name in zip(results(), refs[k], names):
                assert_bits_equal(got, ref, f"replay {replay} {name}")
            issue()
            for got, ref, name in zip(results(), refs[k], names):
                assert_bits_equal(got, ref, f"eager after replay {replay} {name}")
        # the eager backward of set 1 against the oracle
        x, gamma, beta, dy = sets[1][0], sets[0][1], sets[0][2], sets[1][3]
        _, mu_ref, rs_ref = orc.layernorm_forward(x, gamma, beta, 1e-5)
        dx_ref, gg_ref, gb_ref = orc.layernorm_backward(dy, x, gamma, mu_ref, rs_ref)
        fg, fb = _param_floor(dy, x, mu_ref, rs_ref)
        assert rel_err(refs[1][3].reshape(x.shape), dx_ref) <= TOL
        assert rel_err(refs[1][4], gg_ref, floor=fg) <= TOL
        assert rel_err(refs[1][5], gb_ref, floor=fb) <= TOL
    finally:
        if graph:
            L.dll.nnhip_graph_destroy(graph)
        L.dll.nnhip_stream_synchronize(s)
        L.dll.nnhip_stream_destroy(s)
