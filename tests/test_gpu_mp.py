"""Magnitude-preserving rows: mp_cat / mp_channel_cat / mp_channel_split
(reference src/kernels.cu:318-328, 368-378, 1215-1232, 1251-1278) bit-exact,
and forced weight normalisation with gain, forward and backward
(src/kernels.cu:255-297, 330-344; callers src/mp_linear.c:12-38,
src/conv2d.c:24-55) within 1e-5.  Shapes are BASELINE cfg2's."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import TOL, assert_bits_equal, rel_err

pytestmark = pytest.mark.gpu

R2 = 128 * 32 * 32  # cfg2 pixels


@pytest.mark.parametrize("rows,Na,Nb,t", [(R2, 128, 128, 0.3), (7, 3, 5, 0.3), (1000, 64, 192, 0.5),
                                          (33, 1, 1, 0.7)])
def test_mp_cat_bit_exact(L, orc, rng, rows, Na, Nb, t):
    print(f"[case] mp_cat rows={rows} Na={Na} Nb={Nb}", flush=True)
    a = rng.standard_normal((rows, Na), dtype=np.float32)
    b = rng.standard_normal((rows, Nb), dtype=np.float32)
    ad, bd, od = L.to_device(a), L.to_device(b), L.alloc(rows * (Na + Nb))
    L.launch_mp_cat(od.p, ad.p, bd.p, t, rows, Na, Nb, None)
    L.sync()
    ref = orc.mp_cat(a, b, t)
    assert_bits_equal(od.download(shape=ref.shape), ref, "mp_cat")
    # the NHWC channel form is the same placement over spatial = N*H*W pixels
    od.fill_bytes(0)
    L.launch_mp_channel_cat(od.p, ad.p, bd.p, t, rows, Na, Nb, None)
    L.sync()
    assert_bits_equal(od.download(shape=ref.shape), ref, "mp_channel_cat")


@pytest.mark.parametrize("rows,Ca,Cb,t", [(R2, 128, 128, 0.3), (7, 3, 5, 0.3), (1000, 64, 192, 0.5)])
def test_mp_channel_split_bit_exact(L, orc, rng, rows, Ca, Cb, t):
    g = rng.standard_normal((rows, Ca + Cb), dtype=np.float32)
    gd, gad, gbd = L.to_device(g), L.alloc(rows * Ca), L.alloc(rows * Cb)
    L.launch_mp_channel_split(gad.p, gbd.p, gd.p, t, rows, Ca, Cb, None)
    L.sync()
    ga, gb = orc.mp_split(g, Ca, Cb, t)
    assert_bits_equal(gad.download(shape=ga.shape), ga, "grad_a")
    assert_bits_equal(gbd.download(shape=gb.shape), gb, "grad_b")


@pytest.mark.parametrize("n_in,n_out", [(1152, 128), (12, 8), (27, 4), (4, 6), (1, 1), (300, 1000)])
def test_weight_normalize_forward(L, orc, rng, n_in, n_out):
    W = rng.standard_normal((n_in, n_out)).astype(np.float32)
    Wd = L.to_device(W)
    L.launch_weight_normalize(Wd.p, n_in, n_out, 1e-4, None)
    L.sync()
    assert rel_err(Wd.download(shape=W.shape), orc.weight_normalize(W, 1e-4)) <= TOL
    # repeated forwards converge to |W_j|^2 = 1 - eps (the in-place forced form)
    for _ in range(20):
        L.launch_weight_normalize(Wd.p, n_in, n_out, 1e-4, None)
    L.sync()
    ss = np.sum(Wd.download(shape=W.shape).astype(np.float64) ** 2, axis=0)
    np.testing.assert_allclose(ss, 1 - 1e-4, rtol=5e-6)


@pytest.mark.parametrize("n_in,n_out", [(1152, 128), (12, 8), (4, 6), (300, 1000)])
def test_weight_normalize_backward(L, orc, rng, n_in, n_out):
    W = rng.standard_normal((n_in, n_out)).astype(np.float32)
    Wn = orc.weight_normalize(W, 1e-4)
    M = rng.standard_normal((n_in, n_out)).astype(np.float32)
    gain = np.array([1.3], np.float32)
    gWd, Wnd, gaind = L.to_device(M), L.to_device(Wn), L.to_device(gain)
    gg = L.to_device(np.array([0.25], np.float32))  # accumulated onto, as the reference's atomicAdd
    L.launch_weight_normalize_backward(gWd.p, Wnd.p, gaind.p, gg.p, n_in, n_out, None)
    L.sync()
    gW_ref, gg_ref = orc.weight_normalize_backward(M, Wn, float(gain[0]), 0.25)
    terms = (Wn.astype(np.float64) * M)
    dots = terms.sum(axis=0)
    # floor for gW: its RMS; for the gain gradient: sqrt of the summed squared terms
    assert rel_err(gWd.download(shape=M.shape), gW_ref) <= TOL
    floor = float(np.sqrt(np.sum(terms ** 2)) + 0.25)
    assert abs(float(gg.download()[0]) - gg_ref) / max(abs(gg_ref), floor) <= TOL
    assert abs(gg_ref - (0.25 + dots.sum())) < 1e-3


def test_mp_linear_weight_chain(L, orc, rng):
    """The mp_linear sequence (src/mp_linear.c:12-38) minus the GEMM: normalise
    in place, then the backward on the normalised weight with the gain buffer
    zeroed by the caller."""
    n_in, n_out = 1152, 128
    W = rng.standard_normal((n_in, n_out)).astype(np.float32)
    Wd = L.to_device(W)
    L.launch_weight_normalize(Wd.p, n_in, n_out, 1e-4, None)
    M = rng.standard_normal((n_in, n_out)).astype(np.float32)
    gWd = L.to_device(M)
    gain, gg = L.to_device(np.array([1.0], np.float32)), L.alloc(1)
    gg.fill_bytes(0)
    L.launch_weight_normalize_backward(gWd.p, Wd.p, gain.p, gg.p, n_in, n_out, None)
    L.sync()
    Wn_ref = orc.weight_normalize(W, 1e-4)
    gW_ref, gg_ref = orc.weight_normalize_backward(M, Wn_ref, 1.0, 0.0)
    assert rel_err(gWd.download(shape=M.shape), gW_ref) <= TOL
    assert abs(float(gg.download()[0]) - gg_ref) <= TOL * max(abs(gg_ref), float(np.sqrt(n_in * n_out)))


@pytest.mark.parametrize("n_in,n_out", [(1152, 128), (12, 8), (4, 6), (300, 1000), (1, 1)])
def test_weight_normalize_backward_workspace_matches(L, orc, rng, n_in, n_out):
    """The lent-workspace backward (one launch; the gain-gradient sum is done
    by the last workgroup to finish) against the pool launcher and the oracle,
    on two calls in a row through the same workspace, the second smaller: the
    completion counter must re-arm itself."""
    print(f"[case] weight_normalize_backward_ws {n_in}x{n_out}", flush=True)
    ws = L.alloc(int(L.nnhip_weight_normalize_backward_workspace(n_out)))
    ws.fill_bytes(0)
    for k, (ni, no) in enumerate([(n_in, n_out), (max(1, n_in // 2), max(1, n_out // 3))]):
        W = rng.standard_normal((ni, no)).astype(np.float32)
        Wn = orc.weight_normalize(W, 1e-4)
        M = rng.standard_normal((ni, no)).astype(np.float32)
        gain = np.array([0.7 + k], np.float32)
        Wnd, gaind = L.to_device(Wn), L.to_device(gain)
        gA, gB = L.to_device(M), L.to_device(M)
        ggA, ggB = L.to_device(np.array([0.25], np.float32)), L.to_device(np.array([0.25], np.float32))
        L.launch_weight_normalize_backward(gA.p, Wnd.p, gaind.p, ggA.p, ni, no, None)
        L.launch_weight_normalize_backward_ws(gB.p, Wnd.p, gaind.p, ggB.p, ni, no, ws.p, None)
        L.sync()
        # same fixed-order arithmetic as the pool launcher: identical bits
        assert_bits_equal(gB.download(shape=M.shape), gA.download(shape=M.shape), "gW ws vs pool")
        assert_bits_equal(ggB.download(), ggA.download(), "g_gain ws vs pool")
        gW_ref, gg_ref = orc.weight_normalize_backward(M, Wn, float(gain[0]), 0.25)
        assert rel_err(gB.download(shape=M.shape), gW_ref) <= TOL
        terms = Wn.astype(np.float64) * M
        floor = float(np.sqrt(np.sum(terms ** 2)) + 0.25)
        assert abs(float(ggB.download()[0]) - gg_ref) / max(abs(gg_ref), floor) <= TOL


def test_fill_f32(L):
    buf = L.alloc(100003)
    buf.fill_bytes(0xFF)
    L.nnhip_fill_f32(buf.p, 0.0, 100001, None)
    L.sync()
    got = buf.download()
    assert np.all(got[:100001] == 0.0) and np.isnan(got[100001:]).all()
    L.nnhip_fill_f32(buf.p, 2.5, 7, None)
    L.sync()
    assert np.all(buf.download()[:7] == 2.5) and buf.download()[7] == 0.0


def test_launcher_scratch_reuse_across_sizes_and_streams(L, orc, rng):
    """Launchers without a workspace argument keep one cached scratch block per
    stream: calls that grow and shrink it, alternating between the null stream
    and a created one, all match the lent-workspace launcher bit for bit."""
    print("[case] launcher scratch reuse", flush=True)
    s1 = L.dll.nnhip_stream_create()
    assert s1
    try:
        for k, (ni, no) in enumerate([(64, 16), (1152, 640), (300, 1000), (12, 8), (2048, 2048)]):
            stream = s1 if k % 2 else None
            W = orc.weight_normalize(rng.standard_normal((ni, no)).astype(np.float32), 1e-4)
            M = rng.standard_normal((ni, no)).astype(np.float32)
            Wd, gain = L.to_device(W), L.to_device(np.array([1.1], np.float32))
            gA, gB = L.to_device(M), L.to_device(M)
            ggA, ggB = L.to_device(np.zeros(1, np.float32)), L.to_device(np.zeros(1, np.float32))
            ws = L.alloc(int(L.nnhip_weight_normalize_backward_workspace(no)))
            ws.fill_bytes(0)
            L.launch_weight_normalize_backward(gA.p, Wd.p, gain.p, ggA.p, ni, no, stream)
            L.launch_weight_normalize_backward_ws(gB.p, Wd.p, gain.p, ggB.p, ni, no, ws.p, stream)
            L.dll.nnhip_stream_synchronize(s1)
            L.sync()
            assert_bits_equal(gA.download(shape=M.shape), gB.download(shape=M.shape), f"gW call {k}")
            assert_bits_equal(ggA.download(), ggB.download(), f"g_gain call {k}")
    finally:
        L.dll.nnhip_stream_synchronize(s1)
        L.dll.nnhip_stream_destroy(s1)


def test_launcher_scratch_under_graph_capture(L, orc, rng, nn):
    """A launcher without a workspace argument inside a captured graph uses its
    stream's cached scratch block.  The replays keep matching eager after the
    stream's block has grown for a larger eager call (the captured block is
    kept, not freed), and a capture that would need a new or larger block is
    refused on the host with an error instead of allocating."""
    print("[case] scratch under graph capture", flush=True)
    bs, bb, N = 256, 16384, 1024
    g_small = rng.standard_normal((bs, N)).astype(np.float32)
    g_big = rng.standard_normal((bb, N)).astype(np.float32)
    gs, gbig = L.to_device(g_small), L.to_device(g_big)
    out, out_big = L.alloc(N), L.alloc(N)
    s = L.dll.nnhip_stream_create()
    s3 = L.dll.nnhip_stream_create()
    assert s and s3
    graph = None
    try:
        L.launch_bias_grad(out.p, gs.p, bs, N, s)
        L.dll.nnhip_stream_synchronize(s)
        ref = out.download()
        np.testing.assert_allclose(ref, orc.bias_grad(g_small, N), rtol=1e-5, atol=1e-4)
        assert L.dll.nnhip_graph_capture_begin(s) == 0
        L.launch_bias_grad(out.p, gs.p, bs, N, s)
        graph = L.dll.nnhip_graph_capture_end(s)
        assert graph, "graph capture failed"
        for replay in range(3):
            # a larger eager call on the same stream grows its cached block
            L.launch_bias_grad(out_big.p, gbig.p, bb if replay == 0 else bb // 2, N, s)
            out.fill_bytes(0)
            L.dll.nnhip_stream_synchronize(s)
            L.sync()
            assert L.dll.nnhip_graph_launch(graph, s) == 0
            L.dll.nnhip_stream_synchronize(s)
            assert_bits_equal(out.download(), ref, f"replay {replay}")
        np.testing.assert_allclose(out_big.download(), orc.bias_grad(g_big[: bb // 2], N), rtol=1e-4, atol=1e-3)
        # a capture on a stream with no cached block is refused, not allocated
        assert L.dll.nnhip_graph_capture_begin(s3) == 0
        with pytest.raises(nn.NnHipError, match="launch_bias_grad: .*not cached for the capturing stream"):
            L.call("launch_bias_grad", out.p, gs.p, bs, N, s3)
        empty = L.dll.nnhip_graph_capture_end(s3)
        if empty:
            assert L.dll.nnhip_graph_destroy(empty) == 0
        L.launch_bias_grad(out.p, gs.p, bs, N, s3)  # eager again: allocates as usual
        L.dll.nnhip_stream_synchronize(s3)
        assert_bits_equal(out.download(), ref, "eager after refusal")
    finally:
        if graph:
            assert L.dll.nnhip_graph_destroy(graph) == 0
        for st in (s, s3):
            L.dll.nnhip_stream_synchronize(st)
            assert L.dll.nnhip_stream_destroy(st) == 0


def test_launcher_scratch_dropped_with_its_stream(L, orc, rng):
    """Destroying a stream drops its cached scratch block: streams created,
    used by a launcher without a workspace argument and destroyed in turn (a
    new stream may get a recycled handle) keep matching the lent-workspace
    launcher, and nnhip_stream_scratch_release on a live stream is harmless."""
    print("[case] scratch dropped with its stream", flush=True)
    ni, no = 1152, 128
    W = orc.weight_normalize(rng.standard_normal((ni, no)).astype(np.float32), 1e-4)
    M = rng.standard_normal((ni, no)).astype(np.float32)
    Wd, gain = L.to_device(W), L.to_device(np.array([0.9], np.float32))
    ws = L.alloc(int(L.nnhip_weight_normalize_backward_workspace(no)))
    ws.fill_bytes(0)
    gB, ggB = L.to_device(M), L.to_device(np.zeros(1, np.float32))
    L.launch_weight_normalize_backward_ws(gB.p, Wd.p, gain.p, ggB.p, ni, no, ws.p, None)
    L.sync()
    for k in range(4):
        s = L.dll.nnhip_stream_create()
        assert s
        try:
            gA, ggA = L.to_device(M), L.to_device(np.zeros(1, np.float32))
            L.launch_weight_normalize_backward(gA.p, Wd.p, gain.p, ggA.p, ni, no, s)
            if k == 1:
                L.dll.nnhip_stream_scratch_release(s)
                L.launch_weight_normalize_backward(gA.p, Wd.p, gain.p, ggA.p, ni, no, s)
                L.dll.nnhip_stream_synchronize(s)  # the uploads below are not ordered with s
                gA.upload(M)
                ggA.upload(np.zeros(1, np.float32))
                L.launch_weight_normalize_backward(gA.p, Wd.p, gain.p, ggA.p, ni, no, s)
            L.dll.nnhip_stream_synchronize(s)
            L.sync()
            assert_bits_equal(gA.download(shape=M.shape), gB.download(shape=M.shape), f"gW stream {k}")
            assert_bits_equal(ggA.download(), ggB.download(), f"g_gain stream {k}")
        finally:
            L.dll.nnhip_stream_synchronize(s)
            assert L.dll.nnhip_stream_destroy(s) == 0
