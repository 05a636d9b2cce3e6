"""Streaming GroupNorm (+ fused activation) parity: the persistent-grid
kernels that exchange per-tile group statistics through the workspace.

Same maths as the register-resident path (reference src/kernels.cu:622-745,
GN -> activation as in src/conv_residual.c:28-29, 51-52), different schedule:
tiles of 128 (forward) / 64 (backward) pixel rows x 128 channels, records
merged across workgroups.  NNHIP_GN_PATH=stream forces the path for every
shape it accepts; the unset (auto) policy takes it from 4 Mi elements on.

Each case also checks that the streaming kernels really ran (the workspace
holds this launch's epoch-tagged records) and that no statistics wait ran out
of polls (workspace status 0).
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import TOL, assert_bits_equal, gn_param_floor, rel_err
from test_gpu_groupnorm import effective_terms, make_inputs

pytestmark = pytest.mark.gpu

FWD_TP, BWD_TP, COLS = 128, 64, 128  # pixel rows per tile (fwd, bwd), channels per column block

SHAPES = [
    # B, H, W, C, G
    (1, 64, 64, 256, 32),    # cpg 8: fwd 32 / bwd 64 tiles per sample and column block
    (3, 64, 64, 256, 32),    # forward: fewer tiles than workgroups (idle workgroups)
    (2, 32, 32, 128, 32),    # cpg 4, one column block
    (2, 16, 16, 256, 16),    # cpg 16, two forward tiles per sample
    (4, 32, 32, 512, 32),    # cpg 16, four column blocks
    (1, 64, 64, 128, 32),    # cpg 4: backward merges 2 records per lane
    (1, 64, 128, 256, 32),   # cpg 8: backward merges 2 records per lane
    (1, 64, 128, 128, 8),    # cpg 16: backward merges 2 records per lane
    (1, 128, 128, 128, 8),   # cpg 16: forward merges 2 records per lane; backward too large
    (1, 64, 128, 128, 32),   # cpg 4: forward merges 2 records per lane; backward too large -> register/generic
    (1, 128, 128, 128, 32),  # cpg 4: neither direction fits the streaming plan
    (1, 8, 16, 128, 16),     # one forward tile and two backward tiles per sample
    (2, 8, 16, 128, 16),     # the same, two samples
    (1, 8, 8, 128, 16),      # one backward tile; the forward does not stream
]


def tiles(L, B, HW, C, G, tp):
    """(applicable, records) of the streaming plan for this geometry.  The
    persistent grid holds one 1024-thread workgroup per CU (LDS-bound), and a
    multiple of the tiles per sample row must fit in it."""
    cpg = C // G
    if cpg not in (4, 8, 16) or C % COLS or HW % tp:
        return False, 0
    T = HW // tp
    gt = COLS // cpg
    if T & (T - 1) or T > 2 * min(64, 1024 // gt) or T * (C // COLS) > L.device_info()["cus"]:
        return False, 0
    return True, B * (C // COLS) * T * gt * 2


HEADER_WORDS = 8192 // 4  # fixed workspace header: flag word, then arrival counters from byte 256
COUNT_WORD = 256 // 4


def records_tagged(ws, nrec):
    """True when the nrec 64-bit records after the header all carry one
    non-zero epoch in their upper words."""
    u = ws.download().view(np.uint32)
    hi = u[HEADER_WORDS:HEADER_WORDS + 2 * nrec][1::2]
    return hi.size == nrec and hi[0] != 0 and bool(np.all(hi == hi[0]))


def counters_rearmed(ws):
    """The backward's arrival counters are back at zero after a launch."""
    u = ws.download().view(np.uint32)
    return not np.any(u[COUNT_WORD:HEADER_WORDS])


def zeroed(L, n):
    """A workspace to lend: zero-filled before its first use."""
    return L.to_device(np.zeros(n, np.float32))


def run_fwd(L, x, gamma, beta, G, act, ws=None):
    B, HW, C = x.shape
    xd, yd = L.to_device(x), L.alloc(x.size)
    gd, bd = L.to_device(gamma), L.to_device(beta)
    mu, rs = L.alloc(B * G), L.alloc(B * G)
    if ws is None:  # no caller workspace: the launcher draws one from the stream-ordered pool
        L.launch_groupnorm_act_forward(yd.p, mu.p, rs.p, xd.p, gd.p, bd.p, B, HW, C, G, 1e-5, act, None)
    else:
        L.launch_groupnorm_act_forward_ws(yd.p, mu.p, rs.p, xd.p, gd.p, bd.p, B, HW, C, G, 1e-5, act, ws.p, None)
    L.sync()
    return yd.download(shape=x.shape), mu.download(), rs.download()


def run_bwd(L, dy, x, gamma, beta, mu, rs, G, act, ws=None):
    B, HW, C = x.shape
    xd, dyd, dxd = L.to_device(x), L.to_device(dy), L.alloc(x.size)
    gd, bd = L.to_device(gamma), L.to_device(beta)
    mud, rsd = L.to_device(mu), L.to_device(rs)
    ggd, gbd = L.alloc(C), L.alloc(C)
    if ws is None:
        L.launch_groupnorm_act_backward(dxd.p, ggd.p, gbd.p, dyd.p, xd.p, gd.p, bd.p, mud.p, rsd.p, B, HW, C, G,
                                        act, None)
    else:
        L.launch_groupnorm_act_backward_ws(dxd.p, ggd.p, gbd.p, dyd.p, xd.p, gd.p, bd.p, mud.p, rsd.p, B, HW, C,
                                           G, act, ws.p, None)
    L.sync()
    return dxd.download(shape=x.shape), ggd.download(), gbd.download()


def check_case(L, orc, rng, shape, act):
    B, H, W, C, G = shape
    HW = H * W
    x, gamma, beta, dy = make_inputs(rng, B, H, W, C)
    fws = zeroed(L, max(1, L.nnhip_groupnorm_forward_workspace(B, HW, C, G)))
    bws = zeroed(L, L.nnhip_groupnorm_backward_workspace(B, HW, C, G))

    y_ref, mu_ref, rs_ref = orc.groupnorm_forward(x, gamma, beta, G, 1e-5, act)
    y, mu, rs = run_fwd(L, x, gamma, beta, G, act, fws)
    assert rel_err(y, y_ref) <= TOL
    assert rel_err(mu, mu_ref, floor=1e-3) <= TOL
    assert rel_err(rs, rs_ref) <= TOL
    ok, nrec = tiles(L, B, HW, C, G, FWD_TP)
    if ok:
        assert records_tagged(fws, nrec), "forward did not take the streaming path"
        assert L.nnhip_groupnorm_workspace_status(fws.p) == 0

    dx_ref, gg_ref, gb_ref = orc.groupnorm_backward(dy, x, gamma, beta, mu_ref, rs_ref, G, act)
    dx, gg, gb = run_bwd(L, dy, x, gamma, beta, mu_ref, rs_ref, G, act, bws)
    d, xh = effective_terms(orc, x, gamma, beta, mu_ref, rs_ref, dy, G, act)
    fg, fb = gn_param_floor(d, xh, C)
    assert rel_err(dx, dx_ref) <= TOL
    assert rel_err(gg, gg_ref, floor=fg) <= TOL
    assert rel_err(gb, gb_ref, floor=fb) <= TOL
    ok, nrec = tiles(L, B, HW, C, G, BWD_TP)
    if ok:
        assert records_tagged(bws, nrec), "backward did not take the streaming path"
        assert L.nnhip_groupnorm_workspace_status(bws.p) == 0
        assert counters_rearmed(bws), "arrival counters left non-zero"


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("act", [0, 3], ids=["identity", "silu"])
def test_stream_groupnorm(L, orc, rng, monkeypatch, shape, act):
    print(f"[case] stream groupnorm act={act} shape={shape}", flush=True)
    monkeypatch.setenv("NNHIP_GN_PATH", "stream")
    check_case(L, orc, rng, shape, act)


@pytest.mark.parametrize("act", [1, 2, 4, 5], ids=["relu", "gelu", "tanh", "mp_silu"])
def test_stream_groupnorm_other_activations(L, orc, rng, monkeypatch, act):
    print(f"[case] stream groupnorm act={act}", flush=True)
    monkeypatch.setenv("NNHIP_GN_PATH", "stream")
    check_case(L, orc, rng, (2, 32, 32, 256, 32), act)


@pytest.mark.parametrize("act", [3, 0, 1], ids=["silu", "identity", "relu"])
def test_stream_groupnorm_auto_multi_round(L, orc, rng, monkeypatch, act):
    """Auto policy at 64 samples of the north-star sample shape: every
    workgroup walks several samples (16 forward rounds, 32 backward), and both
    directions move >= 512 MB, so the nontemporal instantiations run.  Identity
    and ReLU run the steady loop that issues part of the next tile after
    phase A."""
    print(f"[case] stream groupnorm auto B=64 64x64x256 act={act}", flush=True)
    monkeypatch.delenv("NNHIP_GN_PATH", raising=False)
    check_case(L, orc, rng, (64, 64, 64, 256, 32), act)


@pytest.mark.parametrize("shape", [(32, 64, 64, 128, 32), (32, 32, 32, 512, 32)], ids=["cpg4", "cpg16"])
@pytest.mark.parametrize("act", [3, 0], ids=["silu", "identity"])
def test_stream_groupnorm_multi_round_other_group_widths(L, orc, rng, monkeypatch, shape, act):
    """Several rounds per workgroup at group widths 4 (one column block) and 16
    (four column blocks), forced streaming: 1024 tiles each way."""
    print(f"[case] stream groupnorm multi-round {shape} act={act}", flush=True)
    monkeypatch.setenv("NNHIP_GN_PATH", "stream")
    check_case(L, orc, rng, shape, act)


def test_stream_groupnorm_pool_workspace_and_determinism(L, orc, rng, monkeypatch):
    """No caller workspace (pool-drawn, cleared per launch); two launches give
    bit-identical results (fixed merge and reduction order)."""
    print("[case] stream groupnorm pool workspace", flush=True)
    monkeypatch.setenv("NNHIP_GN_PATH", "stream")
    B, H, W, C, G = 3, 64, 64, 256, 32
    x, gamma, beta, dy = make_inputs(rng, B, H, W, C)
    y1, mu1, rs1 = run_fwd(L, x, gamma, beta, G, 3)
    y2, mu2, rs2 = run_fwd(L, x, gamma, beta, G, 3)
    assert_bits_equal(y1, y2, "y")
    assert_bits_equal(mu1, mu2, "mu")
    assert_bits_equal(rs1, rs2, "rstd")
    y_ref, mu_ref, rs_ref = orc.groupnorm_forward(x, gamma, beta, G, 1e-5, 3)
    assert rel_err(y1, y_ref) <= TOL
    d1 = run_bwd(L, dy, x, gamma, beta, mu_ref, rs_ref, G, 3)
    d2 = run_bwd(L, dy, x, gamma, beta, mu_ref, rs_ref, G, 3)
    for a, b, what in zip(d1, d2, ("dx", "dgamma", "dbeta")):
        assert_bits_equal(a, b, what)
    dx_ref, _, _ = orc.groupnorm_backward(dy, x, gamma, beta, mu_ref, rs_ref, G, 3)
    assert rel_err(d1[0], dx_ref) <= TOL


def test_stream_groupnorm_workspace_reuse_across_shapes(L, orc, rng, monkeypatch):
    """One workspace lent to launches of different shapes and directions in a
    row: records left by an earlier launch never satisfy a later one."""
    print("[case] stream groupnorm workspace reuse", flush=True)
    monkeypatch.setenv("NNHIP_GN_PATH", "stream")
    shapes = [(2, 64, 64, 256, 32), (2, 32, 32, 128, 32), (1, 64, 64, 256, 32)]
    need = max(max(L.nnhip_groupnorm_forward_workspace(B, H * W, C, G),
                   L.nnhip_groupnorm_backward_workspace(B, H * W, C, G)) for B, H, W, C, G in shapes)
    ws = zeroed(L, need)
    for B, H, W, C, G in shapes:
        x, gamma, beta, dy = make_inputs(rng, B, H, W, C)
        y_ref, mu_ref, rs_ref = orc.groupnorm_forward(x, gamma, beta, G, 1e-5, 3)
        y, _, _ = run_fwd(L, x, gamma, beta, G, 3, ws)
        assert rel_err(y, y_ref) <= TOL
        dx_ref, _, _ = orc.groupnorm_backward(dy, x, gamma, beta, mu_ref, rs_ref, G, 3)
        dx, _, _ = run_bwd(L, dy, x, gamma, beta, mu_ref, rs_ref, G, 3, ws)
        assert rel_err(dx, dx_ref) <= TOL
        assert L.nnhip_groupnorm_workspace_status(ws.p) == 0


def test_cooperative_launch_matches_plain(L, rng, monkeypatch):
    """NNHIP_GN_COOPERATIVE=1 launches the same kernels cooperatively: the
    results are bit-identical to the plain launch's."""
    print("[case] stream groupnorm cooperative vs plain", flush=True)
    monkeypatch.setenv("NNHIP_GN_PATH", "stream")
    B, H, W, C, G = 2, 64, 64, 256, 32
    x, gamma, beta, dy = make_inputs(rng, B, H, W, C)
    ws = zeroed(L, L.nnhip_groupnorm_backward_workspace(B, H * W, C, G))
    out = {}
    for coop in ("0", "1"):
        monkeypatch.setenv("NNHIP_GN_COOPERATIVE", coop)
        y, mu, rs = run_fwd(L, x, gamma, beta, G, 3, ws)
        out[coop] = (y, mu, rs) + run_bwd(L, dy, x, gamma, beta, mu, rs, G, 3, ws)
        assert counters_rearmed(ws)
        assert L.nnhip_groupnorm_workspace_status(ws.p) == 0
    for a, b, what in zip(out["0"], out["1"], ("y", "mu", "rstd", "dx", "dgamma", "dbeta")):
        assert_bits_equal(a, b, what)


def test_cooperative_launches_on_two_streams(L, orc, rng, monkeypatch):
    """Streaming GroupNorms issued on two streams at once, each with its own
    workspace, in the cooperative mode that such callers select
    (NNHIP_GN_COOPERATIVE=1): both results match the oracle and no wait ran
    out of polls."""
    print("[case] stream groupnorm cooperative, two streams", flush=True)
    monkeypatch.setenv("NNHIP_GN_PATH", "stream")
    monkeypatch.setenv("NNHIP_GN_COOPERATIVE", "1")
    B, H, W, C, G = 2, 64, 64, 256, 32
    HW = H * W
    streams = [L.dll.nnhip_stream_create() for _ in range(2)]
    try:
        cases = []
        for s in streams:
            x, gamma, beta, dy = make_inputs(rng, B, H, W, C)
            d = {"x": L.to_device(x), "dy": L.to_device(dy), "g": L.to_device(gamma), "b": L.to_device(beta),
                 "y": L.alloc(x.size), "dx": L.alloc(x.size), "mu": L.alloc(B * G), "rs": L.alloc(B * G),
                 "gg": L.alloc(C), "gb": L.alloc(C),
                 "ws": zeroed(L, L.nnhip_groupnorm_backward_workspace(B, HW, C, G)), "s": s}
            cases.append((x, gamma, beta, dy, d))
        for _ in range(3):  # interleaved issue on the two streams
            for *_, d in cases:
                L.launch_groupnorm_act_forward_ws(d["y"].p, d["mu"].p, d["rs"].p, d["x"].p, d["g"].p, d["b"].p, B, HW,
                                                  C, G, 1e-5, 3, d["ws"].p, d["s"])
            for *_, d in cases:
                L.launch_groupnorm_act_backward_ws(d["dx"].p, d["gg"].p, d["gb"].p, d["dy"].p, d["x"].p, d["g"].p,
                                                   d["b"].p, d["mu"].p, d["rs"].p, B, HW, C, G, 3, d["ws"].p, d["s"])
        for s in streams:
            L.dll.nnhip_stream_synchronize(s)
        L.sync()
        for x, gamma, beta, dy, d in cases:
            assert L.nnhip_groupnorm_workspace_status(d["ws"].p) == 0
            y_ref, mu_ref, rs_ref = orc.groupnorm_forward(x, gamma, beta, G, 1e-5, 3)
            assert rel_err(d["y"].download(shape=x.shape), y_ref) <= TOL
            dx_ref, _, _ = orc.groupnorm_backward(dy, x, gamma, beta, mu_ref, rs_ref, G, 3)
            assert rel_err(d["dx"].download(shape=x.shape), dx_ref) <= TOL
    finally:
        for s in streams:
            L.dll.nnhip_stream_synchronize(s)
            L.dll.nnhip_stream_destroy(s)


def test_reg_path_switch_matches_stream(L, rng, monkeypatch):
    """NNHIP_GN_PATH=reg and =stream agree to the parity bar on a shape both take."""
    print("[case] stream vs register path", flush=True)
    B, H, W, C, G = 2, 64, 64, 256, 32
    x, gamma, beta, _ = make_inputs(rng, B, H, W, C)
    monkeypatch.setenv("NNHIP_GN_PATH", "reg")
    y_reg, _, rs_reg = run_fwd(L, x, gamma, beta, G, 3)
    monkeypatch.setenv("NNHIP_GN_PATH", "stream")
    y_str, _, rs_str = run_fwd(L, x, gamma, beta, G, 3)
    assert rel_err(y_str, y_reg) <= TOL
    assert rel_err(rs_str, rs_reg) <= TOL


def test_workspace_status_untouched_by_register_path(L, orc, rng, monkeypatch):
    """A zero-filled lent workspace keeps status 0 through register-path
    launches: their channel partials live past the header and the streaming
    records."""
    print("[case] workspace status after register path", flush=True)
    monkeypatch.setenv("NNHIP_GN_PATH", "reg")
    B, H, W, C, G = 2, 32, 32, 128, 32
    x, gamma, beta, dy = make_inputs(rng, B, H, W, C)
    ws = zeroed(L, L.nnhip_groupnorm_backward_workspace(B, H * W, C, G))
    _, mu_ref, rs_ref = orc.groupnorm_forward(x, gamma, beta, G, 1e-5, 3)
    dx_ref, gg_ref, _ = orc.groupnorm_backward(dy, x, gamma, beta, mu_ref, rs_ref, G, 3)
    dx, gg, _ = run_bwd(L, dy, x, gamma, beta, mu_ref, rs_ref, G, 3, ws)
    d, xh = effective_terms(orc, x, gamma, beta, mu_ref, rs_ref, dy, G, 3)
    fg, _ = gn_param_floor(d, xh, C)
    assert rel_err(dx, dx_ref) <= TOL
    assert rel_err(gg, gg_ref, floor=fg) <= TOL
    assert L.nnhip_groupnorm_workspace_status(ws.p) == 0


def test_stream_groupnorm_graph_replay(L, orc, rng, monkeypatch):
    """The streaming forward + backward captured into a HIP graph and
    replayed with new inputs each time: every replay matches the eager launch
    on the same inputs bit for bit (each replay gets a fresh record tag from
    the workspace), with eager launches on the same workspaces in between."""
    print("[case] stream groupnorm graph capture and replay", flush=True)
    monkeypatch.setenv("NNHIP_GN_PATH", "stream")
    B, H, W, C, G = 16, 64, 64, 256, 32
    HW, act = H * W, 3
    sets = [make_inputs(rng, B, H, W, C) for _ in range(2)]
    xd, dyd = L.alloc(B * HW * C), L.alloc(B * HW * C)
    gd, bd = L.to_device(sets[0][1]), L.to_device(sets[0][2])
    yd, dxd = L.alloc(B * HW * C), L.alloc(B * HW * C)
    mud, rsd, ggd, gbd = L.alloc(B * G), L.alloc(B * G), L.alloc(C), L.alloc(C)
    fws = L.alloc(L.nnhip_groupnorm_forward_workspace(B, HW, C, G))
    bws = L.alloc(L.nnhip_groupnorm_backward_workspace(B, HW, C, G))
    fws.fill_bytes(0)
    bws.fill_bytes(0)
    s = L.dll.nnhip_stream_create()
    assert s
    outs = (yd, mud, rsd, dxd, ggd, gbd)

    def issue():
        L.launch_groupnorm_act_forward_ws(yd.p, mud.p, rsd.p, xd.p, gd.p, bd.p, B, HW, C, G, 1e-5, act, fws.p, s)
        L.launch_groupnorm_act_backward_ws(dxd.p, ggd.p, gbd.p, dyd.p, xd.p, gd.p, bd.p, mud.p, rsd.p, B, HW, C, G,
                                           act, bws.p, s)

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
        for replay in range(6):
            k = replay % 2
            load(k)
            for o in outs:
                o.fill_bytes(0)
            L.sync()
            assert L.dll.nnhip_graph_launch(graph, s) == 0
            for got, ref, name in zip(results(), refs[k], names):
                assert_bits_equal(got, ref, f"replay {replay} {name}")
            issue()  # eager launch on the same workspaces between replays
            for got, ref, name in zip(results(), refs[k], names):
                assert_bits_equal(got, ref, f"eager after replay {replay} {name}")
        assert L.nnhip_groupnorm_workspace_status(fws.p) == 0
        assert L.nnhip_groupnorm_workspace_status(bws.p) == 0
        # the eager reference itself against the oracle (gamma, beta of set 0)
        x, gamma, beta = sets[1][0], sets[0][1], sets[0][2]
        y_ref, mu_ref, rs_ref = orc.groupnorm_forward(x, gamma, beta, G, 1e-5, act)
        assert rel_err(refs[1][0].reshape(x.shape), y_ref) <= TOL
    finally:
        if graph:
            L.dll.nnhip_graph_destroy(graph)
        L.dll.nnhip_stream_synchronize(s)
        L.dll.nnhip_stream_destroy(s)


HIP_ERROR_LAUNCH_TIMEOUT = 702  # hipErrorLaunchTimeOut


def test_wait_failure_surfaces_in_error_record(L, orc, rng, monkeypatch):
    """A statistics wait that gives up is reported, not lost.  With
    NNHIP_GN_SPIN_LIMIT=0 no wait may succeed (each kernel still runs to its
    end); the failure reaches nnhip_get_last_error through the library's
    host-mapped flag, once, for a lent workspace and for the reference-named
    launchers that draw theirs from the stream's pool block.  Back at the
    normal limit the same launches are clean and match the oracle."""
    print("[case] stream groupnorm wait failure -> error record", flush=True)
    monkeypatch.setenv("NNHIP_GN_PATH", "stream")
    B, H, W, C, G = 2, 64, 64, 256, 32
    HW = H * W
    x, gamma, beta, dy = make_inputs(rng, B, H, W, C)
    xd, dyd, yd, dxd = L.to_device(x), L.to_device(dy), L.alloc(x.size), L.alloc(x.size)
    gd, bd, mu, rs, gg, gb = L.to_device(gamma), L.to_device(beta), L.alloc(B * G), L.alloc(B * G), L.alloc(C), L.alloc(C)
    fws = zeroed(L, L.nnhip_groupnorm_forward_workspace(B, HW, C, G))
    bws = zeroed(L, L.nnhip_groupnorm_backward_workspace(B, HW, C, G))

    def fwd(ws):
        if ws is None:
            L.dll.launch_groupnorm_act_forward(yd.p, mu.p, rs.p, xd.p, gd.p, bd.p, B, HW, C, G, 1e-5, 3, None)
        else:
            L.dll.launch_groupnorm_act_forward_ws(yd.p, mu.p, rs.p, xd.p, gd.p, bd.p, B, HW, C, G, 1e-5, 3, ws.p, None)

    def bwd(ws):
        if ws is None:
            L.dll.launch_groupnorm_act_backward(dxd.p, gg.p, gb.p, dyd.p, xd.p, gd.p, bd.p, mu.p, rs.p, B, HW, C, G, 3,
                                                None)
        else:
            L.dll.launch_groupnorm_act_backward_ws(dxd.p, gg.p, gb.p, dyd.p, xd.p, gd.p, bd.p, mu.p, rs.p, B, HW, C, G,
                                                   3, ws.p, None)

    L.sync()
    assert L.last_error()[0] == 0
    monkeypatch.setenv("NNHIP_GN_SPIN_LIMIT", "0")
    for what, launch, ws in (("forward, lent workspace", fwd, fws), ("backward, lent workspace", bwd, bws),
                             ("forward, pool workspace", fwd, None), ("backward, pool workspace", bwd, None)):
        launch(ws)
        L.sync()
        code, msg = L.last_error()
        assert code == HIP_ERROR_LAUNCH_TIMEOUT and "ran out of polls" in msg, (what, code, msg)
        assert L.last_error()[0] == 0, f"{what}: reported more than once"
        if ws is not None:
            assert L.nnhip_groupnorm_workspace_status(ws.p) == 1, what

    monkeypatch.delenv("NNHIP_GN_SPIN_LIMIT")
    fws2 = zeroed(L, L.nnhip_groupnorm_forward_workspace(B, HW, C, G))
    bws2 = zeroed(L, L.nnhip_groupnorm_backward_workspace(B, HW, C, G))
    for ws_f, ws_b in ((fws2, bws2), (None, None)):
        fwd(ws_f)
        bwd(ws_b)
        L.sync()
        assert L.last_error()[0] == 0
        y_ref, mu_ref, rs_ref = orc.groupnorm_forward(x, gamma, beta, G, 1e-5, 3)
        assert rel_err(yd.download(shape=x.shape), y_ref) <= TOL
        dx_ref, _, _ = orc.groupnorm_backward(dy, x, gamma, beta, mu.download(), rs.download(), G, 3)
        assert rel_err(dxd.download(shape=x.shape), dx_ref) <= TOL
    assert L.nnhip_groupnorm_workspace_status(fws2.p) == 0 and L.nnhip_groupnorm_workspace_status(bws2.p) == 0


def test_stream_groupnorm_beside_independent_work(L, orc, rng, monkeypatch):
    """The plain launch's progress argument: workgroups wait only for their
    own team, and whatever else holds the compute units ends by itself.  A
    streaming GroupNorm+SiLU forward and backward (several rounds) runs on one
    stream while another stream keeps the device busy with long elementwise
    kernels.  Every wait finishes (status 0, no error) and the results match
    the oracle."""
    print("[case] stream groupnorm beside elementwise work on another stream", flush=True)
    monkeypatch.setenv("NNHIP_GN_PATH", "stream")
    monkeypatch.delenv("NNHIP_GN_COOPERATIVE", raising=False)
    B, H, W, C, G = 16, 64, 64, 256, 32  # forward 4 rounds, backward 8 rounds of the persistent grid
    HW = H * W
    x, gamma, beta, dy = make_inputs(rng, B, H, W, C)
    xd, dyd, yd, dxd = L.to_device(x), L.to_device(dy), L.alloc(x.size), L.alloc(x.size)
    gd, bd, mu, rs, gg, gb = L.to_device(gamma), L.to_device(beta), L.alloc(B * G), L.alloc(B * G), L.alloc(C), L.alloc(C)
    fws = zeroed(L, L.nnhip_groupnorm_forward_workspace(B, HW, C, G))
    bws = zeroed(L, L.nnhip_groupnorm_backward_workspace(B, HW, C, G))
    n_other = 1 << 27
    a_in, a_out = L.alloc(n_other), L.alloc(n_other)
    a_in.fill_bytes(0)
    s_gn, s_other = L.dll.nnhip_stream_create(), L.dll.nnhip_stream_create()
    try:
        L.launch_activation_forward(a_out.p, a_in.p, n_other, 3, s_other)
        for rep in range(3):
            for _ in range(3):
                L.launch_activation_forward(a_out.p, a_in.p, n_other, 3, s_other)
            L.launch_groupnorm_act_forward_ws(yd.p, mu.p, rs.p, xd.p, gd.p, bd.p, B, HW, C, G, 1e-5, 3, fws.p, s_gn)
            L.launch_groupnorm_act_backward_ws(dxd.p, gg.p, gb.p, dyd.p, xd.p, gd.p, bd.p, mu.p, rs.p, B, HW, C, G, 3,
                                               bws.p, s_gn)
        L.dll.nnhip_stream_synchronize(s_gn)
        L.dll.nnhip_stream_synchronize(s_other)
        L.sync()
        L.check("beside independent work")
        assert L.nnhip_groupnorm_workspace_status(fws.p) == 0 and L.nnhip_groupnorm_workspace_status(bws.p) == 0
        y_ref, mu_ref, rs_ref = orc.groupnorm_forward(x, gamma, beta, G, 1e-5, 3)
        assert rel_err(yd.download(shape=x.shape), y_ref) <= TOL
        dx_ref, _, _ = orc.groupnorm_backward(dy, x, gamma, beta, mu_ref, rs_ref, G, 3)
        assert rel_err(dxd.download(shape=x.shape), dx_ref) <= TOL
    finally:
        for s in (s_gn, s_other):
            L.dll.nnhip_stream_synchronize(s)
            L.dll.nnhip_stream_destroy(s)
