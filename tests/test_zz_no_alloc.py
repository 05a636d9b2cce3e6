"""launch_groupnorm_act_backward_noalloc: the allocation-free variant of
launch_groupnorm_act_backward (its partial sums live in the library's fixed
scratch array instead of a pool block).  Checked against the existing entry
point on the same inputs, bit for bit (same kernels, same reduction orders),
on two calls in a row, the second with a smaller input; plus the refusal of a
shape beyond the scratch's size.  Streaming and register paths both run."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import TOL, assert_bits_equal, rel_err
from test_gpu_groupnorm import make_inputs

pytestmark = pytest.mark.gpu


def _backward(L, launcher, x, gamma, beta, dy, mu, rs, G, act):
    """Runs `launcher`; for the no-allocation entry point also checks that the
    library made no allocation of its own during the call (its pools, their
    blocks, the wait flag: nnhip_launch_allocations)."""
    B, HW, C = x.shape
    xd, dyd, dxd = L.to_device(x), L.to_device(dy), L.alloc(x.size)
    gd, bd, mud, rsd = L.to_device(gamma), L.to_device(beta), L.to_device(mu), L.to_device(rs)
    ggd, gbd = L.alloc(C), L.alloc(C)
    L.sync()
    allocs = L.nnhip_launch_allocations()
    getattr(L, launcher)(dxd.p, ggd.p, gbd.p, dyd.p, xd.p, gd.p, bd.p, mud.p, rsd.p, B, HW, C, G, act, None)
    L.sync()
    L.check(launcher)
    if launcher.endswith("_noalloc"):
        assert L.nnhip_launch_allocations() == allocs, f"{launcher} allocated"
    return dxd.download(shape=x.shape), ggd.download(), gbd.download()


@pytest.mark.parametrize("path", ["stream", "reg"])
def test_noalloc_backward_matches_pool_entry_point(L, orc, rng, monkeypatch, path):
    print(f"[case] groupnorm backward noalloc vs pool entry point, path {path}", flush=True)
    monkeypatch.setenv("NNHIP_GN_PATH", path)
    shapes = [(8, 64, 64, 256, 32), (2, 32, 32, 128, 32)]  # the second call smaller than the first
    for (B, H, W, C, G), act in zip(shapes, (3, 0)):
        x, gamma, beta, dy = make_inputs(rng, B, H, W, C)
        _, mu, rs = orc.groupnorm_forward(x, gamma, beta, G, 1e-5, act)
        got = _backward(L, "launch_groupnorm_act_backward_noalloc", x, gamma, beta, dy, mu, rs, G, act)
        ref = _backward(L, "launch_groupnorm_act_backward", x, gamma, beta, dy, mu, rs, G, act)
        for a, b, what in zip(got, ref, ("dx", "dgamma", "dbeta")):
            assert_bits_equal(a, b, f"{what} {B}x{H}x{W}x{C}")
        dx_ref, _, _ = orc.groupnorm_backward(dy, x, gamma, beta, mu, rs, G, act)
        assert rel_err(got[0], dx_ref) <= TOL


def test_noalloc_size_check_follows_the_path(L, monkeypatch):
    """The streaming workspace limit applies only where the streaming kernels
    run: with the register path forced, the shape the next test refuses
    (streaming plan about 21 MiB; channel partials 1 MiB) passes the size
    check and stops at the null-pointer check, so nothing is launched."""
    print("[case] groupnorm backward noalloc size check on the register path", flush=True)
    B, HW, C, G = 512, 64 * 64, 256, 32
    assert L.nnhip_groupnorm_backward_workspace(B, HW, C, G) * 4 > 12 << 20
    L.sync()
    assert L.last_error()[0] == 0
    monkeypatch.setenv("NNHIP_GN_PATH", "reg")
    L.dll.launch_groupnorm_act_backward_noalloc(None, None, None, None, None, None, None, None, None, B, HW, C, G, 3,
                                                None)
    code, msg = L.last_error()
    assert code != 0 and "null pointer" in msg, (code, msg)


def test_noalloc_backward_refuses_oversized_shape(L, rng):
    print("[case] groupnorm backward noalloc refuses a shape beyond its scratch", flush=True)
    B, HW, C, G = 512, 64 * 64, 256, 32  # streaming workspace of about 21 MiB > 12 MiB
    L.sync()
    assert L.last_error()[0] == 0
    L.dll.launch_groupnorm_act_backward_noalloc(None, None, None, None, None, None, None, None, None, B, HW, C, G, 3,
                                                None)
    code, msg = L.last_error()
    assert code != 0 and "needs" in msg and "scratch" in msg, (code, msg)
