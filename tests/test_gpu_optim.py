"""Optimizer rows: Adam (reference src/kernels.cu:170-183, 241-248 with the
host bias corrections of src/optimizer.c:54-69) and EMA
(src/ema.c:29-35 -> weighted_sum), per tensor and as the one-launch
multi-tensor Adam+EMA over BASELINE cfg5's DDPM-UNet-like tensor list."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import TOL, rel_err

pytestmark = pytest.mark.gpu

LR, B1, B2, EPS, DECAY = 1e-4, 0.9, 0.999, 1e-8, 0.9999


def cfg5_sizes():
    """Parameter sizes of a DDPM UNet with channels (64,128,256,448,512),
    emb_dim 512, C_in = C_out = 3, two res-blocks per level, in the
    reference's parameter order (src/ddpm_unet.c:239-255,
    src/conv_residual.c:68-76), floored at 64 elements."""
    from bench import cfg5_tensor_sizes  # shared with the bench

    return cfg5_tensor_sizes()


def _host_lists(rng, sizes):
    p = [(0.02 * rng.standard_normal(n)).astype(np.float32) for n in sizes]
    return p, [np.zeros(n, np.float32) for n in sizes], [np.zeros(n, np.float32) for n in sizes]


def test_cfg5_list_shape():
    sizes = cfg5_sizes()
    assert len(sizes) == 212 and sum(sizes) == 35_111_104
    assert min(sizes) == 64 and max(sizes) == 2_359_296


@pytest.mark.parametrize("n", [1, 5, 4096, 4097, 100_003])
def test_adam_step_single_tensor(L, orc, rng, n):
    p0 = (0.02 * rng.standard_normal(n)).astype(np.float32)
    pd, md, vd = L.to_device(p0), L.to_device(np.zeros(n, np.float32)), L.to_device(np.zeros(n, np.float32))
    p, m, v = p0, np.zeros(n, np.float32), np.zeros(n, np.float32)
    gd = L.alloc(n)
    for t in range(1, 6):
        g = (1e-3 * rng.standard_normal(n)).astype(np.float32)
        gd.upload(g)
        bc1, bc2 = orc.adam_bias_corrections(B1, B2, t)
        L.launch_adam_step(pd.p, md.p, vd.p, gd.p, LR, B1, B2, EPS, bc1, bc2, n, None)
        p, m, v = orc.adam_step(p, m, v, g, LR, B1, B2, EPS, bc1, bc2)
    L.sync()
    assert rel_err(pd.download(), p) <= TOL
    assert rel_err(md.download(), m) <= TOL
    assert rel_err(vd.download(), v) <= TOL


def _run_plan(L, nn, orc, rng, sizes, steps, with_ema=True, misalign=False):
    ps, ms, vs = _host_lists(rng, sizes)
    shadows = [p.copy() for p in ps]
    off = 1 if misalign else 0
    dev = []
    slots = []
    for p, m, v, s in zip(ps, ms, vs, shadows):
        pd, md, vd, sd, gd = (L.alloc(p.size + off) for _ in range(5))
        for d, h in ((pd, p), (md, m), (vd, v), (sd, s)):
            d.upload(np.concatenate([np.zeros(off, np.float32), h]))
        dev.append((pd, md, vd, sd, gd))
        slots.append({"p": pd.offset(off), "m": md.offset(off), "v": vd.offset(off), "g": gd.offset(off),
                      "shadow": sd.offset(off) if with_ema else None, "n": p.size})
    plan = nn.make_plan(L, slots)
    w1 = float(np.float32(1) - np.float32(DECAY))  # 1.0f - decay in host float (src/ema.c:33)
    try:
        for t in range(1, steps + 1):
            gs = [(1e-3 * rng.standard_normal(n)).astype(np.float32) for n in sizes]
            for (pd, md, vd, sd, gd), g in zip(dev, gs):
                gd.upload(np.concatenate([np.zeros(off, np.float32), g]))
            bc1, bc2 = orc.adam_bias_corrections(B1, B2, t)
            L.launch_adam_ema_step(plan, LR, B1, B2, EPS, bc1, bc2, DECAY if with_ema else 1.0,
                                   w1 if with_ema else 0.0, None)
            for i, g in enumerate(gs):
                ps[i], ms[i], vs[i] = orc.adam_step(ps[i], ms[i], vs[i], g, LR, B1, B2, EPS, bc1, bc2)
                if with_ema:
                    shadows[i] = orc.weighted_sum(shadows[i], ps[i], DECAY, w1)
        L.sync()
    finally:
        L.dll.nnhip_multi_tensor_plan_destroy(plan)
    for i, (pd, md, vd, sd, gd) in enumerate(dev):
        assert rel_err(pd.download()[off:], ps[i]) <= TOL, i
        assert rel_err(md.download()[off:], ms[i]) <= TOL, i
        assert rel_err(vd.download()[off:], vs[i]) <= TOL, i
        if with_ema:
            assert rel_err(sd.download()[off:], shadows[i]) <= TOL, i


def test_multi_tensor_adam_ema_small_lists(L, nn, orc, rng):
    _run_plan(L, nn, orc, rng, [64, 5, 4096, 4097, 12_345, 1], steps=20)
    _run_plan(L, nn, orc, rng, [64, 7, 300], steps=5, with_ema=False)
    _run_plan(L, nn, orc, rng, [64, 7, 4100], steps=5, misalign=True)


def test_multi_tensor_adam_ema_cfg5(L, nn, orc, rng):
    """The full cfg5 list (212 tensors, 35.1M parameters), 3 steps."""
    print("[case] cfg5 adam+ema", flush=True)
    _run_plan(L, nn, orc, rng, cfg5_sizes(), steps=3)


def test_multi_tensor_adam_ema_cfg5_100_steps(L, nn, orc, rng):
    """BASELINE cfg5 as written: the full list (212 tensors, 35,111,104
    parameters, src/ddpm_unet.c:239-255 order), p ~ N(0, 0.02), m = v = 0,
    shadow = p, 100 fused Adam+EMA steps from seed (src/optimizer.c:54-69
    then src/ema.c:29-35, as src/diffusion/train.c:53-54 calls them), checked
    against the oracle's per-element Adam and EMA after the last step.  The
    tensors are consecutive slices of flat device buffers, one plan slot each;
    step t's gradient is the window of a seeded N(0, 1e-3) pool that starts at
    a pseudo-random offset drawn from (seed, t), so that 100 steps of 35.1M
    gradients need neither 100 host draws nor 100 x 212 uploads.  The oracle
    applies the same update to the flat concatenation (the update is
    elementwise with per-step scalars)."""
    print("[case] cfg5 adam+ema, full list, 100 steps", flush=True)
    sizes = cfg5_sizes()
    total = sum(sizes)
    offs = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
    p = (0.02 * rng.standard_normal(total, dtype=np.float32)).astype(np.float32)
    m = np.zeros(total, np.float32)
    v = np.zeros(total, np.float32)
    sh = p.copy()
    pool = (1e-3 * rng.standard_normal(2 * total, dtype=np.float32)).astype(np.float32)
    starts = np.random.default_rng([410293, 5]).integers(0, total, size=101)
    pd, md, vd, sd, gd = L.to_device(p), L.to_device(m), L.to_device(v), L.to_device(sh), L.alloc(total)
    slots = [{"p": pd.offset(o), "m": md.offset(o), "v": vd.offset(o), "g": gd.offset(o), "shadow": sd.offset(o),
              "n": n} for o, n in zip(offs, sizes)]
    plan = nn.make_plan(L, slots)
    w1 = float(np.float32(1) - np.float32(DECAY))  # 1.0f - decay in host float (src/ema.c:33)
    try:
        for t in range(1, 101):
            g = pool[starts[t]:starts[t] + total]
            gd.upload(g)
            bc1, bc2 = orc.adam_bias_corrections(B1, B2, t)
            L.launch_adam_ema_step(plan, LR, B1, B2, EPS, bc1, bc2, DECAY, w1, None)
            p, m, v = orc.adam_step(p, m, v, g, LR, B1, B2, EPS, bc1, bc2)
            sh = orc.weighted_sum(sh, p, DECAY, w1)
            if t % 25 == 0:
                print(f"  step {t}", flush=True)
        L.sync()
    finally:
        L.dll.nnhip_multi_tensor_plan_destroy(plan)
    gp, gm, gv, gs = pd.download(), md.download(), vd.download(), sd.download()
    for o, n in zip(offs, sizes):  # every tensor on its own, as the bar is defined
        for got, ref, what in ((gp, p, "p"), (gm, m, "m"), (gv, v, "v"), (gs, sh, "shadow")):
            assert rel_err(got[o:o + n], ref[o:o + n]) <= TOL, (what, int(o), n)


def test_ema_only_plan(L, nn, orc, rng):
    sizes = [64, 1000, 4099]
    ps = [rng.standard_normal(n).astype(np.float32) for n in sizes]
    ss = [rng.standard_normal(n).astype(np.float32) for n in sizes]
    devs = [(L.to_device(p), L.to_device(s)) for p, s in zip(ps, ss)]
    plan = nn.make_plan(L, [{"p": pd.p, "shadow": sd.p, "n": n} for (pd, sd), n in zip(devs, sizes)])
    w1 = float(np.float32(1) - np.float32(DECAY))
    try:
        L.launch_ema_update(plan, DECAY, w1, None)
        L.sync()
        with pytest.raises(nn.NnHipError):  # no m/v/g in this plan
            L.launch_adam_ema_step(plan, LR, B1, B2, EPS, 0.1, 0.001, DECAY, w1, None)
    finally:
        L.dll.nnhip_multi_tensor_plan_destroy(plan)
    for (pd, sd), p, s in zip(devs, ps, ss):
        assert rel_err(sd.download(), orc.weighted_sum(s, p, DECAY, w1)) <= TOL
