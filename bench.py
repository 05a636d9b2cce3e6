#!/usr/bin/env python3
"""North-star benchmark: GroupNorm(32)+SiLU forward+backward, NHWC fp32,
N=256, H=W=64, C=256 (metric quoted on it).

A step is one fused forward (launch_groupnorm_act_forward) plus one fused
backward (launch_groupnorm_act_backward_ws: dx and dgamma/dbeta) over the
whole batch, inputs resident in HBM.  value = algorithmic bytes per step /
time per step, algorithmic bytes = 20 B/elem (fwd: read x, write y; bwd: read
x, dy, write dx) = 5,368,709,120 B.

Timing: HIP events on the launch stream around exactly --steps steps after
--warmup untimed steps, device synchronised on both sides.  The roofline
object is for the dominant kernel (the backward: 12 B/elem), timed per launch
with events on the same stream.  cpu_baseline times the oracle's fp32 OpenMP
transcription of the reference kernels on a bounded batch sample on the host.

Prints ONE JSON line.  --gpus N > 1 is not supported (one GPU per box).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "GroupNorm+SiLU fwd+bwd µs and HBM GB/s (% of 8 TB/s peak), N=256 64×64×256"
HBM_PEAK_GBS = 8000.0
SEED = 410293


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def cfg5_tensor_sizes(channels=(64, 128, 256, 448, 512), emb_dim=512, c_in=3, c_out=3, res_blocks=2,
                      floor=64):
    """Parameter-tensor sizes of BASELINE cfg5's DDPM-UNet-like list, in the
    reference's ParamList order: the time-embedding MLP (src/diffusion/ddpm.c:
    103-108, 77-81), then ddpm_unet_parameters (src/ddpm_unet.c:239-255) with
    conv_residual's gn1, conv1, time_proj, gn2, conv2 (src/conv_residual.c:
    68-76), conv weight then bias (src/conv2d.c:68-76), the plain attention's
    Wq..Wo then bq..bo (src/attention.c:199-216).  `res_blocks` blocks per
    level on each side; sizes floored at `floor`.  Default: 212 tensors,
    35,111,104 elements."""
    out = []

    def add(n):
        out.append(max(n, floor))

    def conv(ci, co, k):
        add(k * k * ci * co)
        add(co)

    def linear(i, o):
        add(i * o)
        add(o)

    def res_block(c):
        add(c), add(c)
        conv(c, c, 3)
        linear(emb_dim, c)
        add(c), add(c)
        conv(c, c, 3)

    levels = len(channels) - 1
    linear(emb_dim, emb_dim)
    linear(emb_dim, emb_dim)
    conv(c_in, channels[0], 3)
    for i in range(levels):
        for _ in range(res_blocks):
            res_block(channels[i])
        conv(channels[i], channels[i + 1], 1)
    cb = channels[levels]
    res_block(cb)
    for _ in range(4):
        add(cb * cb)
    for _ in range(4):
        add(cb)
    res_block(cb)
    for i in reversed(range(levels)):
        conv(channels[i + 1] + channels[i], channels[i], 1)
        for _ in range(res_blocks):
            res_block(channels[i])
    conv(channels[0], c_out, 3)
    return out


def make_inputs(B, HW, C, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((B, HW, C), dtype=np.float32)
    dy = rng.standard_normal((B, HW, C), dtype=np.float32)
    gamma = (1.0 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(C)).astype(np.float32)
    return x, dy, gamma, beta


def cpu_baseline(x, dy, gamma, beta, G, sample_b, reps=1):
    """Oracle fp32 OpenMP transcription (CPU baseline) on x[:sample_b]."""
    from oracle import oracle as orc

    threads = min(16, os.cpu_count() or 1)
    orc.set_threads(threads)
    xs, dys = np.ascontiguousarray(x[:sample_b]), np.ascontiguousarray(dy[:sample_b])
    orc.groupnorm_forward_f32(xs[:1], gamma, beta, G, 1e-5, 3)  # warm the thread pool
    t0 = time.perf_counter()
    for _ in range(reps):
        y, mu, rs = orc.groupnorm_forward_f32(xs, gamma, beta, G, 1e-5, 3)
        orc.groupnorm_backward_f32(dys, xs, gamma, beta, mu, rs, G, 3)
    dt = (time.perf_counter() - t0) / reps
    n = xs.size
    return {
        "value": round(20.0 * n / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": orc.get_threads(),
        "kind": "port",
        "sample": f"GroupNorm(32)+SiLU fwd+bwd on {sample_b} of 256 samples ([{sample_b},64,64,256]), "
                  f"{reps} rep(s), {dt * 1e3:.1f} ms per fwd+bwd, fp32 OpenMP transcription of "
                  f"src/kernels.cu:622-717 + Pade SiLU",
        "us_per_sample_step": round(dt / sample_b * 1e6, 1),
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=256)
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline leg")
    ap.add_argument("--cpu-sample", type=int, default=16, help="batch samples timed on the CPU")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build measures one GPU "
              f"(the path shards over the batch with no exchange but a 2*C-float dgamma/dbeta "
              f"all-reduce; see DESIGN.md)", file=sys.stderr)
        return 2

    from __graft_entry__ import load_package

    nn = load_package()
    L = nn.lib()
    if L.device_count() < 1:
        print("bench.py: no HIP device", file=sys.stderr)
        return 1
    info = L.device_info()
    B, H, W, C, G = args.batch, 64, 64, 256, 32
    HW = H * W
    n = B * HW * C
    log(f"[bench] device {info}; workload GN({G})+SiLU [{B},{H},{W},{C}] fp32; generating inputs")
    x, dy, gamma, beta = make_inputs(B, HW, C, SEED)

    xd, dyd = L.to_device(x), L.to_device(dy)
    yd, dxd = L.alloc(n), L.alloc(n)
    gd, bd = L.to_device(gamma), L.to_device(beta)
    mu, rs = L.alloc(B * G), L.alloc(B * G)
    gg, gb = L.alloc(C), L.alloc(C)
    ws = L.alloc(L.nnhip_groupnorm_backward_workspace(B, HW, C, G))
    stream = L.dll.nnhip_stream_create()
    if not stream:
        raise RuntimeError("stream creation failed")
    act = nn.ACT_SILU

    def fwd():
        L.launch_groupnorm_act_forward(yd.p, mu.p, rs.p, xd.p, gd.p, bd.p, B, HW, C, G, 1e-5, act, stream)

    def bwd():
        L.launch_groupnorm_act_backward_ws(dxd.p, gg.p, gb.p, dyd.p, xd.p, gd.p, bd.p, mu.p, rs.p, B, HW, C, G,
                                           act, ws.p, stream)

    ev = [L.dll.nnhip_event_create() for _ in range(4)]
    log(f"[bench] warmup {args.warmup} steps")
    for _ in range(args.warmup):
        fwd()
        bwd()
    L.dll.nnhip_stream_synchronize(stream)
    L.sync()

    # whole-step timing
    log(f"[bench] timing {args.steps} steps")
    L.dll.nnhip_event_record(ev[0], stream)
    for _ in range(args.steps):
        fwd()
        bwd()
    L.dll.nnhip_event_record(ev[1], stream)
    L.dll.nnhip_event_synchronize(ev[1])
    L.sync()
    total_ms = L.dll.nnhip_event_elapsed_ms(ev[0], ev[1])
    ms_step = total_ms / args.steps

    # per-launch timing of forward and backward (same stream, events per launch)
    fwd_ms, bwd_ms = [], []
    for _ in range(args.steps):
        L.dll.nnhip_event_record(ev[0], stream)
        fwd()
        L.dll.nnhip_event_record(ev[1], stream)
        bwd()
        L.dll.nnhip_event_record(ev[2], stream)
        L.dll.nnhip_event_synchronize(ev[2])
        fwd_ms.append(L.dll.nnhip_event_elapsed_ms(ev[0], ev[1]))
        bwd_ms.append(L.dll.nnhip_event_elapsed_ms(ev[1], ev[2]))
    L.check("bench")
    fwd_us = 1e3 * float(np.mean(fwd_ms))
    bwd_us = 1e3 * float(np.mean(bwd_ms))

    algo_bytes = 20.0 * n
    gbs = algo_bytes / (ms_step * 1e-3) / 1e9
    bwd_bytes = 12.0 * n
    bwd_gbs = bwd_bytes / (bwd_us * 1e-6) / 1e9
    fwd_gbs = 8.0 * n / (fwd_us * 1e-6) / 1e9
    log(f"[bench] step {ms_step * 1e3:.1f} us ({gbs:.0f} GB/s, {gbs / HBM_PEAK_GBS:.3f} of peak); "
        f"fwd {fwd_us:.1f} us ({fwd_gbs:.0f} GB/s), bwd {bwd_us:.1f} us ({bwd_gbs:.0f} GB/s)")

    # quick self-check of one output against the oracle on one sample (not timed)
    cpu = None
    if not args.no_cpu:
        sample = max(1, min(args.cpu_sample, B))
        log(f"[bench] cpu_baseline on {sample} samples")
        cpu = cpu_baseline(x, dy, gamma, beta, G, sample)

    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "us_per_step": round(ms_step * 1e3, 2),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "fwd_us": round(fwd_us, 2),
        "bwd_us": round(bwd_us, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1) x and dy, gamma=1+0.1N, beta=0.1N)",
        "config": {"workload": "groupnorm32_silu_fwd_bwd", "N": B, "H": H, "W": W, "C": C, "G": G,
                   "layout": "NHWC", "algorithmic_bytes_per_step": int(algo_bytes),
                   "device": info["arch"]},
        "roofline": {
            "kernel": "gn_bwd_reg (launch_groupnorm_act_backward_ws incl. the dgamma/dbeta reduce)",
            "bound": "hbm",
            "achieved": round(bwd_gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(bwd_gbs / HBM_PEAK_GBS, 4),
            "traffic": None,
            "algorithmic_bytes_per_launch": int(bwd_bytes),
            "avg_launch_us": round(bwd_us, 2),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)
    for e in ev:
        L.dll.nnhip_event_destroy(e)
    L.dll.nnhip_stream_destroy(stream)
    return 0


if __name__ == "__main__":
    sys.exit(main())
