#!/usr/bin/env python3
"""Benchmark: TinyMLPHashGrid training step on one MI355X.

Workload (BASELINE configs[1]/[2], the reference's published "Hash + MLP 64x2
train step" row, modules/TinyMLP/tests_kernels/benchCompare.cu:61-84):
  B = 2^18 samples/step, positions U[0,1)^3 (vectorDim 3), L = 16 levels,
  F = 2, T = 2^19 entries/level, base 16, b = (2048/16)^(1/15) (finest 2048),
  density MLP 32 -> 64 ReLU -> 16, fp16 operands / fp32 accumulation,
  table U(+-1e-4), MSE to U[0,1] targets with loss scale 65536, Adam over the
  16.8 M table entries and 3,152 MLP parameters.
One step = zero_grad + forward (fused encode + MLP) + MSE + backward (fused MLP
backward + hash scatter) + Adam, all through the C-ABI library, inputs resident
in HBM.  Prints ONE JSON line.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
from __future__ import annotations

import argparse
import ctypes as C
import importlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
FP16_PEAK_TFLOPS = 2500.0      # MI355X dense fp16 MFMA
REF_TRAIN_MS_2P18 = 12.200     # RTX 4060 Laptop, tinymlp.csv:49

B = 1 << 18
L, F, TBL, BASE = 16, 2, 1 << 19, 16
GROWTH = (2048.0 / 16.0) ** (1.0 / 15.0)
HID, OUT, LAYERS = 64, 16, 2
LOSS_SCALE = 65536.0
LR, B1, B2, EPS = 1e-2, 0.9, 0.99, 1e-15

# Algorithmic counts per unit (SURVEY 8(d) figures for this head).
ENC_BYTES_PER_SAMPLE = 16 + L * 8 * 4 + 2 * L * 2            # 592
SCATTER_BYTES_PER_SAMPLE = 16 + 2 * L * 2 + L * 8 * 2 * 8    # 2,112 (+16 pos: 2,128 with 16-B rows)
ADAM_BYTES_PER_PARAM = 34
MLP_FLOP_FWD = 2 * (32 * 64 + 64 * 16)                       # 6,144 per sample
MLP_FLOP_BWD = 2 * MLP_FLOP_FWD                              # dX + dW: 12,288 per sample


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-oracle baseline leg")
    ap.add_argument("--profile-steps", type=int, default=0, help="only run N steps (for rocprofv3)")
    return ap.parse_args()


def cpu_baseline(pos, tgt, table, W, Bv):
    """The C oracle (oracle/liboracle.so) on the host cores: one full step at N_cpu samples."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as orc
    n = 1 << 16
    p = np.ascontiguousarray(pos[:n])
    t = np.ascontiguousarray(tgt[:n])
    tab = table.copy()
    t16 = tab.astype(np.float16)
    g = np.zeros_like(tab)
    m = np.zeros_like(tab)
    v = np.zeros_like(tab)
    w = W.copy()
    t0 = time.perf_counter()
    enc = orc.hash_encode(p, t16, TBL, L, BASE, GROWTH)
    y, acts = orc.mlp_forward(enc, w.astype(np.float16), Bv, 32, HID, OUT, LAYERS)
    _, dl = orc.mse_loss_grad(y, t, OUT, LOSS_SCALE)
    dW, dB, dx = orc.mlp_backward(dl, enc, acts, w.astype(np.float16), 32, HID, OUT, LAYERS)
    orc.hash_scatter(p, dx, TBL, L, BASE, GROWTH, grads=g)
    bc1, bc2 = orc.adam_bias_corrections(B1, B2, 1)
    orc.adam_hash(tab, g, m, v, LR, B1, B2, EPS, bc1, bc2, 1 / LOSS_SCALE)
    mw = np.zeros_like(w)
    vw = np.zeros_like(w)
    orc.adam_dense(w, dW, mw, vw, LR, B1, B2, EPS, bc1, bc2, 1 / LOSS_SCALE)
    dt = time.perf_counter() - t0
    return {"value": n / dt, "unit": "samples/s", "cores": orc.num_threads(), "kind": "port",
            "sample": f"one full training step at N={n} samples (1/4 of the GPU batch) incl. Adam over the "
                      f"whole T=2^19 x 16-level table; {dt:.2f} s"}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU; multi-GPU sharding is design-only "
                                   "(see DESIGN.md), run with --gpus 1"}))
        sys.exit(2)
    import torch
    P = importlib.import_module("3dmaker_amd")
    assert torch.cuda.is_available(), "bench.py needs cuda:0"
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream

    rng = np.random.default_rng(2024)
    pos = rng.random((B, 3), dtype=np.float32)
    tgt = rng.random((B, OUT), dtype=np.float32).astype(np.float16)
    table = rng.uniform(-1e-4, 1e-4, L * TBL * F).astype(np.float32)
    fan = np.sqrt(6.0 / (32 + HID)), np.sqrt(6.0 / (HID + OUT))
    W = np.concatenate([rng.uniform(-fan[0], fan[0], HID * 32), rng.uniform(-fan[1], fan[1], OUT * HID)]).astype(np.float32)
    Bv = np.zeros(HID + OUT, np.float32)

    opt = P.MLPGridOptions(vectorDim=3, hiddenDim=HID, outputDim=OUT, numLayers=LAYERS, activationType=0,
                           tableSize=TBL, numLevels=L, b=GROWTH, lowestSize=BASE, featuresLevel=F)
    g = P.HashGrid(opt, B, seed=42)
    g.load_hashgrid(table)
    g.load_weights(W, Bv)
    d_pos = torch.from_numpy(pos).to(dev)
    d_tgt = torch.from_numpy(tgt).to(dev)
    d_out = torch.empty((B, OUT), dtype=torch.float32, device=dev)

    def step():
        g.zero_grad(sp)
        g.forward(d_pos, d_out, B, sp)
        g.calculate_loss_and_grad(d_tgt, B, LOSS_SCALE, False, sp)
        g.backward(B, None, sp)
        g.step(LR, B1, B2, EPS, LOSS_SCALE, sp)

    if args.profile_steps:
        for _ in range(args.profile_steps):
            step()
        torch.cuda.synchronize()
        print(json.dumps({"profile_steps": args.profile_steps}))
        return

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / args.steps

    # Per-phase breakdown with HIP events on the launch stream.
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    phases = {"forward": [], "mse": [], "backward": [], "adam": []}
    R = max(5, min(20, args.steps))
    for _ in range(R):
        e = [ev() for _ in range(5)]
        g.zero_grad(sp)
        e[0].record(stream)
        g.forward(d_pos, d_out, B, sp)
        e[1].record(stream)
        g.calculate_loss_and_grad(d_tgt, B, LOSS_SCALE, False, sp)
        e[2].record(stream)
        g.backward(B, None, sp)
        e[3].record(stream)
        g.step(LR, B1, B2, EPS, LOSS_SCALE, sp)
        e[4].record(stream)
        torch.cuda.synchronize()
        for k, name in enumerate(phases):
            phases[name].append(e[k].elapsed_time(e[k + 1]))
    bd = {k: float(np.mean(v)) for k, v in phases.items()}

    # Stand-alone kernels on the same buffers: encode, scatter, hash Adam.
    bufs = g.buffers()
    d_enc = torch.empty((B, 2 * L), dtype=torch.float16, device=dev)
    d_pos4 = torch.zeros((B, 4), dtype=torch.float32, device=dev)
    d_pos4[:, :3] = d_pos

    def timed(fn, reps=20):
        fn()
        a, b = ev(), ev()
        a.record(stream)
        for _ in range(reps):
            fn()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps

    t_enc = timed(lambda: P.launch("launchHashEncodeKernel", C.byref(opt), bufs.fwd_hashtable, d_pos4, 4, d_enc,
                                   B, sp))
    d_grads = torch.zeros(L * TBL * F, dtype=torch.float32, device=dev)
    t_scat = timed(lambda: P.launch("launchHashTableBackwardKernel", bufs.dx_out, d_pos4, d_grads, B, TBL, L,
                                    GROWTH, BASE, F, sp))
    # hash Adam with a realistic (post-scatter) gradient, re-filled before every launch
    d_w = torch.from_numpy(table).to(dev)
    d_w16 = torch.empty(L * TBL * F, dtype=torch.float16, device=dev)
    d_m = torch.zeros_like(d_w)
    d_v = torch.zeros_like(d_w)
    d_g = torch.empty_like(d_w)
    adam_ms = []
    for _ in range(10):
        d_g.copy_(d_grads)
        a, b = ev(), ev()
        a.record(stream)
        P.launch("launchAdamHashGridOptim", C.byref(opt), d_w, d_w16, d_g, d_m, d_v, LR, B1, B2, EPS, 0.1, 0.01,
                 1 / LOSS_SCALE, sp)
        b.record(stream)
        torch.cuda.synchronize()
        adam_ms.append(a.elapsed_time(b))
    t_adam = float(np.mean(adam_ms))
    nz = float((d_grads != 0).float().mean().item())

    kernels = {
        "hash_scatter": {"ms": t_scat, "bytes": SCATTER_BYTES_PER_SAMPLE * B},
        "adam_hash": {"ms": t_adam, "bytes": ADAM_BYTES_PER_PARAM * L * TBL * F},
        "hash_encode": {"ms": t_enc, "bytes": ENC_BYTES_PER_SAMPLE * B},
    }
    dom = max(kernels, key=lambda k: kernels[k]["ms"])
    ach = kernels[dom]["bytes"] / (kernels[dom]["ms"] * 1e-3) / 1e9
    mlp_flop = (MLP_FLOP_FWD + MLP_FLOP_BWD) * B
    roofline = {"bound": "hbm", "kernel": dom, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
                "algorithmic_bytes_per_launch": kernels[dom]["bytes"], "avg_launch_ms": round(kernels[dom]["ms"], 4)}

    value = B / (ms_step * 1e-3)
    out = {
        "metric": "training samples/sec (hash grid + density MLP train step, 2^18 samples/step)",
        "value": round(value, 1),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(value / (B / (REF_TRAIN_MS_2P18 * 1e-3)), 3),
        "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": "TinyMLPHashGrid train step (zero+fwd+MSE+bwd+Adam)", "batch": B,
                   "levels": L, "table_size": TBL, "base": BASE, "growth": round(GROWTH, 6),
                   "mlp": "32-64-16", "loss_scale": LOSS_SCALE},
        "breakdown_ms": {k: round(v, 4) for k, v in bd.items()},
        "kernel_ms": {k: round(v["ms"], 4) for k, v in kernels.items()},
        "hash_encodes_per_s": round(B / (t_enc * 1e-3), 1),
        "mfma_util": round(mlp_flop / ((bd["forward"] + bd["backward"]) * 1e-3) / 1e12 / FP16_PEAK_TFLOPS, 5),
        "grad_nonzero_frac": round(nz, 4),
        "roofline": roofline,
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(pos, tgt, table, W, Bv)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
