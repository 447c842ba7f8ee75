#!/usr/bin/env python3
"""Benchmark: the full NeRF training step of 3DMaker on one MI355X.

Workload (the end-to-end configuration; the reference's
step is InstantNerf::trainWithRaysHit, modules/NeRF/InstantNerf.cu:359-583):
  procedural scene (3 seeded spheres, sigma_max * sigmoid(-sdf / 0.01), 3-band
  sinusoidal colour), ground truth rendered by fixed-step quadrature for a pool
  of rays from 100 cameras at 800x800, fov 50 deg, on a radius-1.5 sphere;
  occupancy 128^3 x 5 cascades x 4 mips, AABB +-1.5, K = 1; hash grid L = 16,
  F = 2, T = 2^19, base 16, b = 1.3819; density 32 -> 64 -> 16, colour
  32 -> 64 -> 64 -> 3 (sigmoid); distortion loss lambda = 0.1; loss scale 128;
  Adam (0.9, 0.999, 1e-8); cosine LR 1e-2 -> 1e-4 over 2000 steps; occupancy
  refreshed every 16 steps (one jittered sample per cell for the first 256
  steps, then half the cells' worth of occupied/uniform samples).
One step = one optimizer step on one hit batch of at most 2^18 compacted
samples: ray setup, DDA count/scan/cutoff/fill, fused hash encode + density
MLP forward, SH gather, colour MLP forward, compositing with distortion,
colour/density gradients, both MLP backwards, hash scatter, Adam over all
parameters (16.8 M table entries), plus the amortised occupancy refresh.
Rays come 2^16 per trainWithRaysHit call (the reference trainer's chunk), the
ray pool and ground truth are resident in HBM before timing starts.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--profile-steps N]

Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import ctypes as C
import importlib
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
FP16_PEAK_TFLOPS = 2500.0      # MI355X dense fp16 MFMA
REF_HASHGRID_TRAIN_MS = 12.200  # TinyMLPHashGrid 64x2 train step at 2^18, RTX 4060 Laptop (tinymlp.csv:49)

BATCH = 1 << 18
RAYS_PER_CALL = 1 << 16
POOL = 1 << 21
L, F, TBL, BASE, GROWTH = 16, 2, 1 << 19, 16, 1.3819
LR_MAX, LR_MIN, ANNEAL = 1e-2, 1e-4, 2000

# Algorithmic counts per unit.
ENC_BYTES_PER_SAMPLE = 16 + L * 8 * 4 + 2 * L * 2                    # 592
SCATTER_BYTES_PER_SAMPLE = 16 + 2 * L * 2 + L * 8 * 2 * 8               # 2,128 (pos 16 + denc 64 + RMW 2,048)
ADAM_BYTES_PER_PARAM = 34
MLP_FLOP_PER_SAMPLE = 3 * (2 * (32 * 64 + 64 * 16) + 2 * (32 * 64 + 64 * 64 + 64 * 3))  # 56,448 fwd + bwd
COPY_BYTES = 256 << 20         # copy-calibration kernel of the PMC runs (read and write each)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC summary, or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        return t["kernels"][kernel]["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=256)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-oracle baseline leg")
    ap.add_argument("--profile-steps", type=int, default=0,
                    help="run --warmup steps, then this many, and exit (for rocprofv3)")
    ap.add_argument("--components", action="store_true",
                    help="only time the stand-alone encode / scatter launches at 2^18 and exit")
    return ap.parse_args()


def options(P):
    o = P.Nerf.default_options()
    o.gridResolution[:] = [128, 128, 128]
    o.aabbMin[:] = [-1.5] * 3
    o.aabbMax[:] = [1.5] * 3
    o.levelsMipmap, o.numCascades, o.samplesPerVoxel = 4, 5, 1
    o.densityHiddenDim, o.densityNumLayers = 64, 2
    o.colorHiddenDim, o.colorNumLayers = 64, 3
    o.hashTableSize, o.numLevels, o.growthFactor, o.baseResolution, o.featuresPerLevel = TBL, L, GROWTH, BASE, F
    # NerfTrainer.cu:72-73: rayChunkSize = batchSize / 4, the rays of one trainWithRaysHit call
    o.batchSize, o.rayChunkSize, o.renderBatchSize = BATCH, RAYS_PER_CALL, BATCH
    o.lambdaDist, o.lambdaDepth = 0.1, 0.0
    o.learningRate, o.beta1, o.beta2, o.epsilon, o.lossScale = LR_MAX, 0.9, 0.999, 1e-8, 128.0
    o.bgColor[:] = [1.0, 1.0, 1.0]
    o.minDensityThreshold, o.decayValue, o.densityBias = 0.01, 0.95, 0.0
    return o


def cosine_lr(step):
    p = min(step / ANNEAL, 1.0)
    return LR_MIN + 0.5 * (LR_MAX - LR_MIN) * (1.0 + math.cos(math.pi * p))


class Trainer:
    """Feeds the ray pool to InstantNerf 2^16 rays per call (NerfTrainer.cu:137-179)."""

    def __init__(self, nerf, o, d, gt, stream):
        self.nerf, self.o, self.d, self.gt, self.stream = nerf, o, d, gt, stream
        self.cursor = 0
        self.step = 0

    def run(self, nsteps):
        hits = []
        while len(hits) < nsteps:
            if self.cursor + RAYS_PER_CALL > self.o.shape[0]:
                self.cursor = 0
            s = slice(self.cursor, self.cursor + RAYS_PER_CALL)
            self.nerf.set_learning_rate(cosine_lr(self.step))
            n, h = self.nerf.train(self.o[s], self.d[s], self.gt[s], RAYS_PER_CALL, stream=self.stream)
            self.cursor += RAYS_PER_CALL
            self.step += n
            hits.extend(h)
        return hits


def cpu_baseline(P, nerf, o, d, gt):
    """The C oracle on the host: one full training step on a bounded ray sample."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as orc
    bits = nerf.occupancy()
    mn, mx = np.float32([-1.5] * 3), np.float32([1.5] * 3)
    R = 1 << 14
    oo, dd, gg = o[:R].cpu().numpy(), d[:R].cpu().numpy(), gt[:R].cpu().numpy()
    dW = np.zeros(64 * 32 + 16 * 64, np.float32)
    dB = np.zeros(80, np.float32)
    nerf.density.save_weights(dW, dB)
    table = np.zeros(L * TBL * F, np.float32)
    nerf.density.save_hashgrid(table)
    cW = np.zeros(64 * 32 + 64 * 64 + 8 * 64, np.float32)
    cB = np.zeros(136, np.float32)
    nerf.color.save_weights(cW, cB)
    t16 = table.astype(np.float16)
    t0 = time.perf_counter()
    di, nr, fr = orc.ray_aabb_inv(oo, dd, mn, mx, 5)
    m = orc.march_hits(oo, dd, di, nr, fr, bits, [128] * 3, mn, mx, 5, 4, 1, 1 << 16)
    N = m["total"]
    enc = orc.hash_encode(m["pos"], t16, TBL, L, BASE, GROWTH)
    dout, dacts = orc.mlp_forward(enc, dW.astype(np.float16), dB, 32, 64, 16, 2)
    cin, sig = orc.sh_gather(dd, m["ray_idx"], dout, 0.0)
    cout, cacts = orc.mlp_forward(cin, cW.astype(np.float16), cB, 32, 64, 8, 3, out_act=1)
    rgb = np.ascontiguousarray(cout[:, :3])
    act = m["active"]
    comp = orc.composite(m["offsets"][:act], m["counts"][:act], m["t"], sig, rgb, gg[:act], 0.1,
                         np.float32([1, 1, 1]))
    cg, ds = orc.color_grad(m["counts"][:act], m["offsets"][:act], m["t"], dout, rgb, comp["phi"], comp["rgb"],
                            comp["dw"], comp["weight_sum"], 128.0, 0.0, R)
    cgp = np.zeros((N, 8), np.float16)
    cgp[:, :3] = cg
    gW, gB, cdx = orc.mlp_backward(cgp, cin, cacts, cW.astype(np.float16), 32, 64, 8, 3)
    dg = orc.density_grad(ds, cdx)
    hW, hB, denc = orc.mlp_backward(dg, enc, dacts, dW.astype(np.float16), 32, 64, 16, 2)
    grads = orc.hash_scatter(m["pos"], denc, TBL, L, BASE, GROWTH)
    bc1, bc2 = orc.adam_bias_corrections(0.9, 0.999, 1)
    z = np.zeros_like(table)
    orc.adam_hash(table, grads, z, z.copy(), 1e-2, 0.9, 0.999, 1e-8, bc1, bc2, 1 / 128.0)
    for w, g in ((dW, hW), (dB, hB), (cW, gW), (cB, gB)):
        orc.adam_dense(w, g, np.zeros_like(w), np.zeros_like(w), 1e-2, 0.9, 0.999, 1e-8, bc1, bc2, 1 / 128.0)
    dt = time.perf_counter() - t0
    return {"value": round(N / dt, 1), "unit": "samples/s", "cores": orc.num_threads(), "kind": "port",
            "sample": f"one full training step (march, encode, both MLPs fwd/bwd, compositing, gradients, scatter, "
                      f"Adam over all 16.8 M table entries) on {R} rays = {N} compacted samples of the same scene "
                      f"and model state, {dt:.2f} s"}


def components(P, torch, stream, sp):
    """Stand-alone launches at BASELINE configs[1]/[2] shapes: encode, scatter, hash Adam (HIP events)."""
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(7)
    pos = np.zeros((BATCH, 4), np.float32)
    pos[:, :3] = rng.random((BATCH, 3), dtype=np.float32)
    table = rng.uniform(-1e-4, 1e-4, L * TBL * F).astype(np.float16)
    opt = P.MLPGridOptions(vectorDim=4, hiddenDim=64, outputDim=16, numLayers=2, activationType=0, tableSize=TBL,
                           numLevels=L, b=(2048 / 16) ** (1 / 15), lowestSize=BASE, featuresLevel=F)
    d_pos = torch.from_numpy(pos).to(dev)
    d_tab = torch.from_numpy(table).to(dev)
    d_enc = torch.empty((BATCH, 2 * L), dtype=torch.float16, device=dev)
    d_denc = torch.from_numpy(rng.normal(0, 1, (BATCH, 2 * L)).astype(np.float16)).to(dev)
    d_grads = torch.zeros(L * TBL * F, dtype=torch.float32, device=dev)
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731

    def timed(fn, reps=20):
        fn()
        a, b = ev(), ev()
        a.record(stream)
        for _ in range(reps):
            fn()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps

    t_enc = timed(lambda: P.launch("launchHashEncodeKernel", C.byref(opt), d_tab, d_pos, 4, d_enc, BATCH, sp))
    t_sc = timed(lambda: P.launch("launchHashTableBackwardKernel", d_denc, d_pos, d_grads, BATCH, TBL, L,
                                  opt.b, BASE, F, sp))
    return {"hash_encode_ms_2p18": round(t_enc, 4), "hash_encodes_per_s": round(BATCH / (t_enc * 1e-3), 1),
            "hash_encode_gbs": round(ENC_BYTES_PER_SAMPLE * BATCH / (t_enc * 1e-3) / 1e9, 1),
            "hash_scatter_ms_2p18": round(t_sc, 4),
            "hash_scatter_gbs": round(SCATTER_BYTES_PER_SAMPLE * BATCH / (t_sc * 1e-3) / 1e9, 1)}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU: multi-GPU sharding is a design only (DESIGN.md); "
                                   "run with --gpus 1"}))
        sys.exit(2)
    import torch
    P = importlib.import_module("3dmaker_amd")
    scenes = importlib.import_module("3dmaker_amd.scenes")
    assert torch.cuda.is_available(), "bench.py needs cuda:0"
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    if args.components:
        print(json.dumps({"components": components(P, torch, stream, sp)}))
        return

    o_np, d_np = scenes.rays_c4(POOL, n_cams=100, seed=2024)
    scene = scenes.SphereScene(seed=5)
    d_o = torch.from_numpy(o_np).to(dev)
    d_d = torch.from_numpy(d_np).to(dev)
    d_gt = scene.render_device(d_o, d_d, steps=1024).contiguous()
    torch.cuda.synchronize()

    nerf = P.Nerf(options(P))
    tr = Trainer(nerf, d_o, d_d, d_gt, sp)
    tr.run(args.warmup)
    torch.cuda.synchronize()
    if args.profile_steps:
        hits = tr.run(args.profile_steps)
        torch.cuda.synchronize()
        # Copy calibration for HBM counters: an elementwise kernel reading and
        # writing exactly COPY_BYTES each (torch's neg), three launches.
        src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        print(json.dumps({"profile_steps": len(hits), "mean_samples": float(np.mean(hits)),
                          "copy_calibration_bytes": COPY_BYTES}))
        return

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    hits = tr.run(args.steps)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    steps = len(hits)
    samples = int(np.sum(hits, dtype=np.int64))
    ms_step = wall * 1e3 / steps

    # Per-stage HIP-event timings on the launch stream over a further profiled window.
    nerf.set_profiling(True)
    nerf.reset_stats()
    prof_hits = tr.run(64)
    torch.cuda.synchronize()
    nerf.set_profiling(False)
    st = nerf.stats()
    n_prof = float(np.mean(prof_hits))
    stage_ms = {k: round(v[0], 4) for k, v in st.items()}
    # per training step: mean per call x calls / steps (march and occupancy run less than once a step)
    stage_ms_per_step = {k: round(v[0] * v[1] / len(prof_hits), 4) for k, v in st.items()}

    # roofline of the dominant kernel of the step (per-call averages of the profiled window)
    candidates = {
        "hashScatter": ("hbm", SCATTER_BYTES_PER_SAMPLE * n_prof),
        "densityFwd": ("hbm", ENC_BYTES_PER_SAMPLE * n_prof),
        "densityOpt": ("hbm", ADAM_BYTES_PER_PARAM * (L * TBL * F)),
    }
    dom = max((k for k in candidates if k in st), key=lambda k: st[k][0])
    bound, algo = candidates[dom]
    dom_ms = st[dom][0]
    ach = algo / (dom_ms * 1e-3) / 1e9
    roofline = {"bound": bound, "kernel": dom, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": measured_traffic(dom),
                "algorithmic_bytes_per_launch": int(algo), "avg_launch_ms": round(dom_ms, 4)}
    mlp_ms = sum(st[k][0] for k in ("densityFwd", "colorFwd", "colorBwd", "densityBwd") if k in st)
    mfma_util = MLP_FLOP_PER_SAMPLE * n_prof / (mlp_ms * 1e-3) / 1e12 / FP16_PEAK_TFLOPS if mlp_ms else None

    out = {
        "metric": "training samples/sec (full NeRF training step, <= 2^18 compacted samples/step)",
        "value": round(samples / wall, 1),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": "InstantNerf.trainWithRaysHit on the procedural 3-sphere scene (BASELINE configs[4])",
                   "batch_samples": BATCH, "rays_per_call": RAYS_PER_CALL, "mean_samples_per_step": round(samples / steps, 1),
                   "grid": "128^3 x 5 cascades x 4 mips", "table_size": TBL, "levels": L, "density": "32-64-16",
                   "color": "32-64-64-3", "lambda_dist": 0.1, "loss_scale": 128.0, "occupancy_refresh": 16},
        "stage_ms": stage_ms,
        "stage_ms_per_step": stage_ms_per_step,
        "hash_encodes_per_s": round(n_prof / (st["densityFwd"][0] * 1e-3), 1) if "densityFwd" in st else None,
        "mfma_util": round(mfma_util, 5) if mfma_util else None,
        "roofline": roofline,
    }
    out["components"] = components(P, torch, stream, sp)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(P, nerf, d_o, d_d, d_gt)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
