#!/usr/bin/env python3
"""Benchmark: the full NeRF training step of 3DMaker on one MI355X.

Workload (the end-to-end configuration; the reference's
step is InstantNerf::trainWithRaysHit, modules/NeRF/InstantNerf.cu:359-583,
driven by INerfTrainer::trainOneChunk, NerfTrainer.cu:137-179):
  procedural scene (3 seeded spheres, sigma_max * sigmoid(-sdf / 0.01), 3-band
  sinusoidal colour) rendered by fixed-step quadrature into 100 RGBA8 views of
  800x800 (fov 50 deg, cameras on a radius-1.5 sphere), resident in HBM; the
  ray feed (launchFetchRayChunk, DataLoader.cu:548-661) draws 2^16 rays per
  trainWithRaysHit call with pcg_hash and composites them over a random
  background colour per call, as the reference trainer does; occupancy
  128^3 x 1 cascade x 4 mips (the reference loader's choice for an orbit),
  AABB +-1.5, K = 1; hash grid L = 16, F = 2,
  T = 2^19, base 16, b = 1.3819; density 32 -> 64 -> 16, colour
  32 -> 64 -> 64 -> 3 (sigmoid); distortion loss lambda = 0.1; loss scale 128;
  Adam (0.9, 0.999, 1e-8); cosine LR 1e-2 -> 1e-4 over 2000 steps; occupancy
  refreshed every 16 steps (one jittered sample per cell for the first 256
  steps, then half the cells' worth of occupied/uniform samples).
One step = one optimizer step on one hit batch of at most 2^18 compacted
samples: ray setup, DDA march (once per ray window and grid version),
compaction, fused hash encode + density MLP forward, SH gather, colour MLP
forward, compositing with distortion, colour/density gradients, both MLP
backwards, hash scatter, Adam over all parameters (16.8 M table entries),
plus the amortised ray fetch and occupancy refresh.

After the timed steps the run continues (untimed) to the end of the 2000-step
cosine schedule and reports PSNR on 12 held-out 800x800 views (their own
camera lattice), rendered with renderImageHit over sequential feed chunks.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--profile-steps N] [--psnr-steps S]

Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import contextlib
import ctypes as C
import gc
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
N_VIEWS, N_HELDOUT, IMG_W, IMG_H, FOV_X = 100, 12, 800, 800, 50.0
L, F, TBL, BASE, GROWTH = 16, 2, 1 << 19, 16, 1.3819
LR_MAX, LR_MIN, ANNEAL = 1e-2, 1e-4, 2000
C5_SEEDS = (1, 2, 3, 4, 5)    # further background-draw seeds of the 5-cascade run
PRETRAIN_STEPS = 256           # optimizer steps before the warm-up (past the early occupancy phase)
# The per-stage HIP-event window (the roofline's kernel times) and a steady-state window of whole refresh
# periods, run after the timed steps: fixed so that the committed kernel trace covers the same steps
# (rocprofv3 ... bench.py --warmup 384 --profile-steps 64: steps 640 .. 703).
PROFILE_FROM, PROFILE_STEPS, STEADY_STEPS = 640, 64, 64
CPU_FEED_CHUNKS = 8            # feed chunks of rays available to the CPU-oracle leg (stops after ~10 s)

# Algorithmic counts per unit.
ENC_BYTES_PER_SAMPLE = 16 + L * 8 * 4 + 2 * L * 2                    # 592
SCATTER_BYTES_PER_SAMPLE = 16 + 2 * L * 2 + L * 8 * 2 * 8               # 2,128 (pos 16 + denc 64 + RMW 2,048)
ADAM_BYTES_PER_PARAM = 34
MLP_FLOP_PER_SAMPLE = 3 * (2 * (32 * 64 + 64 * 16) + 2 * (32 * 64 + 64 * 64 + 64 * 3))  # 56,448 fwd + bwd
# the same minus the colour head's dL/d(SH features), which nothing consumes: 54,400
HEADS_FLOP_PER_SAMPLE = MLP_FLOP_PER_SAMPLE - 2 * 16 * 64
COPY_BYTES = 256 << 20         # copy-calibration kernel of the PMC runs (read and write each)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")
MFMA_FILE = os.path.join(ROOT, "profiles", "mfma_counters.json")
L2_FILE = os.path.join(ROOT, "profiles", "encode_l2_requests.json")


def profile_json(path):
    """A committed counter summary (profiles/*.json), or None."""
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC summary, or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        return t["kernels"][kernel]["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def d2h(ptr, shape, dtype):
    """Copy a device buffer (raw pointer) into a new numpy array."""
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    hip.hipMemcpy.restype = C.c_int
    out = np.empty(shape, dtype)
    if out.nbytes and hip.hipMemcpy(out.ctypes.data, int(ptr), out.nbytes, 2) != 0:
        raise RuntimeError("hipMemcpy device-to-host failed")
    return out


def encode_line_requests(pos, b):
    """64-byte-line requests of the stand-alone encode's corner gathers for points pos [N x >=3] that reach
    the L2: lanes of a wave hold 64 consecutive samples; per level the two x-neighbour corners of each (y, z)
    corner pair are loaded back to back and share their line when they fall in one (the L1 merges them), so
    a request is one distinct line among a wave's 128 addresses of one (level, y/z pair) (forward clamp x0 in
    [0, N_l])."""
    n = pos.shape[0]
    m = (n + 63) // 64 * 64
    p = np.zeros((m, 3), np.float32)
    p[:n] = pos[:, :3]
    valid = (np.arange(m) < n).reshape(-1, 64)
    inner = (np.float32(TBL) ** (1.0 / 3.0) - 1.0) / BASE
    dense_start = max(0, min(int(math.floor(math.log2(inner) / math.log2(b))) + 1, L))
    total = 0
    for lvl in range(L):
        s = np.float32(BASE * b ** lvl)
        res = int(math.floor(s))
        x0 = np.clip(np.floor(p * s).astype(np.int64), 0, res)
        x1 = np.minimum(x0 + 1, res)
        for q in range(4):
            cy = x1[:, 1] if q & 1 else x0[:, 1]
            cz = x1[:, 2] if q & 2 else x0[:, 2]
            lines = []
            for cx in (x0[:, 0], x1[:, 0]):
                if lvl < dense_start:
                    e = cx + cy * (res + 1) + cz * (res + 1) ** 2
                else:
                    e = ((cx.astype(np.uint32) ^ (cy.astype(np.uint32) * np.uint32(2654435761))
                          ^ (cz.astype(np.uint32) * np.uint32(805459861))) & np.uint32(TBL - 1)).astype(np.int64)
                lines.append(np.where(valid, ((lvl * TBL + e) * 4 // 64).reshape(-1, 64), -1))  # 4 B per entry
            line = np.sort(np.concatenate(lines, axis=1), axis=1)
            distinct = (np.diff(line, axis=1) != 0).sum(axis=1) + 1 - (line[:, 0] == -1)
            total += int(distinct.sum())
    return total


_PROBES = None


def probes():
    """bench_probes.so (built by __graft_entry__.build()): device-ceiling probes of this benchmark."""
    global _PROBES
    if _PROBES is None:
        path = os.path.join(ROOT, "bench_probes.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: run __graft_entry__.build() first")
        L_ = C.CDLL(path)
        L_.probe_last_error.restype = C.c_char_p
        L_.probe_stream_copy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.POINTER(C.c_double),
                                         C.c_void_p]
        L_.probe_random_lines.argtypes = [C.c_void_p, C.c_size_t, C.c_int, C.c_int, C.c_void_p, C.c_size_t,
                                          C.POINTER(C.c_double), C.c_void_p]
        L_.probe_atomic_lines.argtypes = [C.c_void_p, C.c_size_t, C.c_int, C.POINTER(C.c_double), C.c_void_p]
        _PROBES = L_
    return _PROBES


def probe(name, *args):
    r = C.c_double(0.0)
    if getattr(probes(), name)(*args[:-1], C.byref(r), args[-1]) != 0:
        raise RuntimeError(f"{name}: {probes().probe_last_error().decode()}")
    return r.value


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256, help="timed optimizer steps")
    ap.add_argument("--warmup", type=int, default=16,
                    help="untimed optimizer steps after the 256 pre-training steps")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-oracle baseline leg")
    ap.add_argument("--profile-steps", type=int, default=0,
                    help="run --warmup steps, then this many, and exit (for rocprofv3)")
    ap.add_argument("--psnr-steps", type=int, default=ANNEAL,
                    help="train (untimed) up to this many steps, then report PSNR on 12 held-out views (-1: skip)")
    ap.add_argument("--cascades", type=int, default=1,
                    help="occupancy cascades of the end-to-end run (1: the reference loader's choice for an orbit)")
    ap.add_argument("--components", action="store_true",
                    help="only time the stand-alone encode / scatter launches at 2^18 and exit")
    return ap.parse_args()


def options(P, cascades=1):
    o = P.Nerf.default_options()
    o.gridResolution[:] = [128, 128, 128]
    o.aabbMin[:] = [-1.5] * 3
    o.aabbMax[:] = [1.5] * 3
    # One cascade: INerfTrainer takes the loader's estimate (NerfTrainer.cu:113-114), and the loader's pose
    # heuristic gives 1 for cameras orbiting the scene, as here (DataLoader.cu:368-376).  With 5 cascades
    # the far field holds a fog shell whose colour follows the random background of the last ray chunk.
    o.levelsMipmap, o.numCascades, o.samplesPerVoxel = 4, cascades, 1
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


@contextlib.contextmanager
def timed_region():
    """Timed steps with no cyclic-garbage collection inside them.  A full collection walks every object the
    process tracks (torch's among them: about 0.05-0.07 s) and stalls the host, and with it the GPU, which
    runs at most a step ahead of the host: one inside a 20-step window would be most of its time.  The
    collector runs before the window instead, and the setup's objects are frozen out of later collections
    (gc.freeze in main)."""
    gc.collect()
    gc.disable()
    try:
        yield
    finally:
        gc.enable()


def cosine_lr(step):
    p = min(step / ANNEAL, 1.0)
    return LR_MIN + 0.5 * (LR_MAX - LR_MIN) * (1.0 + math.cos(math.pi * p))


class RayFeed:
    """Device-resident RGBA8 views + launchFetchRayChunk (DataLoader.cu:548-679), into one of two chunk
    slots (the trainer fills the next chunk's slot while the current one trains); o, d, rgb, dense and
    sigma name the current slot."""

    def __init__(self, P, torch, imgs, transforms, width, height, focal, chunk):
        dev = imgs.device
        self.P, self.imgs, self.w, self.h, self.focal, self.chunk = P, imgs, width, height, focal, chunk
        self.T = torch.from_numpy(transforms).to(dev)
        self.total = int(imgs.shape[0]) * width * height
        self.slots = [{k: torch.empty((chunk, 3) if k in ("o", "d", "rgb") else chunk, device=dev)
                       for k in ("o", "d", "rgb", "dense", "sigma")} for _ in range(2)]
        self.slot = 0

    def __getattr__(self, k):
        if k in ("o", "d", "rgb", "dense", "sigma"):
            return self.slots[self.slot][k]
        raise AttributeError(k)

    def fetch(self, offset, size, seed, bg, stream, sequential=False, slot=None):
        b = self.slots[self.slot if slot is None else slot]
        self.P.lib().launchFetchRayChunk(int(offset), int(size), self.total, int(seed) & 0xffffffff,
                                         0 if sequential else 1, self.w, self.h, float(self.focal),
                                         self.T.data_ptr(), self.imgs.data_ptr(), b["o"].data_ptr(),
                                         b["d"].data_ptr(), b["rgb"].data_ptr(), b["dense"].data_ptr(),
                                         b["sigma"].data_ptr(), None, None, None, None, None, 0, 0.0, 1.0, 1.0,
                                         self.P.Float3(*map(float, bg)), 0, stream)


class Trainer:
    """INerfTrainer::trainOneChunk (NerfTrainer.cu:137-179): per 2^16-ray chunk drawn by the ray feed with
    the epoch's seed, a random background colour (the reference's random-bg augmentation) and the cosine
    LR of the chunk's first step, trainWithRaysHit.

    run(n) trains exactly n optimizer steps: each call is limited to the steps still to go
    (InstantNerf::setStepLimit), and a chunk cut short by the limit is continued, same background and
    LR, by the next call from its first untrained ray.  The next chunk is drawn (same draw order: epoch
    seed at cursor 0, then the background) and fetched into the other feed slot before the current one
    trains, and handed to setNextRays, so that its first hit batch is compacted beside the current
    chunk's last step."""

    def __init__(self, nerf, feed, stream, fixed_bg=None):
        self.nerf, self.feed, self.stream = nerf, feed, stream
        self.rng = np.random.default_rng(42)
        self.cursor = 0      # first ray of the next chunk to draw
        self.step = 0
        self.calls = 0
        self.epoch_seed = 0
        self.fixed_bg = fixed_bg
        self.cur = None      # [offset, size, bg, slot, rays trained, lr] of the chunk in training
        self.ahead = None    # (offset, size, bg, slot) of the chunk fetched ahead

    def _draw_and_fetch(self, slot):
        f = self.feed
        if self.cursor >= f.total:
            self.cursor = 0
        if self.cursor == 0:
            self.epoch_seed = int(self.rng.integers(0, 1 << 32))
        size = min(RAYS_PER_CALL, f.total - self.cursor)
        bg = self.rng.random(3)
        if self.fixed_bg is not None:
            bg = np.asarray(self.fixed_bg, np.float64)
        f.fetch(self.cursor, size, self.epoch_seed, bg, self.stream, slot=slot)
        chunk = (self.cursor, size, bg, slot)
        self.cursor += size
        return chunk

    def run(self, nsteps):
        hits = []
        f = self.feed
        while len(hits) < nsteps:
            if self.cur is None:
                c = self.ahead if self.ahead is not None else self._draw_and_fetch(f.slot)
                self.ahead = self._draw_and_fetch(c[3] ^ 1)
                self.cur = [c[0], c[1], c[2], c[3], 0, cosine_lr(self.step)]
            _, size, bg, slot, done, lr = self.cur
            nb = f.slots[slot ^ 1]
            self.nerf.set_next_rays(nb["o"], nb["d"], self.ahead[1])
            f.slot = slot
            self.nerf.set_learning_rate(lr)
            self.nerf.set_bg_color(*map(float, bg))
            self.nerf.set_step_limit(nsteps - len(hits))
            b = f.slots[slot]
            # the chunk's buffers from its first untrained ray, as device addresses (no tensor views per call)
            at = lambda t, per: t.data_ptr() + done * per * t.element_size()  # noqa: E731
            n, h = self.nerf.train(at(b["o"], 3), at(b["d"], 3), at(b["rgb"], 3), size - done,
                                   rays_depth=at(b["dense"], 1), rays_sigma=at(b["sigma"], 1), stream=self.stream)
            self.calls += 1
            self.step += n
            hits.extend(h)
            self.cur[4] = done + self.nerf.last_rays_trained()
            if self.cur[4] >= size:
                self.cur = None
        self.nerf.set_step_limit(0)
        return hits


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(P, nerf, chunks, min_seconds=10.0, max_steps=64):
    """The C oracle on the host cores: full training steps of up to BATCH compacted
    samples each, chained (each step marches the next rays and trains the
    parameters the previous step updated), until min_seconds have passed.
    chunks: (o, d, rgb, background) per feed chunk, each composited over its own
    random background as the GPU run's feed draws them; a step's rays stay in
    one chunk and composite over its background."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as orc
    bounds = np.cumsum([0] + [c[0].shape[0] for c in chunks])
    o, d, gt = (np.concatenate([c[k] for c in chunks]) for k in range(3))
    bits = nerf.occupancy()
    casc = int(nerf.opts.numCascades)
    mn, mx = np.float32([-1.5] * 3), np.float32([1.5] * 3)
    window = 1 << 14  # rays marched per step; the batch fills from their front
    dW = np.zeros(64 * 32 + 16 * 64, np.float32)
    dB = np.zeros(80, np.float32)
    nerf.density.save_weights(dW, dB)
    table = np.zeros(L * TBL * F, np.float32)
    nerf.density.save_hashgrid(table)
    cW = np.zeros(64 * 32 + 64 * 64 + 8 * 64, np.float32)
    cB = np.zeros(136, np.float32)
    nerf.color.save_weights(cW, cB)
    t16 = table.astype(np.float16)
    mt, vt = np.zeros_like(table), np.zeros_like(table)
    state = [(w, np.zeros_like(w), np.zeros_like(w)) for w in (dW, dB, cW, cB)]
    ray0, steps, samples = 0, 0, 0
    t0 = time.perf_counter()
    while steps < max_steps and ray0 < len(o) and (steps == 0 or time.perf_counter() - t0 < min_seconds):
        ci = int(np.searchsorted(bounds, ray0, side="right")) - 1
        end = min(ray0 + window, int(bounds[ci + 1]))
        bg = np.asarray(chunks[ci][3], np.float32)
        oo, dd, gg = o[ray0:end], d[ray0:end], gt[ray0:end]
        di, nr, fr = orc.ray_aabb_inv(oo, dd, mn, mx, casc)
        m = orc.march_hits(oo, dd, di, nr, fr, bits, [128] * 3, mn, mx, casc, 4, 1, BATCH)
        N, act = m["total"], m["active"]
        dW16, cW16 = dW.astype(np.float16), cW.astype(np.float16)
        enc = orc.hash_encode(m["pos"], t16, TBL, L, BASE, GROWTH)
        dout, dacts = orc.mlp_forward(enc, dW16, dB, 32, 64, 16, 2)
        cin, sig = orc.sh_gather(dd, m["ray_idx"], dout, 0.0)
        cout, cacts = orc.mlp_forward(cin, cW16, cB, 32, 64, 8, 3, out_act=1)
        rgb = np.ascontiguousarray(cout[:, :3])
        comp = orc.composite(m["offsets"][:act], m["counts"][:act], m["t"], sig, rgb, gg[:act], 0.1, bg)
        cg, ds = orc.color_grad(m["counts"][:act], m["offsets"][:act], m["t"], dout, rgb, comp["phi"], comp["rgb"],
                                comp["dw"], comp["weight_sum"], 128.0, 0.0, RAYS_PER_CALL)
        cgp = np.zeros((N, 8), np.float16)
        cgp[:, :3] = cg
        gW, gB, cdx = orc.mlp_backward(cgp, cin, cacts, cW16, 32, 64, 8, 3)
        dg = orc.density_grad(ds, cdx)
        hW, hB, denc = orc.mlp_backward(dg, enc, dacts, dW16, 32, 64, 16, 2)
        grads = orc.hash_scatter(m["pos"], denc, TBL, L, BASE, GROWTH)
        bc1, bc2 = orc.adam_bias_corrections(0.9, 0.999, steps + 1)
        t16 = orc.adam_hash(table, grads, mt, vt, 1e-2, 0.9, 0.999, 1e-8, bc1, bc2, 1 / 128.0, w16_init=t16)
        for (w, mw, vw), g in zip(state, (hW, hB, gW, gB)):
            orc.adam_dense(w, g, mw, vw, 1e-2, 0.9, 0.999, 1e-8, bc1, bc2, 1 / 128.0)
        ray0 += act
        steps += 1
        samples += N
    dt = time.perf_counter() - t0
    return {"value": round(samples / dt, 1), "unit": "samples/s", "cores": orc.num_threads(), "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{steps} chained full training steps (march, encode, both MLPs fwd/bwd, compositing, "
                      f"gradients, scatter, Adam over all 16.8 M table entries) on {ray0} feed rays = "
                      f"{samples} compacted samples, same scene and model state as the GPU run, a random "
                      f"background per 2^16-ray chunk as the GPU run's feed, {dt:.1f} s"}


def cpu_components(gpu):
    """BASELINE configs[0]-[3] on the oracle, each at its full shape: median of 5 runs after 1 warm-up
    (time.perf_counter), beside the GPU's time of the same component from `gpu` (the components leg)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as orc
    scenes = importlib.import_module("3dmaker_amd.scenes")
    rng = np.random.default_rng(7)
    b1 = (2048 / 16) ** (1 / 15)

    def med(fn, reps=5):
        fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts)) * 1e3

    rows = {}
    # N = 4096, T = 2^14, b = 1.447: encode, density MLP forward, MSE, backward, scatter, Adam
    n0, t0_ = 4096, 1 << 14
    p0 = rng.random((n0, 3), dtype=np.float32)
    tab0 = rng.uniform(-1e-4, 1e-4, L * t0_ * F).astype(np.float32)
    w0 = np.concatenate([rng.uniform(-a, a, k) for a, k in ((math.sqrt(6 / 96), 64 * 32), (math.sqrt(6 / 80), 16 * 64))])
    w0 = w0.astype(np.float32)
    bias0 = np.zeros(80, np.float32)
    tgt0 = rng.random((n0, 16)).astype(np.float16)
    st0 = [np.zeros_like(tab0), np.zeros_like(tab0), np.zeros_like(w0), np.zeros_like(w0),
           np.zeros_like(bias0), np.zeros_like(bias0)]

    def c1_step():
        enc = orc.hash_encode(p0, tab0.astype(np.float16), t0_, L, BASE, 1.447)
        y, acts = orc.mlp_forward(enc, w0.astype(np.float16), bias0, 32, 64, 16, 2)
        _, dy = orc.mse_loss_grad(y, tgt0, 16, 128.0)
        gw, gb, dx = orc.mlp_backward(dy, enc, acts, w0.astype(np.float16), 32, 64, 16, 2)
        g = orc.hash_scatter(p0, dx, t0_, L, BASE, 1.447)
        bc1, bc2 = orc.adam_bias_corrections(0.9, 0.99, 1)
        orc.adam_hash(tab0, g, st0[0], st0[1], 1e-2, 0.9, 0.99, 1e-15, bc1, bc2, 1 / 128.0, want_f16=False)
        orc.adam_dense(w0, gw, st0[2], st0[3], 1e-2, 0.9, 0.99, 1e-15, bc1, bc2, 1 / 128.0)
        orc.adam_dense(bias0, gb, st0[4], st0[5], 1e-2, 0.9, 0.99, 1e-15, bc1, bc2, 1 / 128.0)

    rows["c1_train_step_4096_ms"] = med(c1_step)
    # encode and scatter at 2^18 and 2^20, T = 2^19
    tab = rng.uniform(-1e-4, 1e-4, L * TBL * F).astype(np.float16)
    for tag, n in (("2p18", 1 << 18), ("2p20", 1 << 20)):
        pos = rng.random((n, 3), dtype=np.float32)
        denc = rng.normal(0, 1, (n, 2 * L)).astype(np.float16)
        rows[f"c2_encode_{tag}_ms"] = med(lambda: orc.hash_encode(pos, tab, TBL, L, BASE, b1))
        rows[f"c2_scatter_{tag}_ms"] = med(lambda: orc.hash_scatter(pos, denc, TBL, L, BASE, b1))
    # both heads forward + backward at 2^18 (N(0,1) density inputs, SH of unit directions)
    n2 = BATCH
    x = rng.normal(0, 1, (n2, 32)).astype(np.float16)
    dirs = rng.normal(size=(n2, 3)).astype(np.float32)
    dirs /= np.linalg.norm(dirs, axis=1, keepdims=True)
    wd = (rng.normal(0, 0.1, 64 * 32 + 16 * 64)).astype(np.float16)
    bd = np.zeros(80, np.float32)
    wc = (rng.normal(0, 0.1, 64 * 32 + 64 * 64 + 8 * 64)).astype(np.float16)
    bc = np.zeros(136, np.float32)
    ridx = np.arange(n2, dtype=np.uint32)
    cdy = rng.normal(0, 1, (n2, 8)).astype(np.float16)
    cdy[:, 3:] = 0

    def heads():
        dout, dacts = orc.mlp_forward(x, wd, bd, 32, 64, 16, 2)
        cin, sig = orc.sh_gather(dirs, ridx, dout, 0.0)
        cout, cacts = orc.mlp_forward(cin, wc, bc, 32, 64, 8, 3, out_act=1)
        _, _, cdx = orc.mlp_backward(cdy, cin, cacts, wc, 32, 64, 8, 3)
        dg = orc.density_grad(np.zeros(n2, np.float32), cdx)
        orc.mlp_backward(dg, x, dacts, wd, 32, 64, 16, 2)

    rows["c3_heads_fwd_bwd_2p18_ms"] = med(heads)
    # DDA march + compaction of 2^18 camera rays over the 128^3 x 5 Bernoulli grid
    bits = scenes.occupancy_c4(128, 5, 4, 0.1, 0.3, 1.5, seed=0)
    o4, d4 = scenes.rays_c4(1 << 18, n_cams=100, seed=1)
    mn, mx = np.float32([-1.5] * 3), np.float32([1.5] * 3)

    def march():
        di, nr, fr = orc.ray_aabb_inv(o4, d4, mn, mx, 5)
        orc.march_hits(o4, d4, di, nr, fr, bits, [128] * 3, mn, mx, 5, 4, 1, BATCH)

    rows["c4_march_2p18_rays_ms"] = med(march)
    rows = {k: round(v, 2) for k, v in rows.items()}
    pairs = {"c2_encode_2p18_ms": "hash_encode_ms_2p18", "c2_encode_2p20_ms": "hash_encode_ms_2p20",
             "c2_scatter_2p18_ms": "hash_scatter_ms_2p18", "c3_heads_fwd_bwd_2p18_ms": "mlp_fwd_bwd_ms_2p18",
             "c4_march_2p18_rays_ms": "march_compact_ms_2p18_rays"}
    speedup = {k: round(rows[k] / gpu[g], 1) for k, g in pairs.items() if gpu.get(g)}
    return {"components_ms": rows, "component_timing": "median of 5 runs after 1 warm-up, oracle at full shape",
            "gpu_speedup": speedup}


def heldout_psnr(P, torch, nerf, feed, sp):
    """INerfTrainer::validate (NerfTrainer.cu:373-408): sequential ray chunks of
    the held-out views, GT composited over white, renderImageHit in INFERENCE
    mode, PSNR of the mean squared error over all pixels and channels."""
    nerf.set_bg_color(1.0, 1.0, 1.0)
    nerf.set_memory_mode(True)
    se, n, t_render = 0.0, 0, 0.0
    rgb = torch.empty((feed.chunk, 3), device=feed.o.device)
    for off in range(0, feed.total, feed.chunk):
        size = min(feed.chunk, feed.total - off)
        feed.fetch(off, size, 0, (1.0, 1.0, 1.0), sp, sequential=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        nerf.render(feed.o, feed.d, size, rgb, stream=sp)
        torch.cuda.synchronize()
        t_render += time.perf_counter() - t0
        se += float(((rgb[:size] - feed.rgb[:size]) ** 2).sum().item())
        n += 3 * size
    nerf.set_memory_mode(False)
    return {"value": round(-10.0 * math.log10(max(se / n, 1e-12)), 3), "views": int(feed.imgs.shape[0]),
            "resolution": f"{feed.w}x{feed.h}", "render_rays_per_s": round(feed.total / t_render, 1)}


def five_cascades(P, torch, feed, hfeed, sp):
    """The same run at 5 occupancy cascades (the configs[3] grid): step time, held-out PSNR, the PSNR of
    fresh training-view rays (training composite and renderImageHit), occupied cells per cascade; then the
    held-out PSNR of the same training at other seeds of the trainer's background draws.  The step math
    matches the oracle at 5 cascades (tests/test_gpu_c5.py); with random backgrounds the training is
    bistable: at some seeds the outer cascades fill with a fog that follows the backgrounds (held-out PSNR
    under 12 dB), at the others it converges as at one cascade."""
    scenes = importlib.import_module("3dmaker_amd.scenes")
    nerf = P.Nerf(options(P, 5))
    tr = Trainer(nerf, feed, sp)
    tr.run(PRETRAIN_STEPS)
    torch.cuda.synchronize()
    with timed_region():
        t0 = time.perf_counter()
        hits = tr.run(256)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    tr.run(ANNEAL - tr.step)
    torch.cuda.synchronize()
    out = {"ms_per_step": round(wall * 1e3 / len(hits), 4), "samples_per_s": round(float(np.sum(hits)) / wall, 1),
           "mean_samples_per_step": round(float(np.mean(hits)), 1), "after_steps": tr.step}
    out["psnr_heldout"] = heldout_psnr(P, torch, nerf, hfeed, sp)["value"]
    # fresh training-view rays over white: rgb of renderImageHit, then of a training step at LR 0
    n = 1 << 14
    feed.fetch(9 * RAYS_PER_CALL, n, 777, (1.0, 1.0, 1.0), sp, slot=0)
    b = feed.slots[0]
    nerf.set_bg_color(1.0, 1.0, 1.0)
    nerf.set_memory_mode(True)
    rgb_r = torch.zeros((n, 3), device=b["o"].device)
    nerf.render(b["o"][:n], b["d"][:n], n, rgb_r, stream=sp)
    torch.cuda.synchronize()
    nerf.set_memory_mode(False)
    nerf.set_learning_rate(0.0)
    rgb_t = torch.zeros((n, 3), device=b["o"].device)
    nerf.train(b["o"][:n], b["d"][:n], b["rgb"][:n], n, rgb_out=rgb_t, stream=sp)
    torch.cuda.synchronize()
    out["psnr_train_rays_step"] = round(-10 * math.log10(float(((rgb_t - b["rgb"][:n]) ** 2).mean()) + 1e-12), 3)
    out["psnr_train_rays_render"] = round(-10 * math.log10(float(((rgb_r - b["rgb"][:n]) ** 2).mean()) + 1e-12), 3)
    bits = np.unpackbits(nerf.occupancy(), bitorder="little")
    S, G = scenes.pyramid_cells(128, 4), 128 ** 3
    out["occupied_fraction_per_cascade"] = [round(float(bits[c * S: c * S + G].mean()), 4) for c in range(5)]
    nerf.close()
    # the trainer's background draws at other seeds (the run above: 42)
    seeds = {}
    for seed in C5_SEEDS:
        nerf = P.Nerf(options(P, 5))
        tr = Trainer(nerf, feed, sp)
        tr.rng = np.random.default_rng(seed)
        tr.run(ANNEAL)
        torch.cuda.synchronize()
        seeds[str(seed)] = heldout_psnr(P, torch, nerf, hfeed, sp)["value"]
        nerf.close()
    out["psnr_heldout_by_seed"] = seeds
    return out


def heads_components(P, torch, dev, rng, x, d_dirs, ridx, sp, timed):
    """The training step's heads (launchNerfHeads*: density 32-64-16 and colour 32-64-64-3 on the 16x16x32
    MFMA, hidden activations recomputed in the backward) at 2^18, on the same inputs as the TinyMLP leg:
    forward, dX chains, weight gradients, each alone and the three in sequence."""
    lib = P.lib()

    def layers(shape, seed):
        inD, hid, outD, nl = shape
        r = np.random.default_rng(seed)
        ws, bs = [], []
        for l in range(nl):
            o, i = (outD if l == nl - 1 else hid), (inD if l == 0 else hid)
            ws.append(torch.from_numpy(r.uniform(-1, 1, o * i).astype(np.float16) * np.float16(np.sqrt(6 / (o + i))))
                      .to(dev))
            bs.append(torch.zeros(o, device=dev))
        ptrs = lambda ts: torch.tensor([t.data_ptr() for t in ts], dtype=torch.int64, device=dev)  # noqa: E731
        gw = [torch.empty(t.numel(), device=dev) for t in ws]
        gb = [torch.empty(t.numel(), device=dev) for t in bs]
        return (ws, bs, gw, gb), ptrs(ws), ptrs(bs), ptrs(gw), ptrs(gb)

    dkeep, dW, dB, dgW, dgB = layers((32, 64, 16, 2), 1)
    ckeep, cW, cB, cgW, cgB = layers((32, 64, 8, 3), 2)
    packed = torch.empty(lib.nerfHeadsPackedBytes(), dtype=torch.uint8, device=dev)
    lib.launchNerfHeadsPack(dW.data_ptr(), dB.data_ptr(), cW.data_ptr(), cB.data_ptr(), packed.data_ptr(), sp)
    P.check()
    enc = x.view(BATCH, L, 2).transpose(0, 1).contiguous()  # [L][N][2]
    sig = torch.empty(BATCH, device=dev)
    dout = torch.empty((BATCH, 16), device=dev)
    cout = torch.empty((BATCH, 8), device=dev)
    cin = torch.empty((BATCH, 32), dtype=torch.float16, device=dev)
    cdy = torch.zeros((BATCH, 8), dtype=torch.float16, device=dev)
    cdy[:, :3] = torch.from_numpy(rng.normal(0, 0.1, (BATCH, 3)).astype(np.float16)).to(dev)
    ds = torch.from_numpy(rng.normal(0, 0.1, BATCH).astype(np.float32)).to(dev)
    denc = torch.empty((BATCH, 32), dtype=torch.float16, device=dev)
    ddy = torch.empty((BATCH, 16), dtype=torch.float16, device=dev)  # density dL/dy: dX kernel -> dW kernel
    live = torch.empty(BATCH // 16 + 1, dtype=torch.int32, device=dev)  # tiles with a nonzero gradient

    def fwd():
        lib.launchNerfHeadsForward(packed.data_ptr(), enc.data_ptr(), BATCH, L, d_dirs.data_ptr(), ridx.data_ptr(),
                                   BATCH, 0.0, 1, sig.data_ptr(), None, cout.data_ptr(), cin.data_ptr(), sp)

    def dx():
        lib.launchNerfHeadsBackward(packed.data_ptr(), enc.data_ptr(), BATCH, L, cin.data_ptr(), cdy.data_ptr(),
                                    ds.data_ptr(), BATCH, denc.data_ptr(), ddy.data_ptr(), None, live.data_ptr(), sp)

    def dw():
        lib.launchNerfHeadsWeightGrads(packed.data_ptr(), enc.data_ptr(), BATCH, L, cin.data_ptr(), cdy.data_ptr(),
                                       ds.data_ptr(), ddy.data_ptr(), live.data_ptr(), BATCH, dgW.data_ptr(), dgB.data_ptr(),
                                       cgW.data_ptr(), cgB.data_ptr(), sp)

    def step():
        lib.launchNerfHeadsPack(dW.data_ptr(), dB.data_ptr(), cW.data_ptr(), cB.data_ptr(), packed.data_ptr(), sp)
        fwd()
        dx()
        dw()

    t_f, t_x, t_w, t_all = timed(fwd), timed(dx), timed(dw), timed(step)
    P.check()
    fl_f = 2 * (32 * 64 + 64 * 16 + 32 * 64 + 64 * 64 + 64 * 3)          # 18,816
    fl_w = fl_f
    fl_x = HEADS_FLOP_PER_SAMPLE - fl_f - fl_w                           # 16,768
    util = lambda fl, ms: round(fl * BATCH / (ms * 1e-3) / 1e12 / FP16_PEAK_TFLOPS, 5)  # noqa: E731
    del dkeep, ckeep
    return {"mlp_fwd_bwd_ms_2p18": round(t_all, 4),
            "mlp_tflops": round(HEADS_FLOP_PER_SAMPLE * BATCH / (t_all * 1e-3) / 1e12, 2),
            "mlp_mfma_util": util(HEADS_FLOP_PER_SAMPLE, t_all),
            "heads_forward_ms_2p18": round(t_f, 4), "heads_forward_mfma_util": util(fl_f, t_f),
            "heads_dx_ms_2p18": round(t_x, 4), "heads_dx_mfma_util": util(fl_x, t_x),
            "heads_dw_ms_2p18": round(t_w, 4), "heads_dw_mfma_util": util(fl_w, t_w)}


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
    out = {"hash_encode_ms_2p18": round(t_enc, 4), "hash_encodes_per_s": round(BATCH / (t_enc * 1e-3), 1),
           "hash_encode_gbs": round(ENC_BYTES_PER_SAMPLE * BATCH / (t_enc * 1e-3) / 1e9, 1),
           "hash_scatter_ms_2p18": round(t_sc, 4),
           "hash_scatter_gbs": round(SCATTER_BYTES_PER_SAMPLE * BATCH / (t_sc * 1e-3) / 1e9, 1)}
    big = 1 << 20  # BASELINE configs[1] at 2^20
    pos20 = np.zeros((big, 4), np.float32)
    pos20[:, :3] = rng.random((big, 3), dtype=np.float32)
    d_pos20 = torch.from_numpy(pos20).to(dev)
    d_enc20 = torch.empty((big, 2 * L), dtype=torch.float16, device=dev)
    t_enc20 = timed(lambda: P.launch("launchHashEncodeKernel", C.byref(opt), d_tab, d_pos20, 4, d_enc20, big, sp))
    out.update({"hash_encode_ms_2p20": round(t_enc20, 4), "hash_encodes_per_s_2p20": round(big / (t_enc20 * 1e-3), 1)})
    # the encode against its own ceilings, measured in this run: the hand-written streaming copy (bytes)
    # and the rate of 4-byte loads from random 64-byte lines of a 32 MiB table (line requests)
    req18 = encode_line_requests(pos, opt.b)
    req20 = encode_line_requests(pos20, opt.b)
    sink = torch.empty(torch.cuda.get_device_properties(0).multi_processor_count * 16 * 256, dtype=torch.int32,
                       device=dev)
    gather = {}
    for part in (0, 1):
        gather[part] = probe("probe_random_lines", d_tab.data_ptr(), d_tab.numel() * 2, part, 256, sink.data_ptr(),
                             sink.numel() * 4, sp)
    copy_gbs = {}
    for tag, nbytes in (("1gib", 1 << 30), ("32mib", 32 << 20)):
        src = torch.ones(nbytes // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        copy_gbs[tag] = probe("probe_stream_copy", src.data_ptr(), dst.data_ptr(), nbytes, 10, sp) / 1e9
        del src, dst
    enc_gbs20 = ENC_BYTES_PER_SAMPLE * big / (t_enc20 * 1e-3) / 1e9
    out.update({
        "copy_gbs_1gib": round(copy_gbs["1gib"], 1), "copy_gbs_32mib": round(copy_gbs["32mib"], 1),
        "gather_lines_per_s_32mib": round(gather[0], 1), "gather_lines_per_s_32mib_per_xcd": round(gather[1], 1),
        "hash_encode_line_requests_per_sample": round(req18 / BATCH, 2),
        "hash_encode_lines_per_s_2p18": round(req18 / (t_enc * 1e-3), 1),
        "hash_encode_lines_per_s_2p20": round(req20 / (t_enc20 * 1e-3), 1),
        "hash_encode_frac_of_gather_ceiling_2p18": round(req18 / (t_enc * 1e-3) / gather[1], 4),
        "hash_encode_frac_of_gather_ceiling_2p20": round(req20 / (t_enc20 * 1e-3) / gather[1], 4),
        "hash_encode_frac_of_copy_2p20": round(enc_gbs20 / copy_gbs["1gib"], 4),
        "hash_encode_gbs_2p20": round(enc_gbs20, 1)})
    # the same fraction from L2 requests counted by rocprofv3 (TCP_TCC_READ_REQ_sum on these launches, committed
    # summary) instead of the line model: counted requests per sample x samples / this run's time / this run's
    # per-XCD random-line rate
    l2 = profile_json(L2_FILE)
    if l2:
        for tag, n, t in (("2p18", BATCH, t_enc), ("2p20", big, t_enc20)):
            rq = l2["encode"][tag]["l2_requests_per_sample"]
            out[f"hash_encode_l2_requests_per_sample_counted_{tag}"] = rq
            out[f"hash_encode_frac_of_gather_ceiling_counted_{tag}"] = round(rq * n / (t * 1e-3) / gather[1], 4)
    del d_pos20, d_enc20, sink

    # both heads forward + backward at 2^18 (density 32-64-16 on N(0,1) inputs, SH of
    # directions on the sphere, colour 32-64-64-3 sigmoid, L2 to U[0,1] targets), then Adam over both
    # heads and the dense T = 2^19 table gradient of the scatter above.
    dn = P.Net(P.MLPOption(inputDim=32, hiddenDim=64, outputDim=16, numLayers=2, activationType=0,
                           outputActivation=0), BATCH)
    cn = P.Net(P.MLPOption(inputDim=32, hiddenDim=64, outputDim=3, numLayers=3, activationType=0,
                           outputActivation=1), BATCH)
    x = torch.from_numpy(rng.normal(0, 1, (BATCH, 32)).astype(np.float16)).to(dev)
    dirs = rng.normal(size=(BATCH, 3)).astype(np.float32)
    dirs /= np.linalg.norm(dirs, axis=1, keepdims=True)
    d_dirs = torch.from_numpy(dirs).to(dev)
    ridx = torch.arange(BATCH, dtype=torch.int32, device=dev)
    tgt = torch.from_numpy(rng.random((BATCH, 3)).astype(np.float16)).to(dev)
    dout = torch.empty((BATCH, 16), device=dev)
    cin = torch.empty((BATCH, 32), dtype=torch.float16, device=dev)
    sig = torch.empty(BATCH, device=dev)
    cout = torch.empty((BATCH, 3), device=dev)
    cdx = torch.empty((BATCH, 32), dtype=torch.float16, device=dev)
    zero_ds = torch.zeros(BATCH, device=dev)
    dgrad = torch.empty((BATCH, 16), dtype=torch.float16, device=dev)

    def mlp_step():
        dn.zero_grad(sp)
        cn.zero_grad(sp)
        dn.forward(x, dout, BATCH, sp)
        P.launch("launchComputeSHGather", d_dirs, ridx, 0, BATCH, 0.0, dout, cin, sig, sp)
        cn.forward(cin, cout, BATCH, sp)
        cn.calculate_loss_and_grad(tgt, BATCH, 128.0, False, sp)
        cn.backward(BATCH, None, cdx, sp)
        P.launch("launchComputeDensityGrad", BATCH, zero_ds, cdx, dgrad, sp)
        dn.backward(BATCH, dgrad, None, sp)

    t_mlp = timed(mlp_step)
    flops = MLP_FLOP_PER_SAMPLE * BATCH
    out.update({"tinymlp_fwd_bwd_ms_2p18": round(t_mlp, 4),
                "tinymlp_tflops": round(flops / (t_mlp * 1e-3) / 1e12, 2),
                "tinymlp_mfma_util": round(flops / (t_mlp * 1e-3) / 1e12 / FP16_PEAK_TFLOPS, 5)})
    out.update(heads_components(P, torch, dev, rng, x, d_dirs, ridx, sp, timed))
    # Adam over both heads and the dense table gradient (a fresh copy per launch: consumed grads are cleared)
    n_tab = L * TBL * F
    master = torch.from_numpy(rng.uniform(-1e-4, 1e-4, n_tab).astype(np.float32)).to(dev)
    mm, vv = torch.zeros(n_tab, device=dev), torch.zeros(n_tab, device=dev)
    reps = 5
    gcopies = [d_grads.clone() for _ in range(reps + 1)]
    it = iter(range(reps + 1))

    def adam_all():
        k = next(it)
        P.launch("launchAdamHashGridOptim", C.byref(opt), master, d_tab, gcopies[k], mm, vv, 1e-2, 0.9, 0.99,
                 1e-15, 0.1, 0.01, 1.0 / 128.0, sp)
        dn.step(1e-2, 0.9, 0.99, 1e-15, 128.0, sp)
        cn.step(1e-2, 0.9, 0.99, 1e-15, 128.0, sp)

    touched = int((d_grads != 0).sum().item())
    t_adam = timed(adam_all, reps=reps)
    # 34 B per entry the scatter touched, 4 B (the gradient read) per entry it did not: Adam skips those
    adam_bytes = ADAM_BYTES_PER_PARAM * touched + 4 * (n_tab - touched)
    out.update({"adam_all_params_ms": round(t_adam, 4), "adam_touched_entries": touched,
                "adam_gbs": round(adam_bytes / (t_adam * 1e-3) / 1e9, 1)})
    del gcopies, master, mm, vv
    dn.close()
    cn.close()

    # DDA march + compaction of 2^18 camera rays over the C4 grid (processRaysHitLinear,
    # one host read per call), batch 2^18 samples
    scenes = importlib.import_module("3dmaker_amd.scenes")
    bits = scenes.occupancy_c4(128, 5, 4, 0.1, 0.3, 1.5, seed=0)
    o4, d4 = scenes.rays_c4(1 << 18, n_cams=100, seed=1)
    R4 = o4.shape[0]
    t_o, t_d = torch.from_numpy(o4).to(dev), torch.from_numpy(d4).to(dev)
    t_bits = torch.from_numpy(bits).to(dev)
    di = torch.empty((R4, 3), device=dev)
    nr, fr = torch.empty(R4, device=dev), torch.empty(R4, device=dev)
    cnt = torch.empty(R4, dtype=torch.int32, device=dev)
    offs = torch.empty(R4, dtype=torch.int32, device=dev)
    posb = torch.empty((BATCH, 4), device=dev)
    rib = torch.empty(BATCH, dtype=torch.int32, device=dev)
    tsb = torch.empty(BATCH, device=dev)
    act = torch.empty(1, dtype=torch.int32, device=dev)
    total = C.c_uint32(0)
    mn3, mx3 = P.Float3(-1.5, -1.5, -1.5), P.Float3(1.5, 1.5, 1.5)

    def march():
        P.launch("launchComputeRayAabbInv", R4, t_o, t_d, mn3, mx3, 5, di, nr, fr, sp)
        P.lib().processRaysHitLinear(R4, t_o.data_ptr(), t_d.data_ptr(), di.data_ptr(), nr.data_ptr(), fr.data_ptr(),
                                     t_bits.data_ptr(), P.Uint3(128, 128, 128), mn3, mx3, 5, 4, 1, BATCH,
                                     C.byref(total), act.data_ptr(), cnt.data_ptr(), offs.data_ptr(),
                                     posb.data_ptr(), rib.data_ptr(), tsb.data_ptr(), None, sp)
        P.check()

    t_march = timed(march)
    out.update({"march_compact_ms_2p18_rays": round(t_march, 4), "march_rays_per_s": round(R4 / (t_march * 1e-3), 1),
                "march_samples": int(total.value)})
    del t_o, t_d, t_bits, di, nr, fr, cnt, offs, posb, rib, tsb

    # fp16 dense MFMA peak recomputed on the box: CUs x clock x 4,096 flop/clock/CU (gfx950 dense fp16)
    hip = C.CDLL("libamdhip64.so")
    clk = C.c_int(0)
    if hip.hipDeviceGetAttribute(C.byref(clk), 5, 0) == 0 and clk.value > 0:  # 5 = hipDeviceAttributeClockRate (kHz)
        cus = torch.cuda.get_device_properties(0).multi_processor_count
        out["fp16_mfma_peak_tflops_from_clock"] = round(cus * clk.value * 1e3 * 4096 / 1e12, 1)
        out["cus"], out["clock_mhz"] = cus, round(clk.value / 1e3)
    return out


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

    scene = scenes.SphereScene(seed=5)
    focal = scenes.focal_from_fov(IMG_W, FOV_X)
    imgs, tf = scenes.render_views(scene, scenes.cameras(N_VIEWS, 1.5, seed=2024), IMG_W, IMG_H, FOV_X, dev)
    feed = RayFeed(P, torch, imgs, tf, IMG_W, IMG_H, focal, RAYS_PER_CALL)
    torch.cuda.synchronize()

    nerf = P.Nerf(options(P, args.cascades))
    tr = Trainer(nerf, feed, sp)
    gc.collect()
    gc.freeze()
    # the benchmark is quoted past the early occupancy phase (every cell sampled for steps < 256,
    # InstantNerf.cu:488-494), then --warmup untimed steps
    tr.run(PRETRAIN_STEPS)
    tr.run(args.warmup)
    torch.cuda.synchronize()
    if args.profile_steps:
        with timed_region():
            hits = tr.run(args.profile_steps)
            torch.cuda.synchronize()
        # Copy calibration for HBM counters: an elementwise kernel reading and
        # writing exactly COPY_BYTES each (torch's neg), three launches.
        src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        print(json.dumps({"profile_steps": len(hits), "total_steps": tr.step, "mean_samples": float(np.mean(hits)),
                          "copy_calibration_bytes": COPY_BYTES}))
        return

    torch.cuda.synchronize()
    timed_from, calls0 = tr.step, tr.calls
    with timed_region():
        t0 = time.perf_counter()
        hits = tr.run(args.steps)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    calls_timed = tr.calls - calls0
    steps = len(hits)
    samples = int(np.sum(hits, dtype=np.int64))
    ms_step = wall * 1e3 / steps

    # Untimed up to the fixed profiling window, then per-stage HIP-event timings on the launch stream over it
    # (the library waits for a refresh before the scatter stage while profiling, so the stage times its
    # kernels), then a steady-state window of whole refresh periods (timed, no events).
    start = max(PROFILE_FROM, -(-tr.step // 16) * 16)
    if tr.step < start:
        tr.run(start - tr.step)
    torch.cuda.synchronize()
    prof_from = tr.step
    nerf.set_profiling(True)
    nerf.reset_stats()
    with timed_region():
        prof_hits = tr.run(PROFILE_STEPS)
        torch.cuda.synchronize()
    nerf.set_profiling(False)
    st = nerf.stats()
    n_prof = float(np.mean(prof_hits))
    stage_ms = {k: round(v[0], 4) for k, v in st.items()}
    # per training step: mean per call x calls / steps (march and occupancy run less than once a step)
    stage_ms_per_step = {k: round(v[0] * v[1] / len(prof_hits), 4) for k, v in st.items()}
    steady_from = tr.step
    with timed_region():
        t1 = time.perf_counter()
        steady_hits = tr.run(STEADY_STEPS)
        torch.cuda.synchronize()
        steady_wall = time.perf_counter() - t1
    steady = {"window": [steady_from, steady_from + len(steady_hits)],
              "refreshes": sum(1 for k in range(steady_from, steady_from + len(steady_hits)) if k % 16 == 0),
              "ms_per_step": round(steady_wall * 1e3 / len(steady_hits), 4),
              "samples_per_s": round(float(np.sum(steady_hits)) / steady_wall, 1),
              "mean_samples_per_step": round(float(np.mean(steady_hits)), 1)}
    timed_refreshes = sum(1 for k in range(timed_from, timed_from + steps) if k % 16 == 0)

    # roofline of the dominant stage of the step (per-call averages of the profiled window, HIP events on
    # the stream each stage runs on)
    candidates = {
        "hashScatter": ("hbm", SCATTER_BYTES_PER_SAMPLE * n_prof),  # count, prefix, distribute, accumulate
        "encode": ("hbm", ENC_BYTES_PER_SAMPLE * n_prof),  # the step's hash encode (16x16x32 heads)
        "densityOpt": ("hbm", ADAM_BYTES_PER_PARAM * (L * TBL * F)),
    }
    if "encode" not in st:  # other head shapes: encode and heads in one stage
        candidates["forward"] = ("hbm", ENC_BYTES_PER_SAMPLE * n_prof)
    dom = max((k for k in candidates if k in st), key=lambda k: st[k][0])
    bound, algo = candidates[dom]
    dom_ms = st[dom][0]
    ach = algo / (dom_ms * 1e-3) / 1e9
    roofline = {"bound": bound, "kernel": dom, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": measured_traffic(dom),
                "algorithmic_bytes_per_launch": int(algo), "avg_launch_ms": round(dom_ms, 4),
                "window": [prof_from, prof_from + len(prof_hits)], "mean_samples": round(n_prof, 1)}
    # MLP stages: the heads' forward (the encode is a stage of its own with the 16x16x32 heads), the dX
    # chains (main stream) and the weight gradients (side stream, beside the scatter)
    mlp_ms = sum(st[k][0] for k in ("forward", "backwardDx", "colorDx", "densityDx", "colorBwd", "densityBwd",
                                    "headsBwd") if k in st)
    mfma_util = MLP_FLOP_PER_SAMPLE * n_prof / (mlp_ms * 1e-3) / 1e12 / FP16_PEAK_TFLOPS if mlp_ms else None
    mc = profile_json(MFMA_FILE)

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
                   "pretrain_steps": PRETRAIN_STEPS, "timed_window": [timed_from, timed_from + steps],
                   "calls_timed": calls_timed,
                   "grid": f"128^3 x {args.cascades} cascade(s) x 4 mips", "table_size": TBL, "levels": L, "density": "32-64-16",
                   "color": "32-64-64-3", "lambda_dist": 0.1, "loss_scale": 128.0, "occupancy_refresh": 16,
                   "feed": "100 RGBA8 800x800 views in HBM, pcg_hash draws, random background per call"},
        "stage_ms": stage_ms,
        "stage_ms_per_step": stage_ms_per_step,
        "forward_samples_per_s": round(n_prof / ((st["forward"][0] + st.get("encode", (0.0,))[0]) * 1e-3), 1)
        if "forward" in st else None,
        "mfma_util": round(mfma_util, 5) if mfma_util else None,
        # the heads kernels' MFMA flop by counter (SQ_INSTS_VALU_MFMA_MOPS_F16 x 512, every MFMA issued) over
        # their durations, from the committed counter passes: the step's window and the stand-alone 2^18 run
        "mfma_util_counters": {"step_heads": mc["step"]["mfma_util_all_heads"],
                               "standalone_heads_2p18": mc["components"]["mfma_util_heads"],
                               "source": mc["source"]} if mc else None,
        "timed_refreshes": timed_refreshes,
        "steady_state": steady,
        "roofline": roofline,
    }
    # finish the cosine schedule (untimed), then PSNR on 12 held-out views
    if args.psnr_steps > tr.step:
        tr.run(args.psnr_steps - tr.step)
        torch.cuda.synchronize()
    if args.psnr_steps >= 0:
        himgs, htf = scenes.render_views(scene, scenes.cameras(N_HELDOUT, 1.5, seed=4242), IMG_W, IMG_H, FOV_X, dev)
        hfeed = RayFeed(P, torch, himgs, htf, IMG_W, IMG_H, focal, RAYS_PER_CALL)
        out["psnr_heldout"] = dict(heldout_psnr(P, torch, nerf, hfeed, sp), after_steps=tr.step)
        out["cascades5"] = five_cascades(P, torch, feed, hfeed, sp)
        del hfeed, himgs
    out["components"] = components(P, torch, stream, sp)
    if not args.no_cpu:
        # the feed as the GPU run draws it: a random background per chunk, composited at fetch time
        crng = np.random.default_rng(12345)
        chunks = []
        for k in range(CPU_FEED_CHUNKS):
            bg = crng.random(3)
            feed.fetch(k * RAYS_PER_CALL, RAYS_PER_CALL, 12345, bg, sp)
            torch.cuda.synchronize()
            chunks.append((feed.o.cpu().numpy(), feed.d.cpu().numpy(), feed.rgb.cpu().numpy(), bg))
        out["cpu_baseline"] = cpu_baseline(P, nerf, chunks)
        out["cpu_baseline"].update(cpu_components(out["components"]))
    print(json.dumps(out))


if __name__ == "__main__":
    main()
