"""100 chained steps of the training step's fused table update against the oracle.

The step applies the hash table's Adam update (optimizerKernel.cu:116-167) inside the binned scatter of
hashTableScatter_Backward (networkFusionBackwardHashtable.cu:783-910): TinyMLPHashGrid::scatterAdamTable.
Here it runs 100 times in a row at BASELINE configs[1]'s table (T = 2^19, 16 levels, fp16 copy of a
seeded U(+-1e-4) table) with 2^18 fresh seeded samples per step, and the oracle runs the reference's
order -- the scatter summed in fp64, then Adam over the whole table -- from the same initial state on the
same inputs.  Upstream gradients are N(0, 1) scaled per sample by 10^U(-4, 0), so each level's sums span
many decades (the regime of a training step, where the fixed-point quantum is set by the level's largest
gradient).

Bar (north star): Adam parameters within 1e-6 rel (1e-7 abs) after 100 steps, on every entry that some
step touched with a well-conditioned gradient (|g_ref| above 4x the per-word bound of the binned sum
against the oracle's, tests/helpers.scatter_bound); the entries whose gradient was ill-conditioned at some
step (products cancelling to within a few fp32 roundings of their magnitudes) stay below 0.1 % of the
touched ones; entries no step touched keep every bit.  The Adam step count is the reference's (bias
corrections of step k at step k).
"""
import numpy as np
import pytest

import pyoracle as orc
from helpers import assert_close, d2h, make_mlp, pkg, scatter_bound, scatter_quantum

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

LR, B1, B2, EPS, SCALE = 1e-2, 0.9, 0.99, 1e-15, 128.0   # BASELINE configs[0] Adam


@pytest.mark.timeout(900)
def test_fused_table_update_100_steps_matches_oracle():
    assert torch.cuda.is_available(), "GPU tests need cuda:0"
    P = pkg()
    T_, L, b, N, steps = 1 << 19, 16, (2048 / 16) ** (1 / 15), 1 << 18, 100
    n = L * T_ * 2
    opt = P.MLPGridOptions(vectorDim=4, hiddenDim=64, outputDim=16, numLayers=2, activationType=0, tableSize=T_,
                           numLevels=L, b=b, lowestSize=16, featuresLevel=2)
    grid = P.HashGrid(opt, N, seed=11)
    table0 = np.random.default_rng(11).uniform(-1e-4, 1e-4, n).astype(np.float32)
    grid.load_hashgrid(table0)
    W, B = make_mlp(2 * L, 64, 16, 2, seed=12)
    grid.load_weights(W, B)
    bf = grid.buffers()
    w0 = d2h(bf.master_hashtable, (n,), np.float32)
    m0 = d2h(bf.hash_m, (n,), np.float32)
    v0 = d2h(bf.hash_v, (n,), np.float32)
    h0 = d2h(bf.fwd_hashtable, (n,), np.float16)
    w, m, v = w0.copy(), m0.copy(), v0.copy()
    touched_any = np.zeros(n, bool)
    ill_any = np.zeros(n, bool)
    for step in range(steps):
        rng = np.random.default_rng(1000 + step)
        pos = np.zeros((N, 4), np.float32)
        pos[:, :3] = rng.random((N, 3), dtype=np.float32)
        dx = rng.standard_normal((N, 2 * L), dtype=np.float32)
        dx *= (10.0 ** rng.uniform(-4, 0, (N, 1))).astype(np.float32)
        dx = dx.astype(np.float16)
        dx[rng.random(N) < 0.2] = 0   # samples past a ray's saturated transmittance: no gradient
        d_pos = torch.from_numpy(pos).cuda()
        d_dx = torch.from_numpy(dx).cuda()
        grid.scatter_adam_table(d_dx, d_pos, N, 4, LR, B1, B2, EPS, SCALE)
        grid.step_mlp(LR, B1, B2, EPS, SCALE)
        # the oracle's step (runs while the GPU's is in flight)
        g, gabs, cnt = orc.hash_scatter_stats(pos, dx, T_, L, 16, b)
        touched = gabs != 0
        touched_any |= touched
        ill_any |= touched & (np.abs(g) <= 4.0 * scatter_bound(g, gabs, cnt, scatter_quantum(dx, L, T_)))
        bc1, bc2 = orc.adam_bias_corrections(B1, B2, step + 1)
        orc.adam_hash(w, g, m, v, LR, B1, B2, EPS, bc1, bc2, 1.0 / SCALE, want_f16=False)
        if step % 10 == 9:
            torch.cuda.synchronize()
            print(f"[table adam chain] step {step + 1}: {int(touched.sum())} words touched, "
                  f"{int(ill_any.sum())} ill-conditioned so far", flush=True)
    torch.cuda.synchronize()
    assert grid.buffers().step == steps
    wg = d2h(bf.master_hashtable, (n,), np.float32)
    mg = d2h(bf.hash_m, (n,), np.float32)
    vg = d2h(bf.hash_v, (n,), np.float32)
    hg = d2h(bf.fwd_hashtable, (n,), np.float16)
    grid.close()
    # no step touched them: every word as loaded
    un = ~touched_any
    assert un.any()
    for got, ref, what in ((wg, w0, "w"), (mg, m0, "m"), (vg, v0, "v"), (hg, h0, "fp16 copy")):
        bad = np.nonzero(got[un].view(np.uint32 if got.dtype == np.float32 else np.uint16)
                         != ref[un].view(np.uint32 if ref.dtype == np.float32 else np.uint16))[0]
        assert bad.size == 0, f"{bad.size} untouched {what} words changed"
    n_touched = int(touched_any.sum())
    n_ill = int(ill_any.sum())
    print(f"[table adam chain] {n_touched} words touched over {steps} steps, {n_ill} ill-conditioned", flush=True)
    assert n_ill <= 1e-3 * n_touched, f"{n_ill} of {n_touched} touched words ill-conditioned at some step"
    well = touched_any & ~ill_any
    assert_close(wg[well], w[well], atol=1e-7, rtol=1e-6, what=f"table after {steps} fused steps")
    assert_close(mg[well], m[well], atol=1e-7 * float(np.abs(m).max()), rtol=1e-5, what="Adam m")
    assert_close(vg[well], v[well], atol=1e-7 * float(np.abs(v).max()), rtol=1e-5, what="Adam v")
    # the fp16 forward copy is the rounding of the fp32 master wherever a step wrote it
    np.testing.assert_array_equal(hg[touched_any].view(np.uint16),
                                  wg[touched_any].astype(np.float16).view(np.uint16))
