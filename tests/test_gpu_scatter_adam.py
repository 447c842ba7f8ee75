"""GPU parity of the training step's fused table update (TinyMLPHashGrid::scatterAdamTable).

The fused path applies the table's Adam update (optimizerKernel.cu:16-167) inside the binned scatter of
hashTableScatter_Backward (networkFusionBackwardHashtable.cu:783-910), without a gradient array.  Bar:
bit-exact against the stored path it replaces -- the scatter into the zero gradient array
(launchHashTableBackwardKernel) followed by the optimizer step (TinyMLPHashGrid::step) -- on every word of
the fp32 table, its fp16 copy and both moments, over several steps (moments and bias corrections carried),
for single- and multi-chunk bins, ragged batches, and non-finite upstream gradients; the gradient array is
never written.  The stored path itself is pinned against the oracle's Adam in test_gpu_tinymlp.py.
"""
import numpy as np
import pytest

from helpers import d2h, make_mlp, pkg, positions

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

LR, B1, B2, EPS, SCALE = 1e-2, 0.9, 0.99, 1e-15, 128.0


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need cuda:0"
    return torch.device("cuda:0")


def T(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def make_grid(T_, L, b, N, seed):
    P = pkg()
    opt = P.MLPGridOptions(vectorDim=4, hiddenDim=64, outputDim=16, numLayers=2, activationType=0, tableSize=T_,
                           numLevels=L, b=b, lowestSize=16, featuresLevel=2)
    g = P.HashGrid(opt, N, seed=seed)
    rng = np.random.default_rng(seed)
    g.load_hashgrid(rng.uniform(-1e-2, 1e-2, L * T_ * 2).astype(np.float32))
    W, B = make_mlp(2 * L, 64, 16, 2, seed=seed + 1, bias_scale=0.05)
    g.load_weights(W, B)
    return g


def state(g, n):
    bf = g.buffers()
    return {k: d2h(getattr(bf, k), (n,), np.float16 if k == "fwd_hashtable" else np.float32)
            for k in ("master_hashtable", "fwd_hashtable", "hash_m", "hash_v", "hashtable_grads")}


def bits(a):
    return a.view(np.uint16 if a.dtype == np.float16 else np.uint32)


@pytest.mark.parametrize("T_,L,b,N,steps,flags,skew", [(1 << 14, 16, 1.447, 1 << 16, 3, False, False),
                                                       (1 << 19, 16, 1.3819, 3001, 2, False, False),
                                                       (1 << 19, 16, 1.3819, 1 << 17, 2, False, False),
                                                       (1 << 12, 8, 2.0, 777, 2, False, False),
                                                       (1 << 19, 16, 1.3819, 1 << 17, 2, True, False),
                                                       (1 << 14, 16, 1.447, 3001, 2, True, False),
                                                       (1 << 14, 16, 1.447, 1 << 16, 2, False, True),
                                                       (1 << 19, 16, 1.3819, 1 << 17, 2, False, True)])
def test_fused_table_update_equals_scatter_then_step(dev, T_, L, b, N, steps, flags, skew):
    """flags: whole 16-row tiles of dx are +-0 and flagged dead (the dX kernel's tile flags): skipped rows,
    same table.  skew: dx spread over seven decades with one row at 60000 (every level's quantum set by it)
    and half the samples clustered (bins of several chunks): most sums are summed again at their own
    scale, in the fused update as in the stored path."""
    print(f"[scatter adam] T={T_} L={L} N={N} flags={flags} skew={skew}", flush=True)
    P = pkg()
    ga, gb = make_grid(T_, L, b, N, 5), make_grid(T_, L, b, N, 5)
    n = L * T_ * 2
    s0a, s0b = state(ga, n), state(gb, n)
    for k in s0a:
        np.testing.assert_array_equal(bits(s0a[k]), bits(s0b[k]))
    rng = np.random.default_rng(100 + N)
    for step in range(steps):
        pos = positions(N, 7 + step)
        pos[:32, :3] = rng.choice(np.float32([0.0, 1.0, 0.5, np.nextafter(np.float32(1), 0)]), (32, 3))
        dx = rng.normal(0, 0.5, (N, 2 * L)).astype(np.float16)
        dx[rng.random((N, 2 * L)) < 0.3] = 0  # zero gradients: entries no product reaches
        if skew:
            pos[: N // 2, :3] = (0.5 + 0.02 * rng.normal(size=(N // 2, 3))).clip(0, 1)
            dx = (dx.astype(np.float32) * 10.0 ** rng.uniform(-7, 0, (N, 1))).astype(np.float16)
            dx[N // 3] = np.float16(60000.0)
        if step == steps - 1 and N > 40:
            dx[5, 0], dx[17, 3], dx[33, 2 * L - 1] = np.inf, -np.inf, np.nan
        live = None
        if flags:
            ntiles = (N + 15) // 16
            dead = rng.random(ntiles) < 0.5
            dead[:3] = False
            for t in np.nonzero(dead)[0]:
                dx[16 * t:16 * t + 16] = np.where(rng.random(dx[16 * t:16 * t + 16].shape) < 0.5, -0.0, 0.0)
            live = T((~dead).astype(np.uint32), dev)
        d_pos, d_dx = T(pos, dev), T(dx, dev)
        # stored path: scatter into the zero gradient array, then the optimizer step
        ga.zero_grad()
        P.launch("launchHashTableBackwardKernel", d_dx, d_pos, ga.buffers().hashtable_grads, N, T_, L, b, 16, 2, None)
        ga.step(LR, B1, B2, EPS, SCALE)
        # fused path
        gb.zero_grad()
        gb.scatter_adam_table(d_dx, d_pos, N, 4, LR, B1, B2, EPS, SCALE, tile_live=live)
        gb.step_mlp(LR, B1, B2, EPS, SCALE)
        torch.cuda.synchronize()
        sa, sb = state(ga, n), state(gb, n)
        for k in ("master_hashtable", "fwd_hashtable", "hash_m", "hash_v"):
            diff = np.nonzero(bits(sa[k]) != bits(sb[k]))[0]
            assert diff.size == 0, f"step {step} {k}: {diff.size} words differ, first {diff[:8]}"
        assert not sb["hashtable_grads"].any(), "the fused path writes no gradient"
        assert not sa["hashtable_grads"].any()
        moved = (bits(sb["hash_m"]) != bits(s0b["hash_m"])).sum()
        assert moved > 0
    assert ga.buffers().step == gb.buffers().step == steps
    ga.close()
    gb.close()


def test_fused_table_update_rejects_bad_arguments(dev):
    P = pkg()
    g = make_grid(1 << 12, 8, 2.0, 64, 1)
    with pytest.raises(RuntimeError):
        g.scatter_adam_table(None, None, 64)
    with pytest.raises(RuntimeError):
        g.scatter_adam_table(None, None, -1)
    g.scatter_adam_table(None, None, 0)  # nothing to do
    g.close()
