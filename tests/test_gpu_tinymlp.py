"""GPU parity: the gfx950 HIP path (through the C-ABI) against the CPU oracle.

Bars: hash indices / encodings bit-exact (same level
table on both sides); MLP outputs and gradients within 2e-3 abs / 1e-2 rel
(fp16 operands, fp32 accumulation); Adam bit-exact given the same gradients.
"""
import ctypes as C

import numpy as np
import pytest

import pyoracle as orc
from helpers import (assert_close, assert_scatter_close, d2h, h2d, make_mlp, pkg, positions, ptr_array, scatter_bound,
                     scatter_quantum)

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need cuda:0"
    return torch.device("cuda:0")


def T(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def grid_opt(T_, L, b, hidden=64, out=16, layers=2, vec=4, base=16):
    P = pkg()
    return P.MLPGridOptions(vectorDim=vec, hiddenDim=hidden, outputDim=out, numLayers=layers, activationType=0,
                            tableSize=T_, numLevels=L, b=b, lowestSize=base, featuresLevel=2)


def edge_positions(n, seed):
    p = positions(n, seed)
    rng = np.random.default_rng(seed + 1)
    k = min(n, 64)
    p[:k, :3] = rng.choice(np.float32([0.0, 1.0, 0.5, 0.25, 0.75, np.nextafter(np.float32(1), 0)]), (k, 3))
    return p


# --------------------------------------------------------------------------- encode


@pytest.mark.parametrize("N,T_,b,L", [(4096, 1 << 14, 1.447, 16), (1 << 18, 1 << 19, (2048 / 16) ** (1 / 15), 16),
                                      (1 << 20, 1 << 19, (2048 / 16) ** (1 / 15), 16),   # BASELINE C2, second size
                                      (1000, 1 << 12, 1.5, 7), (1, 1 << 14, 1.447, 16)])
def test_encode_bit_exact(dev, N, T_, b, L):
    P = pkg()
    print(f"[encode] N={N} T={T_} L={L}", flush=True)
    pos = edge_positions(N, 3)
    table = np.random.default_rng(4).uniform(-1e-4, 1e-4, L * T_ * 2).astype(np.float16)
    d_enc = torch.empty((N, 2 * L), dtype=torch.float16, device=dev)
    opt = grid_opt(T_, L, b)
    P.launch("launchHashEncodeKernel", C.byref(opt), T(table, dev), T(pos, dev), 4, d_enc, N, None)
    torch.cuda.synchronize()
    want = orc.hash_encode(pos, table, T_, L, 16, b)
    got = d_enc.cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("N,T_,L,b,dist", [
    (1 << 18, 1 << 19, 16, (2048 / 16) ** (1 / 15), "uniform"),   # BASELINE C2 backward
    (1 << 20, 1 << 19, 16, (2048 / 16) ** (1 / 15), "uniform"),   # BASELINE C2, second size
    (1 << 18, 1 << 19, 16, 1.3819, "clustered"),                  # multi-chunk bins at every dense level
    (1 << 16, 1 << 14, 16, 1.447, "clustered"),                   # collision-heavy dense levels
    (3000, 1 << 19, 16, 1.3819, "uniform"),                        # small, ragged batch
    (1 << 16, 1 << 19, 16, 1.3819, "rays"),                        # ray-ordered: merged runs
])
def test_scatter_matches_oracle(dev, N, T_, L, b, dist):
    P = pkg()
    print(f"[scatter] N={N} T={T_} {dist}", flush=True)
    rng = np.random.default_rng(17)
    pos = positions(N, 18)
    if dist == "clustered":
        pos[:, :3] = (0.5 + 0.02 * rng.normal(size=(N, 3))).clip(0, 1).astype(np.float32)
    elif dist == "rays":  # 256 samples per ray, 0.002 apart, as the compaction emits them
        R = N // 256
        o = rng.uniform(0.3, 0.7, (R, 1, 3))
        dirs = rng.normal(size=(R, 1, 3))
        dirs /= np.linalg.norm(dirs, axis=2, keepdims=True)
        tt = 0.002 * np.arange(256)[None, :, None]
        pos[:, :3] = (o + tt * dirs).reshape(N, 3).clip(0, 1).astype(np.float32)
    denc = rng.normal(0, 1, (N, 2 * L)).astype(np.float16)
    grads = torch.zeros(L * T_ * 2, dtype=torch.float32, device=dev)
    grads += 0.5  # the scatter accumulates
    P.launch("launchHashTableBackwardKernel", T(denc, dev), T(pos, dev), grads, N, T_, L, b, 16, 2, None)
    torch.cuda.synchronize()
    g, gabs, cnt = orc.hash_scatter_stats(pos, denc, T_, L, 16, b)
    want = g + np.float32(0.5)
    bound = scatter_bound(g, gabs, cnt, scatter_quantum(denc, L, T_))
    assert_scatter_close(grads.cpu().numpy(), want, bound, base=0.5, what="hash grads")


def _scatter_inputs(N, L, seed, dist):
    rng = np.random.default_rng(seed)
    pos = positions(N, seed + 1)
    if dist == "clustered":
        pos[:, :3] = (0.5 + 0.02 * rng.normal(size=(N, 3))).clip(0, 1).astype(np.float32)
    denc = rng.normal(0, 1, (N, 2 * L)).astype(np.float16)
    return pos, denc


def test_scatter_is_deterministic(dev):
    """Fixed-point sums: bitwise equal results run to run, also for bins split over several chunks."""
    P = pkg()
    N, T_, L, b = 1 << 18, 1 << 19, 16, 1.3819
    pos, denc = _scatter_inputs(N, L, 31, "clustered")
    d_pos, d_denc = T(pos, dev), T(denc, dev)
    outs = []
    for _ in range(2):
        grads = torch.zeros(L * T_ * 2, dtype=torch.float32, device=dev)
        P.launch("launchHashTableBackwardKernel", d_denc, d_pos, grads, N, T_, L, b, 16, 2, None)
        torch.cuda.synchronize()
        outs.append(grads.cpu().numpy())
    np.testing.assert_array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    want, gabs, cnt = orc.hash_scatter_stats(pos, denc, T_, L, 16, b)
    assert_scatter_close(outs[0], want, scatter_bound(want, gabs, cnt, scatter_quantum(denc, L, T_)), what="hash grads")


@pytest.mark.parametrize("N,T_,dist", [(1 << 18, 1 << 19, "uniform"), (1 << 17, 1 << 14, "clustered")])
def test_scatter_small_entries_keep_fp32_precision(dev, N, T_, dist):
    """Upstream gradients spread over seven decades, and one sample per level at 60000, which sets every
    level's fixed-point quantum: most entries' sums are tiny against it (their fixed-point sums fall below
    2^24 quanta, some products below half a quantum) and are summed again at their own scale.  Every word
    stays within the per-word bound of the oracle's fp64 sum, and the sums stay bitwise repeatable."""
    P = pkg()
    L, b = 16, 1.3819
    print(f"[scatter small entries] N={N} T={T_} {dist}", flush=True)
    pos, denc = _scatter_inputs(N, L, 57, dist)
    rng = np.random.default_rng(58)
    denc = (denc.astype(np.float32) * 10.0 ** rng.uniform(-7, 0, (N, 1))).astype(np.float16)
    denc[N // 3] = np.float16(60000.0)
    d_pos, d_denc = T(pos, dev), T(denc, dev)
    outs = []
    for _ in range(2):
        grads = torch.zeros(L * T_ * 2, dtype=torch.float32, device=dev)
        P.launch("launchHashTableBackwardKernel", d_denc, d_pos, grads, N, T_, L, b, 16, 2, None)
        torch.cuda.synchronize()
        outs.append(grads.cpu().numpy())
    np.testing.assert_array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    want, gabs, cnt = orc.hash_scatter_stats(pos, denc, T_, L, 16, b)
    # the regime under test: entries far below the level's largest product
    small = (gabs > 0) & (gabs < 2.0 ** -20 * 60000.0)
    assert small.mean() > 0.05 * (gabs > 0).mean()
    bound = scatter_bound(want, gabs, cnt, scatter_quantum(denc, L, T_))
    # a zero sum on one side only where the bound allows it (exact cancellation in one product order)
    ill = np.abs(want) <= bound
    np.testing.assert_array_equal((outs[0] != 0) | ill, (want != 0) | ill)
    assert_scatter_close(outs[0], want, bound, what="hash grads (small entries)")


def test_scatter_nonfinite_inputs_propagate(dev):
    """Inf / NaN upstream gradients reach exactly the entries the oracle's sums make non-finite."""
    P = pkg()
    N, T_, L, b = 20000, 1 << 19, 16, 1.3819
    pos, denc = _scatter_inputs(N, L, 41, "uniform")
    denc[5, 3] = np.float16(np.inf)
    denc[77, 20] = np.float16(-np.inf)
    denc[900, 31] = np.float16(np.nan)
    denc[1234, 0] = np.float16(65504.0)  # largest finite magnitude sets the level's fixed-point scale
    grads = torch.zeros(L * T_ * 2, dtype=torch.float32, device=dev)
    P.launch("launchHashTableBackwardKernel", T(denc, dev), T(pos, dev), grads, N, T_, L, b, 16, 2, None)
    torch.cuda.synchronize()
    got = grads.cpu().numpy()
    with np.errstate(invalid="ignore"):
        want, gabs, cnt = orc.hash_scatter_stats(pos, denc, T_, L, 16, b)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    np.testing.assert_array_equal(np.isposinf(got), np.isposinf(want))
    np.testing.assert_array_equal(np.isneginf(got), np.isneginf(want))
    fin = np.isfinite(want)
    assert fin.sum() < fin.size and (~fin).sum() >= 3
    q = scatter_quantum(denc, L, T_)
    assert_scatter_close(got[fin], want[fin], scatter_bound(want[fin], gabs[fin], cnt[fin], q[fin]), what="finite grads")


def test_encode_stride3(dev):
    P = pkg()
    N, T_, L, b = 777, 1 << 14, 16, 1.447
    pos = positions(N, 5, stride=3)
    table = np.random.default_rng(6).uniform(-1, 1, L * T_ * 2).astype(np.float16)
    d_enc = torch.empty((N, 2 * L), dtype=torch.float16, device=dev)
    opt = grid_opt(T_, L, b)
    P.launch("launchHashEncodeKernel", C.byref(opt), T(table, dev), T(pos, dev), 3, d_enc, N, None)
    torch.cuda.synchronize()
    want = orc.hash_encode(pos, table, T_, L, 16, b)
    np.testing.assert_array_equal(d_enc.cpu().numpy().view(np.uint16), want.view(np.uint16))


# --------------------------------------------------------------------------- hash grid class


def _grid_with_params(N, T_, L, b, seed, hidden=64, out=16, layers=2, vec=4, table_amp=1e-4):
    P = pkg()
    opt = grid_opt(T_, L, b, hidden, out, layers, vec)
    g = P.HashGrid(opt, N, seed=seed)
    rng = np.random.default_rng(seed)
    table = rng.uniform(-table_amp, table_amp, L * T_ * 2).astype(np.float32)
    g.load_hashgrid(table)
    hw_out = max(8, 1 << (out - 1).bit_length())
    W, B = make_mlp(2 * L, hidden, hw_out, layers, seed=seed + 1, bias_scale=0.05)
    g.load_weights(W, B)
    return g, table, W, B, hw_out


@pytest.mark.parametrize("N", [4096, 1000, 1 << 16])
def test_grid_forward_backward_step(dev, N):
    """C1-shaped step through TinyMLPHashGrid; every stage compared on identical inputs."""
    print(f"[grid step] N={N}", flush=True)
    T_, L, b, scale = 1 << 14, 16, 1.447, 128.0
    g, table, W, B, hw_out = _grid_with_params(N, T_, L, b, seed=11)
    pos = edge_positions(N, 12)
    d_pos = T(pos, dev)
    d_out = torch.empty((N, 16), dtype=torch.float32, device=dev)
    g.zero_grad()
    g.forward(d_pos, d_out, N)
    torch.cuda.synchronize()
    bufs = g.buffers()
    acts = ptr_array(bufs.activations, 2)
    enc = d2h(acts[0], (N, 32), np.float16)
    h1 = d2h(acts[1], (N, 64), np.float16)
    y = d_out.cpu().numpy()

    enc_ref = orc.hash_encode(pos, table.astype(np.float16), T_, L, 16, b)
    np.testing.assert_array_equal(enc.view(np.uint16), enc_ref.view(np.uint16))
    y_ref, a_ref = orc.mlp_forward(enc_ref, W, B, 32, 64, 16, 2)
    assert_close(h1, a_ref[0], what="hidden activation")
    assert_close(y, y_ref, what="density output")

    # MSE: identical predictions in -> bit-exact fp16 gradient out
    tgt = np.random.default_rng(13).random((N, 16), dtype=np.float32).astype(np.float16)
    loss = g.calculate_loss_and_grad(T(tgt, dev), N, scale, fetch_loss=True)
    dloss = d2h(bufs.dloss, (N, 16), np.float16)
    tot, dloss_ref = orc.mse_loss_grad(y, tgt, 16, scale)
    np.testing.assert_array_equal(dloss.view(np.uint16), dloss_ref.view(np.uint16))
    assert abs(loss - tot / (N * 16)) <= 1e-5 * abs(tot / (N * 16)) + 1e-12

    # backward on the GPU's own activations
    g.backward(N)
    torch.cuda.synchronize()
    dx = d2h(bufs.dx_out, (N, 32), np.float16)
    wg = ptr_array(bufs.w_grad, 2)
    bg = ptr_array(bufs.b_grad, 2)
    dW = np.concatenate([d2h(wg[0], (64 * 32,), np.float32), d2h(wg[1], (16 * 64,), np.float32)])
    dB = np.concatenate([d2h(bg[0], (64,), np.float32), d2h(bg[1], (16,), np.float32)])
    dW_ref, dB_ref, dx_ref = orc.mlp_backward(dloss, enc, h1[None], W, 32, 64, 16, 2)
    wscale = np.abs(dW_ref).max()
    assert_close(dW, dW_ref, atol=2e-3 * max(1.0, wscale), what="dW")
    assert_close(dB, dB_ref, atol=2e-3 * max(1.0, np.abs(dB_ref).max()), what="db")
    assert_close(dx, dx_ref, atol=2e-3 * max(1.0, np.abs(dx_ref.astype(np.float32)).max()), what="dL/denc")

    grads = d2h(bufs.hashtable_grads, (L * T_ * 2,), np.float32)
    grads_ref = orc.hash_scatter(pos, dx, T_, L, 16, b)
    gs = np.abs(grads_ref).max()
    assert_close(grads, grads_ref, atol=1e-5 * gs, rtol=1e-4, what="hash grads")

    # Adam on identical gradients: bit-exact, and the grads are cleared
    mw = ptr_array(bufs.master_weights, 2)
    g.step(1e-2, 0.9, 0.99, 1e-15, scale)
    torch.cuda.synchronize()
    bc1, bc2 = orc.adam_bias_corrections(0.9, 0.99, 1)
    tw = table.copy()
    tg = grads.copy()
    tm = np.zeros_like(tw)
    tv = np.zeros_like(tw)
    t16 = orc.adam_hash(tw, tg, tm, tv, 1e-2, 0.9, 0.99, 1e-15, bc1, bc2, 1 / scale,
                        w16_init=table.astype(np.float16))
    np.testing.assert_array_equal(d2h(bufs.master_hashtable, tw.shape, np.float32).view(np.uint32), tw.view(np.uint32))
    np.testing.assert_array_equal(d2h(bufs.fwd_hashtable, tw.shape, np.float16).view(np.uint16), t16.view(np.uint16))
    np.testing.assert_array_equal(d2h(bufs.hash_m, tw.shape, np.float32), tm)
    assert not d2h(bufs.hashtable_grads, tw.shape, np.float32).any()
    w0 = W[:64 * 32].copy()
    m0 = np.zeros_like(w0)
    v0 = np.zeros_like(w0)
    orc.adam_dense(w0, dW[:64 * 32].copy(), m0, v0, 1e-2, 0.9, 0.99, 1e-15, bc1, bc2, 1 / scale)
    np.testing.assert_array_equal(d2h(mw[0], w0.shape, np.float32).view(np.uint32), w0.view(np.uint32))


def test_grid_vectordim3_and_unpadded_out(dev):
    """vectorDim=3 inputs and a non-power-of-two output width (13 -> 16 padded)."""
    N, T_, L, b = 2000, 1 << 14, 16, 1.447
    g, table, W, B, hw_out = _grid_with_params(N, T_, L, b, seed=21, out=13, vec=3)
    assert hw_out == 16
    pos = positions(N, 22, stride=3)
    d_out = torch.empty((N, 13), dtype=torch.float32, device=dev)
    g.forward(T(pos, dev), d_out, N)
    d_inf = torch.empty((N, 13), dtype=torch.float32, device=dev)
    g.inference(T(pos, dev), d_inf, N)
    torch.cuda.synchronize()
    enc_ref = orc.hash_encode(pos, table.astype(np.float16), T_, L, 16, b)
    y_ref, _ = orc.mlp_forward(enc_ref, W, B, 32, 64, 16, 2)
    assert_close(d_out.cpu().numpy(), y_ref[:, :13], what="forward")
    np.testing.assert_array_equal(d_out.cpu().numpy(), d_inf.cpu().numpy())


def test_grid_inference_chunks(dev):
    P = pkg()
    N, T_, L, b = 5000, 1 << 14, 16, 1.447
    opt = grid_opt(T_, L, b)
    g = P.HashGrid(opt, 1024, infer_batch=1024, seed=3, training=False)
    pos = positions(N, 1)
    d_out = torch.empty((N, 16), dtype=torch.float32, device=dev)
    g.inference(T(pos, dev), d_out, N)
    torch.cuda.synchronize()
    table = np.zeros(L * T_ * 2, np.float32)
    g.save_hashgrid(table)
    W = np.zeros(64 * 32 + 16 * 64, np.float32)
    B = np.zeros(80, np.float32)
    g.save_weights(W, B)
    enc_ref = orc.hash_encode(pos, table.astype(np.float16), T_, L, 16, b)
    y_ref, _ = orc.mlp_forward(enc_ref, W, B, 32, 64, 16, 2)
    assert_close(d_out.cpu().numpy(), y_ref, what="chunked inference")


def test_grid_mode_errors(dev):
    P = pkg()
    opt = grid_opt(1 << 14, 16, 1.447)
    g = P.HashGrid(opt, 256, seed=1)
    with pytest.raises(RuntimeError, match="before forward"):
        g.backward(256)
    g.switch_mode(False)
    with pytest.raises(RuntimeError, match="inference mode"):
        g.forward(T(positions(256, 0), dev), None, 256)
    with pytest.raises(RuntimeError, match="inference mode"):
        g.step()
    g.switch_mode(True)
    g.forward(T(positions(256, 0), dev), None, 256)
    with pytest.raises(RuntimeError, match="maxBatchSize"):
        g.forward(T(positions(512, 0), dev), None, 512)


def test_adam_hash_100_steps_bit_exact(dev):
    P = pkg()
    L, T_ = 2, 1 << 12
    n = L * T_ * 2
    opt = grid_opt(T_, L, 1.5)
    rng = np.random.default_rng(99)
    w = rng.standard_normal(n).astype(np.float32)
    w16 = w.astype(np.float16)
    d_w, d_w16 = T(w, dev), T(w16, dev)
    d_m, d_v = torch.zeros(n, device=dev), torch.zeros(n, device=dev)
    d_g = torch.empty(n, device=dev)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    for t in range(1, 101):
        g = (rng.standard_normal(n) * 50).astype(np.float32)
        g[rng.random(n) < 0.3] = 0.0
        if t == 50:
            g[:5] = [np.nan, np.inf, -np.inf, 1e30, -0.0]
        h2d(d_g.data_ptr(), g)
        bc1, bc2 = orc.adam_bias_corrections(0.9, 0.99, t)
        P.launch("launchAdamHashGridOptim", C.byref(opt), d_w, d_w16, d_g, d_m, d_v, 1e-2, 0.9, 0.99, 1e-15,
                 bc1, bc2, 1 / 128.0, None)
        w16 = orc.adam_hash(w, g, m, v, 1e-2, 0.9, 0.99, 1e-15, bc1, bc2, 1 / 128.0, w16_init=w16)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(d_w16.cpu().numpy().view(np.uint16), w16.view(np.uint16))
    np.testing.assert_array_equal(d_w.cpu().numpy().view(np.uint32), w.view(np.uint32))
    np.testing.assert_array_equal(d_m.cpu().numpy().view(np.uint32), m.view(np.uint32))
    np.testing.assert_array_equal(d_v.cpu().numpy().view(np.uint32), v.view(np.uint32))


# --------------------------------------------------------------------------- plain TinyMLP


@pytest.mark.parametrize("inD,hid,outD,nl,act,N", [(32, 64, 3, 3, 1, 4096), (32, 32, 3, 3, 1, 999),
                                                   (64, 64, 64, 2, 0, 2048), (16, 128, 16, 2, 0, 1024),
                                                   (3, 16, 8, 4, 0, 333), (32, 64, 3, 3, 1, 1 << 18),
                                                   (32, 64, 16, 2, 0, 1 << 18)])
def test_net_forward_backward(dev, inD, hid, outD, nl, act, N):
    """TinyMLP (color head and benchmark shapes): forward, MSE/sigmoid', backward with dX."""
    print(f"[net] in={inD} hid={hid} out={outD} layers={nl} act={act} N={N}", flush=True)
    P = pkg()
    opt = P.MLPOption(inputDim=inD, hiddenDim=hid, outputDim=outD, numLayers=nl, activationType=0,
                      outputActivation=act)
    net = P.Net(opt, N, seed=5)
    hw = net.buffers().hw
    hi, hh, ho = hw.inputDim, hw.hiddenDim, hw.outputDim
    W, B = make_mlp(hi, hh, ho, nl, seed=7, bias_scale=0.05)
    net.load_weights(W, B)
    rng = np.random.default_rng(8)
    x = rng.standard_normal((N, inD)).astype(np.float16)
    d_y = torch.empty((N, outD), dtype=torch.float32, device=dev)
    net.zero_grad()
    net.forward(T(x, dev), d_y, N)
    torch.cuda.synchronize()
    xp = np.zeros((N, hi), np.float16)
    xp[:, :inD] = x
    y_ref, acts_ref = orc.mlp_forward(xp, W, B, hi, hh, ho, nl, out_act=act)
    y = d_y.cpu().numpy()
    assert_close(y, y_ref[:, :outD], what="net forward")

    bufs = net.buffers()
    aptr = ptr_array(bufs.activations, nl)
    np.testing.assert_array_equal(d2h(aptr[0], (N, hi), np.float16), xp)
    acts = np.stack([d2h(aptr[l], (N, hh), np.float16) for l in range(1, nl)]) if nl > 1 else None
    for l in range(nl - 1):
        assert_close(acts[l], acts_ref[l], what=f"act {l + 1}")

    tgt = rng.random((N, outD), dtype=np.float32).astype(np.float16)
    net.calculate_loss_and_grad(T(tgt, dev), N, 128.0)
    yp = d2h(bufs.padded_outputs, (N, ho), np.float32)
    tp = np.zeros((N, ho), np.float16)
    tp[:, :outD] = tgt
    _, dl_ref = orc.mse_loss_grad(yp, tp, outD, 128.0, out_act=act)
    dl = d2h(bufs.dloss, (N, ho), np.float16)
    np.testing.assert_array_equal(dl.view(np.uint16), dl_ref.view(np.uint16))

    d_dx = torch.empty((N, hi), dtype=torch.float16, device=dev)
    net.backward(N, dx_out=d_dx)
    torch.cuda.synchronize()
    dW_ref, dB_ref, dx_ref = orc.mlp_backward(dl, xp, acts, W, hi, hh, ho, nl)
    wg = ptr_array(bufs.w_grad, nl)
    bg = ptr_array(bufs.b_grad, nl)
    sizes = [(ho if l == nl - 1 else hh) * (hi if l == 0 else hh) for l in range(nl)]
    dW = np.concatenate([d2h(wg[l], (sizes[l],), np.float32) for l in range(nl)])
    dB = np.concatenate([d2h(bg[l], ((ho if l == nl - 1 else hh),), np.float32) for l in range(nl)])
    assert_close(dW, dW_ref, atol=2e-3 * max(1.0, np.abs(dW_ref).max()), what="dW")
    assert_close(dB, dB_ref, atol=2e-3 * max(1.0, np.abs(dB_ref).max()), what="db")
    dx = d_dx.cpu().numpy()
    assert_close(dx, dx_ref, atol=2e-3 * max(1.0, np.abs(dx_ref.astype(np.float32)).max()), what="dx")


def _net_grads(net, nl):
    bufs = net.buffers()
    hw = bufs.hw
    hi, hh, ho = hw.inputDim, hw.hiddenDim, hw.outputDim
    wg, bg = ptr_array(bufs.w_grad, nl), ptr_array(bufs.b_grad, nl)
    outs = [ho if l == nl - 1 else hh for l in range(nl)]
    ins = [hi if l == 0 else hh for l in range(nl)]
    return np.concatenate([d2h(wg[l], (outs[l] * ins[l],), np.float32) for l in range(nl)] +
                          [d2h(bg[l], (outs[l],), np.float32) for l in range(nl)])


def test_two_instances_on_two_streams_match_serial_runs(dev):
    """Each TinyMLP instance owns the partial-sum workspace of its loss and backward: two instances
    trained at once on two streams give the gradients of serial runs, bit for bit (the reductions
    are fixed-order)."""
    P = pkg()
    N = 1 << 18
    shapes = [(32, 64, 16, 2, 0), (32, 64, 3, 3, 1)]   # the density and colour head shapes
    nets = [P.Net(P.MLPOption(inputDim=i, hiddenDim=h, outputDim=o, numLayers=nl, activationType=0,
                              outputActivation=a), N, seed=11 + k)
            for k, (i, h, o, nl, a) in enumerate(shapes)]
    rng = np.random.default_rng(12)
    xs = [T(rng.standard_normal((N, sh[0])).astype(np.float16), dev) for sh in shapes]
    ts = [T(rng.random((N, sh[2]), dtype=np.float32).astype(np.float16), dev) for sh in shapes]

    def phases(k, stream):
        n = nets[k]
        return [lambda: n.zero_grad(stream), lambda: n.forward(xs[k], None, N, stream),
                lambda: n.calculate_loss_and_grad(ts[k], N, 128.0, stream=stream),
                lambda: n.backward(N, stream=stream)]

    serial = []
    for k in range(2):
        for f in phases(k, 0):
            f()
        torch.cuda.synchronize()
        serial.append(_net_grads(nets[k], shapes[k][3]))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for rep in range(3):
        pa, pb = phases(0, streams[0].cuda_stream), phases(1, streams[1].cuda_stream)
        for fa, fb in zip(pa, pb):   # interleaved: the two backwards run at the same time
            fa()
            fb()
        torch.cuda.synchronize()
        for k in range(2):
            np.testing.assert_array_equal(_net_grads(nets[k], shapes[k][3]), serial[k], err_msg=f"rep {rep} net {k}")
    for n in nets:
        n.close()


def test_net_custom_grad_and_accumulation(dev):
    """backward(custom) twice accumulates dW exactly 2x (deterministic reduction)."""
    P = pkg()
    N = 3000
    opt = P.MLPOption(inputDim=32, hiddenDim=64, outputDim=3, numLayers=3, activationType=0, outputActivation=1)
    net = P.Net(opt, N, seed=9)
    x = np.random.default_rng(1).standard_normal((N, 32)).astype(np.float16)
    net.zero_grad()
    net.forward(T(x, dev), None, N)
    cg = (np.random.default_rng(2).standard_normal((N, 3)) * 100).astype(np.float16)
    net.backward(N, custom_grad=T(cg, dev))
    bufs = net.buffers()
    wg = ptr_array(bufs.w_grad, 3)
    torch.cuda.synchronize()
    g1 = d2h(wg[1], (64 * 64,), np.float32)
    net.backward(N, custom_grad=T(cg, dev))
    torch.cuda.synchronize()
    g2 = d2h(wg[1], (64 * 64,), np.float32)
    np.testing.assert_array_equal(g2, g1 * 2)


def test_launchers_plain_mlp(dev):
    """The reference launchers with raw device pointer arrays (no class)."""
    P = pkg()
    N, inD, hid, outD, nl = 1500, 32, 64, 16, 2
    opt = P.MLPOption(inputDim=inD, hiddenDim=hid, outputDim=outD, numLayers=nl, activationType=0,
                      outputActivation=0)
    W, B = make_mlp(inD, hid, outD, nl, seed=3, bias_scale=0.1)
    w16 = W.astype(np.float16)
    d_w0, d_w1 = T(w16[:hid * inD], dev), T(w16[hid * inD:], dev)
    d_b0, d_b1 = T(B[:hid], dev), T(B[hid:], dev)
    x = np.random.default_rng(4).standard_normal((N, inD)).astype(np.float16)
    d_x = T(x, dev)
    d_h = torch.empty((N, hid), dtype=torch.float16, device=dev)
    Wp = T(np.array([d_w0.data_ptr(), d_w1.data_ptr()], np.uint64).view(np.int64), dev)
    Bp = T(np.array([d_b0.data_ptr(), d_b1.data_ptr()], np.uint64).view(np.int64), dev)
    Ap = T(np.array([d_x.data_ptr(), d_h.data_ptr()], np.uint64).view(np.int64), dev)
    d_y = torch.empty((N, outD), dtype=torch.float32, device=dev)
    d_yi = torch.empty((N, outD), dtype=torch.float32, device=dev)
    P.launch("launchNetworkFusionGradKernel", C.byref(opt), d_x, Ap, Wp, Bp, d_y, N, None)
    P.launch("launchNetworkFusionKernel", C.byref(opt), d_x, Wp, Bp, d_yi, N, None)
    torch.cuda.synchronize()
    y_ref, a_ref = orc.mlp_forward(x, W, B, inD, hid, outD, nl)
    assert_close(d_y.cpu().numpy(), y_ref, what="grad-kernel forward")
    np.testing.assert_array_equal(d_y.cpu().numpy(), d_yi.cpu().numpy())
    dy = (np.random.default_rng(5).standard_normal((N, outD)) * 10).astype(np.float16)
    gw0, gw1 = torch.zeros(hid * inD, device=dev), torch.zeros(outD * hid, device=dev)
    gb0, gb1 = torch.zeros(hid, device=dev), torch.zeros(outD, device=dev)
    GWp = T(np.array([gw0.data_ptr(), gw1.data_ptr()], np.uint64).view(np.int64), dev)
    GBp = T(np.array([gb0.data_ptr(), gb1.data_ptr()], np.uint64).view(np.int64), dev)
    d_dx = torch.empty((N, inD), dtype=torch.float16, device=dev)
    P.launch("launchNetworkFusionBackwardKernel", C.byref(opt), T(dy, dev), Wp, Bp, Ap, GWp, GBp, d_dx, N, None)
    torch.cuda.synchronize()
    h = d_h.cpu().numpy()
    dW_ref, dB_ref, dx_ref = orc.mlp_backward(dy, x, h[None], W, inD, hid, outD, nl)
    dW = np.concatenate([gw0.cpu().numpy(), gw1.cpu().numpy()])
    assert_close(dW, dW_ref, atol=2e-3 * np.abs(dW_ref).max(), what="launcher dW")
    assert_close(d_dx.cpu().numpy(), dx_ref, atol=2e-3 * max(1, np.abs(dx_ref.astype(np.float32)).max()),
                 what="launcher dx")


def test_weight_files_round_trip_and_layout(dev, tmp_path):
    """TinyMLP / TinyMLPHashGrid weight files (TinyMLP.cu:406-481,
    TinyMLPHashGrid.cu:394-455): raw options header of the hardware shape, then
    (grid: the fp32 table, then) per layer W then b, fp32."""
    P = pkg()
    opt = P.MLPOption(inputDim=32, hiddenDim=64, outputDim=3, numLayers=3, activationType=0, outputActivation=1)
    net = P.Net(opt, 256, seed=5)
    hw = net.buffers().hw
    W, B = make_mlp(hw.inputDim, hw.hiddenDim, hw.outputDim, 3, seed=3, bias_scale=0.1)
    net.load_weights(W, B)
    path = str(tmp_path / "color.bin")
    net.save_file(path)
    raw = open(path, "rb").read()
    hdr = P.MLPOption.from_buffer_copy(raw[:C.sizeof(P.MLPOption)])
    assert (hdr.inputDim, hdr.hiddenDim, hdr.outputDim, hdr.numLayers) == (32, 64, 8, 3)
    body = np.frombuffer(raw, np.float32, offset=C.sizeof(P.MLPOption))
    wo = bo = po = 0
    for o, i in [(64, 32), (64, 64), (8, 64)]:
        np.testing.assert_array_equal(body[po:po + o * i], W[wo:wo + o * i])
        np.testing.assert_array_equal(body[po + o * i:po + o * i + o], B[bo:bo + o])
        po += o * i + o
        wo += o * i
        bo += o
    assert po == body.size
    net2 = P.Net(opt, 256, seed=99)
    net2.load_file(path)
    W2, B2 = np.zeros_like(W), np.zeros_like(B)
    net2.save_weights(W2, B2)
    np.testing.assert_array_equal(W2, W)
    np.testing.assert_array_equal(B2, B)

    gopt = grid_opt(1 << 12, 4, 1.5)
    g = P.HashGrid(gopt, 256, seed=1)
    gpath = str(tmp_path / "grid.bin")
    g.save_file(gpath)
    g2 = P.HashGrid(gopt, 256, seed=2)
    g2.load_file(gpath)
    t1, t2 = np.zeros(4 * (1 << 12) * 2, np.float32), np.zeros(4 * (1 << 12) * 2, np.float32)
    g.save_hashgrid(t1)
    g2.save_hashgrid(t2)
    np.testing.assert_array_equal(t1, t2)
    graw = open(gpath, "rb").read()
    off = C.sizeof(P.MLPGridOptions)
    np.testing.assert_array_equal(np.frombuffer(graw, np.float32, t1.size, off), t1)
    bad = P.HashGrid(grid_opt(1 << 12, 4, 1.5), 256, seed=1)
    open(str(tmp_path / "short.bin"), "wb").write(graw[:len(graw) - 100])
    with pytest.raises(RuntimeError):
        bad.load_file(str(tmp_path / "short.bin"))
