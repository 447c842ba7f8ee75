"""Replay of one InstantNerf training step on the CPU oracle, from the GPU's state before it (test helper).

read_state() copies everything a step reads (hash table and its Adam moments, both heads' weights and
moments, occupancy bits and master grid, step counters) back to the host; check_step() then recomputes the
step stage by stage on the oracle and compares it with what the GPU left behind, each stage on the GPU's own
inputs (so that one stage's tolerance does not compound into the next): compaction bit-exact, both heads
within the fp16-MLP tolerance, SH gather and density gradient bit-exact, compositing and gradients within
their rounding bounds, the hash table after scatter + Adam and both heads' weights after Adam.
"""
from __future__ import annotations

import numpy as np

import pyoracle as orc
from helpers import assert_close, d2h, ptr_array, scatter_bound, scatter_quantum

MN = np.float32([-1.5, -1.5, -1.5])
MX = np.float32([1.5, 1.5, 1.5])


def bits_eq(a, b):
    a, b = np.asarray(a), np.asarray(b)
    np.testing.assert_array_equal(a.view(np.uint32) if a.dtype == np.float32 else a,
                                  b.view(np.uint32) if b.dtype == np.float32 else b)


def scan_close(got, want, what, atol_rel=2e-5, rtol=1e-4):
    """Agreement up to fp32 rounding of a different summation/product order."""
    want = np.asarray(want, np.float64)
    scale = float(np.abs(want).max()) if want.size else 0.0
    assert np.isfinite(np.asarray(got, np.float64)).all(), what
    assert_close(got, want, atol=atol_rel * max(scale, 1e-30), rtol=rtol, what=what)


def dsigma_close(got, want, cnt, off, t, dout, phi, dw, loss_scale, total_rays, bias=0.0, what="d sigma"):
    """d sigma subtracts running sums from ray totals (otherKernels.cu:387-400): a different association
    moves it by a few ulp of the totals times delta sigma S / R; bound 32 eps32 delta sigma S/R
    (2 sum|phi| + 2 max|g|) per sample plus the scan_close floor."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert np.isfinite(got).all(), what
    bound = np.zeros_like(want)
    sig = np.exp(np.minimum(dout[:, 0].astype(np.float64) - bias, 8.0))
    for r in range(len(cnt)):
        n, o = int(cnt[r]), int(off[r])
        if n == 0:
            continue
        tt = t[o:o + n].astype(np.float64)
        delta = np.append(np.maximum(np.diff(tt), 0.0), 1e-3)
        amp = 2.0 * np.abs(phi[r]).sum() + 2.0 * np.abs(dw[o:o + n]).max()
        bound[o:o + n] = 32 * 2.0 ** -23 * delta * sig[o:o + n] * (loss_scale / total_rays) * amp
    scale = float(np.abs(want).max()) if want.size else 0.0
    excess = np.abs(got - want) - (bound + 2e-5 * scale + 1e-4 * np.abs(want))
    if (excess > 0).any():
        i = int(np.argmax(excess))
        raise AssertionError(f"{what}: {(excess > 0).sum()} of {want.size} outside; worst at {i}: got {got[i]!r} "
                             f"expected {want[i]!r} bound {bound[i]!r}")


def head_hidden(b, buf, x, W, B, inD, hid, outD, nl, N, out_act=0):
    """The hidden activations [nl-1, N, hid] the step's backward used.  When the step kept them
    (activationsSaved) they are read from the TinyMLP buffers; otherwise the 16x16x32 heads recomputed
    them, and the oracle's forward of the same input stands in (equal up to fp16 rounding of a different
    fp32 summation order)."""
    if b.activationsSaved:
        return np.stack([d2h(q, (N, hid), np.float16) for q in ptr_array(buf.activations, nl)[1:]])
    _, acts = orc.mlp_forward(x, W, B, inD, hid, outD, nl, out_act=out_act)
    return acts


def step_encodings(b, buf, N, levels):
    """The step's fp16 encodings [N, 2 levels]: activation 0 of the density head, or the level-major
    planar copy the 16x16x32 heads read."""
    if b.activationsSaved:
        return d2h(ptr_array(buf.activations, 2)[0], (N, 2 * levels), np.float16)
    pl = d2h(b.encodings, (levels, int(b.encodingPlane), 2), np.float16)[:, :N, :]
    return np.ascontiguousarray(pl.transpose(1, 0, 2).reshape(N, 2 * levels))


def density_outputs(b, N, cin):
    """The step's density head output [N x 16] as the oracle takes it.  With the 16x16x32 heads the step
    stores only the logit 0 (density_stride 1, all the step reads of it); the other 15 outputs then come
    from the colour input, where the forward wrote them sanitised and rounded to fp16 (the values the
    colour head and SH gather use).  Returns (outputs, whether all 16 are the stored fp32 outputs)."""
    ds = int(b.density_stride)
    assert ds in (1, 16), ds
    dout = d2h(b.density_out, (N, ds), np.float32)
    if ds == 16:
        return dout, True
    full = np.asarray(cin, np.float16)[:, :16].astype(np.float32)
    full[:, 0] = dout[:, 0]
    return full, False


def check_density_outputs(b, N, cin, y_ref, what="density output"):
    """The density head's outputs against the oracle's: fp32 where stored; the colour input's fp16 logits
    (rounded) against the sanitised oracle outputs where only the logit 0 is stored."""
    dout, whole = density_outputs(b, N, cin)
    if whole:
        assert_close(dout, y_ref, what=what)
    else:
        assert_close(dout[:, 0], y_ref[:, 0], what=what + " (logit 0)")
        want = np.clip(np.nan_to_num(y_ref[:, 1:], nan=0.0), -64.0, 64.0)
        assert_close(dout[:, 1:], want, atol=2e-3, rtol=1e-2 + 2.0 ** -10, what=what + " (colour input logits)")
    return dout


def color_dx_cols(b):
    """Columns of color_dx the step computes: all 32, or the 16 logit features when the activations are
    recomputed (the SH features get no gradient and are written as 0)."""
    return 32 if b.activationsSaved else 16


def layer_sizes(inD, hid, outD, nl):
    shapes = [((outD if l == nl - 1 else hid), (inD if l == 0 else hid)) for l in range(nl)]
    return [o * i for o, i in shapes], [o for o, _ in shapes]


def _per_layer(arr_ptr, sizes):
    return [d2h(p, (n,), np.float32) for p, n in zip(ptr_array(arr_ptr, len(sizes)), sizes)]


class HeadState:
    """Weights, biases and their Adam moments of one head (fp32 master copies), per layer."""

    def __init__(self, buf, shape):
        inD, hid, outD, nl = shape
        self.ws, self.bs = layer_sizes(inD, hid, outD, nl)
        self.W = _per_layer(buf.master_weights, self.ws)
        self.B = _per_layer(buf.master_biases, self.bs)
        self.Wm, self.Wv = _per_layer(buf.w_m, self.ws), _per_layer(buf.w_v, self.ws)
        self.Bm, self.Bv = _per_layer(buf.b_m, self.bs), _per_layer(buf.b_v, self.bs)
        self.step = int(buf.step)

    def flatW(self):
        return np.concatenate(self.W)

    def flatB(self):
        return np.concatenate(self.B)


def density_shape(opts):
    return (2 * opts.numLevels, 64, 16, 2)


def color_shape(opts):
    return (32, opts.colorHiddenDim, 8, opts.colorNumLayers)


def read_state(nerf, opts):
    g = nerf.density.buffers()
    n = opts.numLevels * opts.hashTableSize * 2
    st = {
        "table": d2h(g.master_hashtable, (n,), np.float32),
        "hash_m": d2h(g.hash_m, (n,), np.float32),
        "hash_v": d2h(g.hash_v, (n,), np.float32),
        "density": HeadState(g, density_shape(opts)),
        "color": HeadState(nerf.color.buffers(), color_shape(opts)),
        "bits": nerf.occupancy(),
        "master": nerf.master_grid(),
        "train_steps": int(nerf.step_buffers().trainSteps),
    }
    return st


def oracle_active(opts, st, o, d):
    """Rays of the first hit batch of (o, d) on the state's occupancy bits, and the oracle's march."""
    res, Cc, L = int(opts.gridResolution[0]), opts.numCascades, opts.levelsMipmap
    m = orc.march_hits(o, d, *orc.ray_aabb_inv(o, d, MN, MX, Cc), st["bits"], [res] * 3, MN, MX, Cc, L,
                       opts.samplesPerVoxel, opts.batchSize)
    return m


def check_adam_head(head_before, buf, lr, opts):
    """Both heads' Adam (bit-exact given the GPU's own gradients)."""
    bc1, bc2 = orc.adam_bias_corrections(opts.beta1, opts.beta2, head_before.step + 1)
    wg = _per_layer(buf.w_grad, head_before.ws)
    bg = _per_layer(buf.b_grad, head_before.bs)
    Wa = _per_layer(buf.master_weights, head_before.ws)
    Ba = _per_layer(buf.master_biases, head_before.bs)
    for l in range(len(head_before.ws)):
        for before, m, v, g, after in ((head_before.W[l], head_before.Wm[l], head_before.Wv[l], wg[l], Wa[l]),
                                       (head_before.B[l], head_before.Bm[l], head_before.Bv[l], bg[l], Ba[l])):
            w = before.copy()
            orc.adam_dense(w, g.copy(), m.copy(), v.copy(), lr, opts.beta1, opts.beta2, opts.epsilon, bc1, bc2,
                           1.0 / opts.lossScale)
            bits_eq(after, w)


def check_step(nerf, opts, st, march, o, d, gt, R, bg, lr, rgb_out):
    """The step the GPU just ran on rays (o, d, gt)[:R] from state st, stage by stage against the oracle."""
    b = nerf.step_buffers()
    N = int(march["total"])
    T_, Lh, base, growth = opts.hashTableSize, opts.numLevels, opts.baseResolution, opts.growthFactor
    # compaction (bit-exact)
    np.testing.assert_array_equal(d2h(b.num_steps, (R,), np.uint32), march["counts"][:R])
    np.testing.assert_array_equal(d2h(b.ray_offsets, (R,), np.uint32), march["offsets"][:R])
    bits_eq(d2h(b.t_sorted, (N,), np.float32), march["t"][:N])
    np.testing.assert_array_equal(d2h(b.ray_indices, (N,), np.uint32), march["ray_idx"][:N])
    pos = d2h(b.positions, (N, 4), np.float32)
    bits_eq(pos, march["pos"][:N])
    cnt, off, t, ridx = march["counts"][:R], march["offsets"][:R], march["t"][:N], march["ray_idx"][:N]
    # density head (hash encode + MLP)
    D, Cs = st["density"], st["color"]
    enc_ref = orc.hash_encode(pos, st["table"].astype(np.float16), T_, Lh, base, growth)
    y_ref, _ = orc.mlp_forward(enc_ref, D.flatW().astype(np.float16), D.flatB(), 32, 64, 16, 2, save_acts=False)
    cin = d2h(b.color_input, (N, 32), np.float16)
    dout = check_density_outputs(b, N, cin, y_ref)
    # SH gather on the GPU's density output (bit-exact)
    w_cin, w_sig = orc.sh_gather(d, ridx, dout, opts.densityBias)
    np.testing.assert_array_equal(cin.view(np.uint16), w_cin.view(np.uint16))
    bits_eq(d2h(b.sigma, (N,), np.float32), w_sig)
    # colour head
    hid, nl = opts.colorHiddenDim, opts.colorNumLayers
    cout = d2h(b.color_output, (N, 8), np.float32)
    c_ref, _ = orc.mlp_forward(cin, Cs.flatW().astype(np.float16), Cs.flatB(), 32, hid, 8, nl, out_act=1,
                               save_acts=False)
    assert_close(cout, c_ref, what="color output")
    # compositing + distortion, colour / density gradients (fused scans: rounding bounds)
    rgb3 = np.ascontiguousarray(cout[:, :3])
    comp = orc.composite(off, cnt, t, w_sig, rgb3, gt[:R], opts.lambdaDist, np.float32(bg))
    scan_close(rgb_out[:R], comp["rgb"], "rgb")
    scan_close(d2h(b.phi, (R, 3), np.float32), comp["phi"], "phi")
    scan_close(d2h(b.dw, (N,), np.float32), comp["dw"], "dL/dw")
    cg, ds = orc.color_grad(cnt, off, t, dout, rgb3, comp["phi"], comp["rgb"], comp["dw"], comp["weight_sum"],
                            opts.lossScale, opts.densityBias, R)
    got_ds = d2h(b.dsigma, (N,), np.float32)
    dsigma_close(got_ds, ds, cnt, off, t, dout, comp["phi"], comp["dw"], opts.lossScale, R, opts.densityBias)
    # colour backward on the GPU's activations
    cgp = np.zeros((N, 8), np.float16)
    cgp[:, :3] = cg
    cbuf = nerf.color.buffers()
    h = head_hidden(b, cbuf, cin, Cs.flatW().astype(np.float16), Cs.flatB(), 32, hid, 8, nl, N, out_act=1)
    cdW_ref, cdB_ref, cdx_ref = orc.mlp_backward(cgp, cin, h, Cs.flatW().astype(np.float16), 32, hid, 8, nl)
    cdx = d2h(b.color_dx, (N, 32), np.float16)
    k = color_dx_cols(b)
    assert_close(cdx[:, :k], cdx_ref[:, :k],
                 atol=2e-3 * max(1.0, float(np.abs(cdx_ref[:, :k].astype(np.float32)).max())), what="color dL/dinput")
    cdW = np.concatenate(_per_layer(cbuf.w_grad, Cs.ws))
    cdB = np.concatenate(_per_layer(cbuf.b_grad, Cs.bs))
    assert_close(cdW, cdW_ref, atol=2e-3 * max(1.0, float(np.abs(cdW_ref).max())), what="color dW")
    assert_close(cdB, cdB_ref, atol=2e-3 * max(1.0, float(np.abs(cdB_ref).max())), what="color db")
    dg = d2h(b.density_grad, (N, 16), np.float16)
    np.testing.assert_array_equal(dg.view(np.uint16), orc.density_grad(got_ds, cdx).view(np.uint16))
    # density backward
    gbuf = nerf.density.buffers()
    enc = step_encodings(b, gbuf, N, Lh)
    np.testing.assert_array_equal(enc.view(np.uint16), enc_ref.view(np.uint16))
    h1 = head_hidden(b, gbuf, enc, D.flatW().astype(np.float16), D.flatB(), 32, 64, 16, 2, N)
    ddW_ref, ddB_ref, denc_ref = orc.mlp_backward(dg, enc, h1, D.flatW().astype(np.float16), 32, 64, 16, 2)
    denc = d2h(gbuf.dx_out, (N, 32), np.float16)
    assert_close(denc, denc_ref, atol=2e-3 * max(1.0, float(np.abs(denc_ref.astype(np.float32)).max())),
                 what="dL/d(encoding)")
    ddW = np.concatenate(_per_layer(gbuf.w_grad, D.ws))
    ddB = np.concatenate(_per_layer(gbuf.b_grad, D.bs))
    assert_close(ddW, ddW_ref, atol=2e-3 * max(1.0, float(np.abs(ddW_ref).max())), what="density dW")
    assert_close(ddB, ddB_ref, atol=2e-3 * max(1.0, float(np.abs(ddB_ref).max())), what="density db")
    # Adam of both heads on the GPU's gradients (bit-exact)
    check_adam_head(D, gbuf, lr, opts)
    check_adam_head(Cs, cbuf, lr, opts)
    # hash table: scatter of the GPU's dL/d(encoding), then Adam from the state before
    t_gpu = d2h(gbuf.master_hashtable, st["table"].shape, np.float32)
    m_gpu = d2h(gbuf.hash_m, st["table"].shape, np.float32)
    n_touched, n_ill = check_table_update(t_gpu, m_gpu, st["table"], st["hash_m"], st["hash_v"], pos, denc, T_, Lh,
                                          base, growth, lr, opts, D.step + 1)
    return {"samples": N, "loss": float(np.mean((comp["rgb"] - gt[:R]) ** 2)),
            "loss_gpu": float(np.mean((rgb_out[:R] - gt[:R]) ** 2)), "touched": n_touched,
            "ill_conditioned": n_ill}


def check_table_update(t_gpu, m_gpu, w0, m0, v0, pos, denc, T_, L, base, growth, lr, opts, step):
    """The fused scatter + Adam of the hash table (optimizerKernel.cu:116-167 on the gradient of
    networkFusionBackwardHashtable.cu:783-910) against the oracle's scatter and Adam from the state before
    (w0, m0, v0), on every touched entry:

    - entries no nonzero product reaches: skipped, bit-identical;
    - entries whose gradient is well conditioned (|g_ref| above 4x the per-word bound of the binned sum
      against the oracle's): the reference updates them, so must the fused path, to the oracle's Adam
      within 1e-6 rel / 1e-7 abs (m within 1e-5 rel);
    - the ill-conditioned rest (products cancelling to within a few fp32 roundings of their magnitudes)
      stays below 0.1 % of the touched entries.
    Returns (touched, ill-conditioned) counts."""
    g_ref, g_abs, cnt = orc.hash_scatter_stats(pos, denc, T_, L, base, growth)
    bc1, bc2 = orc.adam_bias_corrections(opts.beta1, opts.beta2, step)
    t_ref, m_ref, v_ref = w0.copy(), m0.copy(), v0.copy()
    orc.adam_hash(t_ref, g_ref.copy(), m_ref, v_ref, lr, opts.beta1, opts.beta2, opts.epsilon, bc1, bc2,
                  1.0 / opts.lossScale, want_f16=False)
    untouched = g_abs == 0
    moved = np.nonzero(untouched & (t_gpu.view(np.uint32) != w0.view(np.uint32)))[0]
    if moved.size:
        lev = moved // (2 * T_)
        slot = (moved % (2 * T_)) // 2
        raise AssertionError(f"{moved.size} table entries without gradient moved: idx {moved[:8]} level {lev[:8]} "
                             f"slot {slot[:8]} before {w0[moved[:8]]} after {t_gpu[moved[:8]]}")
    ill = ~untouched & (np.abs(g_ref) <= 4.0 * scatter_bound(g_ref, g_abs, cnt, scatter_quantum(denc, L, T_)))
    well = ~untouched & ~ill
    n_touched = int((~untouched).sum())
    assert n_touched > 0
    assert ill.sum() <= 1e-3 * n_touched, f"{int(ill.sum())} of {n_touched} touched entries ill-conditioned"
    assert_close(t_gpu[well], t_ref[well], atol=1e-7, rtol=1e-6, what="hash table after Adam (every touched entry)")
    assert_close(m_gpu[well], m_ref[well], atol=1e-7 * float(np.abs(m_ref).max()), rtol=1e-5,
                 what="hash table Adam m (every touched entry)")
    return n_touched, int(ill.sum())


def refresh_oracle_chunks(opts, st):
    """The occupancy refresh of the state's step on the oracle: per chunk (samples [n, 4], density [n, 16])."""
    res, Cc, L = int(opts.gridResolution[0]), opts.numCascades, opts.levelsMipmap
    G, S = res ** 3, orc.pyramid_cells([res] * 3, L)
    T_ = opts.hashTableSize
    active = orc.active_cells(st["bits"], G, S, Cc)
    D = st["density"]
    chunks = []
    for calls in orc.refresh_schedule(st["train_steps"], Cc, G):
        parts = []
        for mode, n, total, off, seed in calls:
            p, cells = orc.occ_sample(n, mode, total, off, seed, [res] * 3, MN, MX,
                                      cell_list=active if mode == orc.OCC_FROM_LIST else None)
            parts.append(np.concatenate([p[:, :3], cells.view(np.float32)[:, None]], 1))
        smp = np.ascontiguousarray(np.concatenate(parts), np.float32)
        enc = orc.hash_encode(smp, st["table"].astype(np.float16), T_, opts.numLevels, opts.baseResolution,
                              opts.growthFactor)
        y, _ = orc.mlp_forward(enc, D.flatW().astype(np.float16), D.flatB(), 32, 64, 16, 2, save_acts=False)
        chunks.append((smp, y))
    return chunks


def check_refresh(nerf, opts, st):
    """A refresh that ran at the start of the step: last chunk's samples bit-exact, master grid (EMA of the
    sampled sigma maxima) within the density tolerance in log space, bits from the GPU's master grid."""
    res, Cc, L = int(opts.gridResolution[0]), opts.numCascades, opts.levelsMipmap
    G, S = res ** 3, orc.pyramid_cells([res] * 3, L)
    chunks = refresh_oracle_chunks(opts, st)
    rb = nerf.refresh_buffers()
    smp, _ = chunks[-1]
    assert rb.last_count == smp.shape[0]
    np.testing.assert_array_equal(d2h(rb.samples, smp.shape, np.float32).view(np.uint32), smp.view(np.uint32))
    tmp = np.zeros(Cc * G, np.float32)
    for s_, y_ in chunks:
        orc.occ_tmp_max(s_, y_, tmp, opts.densityBias)
    want_master = orc.update_master_grid(tmp, st["master"].copy(), opts.decayValue)
    master = nerf.master_grid()
    np.testing.assert_array_equal(master > 0, want_master > 0)
    pos_ = want_master > 0
    assert_close(np.log(master[pos_]), np.log(want_master[pos_]), what="master grid after the refresh (log)")
    bits = nerf.occupancy()
    want = bits.copy()
    orc.update_occupancy_bits(want, master, np.float32(master.astype(np.float64).sum()), G, S,
                              opts.minDensityThreshold, 3.0 / res)
    orc.build_mipmaps(want, [res] * 3, L, Cc)
    thr = np.minimum((opts.minDensityThreshold / (3.0 / res)) / 2.0 ** (np.arange(Cc * G) // G),
                     master.astype(np.float64).mean())
    near = np.abs(master - thr) <= 1e-5 * np.abs(thr)
    got0 = np.concatenate([np.unpackbits(bits, bitorder="little")[c * S: c * S + G] for c in range(Cc)])
    want0 = np.concatenate([np.unpackbits(want, bitorder="little")[c * S: c * S + G] for c in range(Cc)])
    np.testing.assert_array_equal(got0[~near], want0[~near])
    return int(got0.sum())
