"""Pins of the CPU oracle's fused MLP, MSE and Adam (no GPU).

Independent checks: numpy fp64 matrix products (textbook dense layers), a
finite-difference check of the numpy chain rule, numpy float32 arithmetic
for the element-wise MSE/Adam formulas (IEEE, no FMA), and the special cases
the reference defines (skip-zero, NaN self-heal, 50,000-step cap).
"""
import numpy as np
import pytest

import pyoracle as orc
from helpers import layer_shapes, make_mlp


def np_forward(x16, W, B, inD, hid, outD, nl, out_act=0, round16=True):
    """Textbook dense layers in fp64 with the fp16 rounding points of the kernels."""
    a = x16.astype(np.float64)
    acts = []
    wo = bo = 0
    for l, (o, i) in enumerate(layer_shapes(inD, hid, outD, nl)):
        Wl = W[wo:wo + o * i].astype(np.float16).astype(np.float64).reshape(o, i)
        bl = B[bo:bo + o].astype(np.float64)
        wo += o * i
        bo += o
        z = (a @ Wl.T).astype(np.float32).astype(np.float64) + bl if round16 else a @ Wl.T + bl
        if l < nl - 1:
            z = np.maximum(z, 0.0)
            if round16:
                z = z.astype(np.float32).astype(np.float16).astype(np.float64)
            acts.append(z)
            a = z
        else:
            if out_act == 1:
                z = 1.0 / (1.0 + np.exp(-z))
            return z, acts


def np_backward(dy16, x16, acts, W, inD, hid, outD, nl, round16=True):
    """G_{l-1} = mask(G_l W_l); dW_l = G_l^T X_l; db_l = colsum G_l (fp64)."""
    shapes = layer_shapes(inD, hid, outD, nl)
    offs = np.cumsum([0] + [o * i for o, i in shapes])
    ins = [x16.astype(np.float64)] + acts
    G = dy16.astype(np.float64)
    dW = [None] * nl
    dB = [None] * nl
    dx = None
    for l in range(nl - 1, -1, -1):
        o, i = shapes[l]
        Wl = W[offs[l]:offs[l + 1]].astype(np.float16).astype(np.float64).reshape(o, i)
        dW[l] = G.T @ ins[l]
        dB[l] = G.sum(0)
        d = G @ Wl
        if round16:
            d = d.astype(np.float32).astype(np.float16).astype(np.float64)
        if l > 0:
            G = np.where(ins[l] > 0, d, 0.0)
        else:
            dx = d
    return np.concatenate([w.ravel() for w in dW]), np.concatenate(dB), dx


@pytest.mark.parametrize("inD,hid,outD,nl,act", [(32, 64, 16, 2, 0), (32, 64, 8, 3, 1), (16, 32, 16, 4, 0),
                                                 (8, 16, 8, 2, 1)])
def test_forward_matches_numpy(inD, hid, outD, nl, act):
    rng = np.random.default_rng(inD + hid + nl)
    W, B = make_mlp(inD, hid, outD, nl, seed=3, bias_scale=0.1)
    x = rng.standard_normal((512, inD)).astype(np.float16)
    y, acts = orc.mlp_forward(x, W, B, inD, hid, outD, nl, out_act=act)
    y_np, acts_np = np_forward(x, W, B, inD, hid, outD, nl, out_act=act)
    np.testing.assert_allclose(y, y_np, rtol=1e-5, atol=1e-6)
    for l in range(nl - 1):
        # same fp16 rounding point: equal except for rare fp32 tie flips
        d = np.abs(acts[l].astype(np.float64) - acts_np[l])
        assert (d <= 1e-3 * np.abs(acts_np[l]) + 1e-7).all()


def test_numpy_backward_is_the_gradient():
    """Finite differences of the unrounded fp64 network pin np_backward's chain rule."""
    inD, hid, outD, nl = 8, 16, 4, 3
    rng = np.random.default_rng(1)
    W, B = make_mlp(inD, hid, outD, nl, seed=2, bias_scale=0.3)
    W = W.astype(np.float16).astype(np.float32)
    x = rng.standard_normal((6, inD)).astype(np.float16)
    c = rng.standard_normal((6, outD))
    y, acts = np_forward(x, W, B, inD, hid, outD, nl, round16=False)
    dW, dB, dx = np_backward(c, x, acts, W, inD, hid, outD, nl, round16=False)
    # d/dW of sum(c * y), central differences in fp64 (kept off ReLU kinks by small h)
    Wd = W.astype(np.float64)
    h = 1e-6
    for k in rng.choice(W.size, 25, replace=False):
        Wp, Wm = Wd.copy(), Wd.copy()
        Wp[k] += h
        Wm[k] -= h
        fp = np.sum(c * _fwd64(x, Wp, B, inD, hid, outD, nl))
        fm = np.sum(c * _fwd64(x, Wm, B, inD, hid, outD, nl))
        assert abs((fp - fm) / (2 * h) - dW[k]) < 1e-5 * max(1, abs(dW[k]))


def _fwd64(x, W, B, inD, hid, outD, nl):
    a = x.astype(np.float64)
    wo = bo = 0
    for l, (o, i) in enumerate(layer_shapes(inD, hid, outD, nl)):
        z = a @ W[wo:wo + o * i].reshape(o, i).T + B[bo:bo + o]
        wo += o * i
        bo += o
        a = np.maximum(z, 0) if l < nl - 1 else z
    return a


@pytest.mark.parametrize("inD,hid,outD,nl", [(32, 64, 16, 2), (32, 64, 8, 3), (16, 32, 16, 4)])
def test_backward_matches_numpy(inD, hid, outD, nl):
    rng = np.random.default_rng(7)
    W, B = make_mlp(inD, hid, outD, nl, seed=5, bias_scale=0.1)
    x = rng.standard_normal((1024, inD)).astype(np.float16)
    y, acts = orc.mlp_forward(x, W, B, inD, hid, outD, nl)
    dy = (rng.standard_normal((1024, outD)) * 8).astype(np.float16)
    dW, dB, dx = orc.mlp_backward(dy, x, acts, W, inD, hid, outD, nl)
    acts64 = [a.astype(np.float64) for a in acts[:nl - 1]]
    dW_np, dB_np, dx_np = np_backward(dy, x, acts64, W, inD, hid, outD, nl)
    np.testing.assert_allclose(dW, dW_np, rtol=2e-3, atol=2e-3)
    np.testing.assert_allclose(dB, dB_np, rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(dx.astype(np.float64), dx_np, rtol=1e-2, atol=2e-3)


def test_backward_accumulates():
    inD, hid, outD, nl = 32, 64, 16, 2
    rng = np.random.default_rng(2)
    W, B = make_mlp(inD, hid, outD, nl, seed=5)
    x = rng.standard_normal((64, inD)).astype(np.float16)
    _, acts = orc.mlp_forward(x, W, B, inD, hid, outD, nl)
    dy = rng.standard_normal((64, outD)).astype(np.float16)
    dW1, dB1, _ = orc.mlp_backward(dy, x, acts, W, inD, hid, outD, nl)
    dW2, dB2, _ = orc.mlp_backward(dy, x, acts, W, inD, hid, outD, nl, dW=dW1.copy(), dB=dB1.copy())
    np.testing.assert_allclose(dW2, 2 * dW1, rtol=1e-6)


@pytest.mark.parametrize("act", [0, 1])
def test_mse_closed_form(act):
    rng = np.random.default_rng(4)
    N, P, V, scale = 300, 8, 3, 128.0
    pred = rng.random((N, P), dtype=np.float32)
    tgt = rng.random((N, P), dtype=np.float32).astype(np.float16)
    tot, d = orc.mse_loss_grad(pred, tgt, V, scale, out_act=act)
    gs = np.float32(np.float32(2.0) / np.float32(N * V)) * np.float32(scale)
    diff = np.where(np.arange(P)[None, :] < V, pred - tgt.astype(np.float32), np.float32(0)).astype(np.float32)
    g = (diff * gs).astype(np.float32)
    if act:
        g = (g * (pred * (np.float32(1) - pred)).astype(np.float32)).astype(np.float32)
    np.testing.assert_array_equal(d.view(np.uint16), g.astype(np.float16).view(np.uint16))
    assert abs(tot - float(np.sum((diff * diff).astype(np.float64)))) < 1e-9 * max(1, tot)
    assert (d[:, V:] == 0).all()


def np_adam(w, g, m, v, lr, b1, b2, eps, bc1, bc2, ils):
    f = np.float32
    g = (g * f(ils)).astype(f)
    g = np.where(np.isfinite(g), g, f(0))
    m = np.where(np.isfinite(m), m, f(0))
    v = np.where(np.isfinite(v), v, f(0))
    w = np.where(np.isfinite(w), w, f(0))
    m = (f(b1) * m + (f(1) - f(b1)) * g).astype(f)
    v = (f(b2) * v + ((f(1) - f(b2)) * g) * g).astype(f)
    mh = (m / f(bc1)).astype(f)
    vh = (v / f(bc2)).astype(f)
    w = (w - ((f(lr) * mh) / (np.sqrt(vh) + f(eps)))).astype(f)
    w = np.where(np.isfinite(w), w, f(0))
    return w, m, v


def test_adam_dense_matches_numpy_bitwise_100_steps():
    rng = np.random.default_rng(8)
    n = 5000
    w = rng.standard_normal(n).astype(np.float32)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    wn, mn, vn = w.copy(), m.copy(), v.copy()
    for step in range(1, 101):
        g = (rng.standard_normal(n) * 100).astype(np.float32)
        bc1, bc2 = orc.adam_bias_corrections(0.9, 0.99, step)
        w16 = orc.adam_dense(w, g.copy(), m, v, 1e-2, 0.9, 0.99, 1e-15, bc1, bc2, 1 / 128.0)
        wn, mn, vn = np_adam(wn, g, mn, vn, 1e-2, 0.9, 0.99, 1e-15, bc1, bc2, np.float32(1 / 128.0))
    np.testing.assert_array_equal(w.view(np.uint32), wn.view(np.uint32))
    np.testing.assert_array_equal(m.view(np.uint32), mn.view(np.uint32))
    np.testing.assert_array_equal(w16.view(np.uint16), w.astype(np.float16).view(np.uint16))


def test_adam_matches_kingma_ba_in_fp64():
    """Textbook Adam (fp64, no rescaling rules) agrees to 1e-5 over 100 steps."""
    rng = np.random.default_rng(12)
    n = 1000
    w = rng.standard_normal(n).astype(np.float32)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    w64, m64, v64 = w.astype(np.float64), np.zeros(n), np.zeros(n)
    for t in range(1, 101):
        g = rng.standard_normal(n).astype(np.float32)
        bc1, bc2 = orc.adam_bias_corrections(0.9, 0.999, t)
        orc.adam_dense(w, g, m, v, 1e-3, 0.9, 0.999, 1e-8, bc1, bc2, 1.0, want_f16=False)
        m64 = 0.9 * m64 + 0.1 * g
        v64 = 0.999 * v64 + 0.001 * g.astype(np.float64) ** 2
        w64 -= 1e-3 * (m64 / (1 - 0.9 ** t)) / (np.sqrt(v64 / (1 - 0.999 ** t)) + 1e-8)
    np.testing.assert_allclose(w, w64, rtol=1e-5, atol=1e-6)


def test_adam_hash_skips_zero_and_clears_grad():
    n = 8
    w = np.arange(n, dtype=np.float32)
    g = np.array([0, 1, 0, -2, np.nan, np.inf, -0.0, 3], np.float32)
    m = np.full(n, 0.5, np.float32)
    v = np.full(n, 0.25, np.float32)
    w0, m0, v0 = w.copy(), m.copy(), v.copy()
    orc.adam_hash(w, g, m, v, 0.1, 0.9, 0.99, 1e-8, 0.1, 0.01, 1.0)
    for i in (0, 2, 6):   # exact zeros (incl. -0.0) untouched, grad left as is
        assert w[i] == w0[i] and m[i] == m0[i] and v[i] == v0[i]
    assert np.signbit(g[6])
    for i in (1, 3, 4, 5, 7):
        assert g[i] == 0.0
    # non-finite gradients are treated as 0 but still decay the moments
    assert m[4] == np.float32(np.float32(0.9) * np.float32(0.5))
    assert m[5] == m[4]


def test_adam_self_heals_nonfinite_state():
    w = np.array([np.nan, 1.0, np.inf], np.float32)
    g = np.ones(3, np.float32)
    m = np.array([np.nan, np.inf, 0.0], np.float32)
    v = np.array([np.inf, np.nan, 0.0], np.float32)
    orc.adam_dense(w, g, m, v, 1e-3, 0.9, 0.999, 1e-8, 0.1, 0.001, 1.0, want_f16=False)
    assert np.isfinite(w).all() and np.isfinite(m).all() and np.isfinite(v).all()


def test_adam_step_cap():
    assert orc.adam_bias_corrections(0.9, 0.999, 60000) == orc.adam_bias_corrections(0.9, 0.999, 50000)
    c1, c2 = orc.adam_bias_corrections(0.9, 0.999, 1)
    assert c1 == np.float32(1) - np.float32(0.9) and abs(c2 - 0.001) < 1e-7
