"""Shared helpers for the parity tests (tolerances, seeded inputs)."""
from __future__ import annotations

import importlib

import numpy as np

# Tolerance for fp16-in / fp32-accumulate results.
ATOL = 2e-3
RTOL = 1e-2


def pkg():
    return importlib.import_module("3dmaker_amd")


def assert_close(actual, expected, atol=ATOL, rtol=RTOL, what=""):
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, f"{what}: shape {a.shape} vs {e.shape}"
    excess = np.abs(a - e) - (atol + rtol * np.abs(e))
    bad = excess > 0
    if bad.any():
        i = np.unravel_index(np.argmax(excess), a.shape)
        raise AssertionError(f"{what}: {bad.sum()} of {a.size} outside atol={atol} rtol={rtol}; "
                             f"worst at {i}: got {a[i]!r} expected {e[i]!r}")


def scatter_quantum(denc, L, T, N=None):
    """Per gradient word [L * T * 2], an upper bound on the binned scatter's fixed-point quantum 2^-e of the
    word's level: e = min(49, 60 - ceil(log2(records of the bin))) - E, E the exponent of the level's
    largest fp16 |dL/denc| (non-finite ones count as 2^15), and a bin holds at most 4 records per sample."""
    d = np.ascontiguousarray(denc, np.float16).reshape(-1, L, 2).view(np.uint16) & 0x7fff
    ex = ((d.max(axis=(0, 2)) >> 10) & 31).astype(np.int64)
    E = np.where(ex == 0, -15, np.minimum(ex - 15, 15))
    n = d.shape[0] if N is None else N
    lg = int(np.ceil(np.log2(max(4 * n, 2))))
    return np.repeat(np.ldexp(1.0, E - min(49, 60 - lg)), 2 * T)


def scatter_bound(g, gabs, cnt, quantum=None, extra_roundings=0):
    """Per gradient word, the bound on |binned scatter - oracle| given the oracle's sum (g), sum of
    |products| (gabs) and product count (cnt) of the word (pyoracle.hash_scatter_stats).  Both sides form
    the reference's fp32 products g_f * ((wx * wy) * wz) bit for bit, so only the sums differ:

    - each side rounds its sum to fp32 once: 2^-23 |g| (the oracle's fp64 sum of the products is exact to
      cnt * 2^-52 gabs);
    - the fixed-point sums, cnt / 2 times the smaller of the level's quantum (scatter_quantum; each
      product is within half of it) and 2^-24 gabs (a sum of at least 2^24 quanta has each product within
      2^-25 of the sum, products of at least 2^24 quanta each are within 2^-25 of the smallest; the other
      sums are summed again at the word's own scale, where a product is within 2^-37 of the word's largest
      product for bins of up to 2^22 records);
    - extra_roundings fp32 roundings of gabs for additions the caller makes (sub-batches added one after
      another).
    """
    ga = gabs.astype(np.float64)
    per = np.ldexp(ga, -24)
    if quantum is not None:
        per = np.minimum(per, quantum)
    c = cnt.astype(np.float64)
    return (np.ldexp(np.abs(g.astype(np.float64)), -23) + np.ldexp(extra_roundings + c * 2.0 ** -28, -24) * ga
            + 0.5 * c * per)


def assert_scatter_close(got, want, bound, base=0.0, what=""):
    """got / want: gradient arrays that held `base` before the scatter added to it; every word within its
    bound (plus the fp32 rounding of the addition to a nonzero base)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    allow = bound + (np.ldexp(np.abs(want), -23) if base else 0.0)
    err = np.abs(got - want)
    bad = err > allow
    if bad.any():
        i = int(np.argmax(np.where(bad, err / np.maximum(allow, 1e-300), 0)))
        raise AssertionError(f"{what}: {int(bad.sum())} of {got.size} words outside the per-word bound; worst at "
                             f"{i}: got {got[i]!r} expected {want[i]!r} bound {allow[i]!r}")


def positions(n, seed, stride=4):
    rng = np.random.default_rng(seed)
    p = np.zeros((n, stride), np.float32)
    p[:, :3] = rng.random((n, 3), dtype=np.float32)
    return p


def xavier(fan_in, fan_out, rng):
    bnd = np.sqrt(6.0 / (fan_in + fan_out))
    return rng.uniform(-bnd, bnd, (fan_out, fan_in)).astype(np.float32)


def layer_shapes(inD, hid, outD, nl):
    return [((outD if l == nl - 1 else hid), (inD if l == 0 else hid)) for l in range(nl)]


def make_mlp(inD, hid, outD, nl, seed, bias_scale=0.0):
    rng = np.random.default_rng(seed)
    ws, bs = [], []
    for o, i in layer_shapes(inD, hid, outD, nl):
        ws.append(xavier(i, o, rng).ravel())
        bs.append((rng.uniform(-1, 1, o) * bias_scale).astype(np.float32))
    return np.concatenate(ws), np.concatenate(bs)


# ---- raw HIP memory plumbing for reading library-owned buffers in GPU tests ----
_HIP = None


def hip():
    import ctypes as C
    global _HIP
    if _HIP is None:
        L = C.CDLL("libamdhip64.so")
        L.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        L.hipMemcpy.restype = C.c_int
        L.hipDeviceSynchronize.restype = C.c_int
        _HIP = L
    return _HIP


def d2h(ptr, shape, dtype):
    """Copy a device buffer (raw pointer) into a new numpy array."""
    out = np.empty(shape, dtype)
    if out.nbytes:
        rc = hip().hipMemcpy(out.ctypes.data, int(ptr), out.nbytes, 2)
        assert rc == 0, f"hipMemcpy D2H failed: {rc}"
    return out


def h2d(ptr, arr):
    arr = np.ascontiguousarray(arr)
    rc = hip().hipMemcpy(int(ptr), arr.ctypes.data, arr.nbytes, 1)
    assert rc == 0, f"hipMemcpy H2D failed: {rc}"


def ptr_array(dev_ptr_of_ptrs, count):
    """Read a device array of device pointers."""
    return [int(p) for p in d2h(dev_ptr_of_ptrs, (count,), np.uint64)]
