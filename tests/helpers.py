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
