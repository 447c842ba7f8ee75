"""numpy bindings of the C oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product package.  fp16 arrays are
numpy float16 (their bit patterns are what the C code reads and writes).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")


def build(force: bool = False) -> str:
    path = os.path.join(_HERE, "liboracle.so")
    if force or not os.path.exists(path):
        subprocess.run(["make", "-C", _HERE, "-B" if force else "liboracle.so"],
                       check=True, stdout=subprocess.DEVNULL)
    return path


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        L = C.CDLL(path)
        i, f, d, sz = C.c_int, C.c_float, C.c_double, C.c_size_t
        sig = {
            "orc_f32_to_f16": (C.c_uint16, [f]),
            "orc_f16_to_f32": (f, [C.c_uint16]),
            "orc_hash_coords": (C.c_uint32, [i, i, i, i]),
            "orc_dense_index": (C.c_uint32, [i, i, i, i]),
            "orc_dense_level_start": (i, [i, i, f, i]),
            "orc_level_scales": (None, [i, f, i, _f32p, np.ctypeslib.ndpointer(np.int32)]),
            "orc_hash_corners": (None, [_f32p, i, i, i, i, i, f, i, _u32p, _f32p]),
            "orc_hash_encode_fwd": (None, [_f32p, i, i, _u16p, i, i, i, f, _u16p]),
            "orc_hash_scatter_bwd": (None, [_f32p, i, i, _u16p, i, i, i, f, _f32p]),
            "orc_hash_scatter_stats": (None, [_f32p, i, i, _u16p, i, i, i, f, _f32p, _f32p, _u32p]),
            "orc_mlp_forward": (None, [_u16p, i, i, i, i, i, _u16p, _f32p, i, C.c_void_p, _f32p]),
            "orc_mlp_backward": (None, [_u16p, _u16p, C.c_void_p, i, i, i, i, i, _u16p,
                                        _f32p, _f32p, C.c_void_p]),
            "orc_mse_loss_grad": (d, [_f32p, _u16p, _u16p, i, i, i, f, i]),
            "orc_adam_dense": (None, [_f32p, C.c_void_p, _f32p, _f32p, _f32p, sz,
                                      f, f, f, f, f, f, f]),
            "orc_adam_hash": (None, [_f32p, C.c_void_p, _f32p, _f32p, _f32p, sz,
                                     f, f, f, f, f, f, f]),
            "orc_adam_bias_corrections": (None, [f, f, i, C.POINTER(f), C.POINTER(f)]),
            "orc_expf": (f, [f]),
            "orc_expf_array": (None, [_f32p, _f32p, sz]),
            "orc_get_cascade": (i, [_f32p, _f32p, _f32p, i]),
            "orc_contract_pos": (None, [_f32p, _f32p, _f32p, _f32p]),
            "orc_pyramid_cells": (C.c_uint32, [_u32p, i]),
            "orc_ray_aabb_inv": (None, [C.c_uint32, _f32p, _f32p, _f32p, _f32p, i, _f32p, _f32p, _f32p]),
            "orc_march_count": (None, [C.c_uint32, _f32p, _f32p, _f32p, _f32p, _f32p, _u8p, _u32p, _f32p,
                                       _f32p, i, i, i, _u32p]),
            "orc_march_hits": (C.c_uint32, [C.c_uint32, _f32p, _f32p, _f32p, _f32p, _f32p, _u8p, _u32p, _f32p,
                                            _f32p, i, i, i, C.c_uint32, _u32p, _u32p, C.POINTER(C.c_uint32),
                                            _f32p, _u32p, _f32p]),
            "orc_march_fill": (None, [C.c_uint32, _f32p, _f32p, _f32p, _f32p, _f32p, _u8p, _u32p, _f32p,
                                      _f32p, i, i, i, _u32p, _f32p, _u32p, _f32p]),
            "orc_march_sparse": (None, [C.c_uint32, _f32p, _f32p, _f32p, _f32p, _f32p, _u8p, _u32p, _f32p,
                                        _f32p, i, i, i, _u32p, _f32p, C.c_void_p]),
            "orc_morton30": (C.c_uint32, [C.c_uint32, C.c_uint32, C.c_uint32]),
            "orc_sparse_batch": (None, [C.c_uint32, _u32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _u32p, _f32p]),
            "orc_sh_degree3": (None, [C.c_uint32, _f32p, _f32p]),
            "orc_sh_gather": (None, [C.c_uint32, _f32p, _u32p, f, _f32p, _u16p, _f32p]),
            "orc_composite_distortion": (None, [C.c_uint32, _u32p, _u32p, _f32p, _f32p, C.c_void_p, C.c_void_p,
                                                _f32p, C.c_void_p, _f32p, _f32p, C.c_void_p, _f32p, _f32p, f, f,
                                                _f32p]),
            "orc_composite_infer": (None, [C.c_uint32, C.c_uint32, C.c_uint32, _u32p, _u32p, _f32p, _f32p, _f32p,
                                           i, C.c_void_p, _f32p, _f32p, C.c_void_p, _f32p]),
            "orc_color_grad": (None, [C.c_uint32, _u32p, _u32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p,
                                      _u16p, _f32p, f, f, C.c_uint32]),
            "orc_density_grad": (None, [C.c_uint32, _f32p, _u16p, _u16p]),
            "orc_update_master_grid": (None, [_f32p, _f32p, f, C.c_uint32]),
            "orc_philox4x32_10": (None, [_u32p, C.c_uint32, C.c_uint32]),
            "orc_occ_sample": (None, [_f32p, i, i, i, i, C.c_void_p, i, C.c_uint64, _u32p, _f32p, _f32p]),
            "orc_occ_tmp_max": (None, [_f32p, _f32p, _f32p, f, i]),
            "orc_update_occupancy_bits": (None, [_u8p, _f32p, f, i, i, i, f, f]),
            "orc_build_mipmaps": (None, [_u8p, _u32p, i, i]),
            "orc_pcg_hash": (C.c_uint32, [C.c_uint32]),
            "orc_fetch_ray_chunk": (None, [i, i, i, C.c_uint32, i, i, i, f, _f32p, _u8p, _f32p, _f32p, _f32p,
                                           C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                           C.c_void_p, C.c_uint32, f, f, f, _f32p, i]),
            "orc_num_threads": (i, []),
            "orc_set_num_threads": (None, [i]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def _h(a):
    """float16 array -> uint16 view (C-contiguous)."""
    return np.ascontiguousarray(a, dtype=np.float16).view(np.uint16)


def _vp(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def f32_to_f16_bits(x: float) -> int:
    return lib().orc_f32_to_f16(float(x))


def hash_coords(cx, cy, cz, T):
    return lib().orc_hash_coords(int(cx), int(cy), int(cz), int(T))


def dense_index(cx, cy, cz, N):
    return lib().orc_dense_index(int(cx), int(cy), int(cz), int(N))


def dense_level_start(T, base, b, L):
    return lib().orc_dense_level_start(int(T), int(base), float(b), int(L))


def level_scales(base, b, L):
    s = np.zeros(L, np.float32)
    r = np.zeros(L, np.int32)
    lib().orc_level_scales(int(base), float(b), int(L), s, r)
    return s, r


def _pos(pos):
    pos = np.ascontiguousarray(pos, dtype=np.float32)
    assert pos.ndim == 2 and pos.shape[1] in (3, 4)
    return pos, pos.shape[1]


def hash_corners(pos, T, L, base, b, bwd_clamp=False):
    pos, st = _pos(pos)
    N = pos.shape[0]
    idx = np.zeros((N, L, 8), np.uint32)
    w = np.zeros((N, L, 8), np.float32)
    lib().orc_hash_corners(pos, st, N, T, L, base, float(b), int(bwd_clamp), idx, w)
    return idx, w


def hash_encode(pos, table, T, L, base, b):
    """table: float16 [L*T*2]; returns float16 [N, 2L]."""
    pos, st = _pos(pos)
    N = pos.shape[0]
    out = np.zeros((N, 2 * L), np.uint16)
    lib().orc_hash_encode_fwd(pos, st, N, _h(table).ravel(), T, L, base, float(b), out)
    return out.view(np.float16)


def hash_scatter(pos, denc, T, L, base, b, grads=None):
    pos, st = _pos(pos)
    N = pos.shape[0]
    g = np.zeros(L * T * 2, np.float32) if grads is None else grads
    lib().orc_hash_scatter_bwd(pos, st, N, _h(denc).ravel(), T, L, base, float(b), g)
    return g


def hash_scatter_stats(pos, denc, T, L, base, b):
    """(grads, sum of |products|, product count) per gradient word, each [L * T * 2]."""
    pos, st = _pos(pos)
    N = pos.shape[0]
    g = np.empty(L * T * 2, np.float32)
    ga = np.empty(L * T * 2, np.float32)
    cnt = np.empty(L * T * 2, np.uint32)
    lib().orc_hash_scatter_stats(pos, st, N, _h(denc).ravel(), T, L, base, float(b), g, ga, cnt)
    return g, ga, cnt


def _layer_shapes(inD, hid, outD, nl):
    shapes = []
    for l in range(nl):
        shapes.append((outD if l == nl - 1 else hid, inD if l == 0 else hid))
    return shapes


def mlp_forward(x, W, B, inD, hid, outD, nl, out_act=0, save_acts=True):
    """x float16 [N,in]; W flat float16; B flat float32 -> (y f32 [N,out], acts f16 [nl-1,N,hid])."""
    N = x.shape[0]
    y = np.zeros((N, outD), np.float32)
    acts = np.zeros((max(nl - 1, 1), N, hid), np.uint16) if save_acts else None
    lib().orc_mlp_forward(_h(x).ravel(), N, inD, hid, outD, nl, _h(W).ravel(),
                          np.ascontiguousarray(B, np.float32), int(out_act), _vp(acts), y)
    return y, (acts.view(np.float16) if acts is not None else None)


def mlp_backward(dy, x0, acts, W, inD, hid, outD, nl, dW=None, dB=None, want_dx=True):
    N = dy.shape[0]
    wtot = sum(o * i for o, i in _layer_shapes(inD, hid, outD, nl))
    btot = sum(o for o, _ in _layer_shapes(inD, hid, outD, nl))
    dW = np.zeros(wtot, np.float32) if dW is None else dW
    dB = np.zeros(btot, np.float32) if dB is None else dB
    dx = np.zeros((N, inD), np.uint16) if want_dx else None
    a = _h(acts) if acts is not None else None
    lib().orc_mlp_backward(_h(dy).ravel(), _h(x0).ravel(), _vp(a), N, inD, hid, outD, nl,
                           _h(W).ravel(), dW, dB, _vp(dx))
    return dW, dB, (dx.view(np.float16) if dx is not None else None)


def mse_loss_grad(pred, tgt, valid, loss_scale, out_act=0):
    pred = np.ascontiguousarray(pred, np.float32)
    N, P = pred.shape
    d = np.zeros((N, P), np.uint16)
    tot = lib().orc_mse_loss_grad(pred, _h(tgt).ravel(), d, N, P, valid, float(loss_scale), int(out_act))
    return tot, d.view(np.float16)


def adam_dense(w, g, m, v, lr, b1, b2, eps, bc1, bc2, inv_scale, want_f16=True):
    w16 = np.zeros(w.size, np.uint16) if want_f16 else None
    lib().orc_adam_dense(w, _vp(w16), g, m, v, w.size, lr, b1, b2, eps, bc1, bc2, inv_scale)
    return None if w16 is None else w16.view(np.float16)


def adam_hash(w, g, m, v, lr, b1, b2, eps, bc1, bc2, inv_scale, want_f16=True, w16_init=None):
    """Entries with g == 0 keep their fp16 copy: pass the current fp16 table as
    w16_init to get the full post-step fp16 table (zeros otherwise)."""
    if w16_init is not None:
        w16 = _h(w16_init).copy().ravel()
    else:
        w16 = np.zeros(w.size, np.uint16) if want_f16 else None
    lib().orc_adam_hash(w, _vp(w16), g, m, v, w.size, lr, b1, b2, eps, bc1, bc2, inv_scale)
    return None if w16 is None else w16.view(np.float16)


def adam_bias_corrections(b1, b2, step):
    c1, c2 = C.c_float(), C.c_float()
    lib().orc_adam_bias_corrections(float(b1), float(b2), int(step), C.byref(c1), C.byref(c2))
    return c1.value, c2.value


def num_threads():
    return lib().orc_num_threads()


def set_num_threads(n):
    lib().orc_set_num_threads(int(n))


# ---------------------------------------------------------------------------
# NeRF side (oracle/nerf_oracle.h)
# ---------------------------------------------------------------------------
MAX_HITS = 1024


def _f3(a):
    return np.ascontiguousarray(a, np.float32).reshape(-1)


def expf(x):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().orc_expf_array(x.ravel(), y.ravel(), x.size)
    return y


def get_cascade(pos, aabb_min, aabb_max, cascades):
    return lib().orc_get_cascade(_f3(pos), _f3(aabb_min), _f3(aabb_max), int(cascades))


def contract_pos(pos, aabb_min, aabb_max):
    out = np.zeros(3, np.float32)
    lib().orc_contract_pos(_f3(pos), _f3(aabb_min), _f3(aabb_max), out)
    return out


def pyramid_cells(res, levels):
    return lib().orc_pyramid_cells(np.ascontiguousarray(res, np.uint32), int(levels))


def grid_bytes(res, levels, cascades):
    return (pyramid_cells(res, levels) * cascades + 7) // 8


def ray_aabb_inv(o, d, aabb_min, aabb_max, cascades):
    o, d = _f3(o), _f3(d)
    R = o.size // 3
    di = np.zeros(3 * R, np.float32)
    nr = np.zeros(R, np.float32)
    fr = np.zeros(R, np.float32)
    lib().orc_ray_aabb_inv(R, o, d, _f3(aabb_min), _f3(aabb_max), int(cascades), di, nr, fr)
    return di.reshape(R, 3), nr, fr


def march_count(o, d, di, nears, fars, bits, res, aabb_min, aabb_max, cascades, L, K):
    R = _f3(o).size // 3
    cnt = np.zeros(R, np.uint32)
    lib().orc_march_count(R, _f3(o), _f3(d), _f3(di), _f3(nears), _f3(fars), np.ascontiguousarray(bits, np.uint8),
                          np.ascontiguousarray(res, np.uint32), _f3(aabb_min), _f3(aabb_max), int(cascades),
                          int(L), int(K), cnt)
    return cnt


def march_hits(o, d, di, nears, fars, bits, res, aabb_min, aabb_max, cascades, L, K, batch):
    """processRaysHitLinear -> dict(active, total, counts, offsets, t, ray_idx, pos[N,4])."""
    R = _f3(o).size // 3
    cnt = np.zeros(R, np.uint32)
    off = np.zeros(R, np.uint32)
    tot = C.c_uint32(0)
    need = int(march_count(o, d, di, nears, fars, bits, res, aabb_min, aabb_max, cascades, L, K).sum(dtype=np.int64))
    cap = max(min(int(batch), need), 1)
    t = np.zeros(cap, np.float32)
    ri = np.zeros(cap, np.uint32)
    pos = np.zeros(4 * cap, np.float32)
    act = lib().orc_march_hits(R, _f3(o), _f3(d), _f3(di), _f3(nears), _f3(fars),
                               np.ascontiguousarray(bits, np.uint8), np.ascontiguousarray(res, np.uint32),
                               _f3(aabb_min), _f3(aabb_max), int(cascades), int(L), int(K), int(batch), cnt, off,
                               C.byref(tot), t, ri, pos)
    n = tot.value
    return dict(active=int(act), total=int(n), counts=cnt, offsets=off, t=t[:n], ray_idx=ri[:n],
                pos=pos.reshape(-1, 4)[:n])


def exclusive_scan_u32(counts):
    """custom_exclusive_sum (processRays.cu:486-549): exclusive prefix sums, uint32 wrap-around."""
    c = np.ascontiguousarray(counts, np.uint32)
    out = np.zeros_like(c)
    if c.size > 1:
        out[1:] = np.cumsum(c[:-1], dtype=np.uint64).astype(np.uint32)
    return out


def hit_data(o, d, di, nears, fars, bits, res, aabb_min, aabb_max, cascades, L, K):
    """processRaysHitData (processRays.cu:1042-1081) -> (counts, offsets) over all rays."""
    cnt = march_count(o, d, di, nears, fars, bits, res, aabb_min, aabb_max, cascades, L, K)
    return cnt, exclusive_scan_u32(cnt)


def hit_positions(o, d, di, nears, fars, bits, res, aabb_min, aabb_max, cascades, L, K, counts, offsets,
                  rays_done, batch):
    """processRaysHitPositions (processRays.cu:1083-1174) after hit_data.

    -> dict(rays, next_done, total, base, t, ray_idx (batch-local), pos [total, 4]); rays = 0 (and
    base None) when the first ray from rays_done does not fit or no rays are left.  The cutoff is
    find_cutoff_ray_from_kernel (:771-799): the boundary ray i >= rays_done is the one whose inclusive
    sample count past base fits and whose successor's does not (or that is the last ray)."""
    R = int(np.asarray(counts).size)
    rd = int(rays_done)
    counts = np.ascontiguousarray(counts, np.uint32)
    offsets = np.ascontiguousarray(offsets, np.uint32)
    empty = dict(rays=0, next_done=0, total=0, base=None, t=np.zeros(0, np.float32),
                 ray_idx=np.zeros(0, np.uint32), pos=np.zeros((0, 4), np.float32))
    if rd >= R:
        return empty
    base = offsets[rd]
    incl = (offsets[rd:] + counts[rd:] - base).astype(np.uint32)   # uint32 arithmetic, as on the device
    fits = incl <= np.uint32(batch)
    nxt = np.append(~fits[1:], True)      # successor does not fit, or i is the last ray
    bnd = np.nonzero(fits & nxt)[0]
    if bnd.size == 0:
        return empty
    nb = int(bnd.max()) + 1                # batch rays
    total = int(incl[nb - 1])
    sl = slice(rd, rd + nb)
    t = np.zeros(max(total, 1), np.float32)
    ri = np.zeros(max(total, 1), np.uint32)
    pos = np.zeros(4 * max(total, 1), np.float32)
    ob = (offsets[sl] - base).astype(np.uint32)
    lib().orc_march_fill(nb, _f3(np.asarray(o)[sl]), _f3(np.asarray(d)[sl]), _f3(np.asarray(di)[sl]),
                         _f3(np.asarray(nears)[sl]), _f3(np.asarray(fars)[sl]), np.ascontiguousarray(bits, np.uint8),
                         np.ascontiguousarray(res, np.uint32), _f3(aabb_min), _f3(aabb_max), int(cascades), int(L),
                         int(K), ob, t, ri, pos)
    return dict(rays=nb, next_done=rd + nb, total=total, base=int(base), t=t[:total], ray_idx=ri[:total],
                pos=pos.reshape(-1, 4)[:total])


def march_sparse(o, d, di, nears, fars, bits, res, aabb_min, aabb_max, cascades, L, K, morton=True):
    """launchMarchRaysDDA (processRays.cu:96-265) -> (counts [R], t [R, 1024], morton [R, 1024] or None);
    entries past a ray's count are zero."""
    R = _f3(o).size // 3
    cnt = np.zeros(R, np.uint32)
    t = np.zeros(R * MAX_HITS, np.float32)
    m = np.zeros(R * MAX_HITS, np.uint32) if morton else None
    lib().orc_march_sparse(R, _f3(o), _f3(d), _f3(di), _f3(nears), _f3(fars), np.ascontiguousarray(bits, np.uint8),
                           np.ascontiguousarray(res, np.uint32), _f3(aabb_min), _f3(aabb_max), int(cascades),
                           int(L), int(K), cnt, t, None if m is None else m.ctypes.data_as(C.c_void_p))
    return cnt, t.reshape(R, MAX_HITS), None if m is None else m.reshape(R, MAX_HITS)


def morton30(x, y, z):
    return int(lib().orc_morton30(int(x), int(y), int(z)))


def process_chunk(o, d, di, nears, fars, bits, res, aabb_min, aabb_max, cascades, L, K, sort=True):
    """processRaysChunk (sort, processRays.cu:357-464) / processRaysChunkLinear (:551-624).

    -> dict(counts, offsets, t_sparse, morton, dense_idx (ray-major, ray * 1024 + k), keys_in,
    sorted_idx, keys_out, pos [N, 4], ray_idx, t): every sample of every ray, in ray-major order, or
    stably sorted by Morton code (cub::DeviceRadixSort::SortPairs over 32 bits) when sort."""
    cnt, ts, mor = march_sparse(o, d, di, nears, fars, bits, res, aabb_min, aabb_max, cascades, L, K, morton=sort)
    off = exclusive_scan_u32(cnt)
    rows = np.repeat(np.arange(cnt.size, dtype=np.uint64), cnt.astype(np.int64))
    ks = np.arange(rows.size, dtype=np.uint64) - np.repeat(off.astype(np.uint64), cnt.astype(np.int64))
    dense = (rows * MAX_HITS + ks).astype(np.uint32)
    out = dict(counts=cnt, offsets=off, t_sparse=ts, morton=mor, dense_idx=dense)
    order = dense
    if sort:
        keys = mor.reshape(-1)[dense]
        perm = np.argsort(keys, kind="stable")
        out.update(keys_in=keys, keys_out=keys[perm], sorted_idx=dense[perm])
        order = dense[perm]
    N = int(order.size)
    pos = np.zeros(4 * max(N, 1), np.float32)
    ray = np.zeros(max(N, 1), np.uint32)
    t = np.zeros(max(N, 1), np.float32)
    lib().orc_sparse_batch(N, np.ascontiguousarray(order, np.uint32), np.ascontiguousarray(ts.reshape(-1)), _f3(o),
                           _f3(d), _f3(aabb_min), _f3(aabb_max), pos, ray, t)
    out.update(pos=pos.reshape(-1, 4)[:N], ray_idx=ray[:N], t=t[:N])
    return out


def sh_degree3(dirs):
    """compute_real_sh_degree_3_kernel (otherKernels.cu:18-64) -> [N, 16]."""
    dd = _f3(dirs)
    N = dd.size // 3
    out = np.zeros(16 * max(N, 1), np.float32)
    lib().orc_sh_degree3(N, dd, out)
    return out[:16 * N].reshape(N, 16)


def sh_gather(dirs, ray_idx, density_out, bias=0.0):
    ray_idx = np.ascontiguousarray(ray_idx, np.uint32)
    N = ray_idx.size
    cin = np.zeros((N, 32), np.uint16)
    sig = np.zeros(N, np.float32)
    lib().orc_sh_gather(N, _f3(dirs), ray_idx, float(bias), _f3(density_out), cin, sig)
    return cin.view(np.float16), sig


def composite(offsets, counts, t, sigma, rgb, rgb_true, lambda_dist, bg, depth_prior=None, sigma_prior=None,
              lambda_depth=0.0):
    R = len(counts)
    frgb = np.zeros(3 * R, np.float32)
    fdep = np.zeros(R, np.float32)
    phi = np.zeros(3 * R, np.float32)
    dw = np.zeros(max(len(t), 1), np.float32)
    ws = np.zeros(R, np.float32)
    dp = None if depth_prior is None else _f3(depth_prior)
    sp = None if sigma_prior is None else _f3(sigma_prior)
    rt = None if rgb_true is None else _f3(rgb_true)
    lib().orc_composite_distortion(R, np.ascontiguousarray(offsets, np.uint32), np.ascontiguousarray(counts, np.uint32),
                                   _f3(t) if len(t) else np.zeros(1, np.float32),
                                   _f3(sigma) if len(t) else np.zeros(1, np.float32), _vp(dp), _vp(sp),
                                   _f3(rgb) if len(t) else np.zeros(3, np.float32), _vp(rt), frgb, fdep,
                                   _vp(phi if rt is not None else None), dw, ws, float(lambda_dist),
                                   float(lambda_depth), _f3(bg))
    return dict(rgb=frgb.reshape(R, 3), depth=fdep, phi=phi.reshape(R, 3), dw=dw[:len(t)], weight_sum=ws)


def composite_infer(offsets, counts, t, sigma, rgb, bg, rgb_true=None, base=0, rays_done=0):
    """Inference compositor; offsets indexed from rays_done, counts per ray of this call."""
    R = len(counts)
    rgb = np.ascontiguousarray(rgb, np.float32)
    stride = rgb.shape[1] if rgb.ndim == 2 else 3
    frgb = np.zeros(3 * R, np.float32)
    fdep = np.zeros(R, np.float32)
    phi = np.zeros(3 * R, np.float32)
    rt = None if rgb_true is None else _f3(rgb_true)
    lib().orc_composite_infer(R, int(base), int(rays_done), np.ascontiguousarray(offsets, np.uint32),
                              np.ascontiguousarray(counts, np.uint32),
                              _f3(t) if len(t) else np.zeros(1, np.float32),
                              _f3(sigma) if len(t) else np.zeros(1, np.float32),
                              rgb.reshape(-1) if len(t) else np.zeros(3, np.float32), int(stride), _vp(rt), frgb,
                              fdep, _vp(phi if rt is not None else None), _f3(bg))
    return dict(rgb=frgb.reshape(R, 3), depth=fdep, phi=phi.reshape(R, 3))


def color_grad(counts, offsets, t, density_out, color_out, phi, final_rgb, dw, weight_sum, loss_scale,
               bias, total_rays):
    R = len(counts)
    N = len(t)
    cg = np.zeros((max(N, 1), 3), np.uint16)
    ds = np.zeros(max(N, 1), np.float32)
    lib().orc_color_grad(R, np.ascontiguousarray(counts, np.uint32), np.ascontiguousarray(offsets, np.uint32),
                         _f3(t), _f3(density_out), _f3(color_out), _f3(phi), _f3(final_rgb), _f3(dw),
                         _f3(weight_sum), cg.reshape(-1), ds, float(loss_scale), float(bias), int(total_rays))
    return cg[:N].view(np.float16), ds[:N]


def density_grad(dsigma, color_dx):
    N = len(dsigma)
    out = np.zeros((N, 16), np.uint16)
    lib().orc_density_grad(N, _f3(dsigma), _h(color_dx).reshape(-1), out.reshape(-1))
    return out.view(np.float16)


def update_master_grid(tmp, master, decay):
    lib().orc_update_master_grid(_f3(tmp), master, float(decay), master.size)
    return master


def update_occupancy_bits(bits, master, total_sum, G, S, min_optical, base_voxel):
    lib().orc_update_occupancy_bits(bits, _f3(master), float(total_sum), int(master.size), int(G), int(S),
                                    float(min_optical), float(base_voxel))
    return bits


def build_mipmaps(bits, res, L, cascades):
    lib().orc_build_mipmaps(bits, np.ascontiguousarray(res, np.uint32), int(L), int(cascades))
    return bits


def philox4x32_10(ctr, key):
    c = np.ascontiguousarray(ctr, np.uint32).copy()
    lib().orc_philox4x32_10(c, int(key[0]) & 0xffffffff, int(key[1]) & 0xffffffff)
    return c


# occ_sample modes (otherKernels.cu:591-648, 852-888)
OCC_FROM_LIST, OCC_EVERY_CELL, OCC_RANDOM_CELL = 0, 1, 2


def occ_sample(N, mode, total_cells, cell_offset, seed, res, aabb_min, aabb_max, cell_list=None):
    """-> (positions float32 [N][3] contracted, cells int32 [N]); rows of an empty list stay zero."""
    out = np.zeros((N, 4), np.float32)
    lst = None if cell_list is None else np.ascontiguousarray(cell_list, np.int32)
    lib().orc_occ_sample(out, int(N), int(mode), int(total_cells), int(cell_offset),
                         None if lst is None else lst.ctypes.data, 0 if lst is None else int(lst.size),
                         int(seed) & 0xffffffffffffffff, np.ascontiguousarray(res, np.uint32), _f3(aabb_min),
                         _f3(aabb_max))
    return out, out[:, 3].copy().view(np.int32)


def occ_tmp_max(samples4, density_out, tmp, bias):
    lib().orc_occ_tmp_max(np.ascontiguousarray(samples4, np.float32), np.ascontiguousarray(density_out, np.float32),
                          tmp, float(bias), int(samples4.shape[0]))
    return tmp


def active_cells(bits, G, S, cascades):
    """Cells (cascade * G + local) whose level-0 bit is set, in cell order (extractActiveCells,
    otherKernels.cu:809-834; the reference appends with an atomic counter, this build in order)."""
    b = np.unpackbits(np.ascontiguousarray(bits, np.uint8), bitorder="little")
    cells = []
    for c in range(cascades):
        lvl0 = b[c * S: c * S + G]
        cells.append(np.nonzero(lvl0)[0].astype(np.int64) + c * G)
    return np.concatenate(cells).astype(np.int32)


def refresh_schedule(train_steps, cascades, G):
    """The occupancy refresh's sampling calls (InstantNerf.cu:1009-1171): a list of chunks, each a list of
    (mode, N, total_cells, cell_offset, seed); early (< 256 steps) = every cell of each cascade, late = half
    the cells' worth per refresh split over `cascades` chunks, half from the occupied list, half uniform."""
    if train_steps < 256:
        return [[(OCC_EVERY_CELL, G, G, c * G, train_steps + c)] for c in range(cascades)]
    N = cascades * G
    per = (N // 2) // cascades
    occ = per // 2
    uni = per - occ
    out = []
    for ch in range(cascades):
        seed = train_steps * (2 * cascades) + 2 * ch
        out.append([(OCC_FROM_LIST, occ, 0, 0, seed), (OCC_RANDOM_CELL, uni, N, 0, seed + 1)])
    return out


def pcg_hash(x):
    return lib().orc_pcg_hash(int(x) & 0xffffffff)


def fetch_ray_chunk(offset, size, seed, randomize, transforms, images_rgba, focal, bg, holdout_every=0,
                    records=None, dense_fraction=0.0, uv_scale=(1.0, 1.0)):
    """images_rgba uint8 [n, h, w, 4]; transforms float32 [n, 16]; records = dict(frame, u, v, D, sigma)."""
    imgs = np.ascontiguousarray(images_rgba, np.uint8)
    n, h, w = imgs.shape[:3]
    o = np.zeros((size, 3), np.float32)
    d = np.zeros((size, 3), np.float32)
    rgb = np.zeros((size, 3), np.float32)
    dense = np.zeros(size, np.float32)
    sig = np.zeros(size, np.float32)
    if records is None:
        rec = [None] * 5
        nrec = 0
    else:
        rec = [np.ascontiguousarray(records["frame"], np.int32)] + \
              [np.ascontiguousarray(records[k], np.float32) for k in ("u", "v", "D", "sigma")]
        nrec = len(rec[0])
    lib().orc_fetch_ray_chunk(int(offset), int(size), n * h * w, int(seed) & 0xffffffff, int(bool(randomize)), w, h,
                              float(focal), _f3(transforms), imgs.reshape(-1), o, d, rgb, dense.ctypes.data,
                              sig.ctypes.data, *[_vp(r) for r in rec], nrec, float(dense_fraction),
                              float(uv_scale[0]), float(uv_scale[1]), _f3(bg), int(holdout_every))
    return dict(o=o, d=d, rgb=rgb, dense=dense, sigma=sig)
