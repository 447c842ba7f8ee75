"""Pins of the CPU oracle's hash grid (no GPU).

Each check is independent of the oracle's own code path: integer closed
forms computed here by hand or by Python big-int arithmetic, scipy's
RegularGridInterpolator as a textbook trilinear interpolator, and the
adjoint identity that links the encode to the scatter.
"""
import numpy as np
import pytest
from scipy.interpolate import RegularGridInterpolator

import pyoracle as orc

T19, T14 = 1 << 19, 1 << 14


# Known answers computed arithmetically (uint32 prime-XOR hash, masked to T);
# networkFusionHashtable.cu:62-66.
HASH_KAT = [
    ((0, 0, 0), 0, 0),
    ((1, 0, 0), 1, 1),
    ((0, 1, 0), 489905, 14769),
    ((0, 0, 1), 153493, 6037),
    ((1, 2, 3), 128476, 13788),
    ((100, 200, 300), 110768, 12464),
    ((2047, 2047, 2047), 285147, 6619),
    ((4095, 17, 999), 318797, 7501),
]


@pytest.mark.parametrize("c,h19,h14", HASH_KAT)
def test_hash_known_answers(c, h19, h14):
    assert orc.hash_coords(*c, T19) == h19
    assert orc.hash_coords(*c, T14) == h14


def test_hash_matches_bigint_formula():
    rng = np.random.default_rng(3)
    for _ in range(2000):
        x, y, z = (int(v) for v in rng.integers(0, 1 << 20, 3))
        want = ((x * 1) ^ (y * 2654435761) ^ (z * 805459861)) & 0xFFFFFFFF & (T19 - 1)
        assert orc.hash_coords(x, y, z, T19) == want


def test_dense_index_closed_form():
    for N in (16, 22, 58):
        for (x, y, z) in [(0, 0, 0), (N, 0, 0), (0, N, 0), (0, 0, N), (N, N, N), (3, 5, 7)]:
            assert orc.dense_index(x, y, z, N) == x + y * (N + 1) + z * (N + 1) ** 2


@pytest.mark.parametrize("T,b,want", [(T19, 1.3819, 5), (T19, 1.447, 5), (T14, 1.447, 2), (T14, 1.3819, 2),
                                      (T19, (2048 / 16) ** (1 / 15), 5)])
def test_dense_level_start(T, b, want):
    dls = orc.dense_level_start(T, 16, b, 16)
    assert dls == want
    _, res = orc.level_scales(16, b, 16)
    # every dense level fits its slice 1:1; the first hashed level would not
    for l in range(dls):
        assert (int(res[l]) + 1) ** 3 <= T
    assert (int(res[dls]) + 1) ** 3 > T


def test_level_resolutions():
    _, r = orc.level_scales(16, 1.3819, 16)
    assert list(r) == [16, 22, 30, 42, 58, 80, 111, 153, 212, 294, 406, 561, 775, 1072, 1481, 2047]
    _, r = orc.level_scales(16, 1.447, 16)
    assert list(r) == [16, 23, 33, 48, 70, 101, 146, 212, 307, 444, 643, 931, 1348, 1950, 2822, 4084]
    s, r = orc.level_scales(16, (2048 / 16) ** (1 / 15), 16)
    assert r[-1] == 2047 and abs(s[-1] - 2048.0) < 1e-2


def test_f16_conversion_matches_numpy():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(1e-4),
        rng.standard_normal(20000).astype(np.float32) * np.float32(1e3),
        (rng.standard_normal(20000) * 6e-6).astype(np.float32),
        np.float32([65504, 65519.99, 65520, 1e6, 6e-8, 2.98e-8, 2.9802322e-8, 5.96e-8, 0.0, -0.0]),
    ])
    got = np.array([orc.f32_to_f16_bits(v) for v in x], np.uint16)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, want)


def _lattice_values(table, l, T, res, dense):
    """Values at every lattice corner of level l, via the closed-form index."""
    n = res + 1
    c = np.arange(n, dtype=np.int64)
    X, Y, Z = np.meshgrid(c, c, c, indexing="ij")
    if dense:
        idx = X + Y * n + Z * n * n
    else:
        idx = ((X * 1) ^ (Y * 2654435761) ^ (Z * 805459861)) & 0xFFFFFFFF & (T - 1)
    sl = table.reshape(-1, T, 2)[l].astype(np.float64)
    return sl[idx]  # [n, n, n, 2]


@pytest.mark.parametrize("T,b,L", [(1 << 12, 1.447, 5), (T14, 1.447, 4)])
def test_encode_matches_textbook_trilinear(T, b, L):
    """Encode == scipy trilinear interpolation of the lattice function, per level."""
    rng = np.random.default_rng(11)
    table = rng.uniform(-1, 1, L * T * 2).astype(np.float16)
    pos = rng.random((3000, 3), dtype=np.float32) * np.float32(0.999)
    enc = orc.hash_encode(pos, table, T, L, 16, b).astype(np.float64)
    scale, res = orc.level_scales(16, b, L)
    dls = orc.dense_level_start(T, 16, b, L)
    for l in range(L):
        vals = _lattice_values(table, l, T, int(res[l]), l < dls)
        grid = np.arange(res[l] + 1, dtype=np.float64)
        x = pos.astype(np.float32) * np.float32(scale[l])   # fp32 product, as the kernel
        for f in range(2):
            it = RegularGridInterpolator((grid, grid, grid), vals[..., f])
            want = it(np.clip(x.astype(np.float64), 0, res[l]))
            np.testing.assert_allclose(enc[:, 2 * l + f], want, atol=2e-3, rtol=2e-3,
                                       err_msg=f"level {l} feature {f}")


def test_encode_exact_at_dense_lattice_points():
    T, L, b = T14, 2, 1.447
    rng = np.random.default_rng(5)
    table = rng.uniform(-1, 1, L * T * 2).astype(np.float16)
    scale, res = orc.level_scales(16, b, L)
    N = int(res[0])
    ijk = rng.integers(0, N + 1, (200, 3))
    pos = (ijk / np.float32(scale[0])).astype(np.float32)
    # keep only points whose fp32 product lands exactly on the lattice
    prod = pos * np.float32(scale[0])
    ok = np.all(prod == ijk.astype(np.float32), axis=1)
    enc = orc.hash_encode(pos[ok], table, T, L, 16, b)
    vals = _lattice_values(table, 0, T, N, True)
    want = vals[ijk[ok, 0], ijk[ok, 1], ijk[ok, 2]].astype(np.float16)
    np.testing.assert_array_equal(enc[:, :2], want)


def test_corner_weights_sum_to_one_and_fwd_clamp():
    pos = np.array([[0.1, 0.5, 0.9], [1.0, 1.0, 1.0], [0.0, 0.0, 0.0], [0.999, 0.25, 0.75]], np.float32)
    idx, w = orc.hash_corners(pos, T19, 16, 16, 1.3819)
    np.testing.assert_allclose(w.sum(-1), 1.0, atol=3e-7)
    # at coordinate 1.0 the forward clamp puts both corners on N_l
    _, res = orc.level_scales(16, 1.3819, 16)
    assert (idx[1, 0] == idx[1, 0, 0]).all()   # all 8 corners are (16,16,16) on level 0
    assert idx[1, 0, 0] == orc.dense_index(16, 16, 16, int(res[0])) * 2


def test_encode_is_linear_in_table():
    T, L, b = 1 << 10, 3, 1.5
    rng = np.random.default_rng(9)
    pos = rng.random((500, 3), dtype=np.float32)
    a = rng.integers(-64, 64, L * T * 2).astype(np.float16) / np.float16(64)
    c = rng.integers(-64, 64, L * T * 2).astype(np.float16) / np.float16(64)
    ea = orc.hash_encode(pos, a, T, L, 16, b).astype(np.float64)
    ec = orc.hash_encode(pos, c, T, L, 16, b).astype(np.float64)
    eac = orc.hash_encode(pos, (a + c).astype(np.float16), T, L, 16, b).astype(np.float64)
    np.testing.assert_allclose(eac, ea + ec, atol=4e-3)


@pytest.mark.parametrize("T,b,L", [(1 << 10, 1.5, 4), (T14, 1.447, 6)])
def test_scatter_is_adjoint_of_interpolation(T, b, L):
    """<interp(table), g> == <table, scatter(g)> per level, away from the clamp seam.

    The left side uses scipy's trilinear interpolation in fp64 over the
    closed-form lattice index, so only the scatter comes from the oracle."""
    rng = np.random.default_rng(21)
    scale, res = orc.level_scales(16, b, L)
    dls = orc.dense_level_start(T, 16, b, L)
    # keep x*s < N_l on every level, where the forward and scatter clamps agree
    lim = np.min(res / scale) * 0.999
    pos = (rng.random((4000, 3)) * lim).astype(np.float32)
    table = rng.uniform(-1, 1, L * T * 2).astype(np.float16)
    g = rng.standard_normal((4000, 2 * L)).astype(np.float16)
    sc = orc.hash_scatter(pos, g, T, L, 16, b).astype(np.float64).reshape(L, T * 2)
    tab = table.astype(np.float64).reshape(L, T * 2)
    for l in range(L):
        vals = _lattice_values(table, l, T, int(res[l]), l < dls)
        grid = np.arange(res[l] + 1, dtype=np.float64)
        x = (pos * np.float32(scale[l])).astype(np.float64)
        lhs, mag = 0.0, 0.0
        for f in range(2):
            it = RegularGridInterpolator((grid, grid, grid), vals[..., f])
            t = it(x) * g[:, 2 * l + f].astype(np.float64)
            lhs += t.sum()
            mag += np.abs(t).sum()
        rhs = float(np.dot(tab[l], sc[l]))
        assert abs(lhs - rhs) <= 1e-5 * mag, f"level {l}: {lhs} vs {rhs}"


def test_scatter_clamp_differs_at_seam():
    """At coordinate 1.0 the scatter clamps x0 to N_l-1 (networkFusionBackwardHashtable.cu:816-818)."""
    _, res = orc.level_scales(16, 1.3819, 16)
    pos = np.array([[1.0, 1.0, 1.0]], np.float32)
    idx, w = orc.hash_corners(pos, T19, 16, 16, 1.3819, bwd_clamp=True)
    N = int(res[0])
    assert idx[0, 0, 0] == orc.dense_index(N - 1, N - 1, N - 1, N) * 2
    assert w[0, 0, 0] == 1.0


@pytest.mark.parametrize("T,b,L", [(1 << 10, 1.5, 4), (T14, 1.447, 16)])
def test_scatter_stats_sums_magnitudes_and_counts(T, b, L):
    """hash_scatter_stats: its sums are hash_scatter's bit for bit, its magnitudes are the scatter of |g|
    (the corner weights are non-negative), and its counts are a bincount of the backward corner indices
    (two words per corner, zero products included)."""
    rng = np.random.default_rng(23)
    N = 3000
    pos = rng.random((N, 3)).astype(np.float32)
    pos[:16] = rng.choice(np.float32([0.0, 1.0, 0.5]), (16, 3))
    g = rng.standard_normal((N, 2 * L)).astype(np.float16)
    g[rng.random((N, 2 * L)) < 0.2] = 0
    s, sa, cnt = orc.hash_scatter_stats(pos, g, T, L, 16, b)
    np.testing.assert_array_equal(s.view(np.uint32), orc.hash_scatter(pos, g, T, L, 16, b).view(np.uint32))
    np.testing.assert_array_equal(sa.view(np.uint32), orc.hash_scatter(pos, np.abs(g), T, L, 16, b).view(np.uint32))
    idx, w = orc.hash_corners(pos, T, L, 16, b, bwd_clamp=True)
    assert (w >= 0).all()
    want = np.bincount(idx.ravel().astype(np.int64), minlength=L * T * 2)
    want[1:] += np.bincount(idx.ravel().astype(np.int64) + 1, minlength=L * T * 2)[1:L * T * 2]
    np.testing.assert_array_equal(cnt, want[:L * T * 2])
