"""GPU parity of the training ray feed (fetchRayChunkStreamingKernel,
DataLoader.cu:548-661) through launchFetchRayChunk: ray origins, directions,
composited colours and depth-prior fields bit-exact with the oracle (same fp32
operations; integer draws from pcg_hash)."""
import numpy as np
import pytest

import pyoracle as orc
from helpers import pkg

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need cuda:0"
    return torch.device("cuda:0")


def T(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("offset,size,seed,randomize,holdout,dense_fraction",
                         [(0, 5000, 0, False, 0, 0.0), (123456, 7001, 77, True, 0, 0.0),
                          (0, 65536, 2024, True, 8, 0.0), (64, 4096, 5, True, 4, 0.5)])
def test_fetch_ray_chunk_bit_exact(dev, offset, size, seed, randomize, holdout, dense_fraction):
    P = pkg()
    print(f"[feed] offset={offset} size={size} randomize={randomize} holdout={holdout}", flush=True)
    rng = np.random.default_rng(seed + 1)
    n, h, w = 17, 48, 64
    imgs = rng.integers(0, 256, (n, h, w, 4), dtype=np.uint8)
    Tm = np.zeros((n, 16), np.float32)
    for i in range(n):
        q, _ = np.linalg.qr(rng.normal(size=(3, 3)))
        Tm[i] = np.concatenate([np.concatenate([q, rng.normal(size=(3, 1))], 1), [[0, 0, 0, 1]]]).reshape(-1)
    nrec = 50 if dense_fraction > 0 else 0
    rec = None
    if nrec:
        rec = dict(frame=rng.integers(0, n, nrec).astype(np.int32), u=rng.uniform(-2, 70, nrec).astype(np.float32),
                   v=rng.uniform(-2, 50, nrec).astype(np.float32), D=rng.uniform(0.1, 3, nrec).astype(np.float32),
                   sigma=rng.uniform(0.01, 0.2, nrec).astype(np.float32))
    bg = np.float32([0.3, 0.1, 0.9])
    focal = 55.5
    out = {k: torch.zeros(s, device=dev) for k, s in [("o", (size, 3)), ("d", (size, 3)), ("rgb", (size, 3)),
                                                      ("dense", size), ("sigma", size)]}
    keep = [T(Tm, dev), T(imgs, dev)]
    recd = [T(rec[k], dev) for k in ("frame", "u", "v", "D", "sigma")] if rec else [None] * 5
    P.lib().launchFetchRayChunk(offset, size, n * h * w, seed, int(randomize), w, h, focal, keep[0].data_ptr(),
                                keep[1].data_ptr(), out["o"].data_ptr(), out["d"].data_ptr(), out["rgb"].data_ptr(),
                                out["dense"].data_ptr(), out["sigma"].data_ptr(),
                                *[r.data_ptr() if r is not None else None for r in recd], nrec, dense_fraction,
                                0.9, 1.1, P.Float3(*map(float, bg)), holdout, None)
    P.check()
    torch.cuda.synchronize()
    want = orc.fetch_ray_chunk(offset, size, seed, randomize, Tm, imgs, focal, bg, holdout_every=holdout,
                               records=rec, dense_fraction=dense_fraction, uv_scale=(0.9, 1.1))
    for k in ("o", "d", "rgb", "dense", "sigma"):
        np.testing.assert_array_equal(out[k].cpu().numpy().view(np.uint32), want[k].view(np.uint32), err_msg=k)
    if dense_fraction:
        assert (want["dense"] >= 0).any()
