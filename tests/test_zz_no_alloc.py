"""The allocation-free scatter entry point (launchHashTableBackwardKernelNoAlloc) against the regular one."""
import numpy as np
import pytest

import pyoracle as orc
from helpers import assert_scatter_close, pkg, positions, scatter_bound, scatter_quantum

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _run(P, name, denc, pos, T_, L, b, N, fill):
    grads = torch.full((L * T_ * 2,), fill, dtype=torch.float32, device="cuda:0")
    P.launch(name, denc, pos, grads, N, T_, L, b, 16, 2, None)
    torch.cuda.synchronize()
    return grads.cpu().numpy()


def test_no_alloc_scatter_matches_the_allocating_entry_point():
    """Two calls in a row, the second smaller; the first spans several sub-batches of the fixed scratch."""
    assert torch.cuda.is_available()
    P = pkg()
    T_, L, b = 1 << 19, 16, (2048 / 16) ** (1 / 15)
    rng = np.random.default_rng(91)
    for N in (100000, 5000):
        print(f"[no-alloc scatter] N={N}", flush=True)
        pos = positions(N, 92 + N)
        pos[: N // 2, :3] = (0.5 + 0.03 * rng.normal(size=(N // 2, 3))).clip(0, 1)  # dense-level hot bins
        denc = rng.normal(0, 1, (N, 2 * L)).astype(np.float16)
        d_pos, d_denc = torch.from_numpy(pos).cuda(), torch.from_numpy(denc).cuda()
        want = _run(P, "launchHashTableBackwardKernel", d_denc, d_pos, T_, L, b, N, 0.25)
        got = _run(P, "launchHashTableBackwardKernelNoAlloc", d_denc, d_pos, T_, L, b, N, 0.25)
        g, gabs, cnt = orc.hash_scatter_stats(pos, denc, T_, L, 16, b)
        # sub-batches of at most 32768 samples, each added to the array in fp32
        subs = -(-N // 32768)
        bound = scatter_bound(g, gabs, cnt, scatter_quantum(denc, L, T_), extra_roundings=2 * subs)
        assert_scatter_close(got, g + np.float32(0.25), bound, base=0.25, what=f"no-alloc vs oracle N={N}")
        assert_scatter_close(got, want, 2 * bound, base=0.25, what=f"no-alloc vs allocating entry point N={N}")


def test_no_alloc_scatter_rejects_grids_beyond_its_scratch():
    P = pkg()
    T_, L = 1 << 24, 16   # 16 levels x 4096 slices > 8192 bins
    pos = torch.zeros((8, 4), dtype=torch.float32, device="cuda:0")
    denc = torch.zeros((8, 2 * L), dtype=torch.float16, device="cuda:0")
    grads = torch.zeros(16, dtype=torch.float32, device="cuda:0")  # never touched: the call is rejected first
    with pytest.raises(RuntimeError, match="beyond the fixed scratch"):
        P.launch("launchHashTableBackwardKernelNoAlloc", denc, pos, grads, 8, T_, L, 1.3819, 16, 2, None)
