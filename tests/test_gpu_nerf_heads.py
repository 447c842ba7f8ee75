"""GPU parity of the NeRF step's two heads on the 16x16x32 MFMA (launchNerfHeads*) against the oracle.

The heads replace the density head's forward, compute_SH_gather, the colour head's forward and, in the
backward, the colour dX chain, compute_density_grad and the density dX chain
(networkFusionHashtable.cu:441-682, networkFusion.cu:197-355, networkFusionBackward.cu:49-646,
networkFusionBackwardHashtable.cu:71-781, otherKernels.cu compute_SH_gather / compute_density_grad).
Bars: the MLP outputs and gradients within 2e-3 abs (relative to the largest value) / 1e-2 rel (fp16
operands, fp32 accumulation, the north star's tolerance); sigma and the colour input bit-exact against
the oracle's SH gather of the kernel's own density output, and the density dL/dy bit-exact against the
oracle's density-gradient glue of the kernel's own colour dL/dx (same fp32 operations in the same
order); the SH features of the colour dL/dx are 0 by contract.
"""
import numpy as np
import pytest

import pyoracle as orc
from helpers import assert_close, d2h, make_mlp, pkg

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

DSHAPE = (32, 64, 16, 2)
CSHAPE = (32, 64, 8, 3)


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need cuda:0"
    return torch.device("cuda:0")


def T(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


class Head:
    """One head's per-layer fp16 weights / fp32 biases on the device, with device arrays of their pointers
    (the layout the TinyMLP classes keep), and per-layer fp32 gradient arrays."""

    def __init__(self, shape, seed, dev):
        inD, hid, outD, nl = shape
        self.shape = shape
        self.W, self.B = make_mlp(inD, hid, outD, nl, seed, bias_scale=0.2)
        self.W16 = self.W.astype(np.float16)
        sizes = [((outD if l == nl - 1 else hid), (inD if l == 0 else hid)) for l in range(nl)]
        self.wsz = [o * i for o, i in sizes]
        self.bsz = [o for o, _ in sizes]
        wo, bo = np.cumsum([0] + self.wsz), np.cumsum([0] + self.bsz)
        self.dw = [T(self.W16[wo[l]:wo[l + 1]], dev) for l in range(nl)]
        self.db = [T(self.B[bo[l]:bo[l + 1]], dev) for l in range(nl)]
        self.gw = [torch.full((n,), float("nan"), dtype=torch.float32, device=dev) for n in self.wsz]
        self.gb = [torch.full((n,), float("nan"), dtype=torch.float32, device=dev) for n in self.bsz]
        self.pw = self._ptrs(self.dw, dev)
        self.pb = self._ptrs(self.db, dev)
        self.pgw = self._ptrs(self.gw, dev)
        self.pgb = self._ptrs(self.gb, dev)

    @staticmethod
    def _ptrs(ts, dev):
        return torch.tensor([t.data_ptr() for t in ts], dtype=torch.int64, device=dev)

    def grads(self):
        torch.cuda.synchronize()
        return (np.concatenate([g.cpu().numpy() for g in self.gw]), np.concatenate([g.cpu().numpy() for g in self.gb]))


def check(L, what):
    assert L.tinymlp_last_error() == 0, f"{what}: {L.tinymlp_last_error_message()}"


def big_close(got, want, what):
    want = np.asarray(want, np.float32)
    assert_close(got, want, atol=2e-3 * max(1.0, float(np.abs(want).max())), what=what)


def make_case(N, levels, plane_pad, seed, dev, zero_tiles=False):
    rng = np.random.default_rng(seed)
    R = max(1, N // 7)
    enc = np.zeros((N, 32), np.float16)
    enc[:, :2 * levels] = rng.uniform(-1, 1, (N, 2 * levels)).astype(np.float16)
    plane = N + plane_pad
    planar = np.zeros((levels, plane, 2), np.float16)
    planar[:, :N, :] = enc[:, :2 * levels].reshape(N, levels, 2).transpose(1, 0, 2)
    dirs = rng.normal(size=(R, 3)).astype(np.float32)
    dirs /= np.linalg.norm(dirs, axis=1, keepdims=True)
    n1 = max(N, 1)  # a zero-sample case still passes non-null inputs
    ridx = rng.integers(0, R, n1).astype(np.uint32)
    cdy = np.zeros((n1, 8), np.float16)
    cdy[:, :3] = rng.uniform(-0.5, 0.5, (n1, 3)).astype(np.float16)
    dsig = rng.uniform(-1, 1, n1).astype(np.float32)
    if zero_tiles:
        # tiles past a saturated transmittance: zero colour dL/dy and a d sigma that rounds to +-0 in fp16
        # (skipped tiles); tiles with zero colour dL/dy but one live d sigma; a zero run across a tile edge
        for t in range((n1 + 15) // 16):
            sl = slice(16 * t, min(16 * t + 16, n1))
            if t % 3 == 0:
                cdy[sl] = 0
                dsig[sl] = rng.choice([0.0, -0.0, 1e-30, -1e-30, 2e-8, -2e-8], sl.stop - sl.start).astype(np.float32)
            elif t % 3 == 1:
                cdy[sl] = 0
                dsig[sl] = 0.0
                dsig[16 * t] = 0.25
        cdy[8:24] = 0
    return dict(N=N, levels=levels, plane=plane, enc=enc, planar=planar, dirs=dirs, ridx=ridx, cdy=cdy, dsig=dsig)


class Run:
    def __init__(self, case, dh, ch, dev, bias=0.5, act=1, stored_dy=False, tile_flags=False):
        P = pkg()
        self.L = L = P.lib()
        N = case["N"]
        self.c = case
        self.packed = torch.zeros(L.nerfHeadsPackedBytes(), dtype=torch.uint8, device=dev)
        L.launchNerfHeadsPack(dh.pw.data_ptr(), dh.pb.data_ptr(), ch.pw.data_ptr(), ch.pb.data_ptr(),
                              self.packed.data_ptr(), None)
        check(L, "pack")
        self.enc = T(case["planar"], dev)
        self.dirs = T(case["dirs"], dev)
        self.ridx = T(case["ridx"].view(np.int32), dev)
        n1 = max(N, 1)
        self.sigma = torch.full((n1,), float("nan"), dtype=torch.float32, device=dev)
        self.dout = torch.full((n1, 16), float("nan"), dtype=torch.float32, device=dev)
        self.cout = torch.full((n1, 8), float("nan"), dtype=torch.float32, device=dev)
        self.cin = torch.full((n1, 32), float("nan"), dtype=torch.float16, device=dev)
        L.launchNerfHeadsForward(self.packed.data_ptr(), self.enc.data_ptr(), case["plane"], case["levels"],
                                 self.dirs.data_ptr(), self.ridx.data_ptr(), N, bias, act, self.sigma.data_ptr(),
                                 self.dout.data_ptr(), self.cout.data_ptr(), self.cin.data_ptr(), None)
        check(L, "forward")
        self.cdy = T(case["cdy"], dev)
        self.dsig = T(case["dsig"], dev)
        self.denc = torch.full((n1, 32), float("nan"), dtype=torch.float16, device=dev)
        self.ddy = torch.full((n1, 16), float("nan"), dtype=torch.float16, device=dev)
        self.cdx = torch.full((n1, 32), float("nan"), dtype=torch.float16, device=dev)
        # tile_flags: the backward flags the tiles with a nonzero gradient, the weight gradients visit those
        self.live = torch.full(((n1 + 15) // 16,), 7, dtype=torch.int32, device=dev)
        L.launchNerfHeadsBackward(self.packed.data_ptr(), self.enc.data_ptr(), case["plane"], case["levels"],
                                  self.cin.data_ptr(), self.cdy.data_ptr(), self.dsig.data_ptr(), N,
                                  self.denc.data_ptr(), self.ddy.data_ptr(), self.cdx.data_ptr(),
                                  self.live.data_ptr() if tile_flags else None, None)
        check(L, "backward")
        # stored_dy: the density head's gradients start from the density dL/dy the backward stored
        L.launchNerfHeadsWeightGrads(self.packed.data_ptr(), self.enc.data_ptr(), case["plane"], case["levels"],
                                     self.cin.data_ptr(), self.cdy.data_ptr(), self.dsig.data_ptr(),
                                     self.ddy.data_ptr() if stored_dy else None,
                                     self.live.data_ptr() if tile_flags else None, N,
                                     dh.pgw.data_ptr(), dh.pgb.data_ptr(), ch.pgw.data_ptr(), ch.pgb.data_ptr(), None)
        check(L, "weight grads")
        torch.cuda.synchronize()
        self.bias, self.act = bias, act

    def host(self):
        N = self.c["N"]
        return {k: getattr(self, k)[:N].cpu().numpy() for k in ("sigma", "dout", "cout", "cin", "denc", "ddy", "cdx")}


def check_against_oracle(run, dh, ch):
    c, g = run.c, run.host()
    N, enc = c["N"], c["enc"]
    # density head forward
    y_ref, h1 = orc.mlp_forward(enc, dh.W16, dh.B, *DSHAPE, save_acts=True)
    big_close(g["dout"], y_ref, "density output")
    # SH gather of the kernel's own density output (bit-exact)
    w_cin, w_sig = orc.sh_gather(c["dirs"], c["ridx"], g["dout"], run.bias)
    np.testing.assert_array_equal(g["cin"].view(np.uint16), w_cin.view(np.uint16))
    np.testing.assert_array_equal(g["sigma"].view(np.uint32), w_sig.view(np.uint32))
    # colour head forward on the kernel's colour input
    c_ref, h2 = orc.mlp_forward(g["cin"], ch.W16, ch.B, *CSHAPE, out_act=run.act, save_acts=True)
    big_close(g["cout"], c_ref, "colour output")
    # colour dX chain (the SH features get no gradient: 0)
    cdW_ref, cdB_ref, cdx_ref = orc.mlp_backward(c["cdy"], g["cin"], h2, ch.W16, *CSHAPE)
    big_close(g["cdx"][:, :16], cdx_ref[:, :16], "colour dL/dinput")
    assert not g["cdx"][:, 16:].any(), "SH features of the colour dL/dinput are written as 0"
    # density-gradient glue on the kernel's own colour dL/dx (bit-exact)
    dg = orc.density_grad(c["dsig"], g["cdx"])
    np.testing.assert_array_equal(g["ddy"].view(np.uint16), dg.view(np.uint16))
    # density dX chain
    ddW_ref, ddB_ref, denc_ref = orc.mlp_backward(g["ddy"], enc, h1, dh.W16, *DSHAPE)
    big_close(g["denc"], denc_ref, "dL/d(encoding)")
    # weight gradients of both heads
    ddW, ddB = dh.grads()
    cdW, cdB = ch.grads()
    big_close(ddW, ddW_ref, "density dW")
    big_close(ddB, ddB_ref, "density db")
    big_close(cdW, cdW_ref, "colour dW")
    big_close(cdB, cdB_ref, "colour db")


@pytest.mark.parametrize("N,levels,pad,act,stored_dy", [(1, 16, 0, 1, False), (17, 16, 5, 1, True),
                                                        (5003, 16, 0, 1, False), (5003, 16, 0, 1, True),
                                                        (4096, 16, 64, 0, True), (3001, 9, 3, 1, True),
                                                        (40000, 16, 0, 1, False), (40000, 16, 0, 1, True)])
def test_heads_match_oracle(dev, N, levels, pad, act, stored_dy):
    print(f"heads N={N} levels={levels} pad={pad} act={act} stored_dy={stored_dy}", flush=True)
    dh, ch = Head(DSHAPE, 11, dev), Head(CSHAPE, 12, dev)
    run = Run(make_case(N, levels, pad, 100 + N, dev), dh, ch, dev, act=act, stored_dy=stored_dy)
    check_against_oracle(run, dh, ch)


@pytest.mark.parametrize("stored_dy,tile_flags", [(False, False), (True, False), (False, True), (True, True)])
def test_heads_skip_zero_gradient_tiles(dev, stored_dy, tile_flags):
    """Tiles whose colour dL/dy is zero and whose density dL/dy rounds to +-0 are skipped by the dX kernel and,
    with its tile flags, by the weight-gradient kernel: same results as the chain (zero dL/d(encoding), the
    glue of +0 and d sigma, zero dW terms), against the oracle; the flags mark exactly the live tiles."""
    dh, ch = Head(DSHAPE, 51, dev), Head(CSHAPE, 52, dev)
    case = make_case(3001, 16, 7, 77, dev, zero_tiles=True)
    run = Run(case, dh, ch, dev, stored_dy=stored_dy, tile_flags=tile_flags)
    check_against_oracle(run, dh, ch)
    g = run.host()
    ntiles = (3001 + 15) // 16
    cdy = np.zeros((ntiles * 16, 8), np.float16)
    cdy[:3001] = case["cdy"][:3001]
    glue = np.zeros(ntiles * 16, np.float16)
    glue[:3001] = np.clip(np.nan_to_num(np.float32(0.0) + case["dsig"][:3001], nan=0.0), -65504, 65504)
    live = ((cdy.view(np.uint16) & 0x7fff).reshape(ntiles, -1).any(1) |
            (glue.view(np.uint16) & 0x7fff).reshape(ntiles, 16).any(1))
    assert (~live).sum() > ntiles // 4
    rows = np.concatenate([np.arange(16 * t, min(16 * t + 16, 3001)) for t in np.nonzero(~live)[0]])
    assert not (g["denc"][rows].view(np.uint16) & 0x7fff).any()
    if tile_flags:
        np.testing.assert_array_equal(run.live.cpu().numpy() != 0, live)


def test_heads_density_grads_from_stored_dy_match_the_recomputed_ones(dev):
    """The density head's dW/db from the stored density dL/dy equal those of the recomputed colour chain
    (the dX kernel's operations: the same per-sample values); the two paths split the blocks between the
    heads differently, so the fixed-order sums of the block partials agree to fp32 rounding."""
    case = make_case(20011, 16, 0, 13, dev)
    dh, ch = Head(DSHAPE, 41, dev), Head(CSHAPE, 42, dev)
    Run(case, dh, ch, dev, stored_dy=False)
    rec = dh.grads() + ch.grads()
    dh2, ch2 = Head(DSHAPE, 41, dev), Head(CSHAPE, 42, dev)
    Run(case, dh2, ch2, dev, stored_dy=True)
    got = dh2.grads() + ch2.grads()
    for a, b, what in zip(rec, got, ("density dW", "density db", "colour dW", "colour db")):
        np.testing.assert_allclose(b, a, rtol=0, atol=1e-5 * float(np.abs(a).max()), err_msg=what)


def test_heads_zero_samples_store_zero_gradients(dev):
    dh, ch = Head(DSHAPE, 21, dev), Head(CSHAPE, 22, dev)
    Run(make_case(0, 16, 8, 5, dev), dh, ch, dev)
    for g in dh.grads() + ch.grads():
        assert not g.any() and np.isfinite(g).all()


def test_heads_weight_grads_are_deterministic_and_overwrite(dev):
    """Two runs on the same inputs give bit-identical gradients (fixed-order reduction), whatever the
    gradient arrays held before."""
    dh, ch = Head(DSHAPE, 31, dev), Head(CSHAPE, 32, dev)
    case = make_case(20011, 16, 0, 9, dev)
    run = Run(case, dh, ch, dev)
    first = dh.grads() + ch.grads()
    for t in dh.gw + dh.gb + ch.gw + ch.gb:
        t.fill_(123.0)
    L = run.L
    L.launchNerfHeadsWeightGrads(run.packed.data_ptr(), run.enc.data_ptr(), case["plane"], case["levels"],
                                 run.cin.data_ptr(), run.cdy.data_ptr(), run.dsig.data_ptr(), None, None, case["N"],
                                 dh.pgw.data_ptr(), dh.pgb.data_ptr(), ch.pgw.data_ptr(), ch.pgb.data_ptr(), None)
    check(L, "weight grads")
    second = dh.grads() + ch.grads()
    for a, b in zip(first, second):
        np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
