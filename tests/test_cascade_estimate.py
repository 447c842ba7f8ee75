"""DataLoader::getNumCascades: the reference loader's pose-only cascade estimate
(DataLoader.cu:213-271 regime signals, 367-377 the estimate), applied by the
trainer when its config asks for 0 cascades (NerfTrainer.cu:113-114).

Host logic through the C-ABI (ntr_estimate_num_cascades), no GPU.  Each pose set
is built so that the regime, and with it the answer, is fixed by geometry alone:
cameras on a sphere looking at its centre (orbit: 1), a planar rig of parallel
cameras (forward-facing: 4), cameras at the origin looking outward (panorama: 3).
The determinant threshold is pinned from both sides with one rig of converging
cameras: a narrow one stays forward-facing, a wide one becomes bounded (and its
mirror image, rays meeting behind the rig, a panorama).
"""
import importlib

import numpy as np
import pytest

scenes = importlib.import_module("3dmaker_amd.scenes")


def pkg():
    return importlib.import_module("3dmaker_amd")


def look_at(eye, target, up=(0.0, 0.0, 1.0)):
    """Row-major camera-to-world matrix of a camera at eye looking at target (NeRF: view along -z)."""
    eye, target, up = (np.asarray(v, np.float64) for v in (eye, target, up))
    f = target - eye
    f /= np.linalg.norm(f)
    r = np.cross(f, up)
    if np.linalg.norm(r) < 1e-9:
        r = np.cross(f, (0.0, 1.0, 0.0))
    r /= np.linalg.norm(r)
    u = np.cross(r, f)
    m = np.eye(4)
    m[:3, 0], m[:3, 1], m[:3, 2], m[:3, 3] = r, u, -f, eye
    return m.astype(np.float32).reshape(16)


def est(tfs):
    return pkg().estimate_num_cascades(np.stack(tfs))


def as_4x4(c2w34):
    """[n, 3, 4] camera-to-world matrices as [n, 16] row-major 4x4."""
    n = c2w34.shape[0]
    m = np.tile(np.eye(4), (n, 1, 1))
    m[:, :3, :] = c2w34
    return m.astype(np.float32).reshape(n, 16)


def test_orbit_is_bounded():
    # the bench's 100 orbit cameras (radius 1.5, looking at the origin)
    assert est(list(as_4x4(scenes.cameras(100, 1.5, seed=2024)))) == 1
    rng = np.random.default_rng(0)
    centre = np.array([0.3, -0.2, 0.1])
    poses = []
    for _ in range(40):
        d = rng.normal(size=3)
        d /= np.linalg.norm(d)
        poses.append(look_at(centre + 4.0 * d, centre))
    assert est(poses) == 1


def test_forward_facing_rig():
    poses = [look_at((x, y, 0.0), (x, y, -5.0)) for x in np.linspace(-1, 1, 4) for y in np.linspace(-0.5, 0.5, 3)]
    assert est(poses) == 4


def test_outward_panorama():
    rng = np.random.default_rng(1)
    poses = []
    for _ in range(30):
        d = rng.normal(size=3)
        d /= np.linalg.norm(d)
        poses.append(look_at(0.05 * d, 10.0 * d))
    assert est(poses) == 3


def test_toed_in_and_toed_out_rigs():
    # A horizontal row of cameras whose view rays meet in one point.  The mean projector
    # (1/n) sum (I - f f^T) has a near-zero eigenvalue while the directions spread little: a
    # determinant below 0.02 makes the rig "parallel", its centre the cameras' mean and its
    # inwardness about 0 (forward-facing, 4), however the rays converge.  With a wider spread the
    # rays' meeting point is solved for: in front of the rig the inwardness is 1 (bounded, 1),
    # behind it -1 (panorama, 3).
    narrow = np.linspace(-0.5, 0.5, 9)   # directions within +-0.17 rad: determinant 0.011
    assert est([look_at((x, 0.0, 0.0), (0.0, -3.0, 0.0)) for x in narrow]) == 4
    wide = np.linspace(-1.5, 1.5, 9)     # within +-0.64 rad: determinant 0.14
    assert est([look_at((x, 0.0, 0.0), (0.0, -2.0, 0.0)) for x in wide]) == 1
    # rays from (x, 0, 0) towards (6 x, -3, 0) meet at (0, 0.6, 0), behind the rig: determinant 0.16
    assert est([look_at((x, 0.0, 0.0), (6 * x, -3.0, 0.0)) for x in narrow]) == 3
    assert est([look_at((x, 0.0, 0.0), (x, -3.0, 0.0)) for x in narrow]) == 4


def test_too_few_poses_keep_the_default():
    poses = [look_at((x, 0.0, 0.0), (x, -1.0, 0.0)) for x in (0.0, 0.1, 0.2)]
    assert est(poses) == 1
    assert pkg().estimate_num_cascades(np.zeros((0, 16), np.float32)) == 1


@pytest.mark.parametrize("seed", [3, 4])
def test_invariant_under_rigid_motion(seed):
    # the regime does not depend on the frame: rotate and translate every pose
    rng = np.random.default_rng(seed)
    q, _ = np.linalg.qr(rng.normal(size=(3, 3)))
    if np.linalg.det(q) < 0:
        q[:, 0] = -q[:, 0]  # a proper rotation
    G = np.eye(4)
    G[:3, :3], G[:3, 3] = q, rng.normal(size=3)
    sets = {
        1: [look_at(3 * d / np.linalg.norm(d), (0, 0, 0)) for d in rng.normal(size=(20, 3))],
        4: [look_at((x, y, 0.0), (x, y, -5.0)) for x in np.linspace(-1, 1, 4) for y in np.linspace(-0.5, 0.5, 3)],
    }
    for want, poses in sets.items():
        moved = [(G @ p.reshape(4, 4).astype(np.float64)).astype(np.float32).reshape(16) for p in poses]
        assert est(moved) == want
