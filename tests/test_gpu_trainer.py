"""INerfTrainer (NerfTrainer.cu) end to end on a small in-memory dataset: the
training loop lowers the loss, validate() scores the held-out views, .inerf
save/load with the scene footer round-trips, and the render entry points
produce images."""
import importlib

import numpy as np
import pytest

from helpers import pkg

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
scenes = importlib.import_module("3dmaker_amd.scenes")


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need cuda:0"
    return torch.device("cuda:0")


def test_trainer_loop_validate_save_load_render(dev, tmp_path):
    P = pkg()
    W = H = 96
    n = 24
    scene = scenes.SphereScene(seed=5)
    imgs, tf = scenes.render_views(scene, scenes.cameras(n, 1.5, seed=8), W, H, 50.0, dev, steps=256)
    focal = scenes.focal_from_fov(W, 50.0)
    cfg = P.NerfTrainer.default_config()
    cfg.numCascades, cfg.batchSize, cfg.renderBatchSize = 2, 1 << 15, 1 << 15
    cfg.shouldValidate, cfg.maxLR, cfg.minLR, cfg.annealSteps = 1, 1e-2, 1e-4, 300
    tr = P.NerfTrainer(cfg)
    tr.load_dataset(imgs.cpu().numpy(), tf, focal)
    assert tr.num_train_views() == n
    tr.begin_training(300)
    losses = []
    while tr.step() < 300:
        st = tr.train_steps(30)
        print(f"[trainer] step {st.step} loss {st.loss:.5f} lr {st.lr:.5f} ms/step {st.msPerStep:.3f}", flush=True)
        assert np.isfinite(st.loss) and st.loss > 0
        losses.append(st.loss)
    assert st.step >= 300 and st.targetSteps == 300
    assert min(losses[-3:]) < 0.5 * losses[0]
    # validate() renders with the model's current background (the last chunk's
    # random colour, as in the reference) against ground truth over white
    psnr = tr.validate()
    assert np.isfinite(psnr) and psnr > 0.0

    path = str(tmp_path / "scene.inerf")
    tr.save(path)
    raw = open(path, "rb").read()
    assert raw[:6] == b"INERF1" and raw[-36:-32] == b"SCN1"
    tr2 = P.NerfTrainer(cfg)
    tr2.load(path)
    # the loaded trainer has no dataset: validate() returns 0, as in the reference
    assert tr2.validate() == 0.0
    img = tr.render_orbit(30.0, 20.0, 1.5, 50.0, 64, 48)
    img2 = tr2.render_orbit(30.0, 20.0, 1.5, 50.0, 64, 48)
    assert img.shape == (48, 64, 3) and np.isfinite(img).all()
    np.testing.assert_array_equal(img, img2)
    view = tr.render_train_view(3, W, H)
    assert view.shape == (H, W, 3) and np.isfinite(view).all()
    assert view.min() >= 0.0 and view.max() <= 1.0 + 1e-6
    assert tr2.train_steps(1).step == 0  # no dataset on the loaded trainer: nothing to train (as the reference)
    tr.close()
    tr2.close()


@pytest.mark.parametrize("kind,want", [("orbit", 1), ("forward", 4)])
def test_trainer_takes_the_loaders_cascade_estimate(dev, kind, want):
    # numCascades 0: the model is built with the loader's pose estimate (NerfTrainer.cu:113-114)
    P = pkg()
    n, W, H = 12, 16, 16
    if kind == "orbit":
        tf = np.tile(np.eye(4, dtype=np.float32), (n, 1, 1))
        tf[:, :3, :] = scenes.cameras(n, 1.5, seed=3)
        tf = tf.reshape(n, 16)
    else:
        tf = np.tile(np.eye(4, dtype=np.float32).reshape(16), (n, 1))
        tf[:, 3] = np.linspace(-1.0, 1.0, n)   # a row of parallel cameras looking down -z
        tf[:, 11] = 2.0
    rgba = np.full((n, H, W, 4), 255, np.uint8)
    cfg = P.NerfTrainer.default_config()
    cfg.numCascades, cfg.batchSize, cfg.renderBatchSize = 0, 1 << 14, 1 << 14
    tr = P.NerfTrainer(cfg)
    tr.load_dataset(rgba, tf, scenes.focal_from_fov(W, 50.0))
    assert tr.num_cascades() == want == P.estimate_num_cascades(tf)
    tr.close()
