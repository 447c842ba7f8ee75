"""Synthetic, seeded inputs for the NeRF hot path (no datasets are available).

* occupancy_c4: a cascaded occupancy bitfield in the reference layout
  (InstantNerf.cu:286-299; cell z*res^2 + y*res + x, LSB-first bytes, per
  cascade a mip pyramid whose level l+1 is the OR of 2x2x2 cells of level l,
  otherKernels.cu:752-807) with Bernoulli(p) level-0 cells inside a sphere.
* cameras / camera_rays: pinhole cameras on a sphere looking at the origin and
  pixel-centre rays through them (ray formula of NerfTrainer.cu:37-46).
* SphereScene: the procedural scene of the end-to-end configuration, a union
  of spheres as density sigma_max * sigmoid(-sdf / width) and a 3-band
  sinusoidal colour field, with ground-truth pixels rendered by fixed-step
  quadrature.

Everything here is numpy on the host; it produces inputs, it computes nothing
of the training path.
"""
from __future__ import annotations

import math

import numpy as np


def pyramid_cells(res: int, levels: int) -> int:
    return sum((res >> l) ** 3 for l in range(levels))


def mip_pyramid(level0: np.ndarray, levels: int) -> list[np.ndarray]:
    """level0: bool [res, res, res] indexed [z, y, x] -> [level0, level1, ...]."""
    out = [level0]
    cur = level0
    for _ in range(levels - 1):
        r = cur.shape[0] // 2
        cur = cur.reshape(r, 2, r, 2, r, 2).any(axis=(1, 3, 5))
        out.append(cur)
    return out


def pack_grid(level0_per_cascade: list[np.ndarray], levels: int) -> np.ndarray:
    """Bitfield bytes of all cascades (cascade c at bit c * pyramid_cells)."""
    bits = []
    for l0 in level0_per_cascade:
        for lv in mip_pyramid(l0, levels):
            bits.append(lv.reshape(-1))
    flat = np.concatenate(bits).astype(np.uint8)
    return np.packbits(flat, bitorder="little")


def occupancy_c4(res=128, cascades=5, levels=4, p=0.1, radius=0.3, aabb=1.5, seed=0):
    """Level-0 cells of cascade 0 whose centre lies within `radius` of the origin
    are occupied with probability p; every other cell is empty."""
    rng = np.random.default_rng(seed)
    c = (np.arange(res, dtype=np.float64) + 0.5) / res * (2 * aabb) - aabb
    z, y, x = np.meshgrid(c, c, c, indexing="ij")
    inside = x * x + y * y + z * z <= radius * radius
    l0 = inside & (rng.random((res, res, res)) < p)
    per = [l0] + [np.zeros((res, res, res), bool) for _ in range(cascades - 1)]
    return pack_grid(per, levels)


def _look_at(eye: np.ndarray) -> np.ndarray:
    """Camera-to-world rotation, camera looking down -z at the origin."""
    fwd = -eye / np.linalg.norm(eye)
    up = np.array([0.0, 1.0, 0.0])
    if abs(float(np.dot(fwd, up))) > 0.999:
        up = np.array([1.0, 0.0, 0.0])
    right = np.cross(fwd, up)
    right /= np.linalg.norm(right)
    true_up = np.cross(right, fwd)
    return np.stack([right, true_up, -fwd], axis=1)  # columns: x, y, z axes


def cameras(n=100, radius=1.5, seed=0, jitter=0.05):
    """n camera-to-world 3x4 matrices on a Fibonacci lattice with seeded jitter."""
    rng = np.random.default_rng(seed)
    out = []
    golden = math.pi * (3.0 - math.sqrt(5.0))
    for i in range(n):
        yv = 1.0 - 2.0 * (i + 0.5) / n
        r = math.sqrt(max(0.0, 1.0 - yv * yv))
        th = golden * i
        d = np.array([math.cos(th) * r, yv, math.sin(th) * r]) + rng.normal(0, jitter, 3)
        eye = d / np.linalg.norm(d) * radius
        m = np.zeros((3, 4))
        m[:, :3] = _look_at(eye)
        m[:, 3] = eye
        out.append(m)
    return np.stack(out)


def focal_from_fov(width: int, fov_x_deg: float) -> float:
    return 0.5 * width / math.tan(math.radians(fov_x_deg) * 0.5)


def camera_rays(c2w: np.ndarray, cam: np.ndarray, px: np.ndarray, py: np.ndarray, width: int, height: int,
                focal: float):
    """Unit rays through pixel centres (px + 0.5, py + 0.5) of cameras cam[i]."""
    dx = (px + 0.5 - width * 0.5) / focal
    dy = -(py + 0.5 - height * 0.5) / focal
    dz = -np.ones_like(dx)
    v = np.stack([dx, dy, dz], axis=1)
    v /= np.linalg.norm(v, axis=1, keepdims=True)
    R = c2w[cam, :, :3]
    d = np.einsum("nij,nj->ni", R, v)
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    o = c2w[cam, :, 3]
    return o.astype(np.float32), d.astype(np.float32)


def rays_c4(num_rays=1 << 18, n_cams=100, width=800, height=800, fov_x=50.0, radius=1.5, seed=0):
    """Uniformly random (camera, pixel) pairs; returns (o, d) float32 [R, 3]."""
    rng = np.random.default_rng(seed)
    c2w = cameras(n_cams, radius, seed)
    cam = rng.integers(0, n_cams, num_rays)
    px = rng.integers(0, width, num_rays).astype(np.float64)
    py = rng.integers(0, height, num_rays).astype(np.float64)
    return camera_rays(c2w, cam, px, py, width, height, focal_from_fov(width, fov_x))


class SphereScene:
    """Union of 3 seeded spheres: sigma = sigma_max * sigmoid(-sdf / width); colour
    c_k(x) = 0.5 + 0.5 sin(f_k . x + p_k) for 3 bands."""

    def __init__(self, seed=0, sigma_max=200.0, width=0.01):
        rng = np.random.default_rng(seed)
        self.centres = rng.uniform(-0.6, 0.6, (3, 3))
        self.radii = rng.uniform(0.15, 0.35, 3)
        self.freq = rng.normal(0, 4.0, (3, 3))
        self.phase = rng.uniform(0, 2 * math.pi, 3)
        self.sigma_max = sigma_max
        self.width = width

    def sdf(self, p):
        d = np.linalg.norm(p[..., None, :] - self.centres, axis=-1) - self.radii
        return d.min(axis=-1)

    def density(self, p):
        z = np.clip(-self.sdf(p) / self.width, -60, 60)
        return self.sigma_max / (1.0 + np.exp(-z))

    def colour(self, p):
        return 0.5 + 0.5 * np.sin(p @ self.freq.T + self.phase)

    def render(self, o, d, near=0.0, far=3.5, steps=1024, bg=(1.0, 1.0, 1.0), chunk=1 << 14):
        """Ground-truth pixels by midpoint quadrature of the volume-rendering integral."""
        o = np.asarray(o, np.float64)
        d = np.asarray(d, np.float64)
        out = np.zeros((o.shape[0], 3))
        dt = (far - near) / steps
        ts = near + (np.arange(steps) + 0.5) * dt
        bgv = np.asarray(bg, np.float64)
        for s in range(0, o.shape[0], chunk):
            oo, dd = o[s:s + chunk], d[s:s + chunk]
            p = oo[:, None, :] + ts[None, :, None] * dd[:, None, :]
            sig = self.density(p)
            alpha = 1.0 - np.exp(-sig * dt)
            T = np.cumprod(np.concatenate([np.ones((len(oo), 1)), 1.0 - alpha[:, :-1]], axis=1), axis=1)
            w = T * alpha
            c = self.colour(p)
            out[s:s + chunk] = (w[..., None] * c).sum(1) + (T[:, -1] * (1.0 - alpha[:, -1]))[:, None] * bgv
        return out.astype(np.float32)

    def render_device_rgba(self, o, d, near=0.0, far=3.5, steps=1024, chunk=1 << 16):
        """(colour over a black background [N, 3], opacity 1 - T [N]) by the
        quadrature of render(), evaluated with torch on the tensors' device (fp32)."""
        import torch
        dev = o.device
        cen = torch.tensor(self.centres, dtype=torch.float32, device=dev)
        rad = torch.tensor(self.radii, dtype=torch.float32, device=dev)
        fr = torch.tensor(self.freq, dtype=torch.float32, device=dev)
        ph = torch.tensor(self.phase, dtype=torch.float32, device=dev)
        dt = (far - near) / steps
        ts = near + (torch.arange(steps, device=dev, dtype=torch.float32) + 0.5) * dt
        col = torch.empty((o.shape[0], 3), dtype=torch.float32, device=dev)
        alpha_out = torch.empty(o.shape[0], dtype=torch.float32, device=dev)
        for s in range(0, o.shape[0], chunk):
            oo, dd = o[s:s + chunk], d[s:s + chunk]
            p = oo[:, None, :] + ts[None, :, None] * dd[:, None, :]
            sdf = (torch.linalg.norm(p[..., None, :] - cen, dim=-1) - rad).min(dim=-1).values
            sig = self.sigma_max * torch.sigmoid(-sdf / self.width)
            alpha = 1.0 - torch.exp(-sig * dt)
            T = torch.cumprod(torch.cat([torch.ones_like(alpha[:, :1]), 1.0 - alpha[:, :-1]], dim=1), dim=1)
            w = T * alpha
            c = 0.5 + 0.5 * torch.sin(p @ fr.T + ph)
            col[s:s + chunk] = (w[..., None] * c).sum(1)
            alpha_out[s:s + chunk] = 1.0 - T[:, -1] * (1.0 - alpha[:, -1])
        return col, alpha_out

    def render_device(self, o, d, near=0.0, far=3.5, steps=1024, bg=(1.0, 1.0, 1.0), chunk=1 << 16):
        """render() evaluated with torch on the tensors' device (fp32): the same
        quadrature for ray pools too large for the host."""
        import torch
        col, a = self.render_device_rgba(o, d, near, far, steps, chunk)
        bgv = torch.tensor(bg, dtype=torch.float32, device=o.device)
        return col + (1.0 - a)[:, None] * bgv

def feed_pixel_rays(c2w: np.ndarray, cam: int, width: int, height: int, focal: float):
    """Rays of every pixel of camera cam as the training ray feed builds them
    (DataLoader.cu:623-641): pixel (px, py) -> ((px - w/2)/f, -(py - h/2)/f, -1)."""
    py, px = np.meshgrid(np.arange(height, dtype=np.float64), np.arange(width, dtype=np.float64), indexing="ij")
    dx = (px.ravel() - width * 0.5) / focal
    dy = -(py.ravel() - height * 0.5) / focal
    v = np.stack([dx, dy, -np.ones_like(dx)], axis=1)
    v /= np.linalg.norm(v, axis=1, keepdims=True)
    d = v @ c2w[cam, :, :3].T
    o = np.broadcast_to(c2w[cam, :, 3], d.shape)
    return np.ascontiguousarray(o, np.float32), np.ascontiguousarray(d, np.float32)


def render_views(scene: "SphereScene", c2w: np.ndarray, width: int, height: int, fov_x: float, device, steps=1024):
    """A dataset for the ray feed: RGBA8 images [n, h, w, 4] (uint8 tensor on device,
    straight colour + opacity) and camera-to-world matrices [n, 16] (float32,
    row-major 4x4) of the analytic scene seen from cameras c2w [n, 3, 4]."""
    import torch
    focal = focal_from_fov(width, fov_x)
    n = c2w.shape[0]
    imgs = torch.empty((n, height, width, 4), dtype=torch.uint8, device=device)
    for k in range(n):
        o, d = feed_pixel_rays(c2w, k, width, height, focal)
        c0, a = scene.render_device_rgba(torch.from_numpy(o).to(device), torch.from_numpy(d).to(device), steps=steps)
        straight = torch.where(a[:, None] > 1e-6, c0 / a.clamp_min(1e-6)[:, None], torch.zeros_like(c0))
        rgba = torch.cat([straight.clamp(0, 1), a[:, None]], dim=1)
        imgs[k] = torch.round(rgba * 255.0).to(torch.uint8).view(height, width, 4)
    T = np.zeros((n, 16), np.float32)
    for k in range(n):
        m = np.eye(4)
        m[:3, :] = c2w[k]
        T[k] = m.reshape(-1)
    return imgs, T
