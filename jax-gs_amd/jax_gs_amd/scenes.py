"""Seeded synthetic scenes of the benchmark configurations (NumPy, host side).

Every configuration draws from ``numpy.random.default_rng(seed)`` (seed = config
index by default) in a fixed order, in float32, with identity extrinsics and a
black background:
  cfg0  16,384 Gaussians, 256x256, SH0, forward (x,y ~ U(-1,1), z ~ U(2,6),
        log-scale ~ N(-3.5, 0.5), 60 deg FOV)
  cfg1  200,000 Gaussians in 32 clusters (sigma 0.3, centres U([-1.5,1.5]^2 x [2,8])),
        504x378, f=407, SH3, log-scale ~ N(-4, 0.7), L1 vs U(0,1) target
  cfg2  1,000,000 Gaussians, as cfg1 with centre z ~ U(1.5, 12), 1920x1080,
        f = 407*1920/504 (cfg1's field of view)
  cfg3  3,000,000 Gaussians, SH1, 1280x720: 70% in 4 tight clusters (sigma 0.05)
        near the optical axis, 30% uniform in the frustum (z ~ U(2, 8)); forward
  cfg4  capacity 2,097,152, 60% active (Bernoulli), SH3, 1280x720, as cfg1
        (inactive entries: logit -20, identity rotation)
Common: quaternions ~ N(0,1)^4 normalised; opacity logit ~ N(0,1); DC colour
c ~ U(0,1) stored as (c - 0.5) / C0 (gaussians.py:46); higher SH ~ N(0, 0.05).
"""
from __future__ import annotations

import math

import numpy as np

SH_C0 = 0.28209479177387814


def _camera(W, H, f):
    return dict(W=int(W), H=int(H), fx=float(f), fy=float(f), cx=W / 2.0, cy=H / 2.0,
                W2C=np.eye(4, dtype=np.float32))


def _common(rng, n, K, log_scale_mu, log_scale_sigma, sh_degree):
    scales = rng.normal(log_scale_mu, log_scale_sigma, (n, 3)).astype(np.float32)
    q = rng.normal(0.0, 1.0, (n, 4)).astype(np.float32)
    q /= np.linalg.norm(q, axis=1, keepdims=True).astype(np.float32)
    opac = rng.normal(0.0, 1.0, (n, 1)).astype(np.float32)
    sh = np.zeros((n, K, 3), np.float32)
    c = rng.uniform(0.0, 1.0, (n, 3)).astype(np.float32)
    sh[:, 0, :] = (c - np.float32(0.5)) / np.float32(SH_C0)
    nb = (sh_degree + 1) ** 2
    if nb > 1:
        sh[:, 1:nb, :] = rng.normal(0.0, 0.05, (n, nb - 1, 3)).astype(np.float32)
    return scales, q.astype(np.float32), opac, sh


def _clustered(rng, n, n_clusters, sigma, zlo, zhi):
    centres = np.stack([rng.uniform(-1.5, 1.5, n_clusters), rng.uniform(-1.5, 1.5, n_clusters),
                        rng.uniform(zlo, zhi, n_clusters)], axis=1)
    idx = rng.integers(0, n_clusters, n)
    return (centres[idx] + rng.normal(0.0, sigma, (n, 3))).astype(np.float32)


def make_scene(cfg: int, n: int | None = None, seed: int | None = None, width: int | None = None,
               height: int | None = None) -> dict:
    """Return dict(params=..., cam=..., sh_degree=..., target=..., mask=..., name=...).

    ``n``/``width``/``height`` shrink a configuration with the same distributions
    (for tests); the defaults are the full configuration."""
    rng = np.random.default_rng(cfg if seed is None else seed)
    mask = None
    target = None
    if cfg == 0:
        N = 16384 if n is None else n
        W, H = width or 256, height or 256
        f = (W / 2.0) / math.tan(math.radians(30.0))
        D = 0
        means = np.stack([rng.uniform(-1, 1, N), rng.uniform(-1, 1, N), rng.uniform(2, 6, N)], 1).astype(np.float32)
        scales, q, opac, sh = _common(rng, N, (D + 1) ** 2, -3.5, 0.5, D)
    elif cfg in (1, 2, 4):
        D = 3
        if cfg == 1:
            N = 200_000 if n is None else n
            W, H = width or 504, height or 378
            f = 407.0 * W / 504.0
            zlo, zhi = 2.0, 8.0
        elif cfg == 2:
            N = 1_000_000 if n is None else n
            W, H = width or 1920, height or 1080
            f = 407.0 * W / 504.0
            zlo, zhi = 1.5, 12.0
        else:
            N = 2_097_152 if n is None else n
            W, H = width or 1280, height or 720
            f = 407.0 * W / 504.0
            zlo, zhi = 2.0, 8.0
        means = _clustered(rng, N, 32, 0.3, zlo, zhi)
        scales, q, opac, sh = _common(rng, N, 16, -4.0, 0.7, D)
        if cfg == 4:
            mask = rng.uniform(0.0, 1.0, N) < 0.6
            opac[~mask] = -20.0
            q[~mask] = np.array([1, 0, 0, 0], np.float32)
        target = rng.uniform(0.0, 1.0, (H, W, 3)).astype(np.float32)
    elif cfg == 3:
        D = 1
        N = 3_000_000 if n is None else n
        W, H = width or 1280, height or 720
        f = 407.0 * W / 504.0
        n_cl = int(round(0.7 * N))
        # 4 cluster centres near the optical axis at depth ~4: they project into a
        # few percent of the frame
        centres = np.stack([rng.uniform(-0.15, 0.15, 4), rng.uniform(-0.1, 0.1, 4), rng.uniform(3.5, 4.5, 4)], 1)
        idx = rng.integers(0, 4, n_cl)
        pts_cl = centres[idx] + rng.normal(0.0, 0.05, (n_cl, 3))
        n_un = N - n_cl
        z = rng.uniform(2.0, 8.0, n_un)
        x = rng.uniform(-1.0, 1.0, n_un) * z * (W / 2.0) / f
        y = rng.uniform(-1.0, 1.0, n_un) * z * (H / 2.0) / f
        pts_un = np.stack([x, y, z], 1)
        means = np.concatenate([pts_cl, pts_un], 0).astype(np.float32)
        scales, q, opac, sh = _common(rng, N, 4, -4.0, 0.7, D)
    else:
        raise ValueError(f"unknown configuration {cfg}")
    params = dict(means=means, scales=scales, quaternions=q, opacities=opac, sh_coeffs=sh)
    return dict(params=params, cam=_camera(W, H, f), sh_degree=D, target=target, mask=mask, name=f"cfg{cfg}")


def to_torch(scene: dict, device="cuda"):
    """(Gaussians, Camera, target tensor or None, mask tensor or None) on `device`."""
    import torch

    from .core.camera import Camera
    from .core.gaussians import Gaussians

    p = scene["params"]
    g = Gaussians(**{k: torch.from_numpy(np.ascontiguousarray(v)).to(device) for k, v in p.items()})
    c = scene["cam"]
    cam = Camera(W=c["W"], H=c["H"], fx=c["fx"], fy=c["fy"], cx=c["cx"], cy=c["cy"],
                 W2C=torch.from_numpy(c["W2C"]).to(device), full_proj=torch.eye(4, device=device))
    tgt = None if scene["target"] is None else torch.from_numpy(scene["target"]).to(device)
    m = None if scene["mask"] is None else torch.from_numpy(scene["mask"]).to(device)
    return g, cam, tgt, m
