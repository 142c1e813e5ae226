"""Writes the golden fixtures of this directory (run from the repository root:
``python tests/golden/make_golden.py``).

Each fixture is a tiny scene (inputs) with the reference path's outputs as the CPU oracle
computes them -- the oracle's float32 restatement for the forward (projection, the full
get_tile_interactions arrays, the image of rasterizer.py's default path and of the TPU
path, n_contrib, the extras) and its float64 reverse mode for the cotangents of a fixed
image cotangent (the five Gaussian arrays and W2C).  The oracle is pinned separately
(tests/test_oracle.py: known answers KA1-KA5, brute force, central differences); the
fixtures freeze its outputs so that a later change of the oracle or of the GPU path is
caught against data that does not move.  JAX is not installed anywhere this build runs,
so no fixture comes from the reference itself.
"""
import math
import os
import sys

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(_HERE)))
import oracle  # noqa: E402

F32 = np.float32
C0 = 0.28209479177387814


def _rot(axis, th):
    ax = np.asarray(axis, np.float64)
    ax /= np.linalg.norm(ax)
    K = np.array([[0, -ax[2], ax[1]], [ax[2], 0, -ax[0]], [-ax[1], ax[0], 0]])
    return np.eye(3) + math.sin(th) * K + (1 - math.cos(th)) * K @ K


def scene(seed, n, W, H, deg, oblique, behind, masked):
    rng = np.random.default_rng(seed)
    means = np.stack([rng.uniform(-0.7, 0.7, n), rng.uniform(-0.5, 0.5, n), rng.uniform(2.5, 5.0, n)], 1)
    means[:behind, 2] = -rng.uniform(1.0, 3.0, behind)  # behind the camera: tile -1 slots
    K = 16
    sh = np.zeros((n, K, 3))
    sh[:, 0, :] = (rng.uniform(0.1, 0.9, (n, 3)) - 0.5) / C0
    sh[:, 1:, :] = rng.normal(0, 0.08, (n, K - 1, 3))
    params = dict(means=means.astype(F32), scales=rng.normal(-2.4, 0.4, (n, 3)).astype(F32),
                  quaternions=rng.normal(0, 1, (n, 4)).astype(F32), opacities=rng.normal(0.5, 1.5, (n, 1)).astype(F32),
                  sh_coeffs=sh.astype(F32))
    w2c = np.eye(4)
    if oblique:
        w2c[:3, :3] = _rot([0.2, -0.6, 0.75], 0.12)
        w2c[:3, 3] = [0.03, -0.02, 0.1]
    f = 0.9 * W
    cam = dict(W=W, H=H, fx=f, fy=f, cx=W / 2.0, cy=H / 2.0, W2C=w2c.astype(F32))
    mask = None
    if masked:
        mask = rng.uniform(0, 1, n) < 0.8
    return params, cam, deg, mask


CASES = {
    "small_sh3": dict(seed=1, n=48, W=64, H=48, deg=3, oblique=False, behind=0, masked=False),
    "oblique_behind_masked": dict(seed=2, n=40, W=56, H=40, deg=2, oblique=True, behind=3, masked=True),
}


def make(name):
    params, cam, deg, mask = scene(**CASES[name])
    img, ex, res = oracle.render(params, cam, mask=mask, sh_degree=deg)
    img_t, _, res_t = oracle.render(params, cam, mask=mask, sh_degree=deg, tpu_gather=True)
    g_img = np.random.default_rng(100).normal(0, 1, img.shape).astype(F32)
    p64 = {k: v.astype(np.float64) for k, v in params.items()}
    c64 = dict(cam, W2C=cam["W2C"].astype(np.float64))
    _, _, r64 = oracle.render(p64, c64, mask=mask, sh_degree=deg, dtype=np.float64)
    g64 = oracle.render_vjp(p64, c64, r64, g_img.astype(np.float64), sh_degree=deg, dtype=np.float64)
    pre = res["pre"]
    out = dict(W=cam["W"], H=cam["H"], fx=cam["fx"], fy=cam["fy"], cx=cam["cx"], cy=cam["cy"], W2C=cam["W2C"],
               sh_degree=deg, mask=(np.ones(len(params["means"]), bool) if mask is None else mask),
               means2d=pre["means2d"], radii=pre["radii"], valid=pre["valid"], depths=pre["depths"],
               colors=pre["colors"], sorted_tiles=res["sorted_tiles"], sorted_gids=res["sorted_gids"],
               n_interactions=np.int32(ex["n_interactions"]), image=img, final_T=res["final_T"],
               n_contrib=res["n_contrib"], image_tpu=img_t, g_image=g_img)
    for k, v in params.items():
        out["in_" + k] = v
    for k in ("means", "scales", "quaternions", "opacities", "sh_coeffs", "W2C"):
        out["grad_" + k] = g64[k]
    np.savez_compressed(os.path.join(_HERE, name + ".npz"), **out)


if __name__ == "__main__":
    for name in CASES:
        make(name)
        print("wrote", name)
