"""eval_sh on its own (sh.py:25-74) and the camera cotangent dL/dW2C, on the GPU against
the oracle (both pinned on the CPU: scipy's real harmonics and central differences)."""
import math

import numpy as np
import pytest
import torch

import oracle
from gpu_helpers import FIELDS, GRAD_TOL, IMG_TOL, log, np_, rel
from jax_gs_amd import render, scenes
from jax_gs_amd.renderer.sh import eval_sh

pytestmark = pytest.mark.gpu
F32 = np.float32


@pytest.mark.parametrize("deg,K", [(0, 1), (0, 16), (1, 4), (2, 9), (3, 16), (2, 16)])
def test_eval_sh_and_vjp_match_oracle(cuda, deg, K):
    """Colours bit-identical to the oracle's (the reference's association order, no FMA);
    the SH cotangent bit-identical (the signed basis times the colour cotangent); the
    direction cotangent within 1e-5 relative L2."""
    log(f"eval_sh deg={deg} K={K}")
    rng = np.random.default_rng(50 + 4 * deg + K)
    n = 5000
    d = rng.normal(0, 1, (n, 3)).astype(F32)
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    sh = rng.normal(0, 0.3, (n, K, 3)).astype(F32)
    g = rng.normal(0, 1, (n, 3)).astype(F32)
    sh_t = torch.from_numpy(sh).to(cuda).requires_grad_(True)
    d_t = torch.from_numpy(d).to(cuda).requires_grad_(True)
    col = eval_sh(deg, sh_t, d_t)
    np.testing.assert_array_equal(np_(col), oracle.eval_sh(deg, sh, d))
    col.backward(torch.from_numpy(g).to(cuda))
    g_sh, g_d = oracle.eval_sh_vjp(deg, sh, d, g)
    np.testing.assert_array_equal(np_(sh_t.grad), g_sh)
    if deg == 0:
        assert np.all(np_(d_t.grad) == 0)
    else:
        assert rel(np_(d_t.grad), g_d) <= 1e-5


def _oblique(sc):
    """The scene's camera turned 0.15 rad about an oblique axis and moved, so that every
    entry of W2C's first three rows enters."""
    ax = np.array([0.3, -0.5, 0.8])
    ax /= np.linalg.norm(ax)
    Kx = np.array([[0, -ax[2], ax[1]], [ax[2], 0, -ax[0]], [-ax[1], ax[0], 0]])
    w = np.eye(4)
    w[:3, :3] = np.eye(3) + math.sin(0.15) * Kx + (1 - math.cos(0.15)) * Kx @ Kx
    w[:3, 3] = [0.05, -0.03, 0.2]
    sc["cam"]["W2C"] = w.astype(F32)
    return sc


@pytest.mark.parametrize("cfg,n,W,H", [(1, 3000, 200, 150), (0, 2000, 96, 64)])
def test_render_w2c_cotangent_matches_oracle(cuda, cfg, n, W, H):
    """render with a W2C that requires grad: the image, the five cotangents and dL/dW2C
    (row 3 exactly 0) against the oracle's VJP."""
    log(f"w2c cfg={cfg} n={n} {W}x{H}")
    sc = _oblique(scenes.make_scene(cfg, n=n, width=W, height=H))
    g, cam, _, m = scenes.to_torch(sc, cuda)
    for f in FIELDS:
        getattr(g, f).requires_grad_(True)
    cam = cam._replace(W2C=cam.W2C.clone().requires_grad_(True))
    image, _ = render(g, cam, mask=m, sh_degree=sc["sh_degree"])
    img_o, _, res = oracle.render(sc["params"], sc["cam"], mask=sc["mask"], sh_degree=sc["sh_degree"])
    assert float(np.abs(np_(image) - img_o).max()) <= IMG_TOL
    seed = np.random.default_rng(9).normal(0, 1, img_o.shape).astype(F32)
    image.backward(torch.from_numpy(seed).to(cuda))
    gr_o = oracle.render_vjp(sc["params"], sc["cam"], res, seed, sh_degree=sc["sh_degree"])
    for f in FIELDS:
        assert rel(np_(getattr(g, f).grad), gr_o[f]) <= GRAD_TOL, f
    gw = np_(cam.W2C.grad)
    assert np.all(gw[3] == 0)
    assert rel(gw, gr_o["W2C"]) <= GRAD_TOL, (gw, gr_o["W2C"])
