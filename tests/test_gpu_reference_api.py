"""The reference's own renderer tests (jax-gs tests/test_renderer.py:11-158) run through
this package's module API on the GPU, with the hand-derived known answers:

  KA1 project_gaussians      means2D (50, 50), depth 5, cov2D diag(0.5478752), radius 3
  KA2 get_tile_interactions  entries [(0,g0),(0,g1),(1,g0),(2,g0),(3,g0)], 512 slots,
                             tile ranges [0, 2, 3, 4, 5]
  KA3 render                 pixel (32, 32) ~ (0.99, 0, 0) with the alpha cap binding, so
                             d pixel / d opacity = 0
  KA4 render_tiles           the single-Gaussian alpha 0.9752656 at pixel (16, 16)
  KA5 render_tiles           520 co-located Gaussians: exactly 48 blends, then T <= 1e-4:
                             (0.0090747, 0.9908275, 0)

and the public drop-ins (tile_ranges, render_tiles) on arrays in the reference's full
layout, including Gaussians behind the camera (tile -1 prefix) and the sentinel tail.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from gpu_helpers import IMG_TOL, np_
from jax_gs_amd import Camera, init_gaussians_from_pcd, render
from jax_gs_amd.renderer import rasterizer
from jax_gs_amd.renderer.projection import project_gaussians

pytestmark = pytest.mark.gpu
F32 = np.float32


def _t(a, cuda, dtype=torch.float32):
    return torch.as_tensor(np.asarray(a), dtype=dtype, device=cuda)


def _cam(W, H, f, c, cuda):
    eye = torch.eye(4, device=cuda)
    return Camera(W=W, H=H, fx=f, fy=f, cx=c, cy=c, W2C=eye, full_proj=eye)


def test_ka1_projection(cuda):
    """test_renderer.py:11-33."""
    g = init_gaussians_from_pcd(_t([[0.0, 0.0, 5.0]], cuda), _t([[1.0, 1.0, 1.0]], cuda))
    means2D, cov2D, radii, valid, depths = project_gaussians(g, _cam(100, 100, 50.0, 50.0, cuda))
    np.testing.assert_array_equal(np_(means2D)[0], [50.0, 50.0])
    assert bool(valid[0]) and float(depths[0]) == 5.0
    c = (50.0 / 5.0) ** 2 * math.exp(-6.0) + 0.3
    np.testing.assert_allclose(np_(cov2D)[0], [[c, 0], [0, c]], rtol=2e-6, atol=1e-7)
    assert abs(c - 0.5478752) < 1e-7
    assert float(radii[0]) == 3.0


def test_ka2_tile_interactions(cuda):
    """test_renderer.py:35-51 (integer radii as in the reference test)."""
    st, sg, n = rasterizer.get_tile_interactions(_t([[16.0, 16.0], [0.0, 0.0]], cuda),
                                                 _t([4, 2], cuda, torch.int32), _t([True, True], cuda, torch.bool),
                                                 _t([5.0, 10.0], cuda), 32, 32, rasterizer.TILE_SIZE)
    assert int(n) == 5 and st.shape == (512,) and sg.shape == (512,)
    st, sg = np_(st), np_(sg)
    np.testing.assert_array_equal(st[:5], [0, 0, 1, 2, 3])
    np.testing.assert_array_equal(sg[:5], [0, 1, 0, 0, 0])
    assert np.all(st[5:] == 4)
    # the empty slots in the reference's order: g0's 252 (depth 5) before g1's 255 (depth 10)
    np.testing.assert_array_equal(sg[5:], [0] * 252 + [1] * 255)
    b = rasterizer.tile_ranges(_t(st, cuda, torch.int32), 4)
    np.testing.assert_array_equal(np_(b), [0, 2, 3, 4, 5])
    st_o, sg_o, n_o = oracle.tile_interactions(np.array([[16, 16], [0, 0]], F32), np.array([4, 2], F32),
                                               np.array([True, True]), np.array([5.0, 10.0], F32), 32, 32)
    np.testing.assert_array_equal(st, st_o)
    np.testing.assert_array_equal(sg, sg_o)


def test_ka3_full_render_and_capped_alpha(cuda):
    """test_renderer.py:78-113, and the gradient the alpha cap min(0.99, .) passes: none."""
    g = init_gaussians_from_pcd(_t([[0.0, 0.0, 5.0]], cuda), _t([[1.0, 0.0, 0.0]], cuda))
    g = g.replace(opacities=_t([[10.0]], cuda), scales=_t([[-1.0, -1.0, -1.0]], cuda))
    for f in ("means", "scales", "quaternions", "opacities", "sh_coeffs"):
        getattr(g, f).requires_grad_(True)
    image, extras = render(g, _cam(64, 64, 100.0, 32.0, cuda))
    img = np_(image)
    assert img.shape == (64, 64, 3)
    np.testing.assert_allclose(img[32, 32], [0.99, 0.0, 0.0], atol=1e-6)
    assert int(extras["radii"][0]) == 23
    seed = torch.zeros_like(image)
    seed[32, 32, 0] = 1.0
    image.backward(seed)
    assert float(g.opacities.grad[0, 0]) == 0.0
    # every cotangent against the oracle's VJP (the red channel sits on the clip bound
    # clip(., 0, 1) = 1 exactly: half of its cotangent passes)
    params = {f: np_(getattr(g, f)) for f in ("means", "scales", "quaternions", "opacities", "sh_coeffs")}
    cam_o = dict(W=64, H=64, fx=100.0, fy=100.0, cx=32.0, cy=32.0, W2C=np.eye(4, dtype=F32))
    img_o, _, res = oracle.render(params, cam_o)
    np.testing.assert_allclose(img, img_o, atol=IMG_TOL)
    gr_o = oracle.render_vjp(params, cam_o, res, np_(seed))
    assert gr_o["opacities"][0, 0] == 0.0 and gr_o["sh_coeffs"][0, 0, 0] != 0.0
    for f in params:
        got, want = np_(getattr(g, f).grad), gr_o[f]
        assert np.linalg.norm(got - want) <= 1e-3 * max(np.linalg.norm(want), 1e-30), f


def test_ka4_render_tiles_single_gaussian(cuda):
    """test_renderer.py:53-76 (cov 10 I, logit 10, red, four tiles)."""
    img = rasterizer.render_tiles(_t([[16.0, 16.0]], cuda), _t([[[10.0, 0.0], [0.0, 10.0]]], cuda),
                                  _t([[10.0]], cuda), _t([[1.0, 0.0, 0.0]], cuda), _t([0, 1, 2, 3], cuda, torch.int32),
                                  _t([0, 0, 0, 0], cuda, torch.int32), 32, 32, rasterizer.TILE_SIZE,
                                  _t([0.0, 0.0, 0.0], cuda))
    want = math.exp(-0.5 * 0.5 / 10) * (1 / (1 + math.exp(-10)))
    assert abs(want - 0.9752656) < 1e-7
    np.testing.assert_allclose(np_(img)[16, 16], [want, 0, 0], rtol=0, atol=1e-6)


def test_ka5_chunked_gated_composite(cuda):
    """test_renderer.py:115-158: 520 co-located Gaussians in one tile; the gated result
    (48 blends until T <= 1e-4)."""
    N = 520
    col = np.stack([np.linspace(0, 1, N, dtype=F32), np.linspace(1, 0, N, dtype=F32), np.zeros(N, F32)], -1)
    img = rasterizer.render_tiles(_t(np.tile([[8.0, 8.0]], (N, 1)), cuda),
                                  _t(np.tile([[[6.0, 0.0], [0.0, 6.0]]], (N, 1, 1)), cuda),
                                  _t(np.full((N, 1), -1.5), cuda), _t(col, cuda), _t(np.zeros(N), cuda, torch.int32),
                                  _t(np.arange(N), cuda, torch.int32), 16, 16, rasterizer.TILE_SIZE,
                                  _t([0.0, 0.0, 0.0], cuda))
    a = math.exp(-0.5 * 0.5 / 6) / (1 + math.exp(1.5))
    C, Tr, k = np.zeros(3), 1.0, 0
    while Tr > 1e-4:
        C += a * Tr * col[k].astype(np.float64)
        Tr *= 1 - a
        k += 1
    assert k == 48
    np.testing.assert_allclose(np_(img)[8, 8], C, atol=2e-6)
    np.testing.assert_allclose(np_(img)[8, 8], [0.0090747, 0.9908275, 0.0], atol=1e-6)
    # every pixel against the oracle: the array is 520 entries long, so the tile's second
    # chunk (entries 512-519) starts within 512 of its end and the default path reads it
    # through the clamped slice [8, 520) (entries 8-15), the TPU path entry by entry;
    # the pixels that stay open after 512 blends (the tile's rim) differ between the two
    args = (np.tile(np.array([[8.0, 8.0]], F32), (N, 1)), np.tile(np.array([[[6.0, 0.0], [0.0, 6.0]]], F32), (N, 1, 1)),
            np.full((N, 1), -1.5, F32), col, np.zeros(N, np.int32), np.arange(N, dtype=np.int32), 16, 16)
    img_std, _, _ = oracle.render_tiles(*args)
    img_tpu, _, _ = oracle.render_tiles(*args, tpu_gather=True)
    assert np.abs(img_std - img_tpu).max() > 1e-3
    assert np.abs(np_(img) - img_std).max() <= IMG_TOL
    img_t = rasterizer.render_tiles_tpu(*[_t(a, cuda, torch.int32 if a.dtype == np.int32 else torch.float32)
                                          for a in args[:6]], 16, 16, _t([0.0, 0.0, 0.0], cuda))
    assert np.abs(np_(img_t) - img_tpu).max() <= IMG_TOL


@pytest.mark.parametrize("n_behind", [0, 3])
def test_reference_layout_arrays_through_drop_ins(cuda, n_behind):
    """tile_ranges and render_tiles on the oracle's arrays in the reference's own layout
    (all 256 N slots: tile -1 slots of Gaussians behind the camera first, then the
    valid entries, then the sentinel tail): ranges bit-exact, image within 1e-4."""
    from jax_gs_amd import scenes

    sc = scenes.make_scene(1, n=3000, width=200, height=150)
    p = sc["params"]
    p["means"][:n_behind, 2] = -np.abs(p["means"][:n_behind, 2])
    c = sc["cam"]
    W, H = c["W"], c["H"]
    pre = oracle.preprocess(p["means"], p["scales"], p["quaternions"], p["sh_coeffs"], c["W2C"], W, H, F32(c["fx"]),
                            F32(c["fy"]), F32(c["cx"]), F32(c["cy"]), sc["sh_degree"])
    st, sg, n_int = oracle.tile_interactions(pre["means2d"], pre["radii"], pre["valid"], pre["depths"], H, W)
    assert int((st == -1).sum()) == 256 * n_behind
    T = ((W + 15) // 16) * ((H + 15) // 16)
    b = rasterizer.tile_ranges(_t(st, cuda, torch.int32), T)
    np.testing.assert_array_equal(np_(b), oracle.tile_boundaries(st, T))
    dev = [_t(pre["means2d"], cuda), _t(pre["cov2d"], cuda), _t(p["opacities"], cuda), _t(pre["colors"], cuda),
           _t(st, cuda, torch.int32), _t(sg, cuda, torch.int32)]
    img_o, _, _ = oracle.render_tiles(pre["means2d"], pre["cov2d"], p["opacities"], pre["colors"], st, sg, H, W)
    assert np.abs(np_(rasterizer.render_tiles(*dev, H, W)) - img_o).max() <= IMG_TOL
    assert np.abs(np_(rasterizer.render_tiles_tpu(*dev, H, W)) - img_o).max() <= IMG_TOL


def _reference_arrays_case(cuda, means2d, radii, valid, depths, H, W):
    st, sg, n = rasterizer.get_tile_interactions(_t(means2d, cuda), _t(radii, cuda), _t(valid, cuda, torch.bool),
                                                 _t(depths, cuda), H, W)
    st_o, sg_o, n_o = oracle.tile_interactions(means2d, radii, valid, depths, H, W)
    assert int(n) == n_o
    np.testing.assert_array_equal(np_(st), st_o)
    np.testing.assert_array_equal(np_(sg), sg_o)
    T = ((W + 15) // 16) * ((H + 15) // 16)
    np.testing.assert_array_equal(np_(rasterizer.tile_ranges(st, T)), oracle.tile_boundaries(st_o, T))
    return st_o, n_o


@pytest.mark.parametrize("n,seed", [(1, 0), (2, 1), (3, 2), (57, 3), (3000, 4)])
def test_get_tile_interactions_reference_arrays(cuda, n, seed):
    """rasterizer.py:12-116 slot for slot on arbitrary inputs: negative depths (their 256
    slots first, tile -1), -0.0, depths below the 0.01 near plane that the caller marks
    valid, valid Gaussians behind the camera (counted in n, sorted with tile -1), radii past
    the 16-tile cap, boxes off the image, equal depth quanta (ties by id), and the padding
    to 512 slots for n <= 1."""
    rng = np.random.default_rng(seed)
    W, H = 200, 150
    means2d = rng.uniform(-60, 260, (n, 2)).astype(F32)
    radii = np.ceil(rng.uniform(0, 70, n)).astype(F32)
    radii[rng.uniform(size=n) < 0.05] = 400.0
    valid = rng.uniform(size=n) < 0.8
    depths = rng.uniform(0.02, 20, n).astype(F32)
    k = rng.uniform(size=n)
    depths[k < 0.1] = -rng.uniform(0.01, 5, int((k < 0.1).sum())).astype(F32)
    depths[(k >= 0.1) & (k < 0.13)] = np.float32(-0.0)
    depths[(k >= 0.13) & (k < 0.16)] = rng.uniform(0, 0.01, int(((k >= 0.13) & (k < 0.16)).sum())).astype(F32)
    if n > 4:
        depths[1] = depths[3]
        valid[1] = valid[3] = True
    st_o, n_o = _reference_arrays_case(cuda, means2d, radii, valid, depths, H, W)
    if n >= 57:
        assert (st_o == -1).sum() > 0 and n_o > 0


def test_get_tile_interactions_reference_arrays_cfg1(cuda):
    """The configuration-1 scene (200k Gaussians, 51.2M slots) with a fifth of it moved
    behind the camera: the projection's outputs through get_tile_interactions."""
    from jax_gs_amd import scenes

    sc = scenes.make_scene(1)
    p = sc["params"]
    p["means"][::5, 2] = -p["means"][::5, 2]
    c = sc["cam"]
    pre = oracle.preprocess(p["means"], p["scales"], p["quaternions"], p["sh_coeffs"], c["W2C"], c["W"], c["H"],
                            F32(c["fx"]), F32(c["fy"]), F32(c["cx"]), F32(c["cy"]), sc["sh_degree"])
    st_o, n_o = _reference_arrays_case(cuda, pre["means2d"], pre["radii"], pre["valid"], pre["depths"], c["H"],
                                       c["W"])
    assert (st_o == -1).sum() == 256 * len(range(0, p["means"].shape[0], 5))
