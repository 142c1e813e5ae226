"""The HIP path against the committed golden fixtures (tests/golden/): preprocessing and the
full get_tile_interactions arrays bit for bit, both compositing paths' images within 1e-4,
n_contrib exactly, and the five Gaussian cotangents plus dL/dW2C within 1e-3 relative L2 of
the fixtures' float64 values."""
import numpy as np
import pytest
import torch

from gpu_helpers import FIELDS, GRAD_TOL, IMG_TOL, log, np_, rel
from jax_gs_amd import Camera, Gaussians, render
from jax_gs_amd.renderer import rasterizer
from jax_gs_amd.renderer.projection import preprocess
from test_golden import CASES, load

pytestmark = pytest.mark.gpu


def _torch_inputs(params, cam, mask, cuda, w2c_grad=False):
    g = Gaussians(*[torch.from_numpy(params[f]).to(cuda).requires_grad_(True) for f in FIELDS])
    w2c = torch.from_numpy(cam["W2C"]).to(cuda)
    if w2c_grad:
        w2c.requires_grad_(True)
    c = Camera(W=cam["W"], H=cam["H"], fx=cam["fx"], fy=cam["fy"], cx=cam["cx"], cy=cam["cy"], W2C=w2c,
               full_proj=torch.eye(4, device=cuda))
    return g, c, torch.from_numpy(mask).to(cuda)


@pytest.mark.parametrize("name", CASES)
def test_hip_path_reproduces_the_fixture(cuda, name):
    log(f"golden {name}")
    z, params, cam, deg, mask = load(name)
    g, c, m = _torch_inputs(params, cam, mask, cuda, w2c_grad=True)
    with torch.no_grad():
        pre = preprocess(g, c, mask=m, sh_degree=deg)
    for k in ("means2d", "radii", "depths", "colors"):
        np.testing.assert_array_equal(np_(pre[k]), z[k], err_msg=k)
    np.testing.assert_array_equal(np_(pre["valid"]).astype(bool), z["valid"])
    st, sg, n = rasterizer.get_tile_interactions(pre["means2d"], pre["radii"], pre["valid"], pre["depths"],
                                                 cam["H"], cam["W"])
    np.testing.assert_array_equal(np_(st), z["sorted_tiles"])
    np.testing.assert_array_equal(np_(sg), z["sorted_gids"])
    assert int(n) == int(z["n_interactions"])
    with torch.no_grad():
        b = rasterizer.bin_gaussians(pre["means2d"], pre["radii"], pre["valid"], pre["depths"], cam["H"], cam["W"],
                                     window=True)
        bg = torch.zeros(3, device=cuda)
        img, fT, nc, _ = rasterizer.composite(pre["records"], b["sorted_gids"], b["ranges"], cam["H"], cam["W"], bg,
                                              window=b["window"])
    np.testing.assert_array_equal(np_(nc), z["n_contrib"])
    assert float(np.abs(np_(img) - z["image"]).max()) <= IMG_TOL
    for tpu, key in ((False, "image"), (True, "image_tpu")):
        g2, c2, m2 = _torch_inputs(params, cam, mask, cuda, w2c_grad=not tpu)
        image, extras = render(g2, c2, mask=m2, sh_degree=deg, fast_tpu_rasterizer=tpu)
        assert float(np.abs(np_(image) - z[key]).max()) <= IMG_TOL, key
        assert int(extras["n_interactions"]) == int(z["n_interactions"])
        if not tpu:
            image.backward(torch.from_numpy(z["g_image"]).to(cuda))
            for f in FIELDS:
                assert rel(np_(getattr(g2, f).grad), z["grad_" + f]) <= GRAD_TOL, f
            assert rel(np_(c2.W2C.grad), z["grad_W2C"]) <= GRAD_TOL
