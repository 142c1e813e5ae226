"""The committed golden fixtures (tests/golden/, written by make_golden.py) against the CPU
oracle: the forward outputs of the float32 restatement bit for bit (projection, the full
get_tile_interactions arrays, both compositing paths' images, n_contrib), and the float64
cotangents of the fixed image cotangent (five Gaussian arrays and W2C)."""
import os

import numpy as np
import pytest

import oracle

_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CASES = sorted(f[:-4] for f in os.listdir(_DIR) if f.endswith(".npz"))
FIELDS = ("means", "scales", "quaternions", "opacities", "sh_coeffs")


def load(name):
    z = np.load(os.path.join(_DIR, name + ".npz"))
    params = {k: z["in_" + k] for k in FIELDS}
    cam = dict(W=int(z["W"]), H=int(z["H"]), fx=float(z["fx"]), fy=float(z["fy"]), cx=float(z["cx"]),
               cy=float(z["cy"]), W2C=z["W2C"])
    return z, params, cam, int(z["sh_degree"]), z["mask"]


def test_fixtures_present():
    assert set(CASES) == {"small_sh3", "oblique_behind_masked"}


@pytest.mark.parametrize("name", CASES)
def test_oracle_reproduces_the_fixture(name):
    z, params, cam, deg, mask = load(name)
    img, ex, res = oracle.render(params, cam, mask=mask, sh_degree=deg)
    pre = res["pre"]
    for k in ("means2d", "radii", "depths", "colors"):
        np.testing.assert_array_equal(pre[k], z[k], err_msg=k)
    np.testing.assert_array_equal(pre["valid"], z["valid"])
    np.testing.assert_array_equal(res["sorted_tiles"], z["sorted_tiles"])
    np.testing.assert_array_equal(res["sorted_gids"], z["sorted_gids"])
    assert ex["n_interactions"] == int(z["n_interactions"])
    np.testing.assert_array_equal(img, z["image"])
    np.testing.assert_array_equal(res["n_contrib"], z["n_contrib"])
    img_t, _, _ = oracle.render(params, cam, mask=mask, sh_degree=deg, tpu_gather=True)
    np.testing.assert_array_equal(img_t, z["image_tpu"])
    p64 = {k: v.astype(np.float64) for k, v in params.items()}
    c64 = dict(cam, W2C=cam["W2C"].astype(np.float64))
    _, _, r64 = oracle.render(p64, c64, mask=mask, sh_degree=deg, dtype=np.float64)
    g = oracle.render_vjp(p64, c64, r64, z["g_image"].astype(np.float64), sh_degree=deg, dtype=np.float64)
    for k in FIELDS + ("W2C",):
        want = z["grad_" + k]
        assert np.linalg.norm(g[k] - want) <= 1e-10 * max(np.linalg.norm(want), 1e-30), k
    # the scenes exercise what they are meant to
    if name == "oblique_behind_masked":
        assert (z["depths"] < 0).sum() == 3 and not z["mask"].all() and not np.allclose(z["W2C"], np.eye(4))
        assert np.abs(z["grad_W2C"][:3]).max() > 0
