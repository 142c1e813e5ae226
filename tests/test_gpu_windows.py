"""The reference's default compositing path with its clamped chunk windows, on the GPU.

rasterizer.py:184-190 slices chunk c of tile t at min(start + 512 c, L - 512) of the
L = max(256 N, 512)-slot arrays of get_tile_interactions; a chunk that starts past L - 512
blends the arrays' last 512 slots -- other tiles' entries, Gaussians' empty slots (their
ids in (depth quantum, id) order), the slots of Gaussians behind the camera -- instead of
its own entries.  render(fast_tpu_rasterizer=False) reproduces that through the window of
gs_window_from_bins; fast_tpu_rasterizer=True reads each tile's own entries
(rasterizer_tpu.py:90-97).  Each scene below makes the clamp bite, and the two paths
differ there; each is checked against the oracle's own path (image and every cotangent),
and the window itself against the oracle's full arrays.
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_helpers import FIELDS, GRAD_TOL, IMG_TOL, log, np_, rel
from jax_gs_amd import _lib, render, scenes
from jax_gs_amd.renderer import rasterizer
from jax_gs_amd.renderer.projection import preprocess

pytestmark = pytest.mark.gpu
F32 = np.float32
SH_C0 = 0.28209479177387814


def _scene(means, log_scales, opac, rgb, W, H, f, mask=None):
    n = len(means)
    sh = np.zeros((n, 1, 3), F32)
    sh[:, 0, :] = (np.asarray(rgb, F32) - F32(0.5)) / F32(SH_C0)
    q = np.zeros((n, 4), F32)
    q[:, 0] = 1.0
    params = dict(means=np.asarray(means, F32), scales=np.broadcast_to(np.asarray(log_scales, F32)[:, None],
                                                                        (n, 3)).copy(),
                  quaternions=q, opacities=np.asarray(opac, F32).reshape(n, 1), sh_coeffs=sh)
    cam = dict(W=W, H=H, fx=float(f), fy=float(f), cx=W / 2.0, cy=H / 2.0, W2C=np.eye(4, dtype=F32))
    return dict(params=params, cam=cam, sh_degree=0, target=None, mask=mask, name="window")


def _two():
    """L = 512: every tile but tile 0 starts past L - 512 = 0 and blends entries from
    the front of the list (the other Gaussian's among them)."""
    return _scene([[0.0, 0.0, 5.0], [0.3, 0.25, 4.0]], [-1.3, -1.6], [1.0, 2.0],
                  [[0.9, 0.1, 0.1], [0.1, 0.2, 0.9]], 64, 64, 100.0)


def _two_one_behind():
    """One Gaussian behind the camera: its 256 slots (tile -1) open the arrays, so every
    chunk (thr = -256 in the list's coordinates) blends it."""
    return _scene([[0.0, 0.0, 5.0], [0.1, -0.1, -3.0]], [-1.2, -1.0], [1.5, 1.0],
                  [[0.9, 0.8, 0.1], [0.1, 0.9, 0.4]], 64, 64, 100.0)


def _three_two_behind():
    """Two behind the camera: the window opens with the second of them in (depth
    quantum, id) order (z = -5 sorts after z = -3), then the entries and the empty slots."""
    return _scene([[0.05, 0.0, -3.0], [0.0, 0.05, 5.0], [-0.05, 0.0, -5.0]], [-1.0, -1.2, -0.8], [1.0, 1.5, 1.0],
                  [[0.9, 0.1, 0.1], [0.2, 0.9, 0.2], [0.1, 0.1, 0.9]], 64, 64, 100.0)


def _big(seed=0):
    """304 Gaussians, 300 of them covering 16x16 tiles of a 512x512 image, one more
    reaching three further tile rows and columns alone (its last tiles hold one entry each),
    one masked out (256 empty slots) and two behind the camera (256 slots each, tile -1):
    fewer than 512 empty slots in all, so the last tiles' chunks are clamped."""
    rng = np.random.default_rng(seed)
    m = np.zeros((304, 3), F32)
    m[:300, :2] = rng.uniform(-0.05, 0.05, (300, 2))
    m[:300, 2] = rng.uniform(4.8, 5.2, 300)
    m[300] = [0.6, 0.6, 5.0]
    m[301] = [0.0, 0.0, 5.0]
    m[302] = [0.1, 0.0, -4.0]
    m[303] = [0.0, 0.1, -6.0]
    opac = rng.uniform(-4.5, -3.5, 304)
    rgb = rng.uniform(0.0, 1.0, (304, 3))
    mask = np.ones(304, bool)
    mask[301] = False
    return _scene(m, np.zeros(304), opac, rgb, 512, 512, 400.0, mask=mask)


CASES = {"two": _two, "two_one_behind": _two_one_behind, "three_two_behind": _three_two_behind, "big": _big}


def _oracle_layout(sc):
    c = sc["cam"]
    pre = oracle.preprocess(sc["params"]["means"], sc["params"]["scales"], sc["params"]["quaternions"],
                            sc["params"]["sh_coeffs"], c["W2C"], c["W"], c["H"], F32(c["fx"]), F32(c["fy"]),
                            F32(c["cx"]), F32(c["cy"]), 0, mask=sc["mask"])
    st, sg, _ = oracle.tile_interactions(pre["means2d"], pre["radii"], pre["valid"], pre["depths"], c["H"], c["W"])
    return pre, st, sg


def _clamped(st, T):
    """Whether some tile's chunk starts past L - 512 (rasterizer.py:169-190)."""
    L = st.shape[0]
    b = oracle.tile_boundaries(st, T)
    for t in range(T):
        cnt = min(int(b[t + 1] - b[t]), 4096)
        if cnt > 0 and int(b[t]) + 512 * ((cnt - 1) // 512) > L - 512:
            return True
    return False


@pytest.mark.parametrize("case", list(CASES))
def test_window_from_bins_is_the_reference_tail(cuda, case):
    """gs_window_from_bins: thr = L - 512 - 256 (behind the camera), ids = the oracle's
    full arrays' last 512 slots, and the clamp flag in the stats as the arrays set it."""
    sc = CASES[case]()
    log(f"window case={case}")
    g, cam, _, m = scenes.to_torch(sc, cuda)
    with torch.no_grad():
        pre = preprocess(g, cam, mask=m, sh_degree=0)
        b = rasterizer.bin_gaussians(pre["means2d"], pre["radii"], pre["valid"], pre["depths"], cam.H, cam.W,
                                     window=True)
    pre_o, st, sg = _oracle_layout(sc)
    T = ((cam.W + 15) // 16) * ((cam.H + 15) // 16)
    n_neg = int(np.signbit(pre_o["depths"]).sum())
    L = st.shape[0]
    assert L == max(256 * len(pre_o["depths"]), 512)
    win = np_(b["window"])
    thr = int(win[:8].view(np.int64)[0])
    assert thr == L - 512 - 256 * n_neg
    flag = int(np_(b["stats"])[_lib.STAT["window_clamped"]])
    assert flag == int(_clamped(st, T)) == 1
    np.testing.assert_array_equal(win[16:].view(np.int32), sg[L - 512:])


@pytest.mark.parametrize("case", list(CASES))
def test_render_paths_match_the_oracle(cuda, case):
    """render with the default rasterizer (clamped windows) and with fast_tpu_rasterizer
    against the oracle's two paths: image and the five cotangents."""
    sc = CASES[case]()
    g0, cam, _, m = scenes.to_torch(sc, cuda)
    imgs = {}
    for tpu in (False, True):
        log(f"render case={case} fast_tpu_rasterizer={tpu}")
        g = type(g0)(*[getattr(g0, f).detach().clone().requires_grad_(True) for f in FIELDS])
        image, extras = render(g, cam, mask=m, sh_degree=0, fast_tpu_rasterizer=tpu)
        img_o, _, res = oracle.render(sc["params"], sc["cam"], mask=sc["mask"], tpu_gather=tpu)
        err = float(np.abs(np_(image) - img_o).max())
        assert err <= IMG_TOL, (tpu, err)
        seed = np.random.default_rng(3).normal(0, 1, img_o.shape).astype(F32)
        image.backward(torch.from_numpy(seed).to(cuda))
        gr_o = oracle.render_vjp(sc["params"], sc["cam"], res, seed, tpu_gather=tpu)
        for f in FIELDS:
            e = rel(np_(getattr(g, f).grad), gr_o[f])
            assert e <= GRAD_TOL, (tpu, f, e)
        imgs[tpu] = img_o
    # the clamp changes the image: the default path is not the per-tile one here
    assert np.abs(imgs[False] - imgs[True]).max() > 1e-3


def test_window_from_list_matches_caller_arrays(cuda):
    """gs_window_from_list on a list of 700 ids: thr = 188 and the last 512 ids; a list
    shorter than 512 is never clamped."""
    ids = torch.arange(700, dtype=torch.int32, device=cuda) * 3
    win = np_(rasterizer.window_from_list(ids))
    assert int(win[:8].view(np.int64)[0]) == 188
    np.testing.assert_array_equal(win[16:].view(np.int32), np_(ids)[188:])
    win = np_(rasterizer.window_from_list(ids[:100].contiguous()))
    assert int(win[:8].view(np.int64)[0]) == np.iinfo(np.int64).max
