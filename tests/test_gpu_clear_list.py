"""The compositing VJP's clear list and the preprocessing VJP's zeroed mode.

render's backward lets gs_composite_bwd set the five cotangent arrays to zero on the side
(gs_clear_list_t) and calls gs_preprocess_bwd with zeroed = 1, which then writes only the
rows of the Gaussians some pixel reached.  Checked here through the C ABI:
  * every listed array is zero afterwards, also arrays whose start is not 16-byte aligned
    and whose length is not a multiple of four floats, and the floats just outside them are
    untouched;
  * the gradient records are those of a launch without a clear list, up to the order of the
    launch's float atomics (the clear stores come after each workgroup's walk);
  * gs_preprocess_bwd(zeroed = 1) on cleared arrays writes the same arrays, bit for bit, as
    gs_preprocess_bwd(zeroed = 0) on arrays full of NaN, with and without the camera
    cotangent (the reference's VJP, projection.py:6-79 with renderer.py:40-49, the same either
    way; its parity with the oracle is what the render tests check);
  * bad clear lists are rejected before anything is launched.
"""
import ctypes

import numpy as np
import pytest
import torch

from gpu_helpers import FIELDS, log, np_, rel
from jax_gs_amd import _lib, scenes
from jax_gs_amd.renderer import rasterizer
from jax_gs_amd.renderer.projection import preprocess

pytestmark = pytest.mark.gpu

# two launches of the compositing VJP add their float atomics in different orders
ATOMIC_ORDER_TOL = 2e-5


def _scene(cuda, cfg, n, w, h):
    sc = scenes.make_scene(cfg, n=n, width=w, height=h)
    g, cam, _, m = scenes.to_torch(sc, cuda)
    pre = preprocess(g, cam, mask=m, sh_degree=sc["sh_degree"], records=True, projected=False)
    b = rasterizer.bin_gaussians(pre["means2d"], pre["radii"], pre["valid"], pre["depths"], cam.H, cam.W,
                                 want_tiles=False, window=True, deferred=True)
    bg = torch.zeros(3, device=cuda)
    image, fT, nc, order = rasterizer.composite(pre["records"], b["sorted_gids"], b["ranges"], cam.H, cam.W, bg,
                                                residuals=True, window=b["window"], bins=b)[:4]
    seed = torch.from_numpy(np.random.default_rng(11).normal(0, 1, (cam.H, cam.W, 3)).astype(np.float32)).to(cuda)
    return sc, g, cam, pre, b, bg, fT, nc, order, seed


def _composite_bwd(cuda, pre, b, cam, bg, seed, fT, nc, order, clear):
    n = pre["records"].shape[0]
    grec = torch.empty((n, _lib.GS_REC_STRIDE), device=cuda)
    _lib.call("gs_composite_bwd", _lib.stream_handle(cuda), n, _lib.ptr(pre["records"]), _lib.ptr(b["sorted_gids"]),
              b["sorted_gids"].shape[0], _lib.ptr(b["ranges"]), cam.W, cam.H, _lib.ptr(bg), _lib.ptr(seed),
              _lib.ptr(fT), _lib.ptr(nc), _lib.ptr(order), _lib.ptr(grec), None, 0, _lib.ptr(b["window"]),
              None if clear is None else ctypes.byref(clear))
    return grec


@pytest.mark.parametrize("cfg,n,w,h", [(2, 30000, 1024, 768), (1, 4000, 200, 150)])
def test_clear_list_zeroes_every_listed_array(cuda, cfg, n, w, h):
    """Four-pixel (3072 tiles) and one-pixel (130 tiles) builds; arrays at offsets 0..3 floats
    from an aligned start, of lengths 0, 1, 3, 5 and larger odd ones."""
    sc, g, cam, pre, b, bg, fT, nc, order, seed = _scene(cuda, cfg, n, w, h)
    log(f"clear list: cfg{cfg} n={n} {w}x{h}")
    lengths = [12345, 3 * n + 1, 7, 1, 0, 5, 3, 100003]
    bufs, views = [], []
    for i, ln in enumerate(lengths):
        off = i % 4
        buf = torch.full((ln + off + 8,), 7.0, device=cuda)
        bufs.append((buf, off, ln))
        views.append(buf[off:off + ln])
    cl = _lib.clear_list(*views)
    g_ref = _composite_bwd(cuda, pre, b, cam, bg, seed, fT, nc, order, None)
    g_cl = _composite_bwd(cuda, pre, b, cam, bg, seed, fT, nc, order, cl)
    torch.cuda.synchronize()
    assert rel(np_(g_cl), np_(g_ref)) <= ATOMIC_ORDER_TOL
    for buf, off, ln in bufs:
        a = np_(buf)
        assert (a[off:off + ln] == 0.0).all(), (off, ln)
        assert (a[:off] == 7.0).all() and (a[off + ln:] == 7.0).all(), (off, ln)


@pytest.mark.parametrize("w2c_grad", [False, True])
def test_preprocess_bwd_zeroed_matches_the_full_write(cuda, w2c_grad):
    sc, g, cam, pre, b, bg, fT, nc, order, seed = _scene(cuda, 2, 20000, 640, 480)
    n = g.means.shape[0]
    grec = _composite_bwd(cuda, pre, b, cam, bg, seed, fT, nc, order, None)
    reached = int((np_(grec)[:, :9] != 0).any(axis=1).sum())
    log(f"preprocess VJP zeroed: {reached} of {n} Gaussians reached, camera cotangent {w2c_grad}")
    assert 0 < reached < n
    params = [getattr(g, f).detach().contiguous() for f in FIELDS]
    w2c = torch.as_tensor(cam.W2C, dtype=torch.float32, device=cuda).contiguous()
    outs = {}
    for zeroed in (0, 1):
        arrs = [torch.full_like(p, float("nan")) for p in params]
        if zeroed:
            cl = _lib.clear_list(*arrs)
            _composite_bwd(cuda, pre, b, cam, bg, seed, fT, nc, order, cl)
        args = (_lib.stream_handle(cuda), n, params[4].shape[1], sc["sh_degree"], *[_lib.ptr(p) for p in params],
                _lib.ptr(w2c), cam.W, cam.H, float(cam.fx), float(cam.fy), float(cam.cx), float(cam.cy),
                _lib.ptr(grec), *[_lib.ptr(a) for a in arrs])
        gw = None
        if w2c_grad:
            gw = torch.empty((4, 4), device=cuda)
            nb = _lib.lib().gs_preprocess_bwd_w2c_workspace_size(n)
            ws = torch.empty((nb,), dtype=torch.uint8, device=cuda)
            _lib.call("gs_preprocess_bwd_w2c", *args, _lib.ptr(gw), _lib.ptr(ws), nb, zeroed)
        else:
            _lib.call("gs_preprocess_bwd", *args, zeroed)
        torch.cuda.synchronize()
        outs[zeroed] = ([np_(a) for a in arrs], None if gw is None else np_(gw))
    for f, a0, a1 in zip(FIELDS, outs[0][0], outs[1][0]):
        assert not np.isnan(a1).any(), f
        assert np.array_equal(a0, a1), f
    if w2c_grad:
        assert np.array_equal(outs[0][1], outs[1][1])


def test_bad_clear_lists_are_rejected(cuda):
    sc, g, cam, pre, b, bg, fT, nc, order, seed = _scene(cuda, 1, 1000, 128, 96)
    cl = _lib.ClearList()
    cl.count[2] = -1
    with pytest.raises(ValueError, match="negative count"):
        _composite_bwd(cuda, pre, b, cam, bg, seed, fT, nc, order, cl)
    cl = _lib.ClearList()
    cl.count[5] = 10  # NULL pointer with a count
    with pytest.raises(ValueError, match="is NULL"):
        _composite_bwd(cuda, pre, b, cam, bg, seed, fT, nc, order, cl)
    with pytest.raises(ValueError):
        _lib.clear_list(torch.zeros(4, dtype=torch.float64, device=cuda))
