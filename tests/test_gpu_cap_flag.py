"""The compositing records' cap flag on long thin ("needle") Gaussians, on the GPU.

composite_bwd_wide_kernel (images of 2048 tiles or more) skips the 0.99 alpha cap
(rasterizer.py:211) for records whose slot 11 holds 1.0 (gs::record_cannot_cap: the conic
is positive definite and log2(op) plus a bound of the exponent's float32 rounding stays
below log2(0.99)).  Needles at opacities 0.95-0.98 are where a rule that ignores the rounding
fails: the exponent's terms reach 1e5 and more along the needle and cancel, so gated pixels
reach exp2(q) >= 0.99 although op < 0.98.  The CPU fuzz (tests/cap_fuzz.cpp) checks the flag
against the kernels' own expressions; here the scene is rendered and differentiated on the
GPU:
  * the scene holds such pixels (checked on the host from the GPU's own records and entry
    list, with the kernels' expression for q), so the flag decides something;
  * those needles' records carry 0.0, ordinary records 1.0;
  * the backward with the flags as written equals the backward with every flag cleared
    (the per-wave cap test for every entry), and all gradients are finite;
  * against the oracle: the image within 1e-4 outside the needles' tiles and the gradients
    within 1e-3 for the Gaussians with no entry in them.  Inside, the reference's own
    power expression and the kernels' exponent round differently by whole percent of
    alpha (the terms cancel from 1e5), so the oracle is no bar there; the errors are logged.
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_helpers import FIELDS, GRAD_TOL, IMG_TOL, log, np_, rel
from jax_gs_amd import _lib, scenes
from jax_gs_amd.renderer import rasterizer
from jax_gs_amd.renderer.projection import preprocess

pytestmark = pytest.mark.gpu
F32 = np.float32
L2E = F32(1.4426950408889634)


def _fma32(a, b, c):
    # float32 fused multiply-add: the float64 product of two float32 values is exact
    return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(F32)


def _q_kernel(rec, px, py):
    """The kernels' exponent (gs_cull.h q_of with the shared row terms) for one record."""
    mx, my, A, B, C, lop = (F32(v) for v in rec[:6])
    dx = (px - mx).astype(F32)
    adx = (A * dx).astype(F32)
    adx2l = _fma32(adx, dx, np.full_like(dx, lop))
    bdx = (B * dx).astype(F32)
    dy = (py - my).astype(F32)
    return _fma32(_fma32(np.full_like(dy, C), dy, bdx), dy, adx2l)


def _needle_scene(n=20000, n_needles=400):
    """cfg1-family Gaussians on a 1024 x 768 image (3072 tiles: the wide backward) and
    n_needles needles: one axis of 2000-3000 px (projected), the others 1e-4 (the 0.3
    low-pass then sets the width, 0.55 px), at 40-50 degrees in the image, centred on the
    diagonal 400-700 px from the corner, opacity 0.95-0.98.  The binning gives each one the
    image's top-left 16 x 16 tiles (its rectangle clipped, first 16 tiles a side), 550-1000 px
    from its centre along its axis: there the exponent's terms reach 1e5 and cancel."""
    sc = scenes.make_scene(1, n=n, width=1024, height=768, seed=31)
    rng = np.random.default_rng(32)
    p = sc["params"]
    c = sc["cam"]
    f = c["fx"]
    idx = rng.choice(n, n_needles, replace=False)
    z = rng.uniform(3.0, 6.0, n_needles)
    m = rng.uniform(400.0, 700.0, n_needles)
    px = m + rng.uniform(-20.0, 20.0, n_needles)
    py = m + rng.uniform(-20.0, 20.0, n_needles)
    p["means"][idx] = np.stack([(px - c["cx"]) * z / f, (py - c["cy"]) * z / f, z], 1).astype(F32)
    s = np.full((n_needles, 3), np.log(1e-4), F32)
    s[:, 0] = np.log(rng.uniform(2000.0, 3000.0, n_needles) * z / f).astype(F32)
    p["scales"][idx] = s
    th = np.radians(rng.uniform(40.0, 50.0, n_needles))  # about the camera's z axis
    zero = np.zeros(n_needles)
    p["quaternions"][idx] = np.stack([np.cos(th / 2), zero, zero, np.sin(th / 2)], 1).astype(F32)
    op = rng.uniform(0.95, 0.98, n_needles)
    p["opacities"][idx, 0] = np.log(op / (1.0 - op)).astype(F32)
    return sc, np.sort(idx)


def _bwd(rec, b, H, W, bg, seed, fT, nc, order, n):
    dev = rec.device
    grec = torch.empty((n, _lib.GS_REC_STRIDE), dtype=torch.float32, device=dev)
    gbg = torch.empty((3,), dtype=torch.float32, device=dev)
    _lib.call("gs_composite_bwd", _lib.stream_handle(dev), n, _lib.ptr(rec), _lib.ptr(b["sorted_gids"]),
              b["sorted_gids"].shape[0], _lib.ptr(b["ranges"]), int(W), int(H), _lib.ptr(bg), _lib.ptr(seed),
              _lib.ptr(fT), _lib.ptr(nc), _lib.ptr(order), _lib.ptr(grec), _lib.ptr(gbg), 0, None, None)
    torch.cuda.synchronize()
    return np_(grec), np_(gbg)


def test_needles_cap_flag_and_wide_backward(cuda):
    sc, needles = _needle_scene()
    c = sc["cam"]
    W, H = c["W"], c["H"]
    n = sc["params"]["means"].shape[0]
    log(f"needles: N={n} ({needles.size} needles) {W}x{H}")
    g, cam, _, _ = scenes.to_torch(sc, cuda)
    with torch.no_grad():
        pre = preprocess(g, cam, sh_degree=sc["sh_degree"])
        b = rasterizer.bin_gaussians(pre["means2d"], pre["radii"], pre["valid"], pre["depths"], H, W)
        bg = torch.zeros(3, device=cuda)
        rec = pre["records"]
        image, fT, nc, order = rasterizer.composite(rec, b["sorted_gids"], b["ranges"], H, W, bg)
    R = np_(rec)
    flag = R[:, 11]
    assert set(np.unique(flag)) <= {0.0, 1.0}
    cov = np_(pre["cov2d"]).astype(np.float64)
    op = R[:, 9]
    pd = (cov[:, 0, 0] > 0) & (cov[:, 0, 0] * cov[:, 1, 1] - cov[:, 0, 1] * cov[:, 1, 0] > 0)
    old_rule = (op < 0.98) & pd
    ordinary = np.setdiff1d(np.arange(n), needles)
    # ordinary Gaussians below 0.98 are flagged; needles mostly are not
    assert flag[ordinary][old_rule[ordinary]].mean() > 0.99
    assert flag[needles].mean() < 0.5
    # the scene has gated pixels above the cap's exponent for needles the old rule calls safe
    n_int = int(np_(b["n_interactions"]))
    st = np_(b["sorted_tiles"][:n_int])
    sg = np_(b["sorted_gids"][:n_int])
    tx = W // 16
    hits = 0
    lane = np.arange(16, dtype=F32) + F32(0.5)
    for gid in needles:
        if not old_rule[gid]:
            continue
        tiles = st[sg == gid]
        if tiles.size == 0:
            continue
        px = ((tiles % tx) * 16).astype(F32)[:, None, None] + lane[None, None, :]
        py = ((tiles // tx) * 16).astype(F32)[:, None, None] + lane[None, :, None]
        px, py = np.broadcast_arrays(px, py)
        q = _q_kernel(R[gid], px.astype(F32), py.astype(F32))
        hits += int(((q > R[gid, 10]) & (q >= F32(-0.015))).sum())
    log(f"gated pixels of old-rule-safe needles at or above the cap's exponent: {hits}")
    assert hits > 0
    # the wide backward (3072 tiles) with the flags as written vs every flag cleared
    seed = torch.from_numpy(np.random.default_rng(11).normal(0, 1, (H, W, 3)).astype(F32)).to(cuda)
    g1, b1 = _bwd(rec, b, H, W, bg, seed, fT, nc, order, n)
    rec0 = rec.clone()
    rec0[:, 11] = 0.0
    g0, b0 = _bwd(rec0, b, H, W, bg, seed, fT, nc, order, n)
    assert np.isfinite(g1).all() and np.isfinite(g0).all()
    e = rel(g1, g0)
    log(f"flags as written vs cleared: gradient records rel L2 {e:.2e}")
    assert e <= 1e-5 and rel(b1, b0) <= 1e-5
    # against the oracle (float32 reference semantics), where the needles do not enter: the
    # pixels outside their tiles, and the Gaussians with no entry in those tiles
    img_o, ex_o, res = oracle.render(sc["params"], c, sh_degree=sc["sh_degree"])
    assert int(ex_o["n_interactions"]) == n_int
    ntiles = np.unique(np.concatenate([st[sg == gid] for gid in needles]))
    touched = np.zeros((H // 16) * tx, bool)
    touched[ntiles] = True
    pix = np.repeat(np.repeat(touched.reshape(H // 16, tx), 16, 0), 16, 1)
    diff = np.abs(np_(image) - img_o)
    log(f"image max-abs {diff.max():.2e} (outside the needles' {ntiles.size} tiles {diff[~pix].max():.2e})")
    assert diff[~pix].max() <= IMG_TOL
    from jax_gs_amd import render

    for f in FIELDS:
        getattr(g, f).requires_grad_(True)
    image2, _ = render(g, cam, sh_degree=sc["sh_degree"])
    image2.backward(seed)
    gr_o = oracle.render_vjp(sc["params"], c, res, np_(seed), sh_degree=sc["sh_degree"])
    far = np.setdiff1d(np.arange(n), np.unique(sg[touched[st]]))
    log(f"{far.size} Gaussians with no entry in the needles' tiles")
    assert far.size > n // 2
    for f in FIELDS:
        a = np_(getattr(g, f).grad)
        assert np.isfinite(a).all(), f
        e_all, e_far = rel(a, gr_o[f]), rel(a[far], gr_o[f][far])
        log(f"{f}: rel L2 {e_all:.1e}, on the Gaussians away from the needles {e_far:.1e}")
        assert e_far <= GRAD_TOL, f
