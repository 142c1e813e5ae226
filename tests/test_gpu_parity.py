"""GPU parity: the HIP path (through the C ABI) against the CPU oracle.

The bars and the reference-order note are in gpu_helpers.py; scenes here are the
configurations' families at reduced sizes plus the full sizes of configurations 0 and 1
(configurations 2-4 at full size: test_gpu_fullsize.py).
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_helpers import FIELDS, GRAD_TOL, IMG_TOL
from gpu_helpers import check_binning as _check_binning
from gpu_helpers import check_preprocess as _check_preprocess
from gpu_helpers import np_ as _np
from gpu_helpers import rel as _rel
from gpu_helpers import render_both as _render_both
from jax_gs_amd import render, scenes
from jax_gs_amd.renderer import rasterizer
from jax_gs_amd.renderer.projection import preprocess

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("cfg,n,w,h", [(0, 3000, 128, 96), (1, 4000, 200, 150), (3, 6000, 160, 96),
                                       (4, 5000, 160, 90), (2, 3000, 1024, 768)])
def test_small_scene_parity(cuda, cfg, n, w, h):
    sc = scenes.make_scene(cfg, n=n, width=w, height=h)
    pre, pre_o = _check_preprocess(sc, cuda)
    _check_binning(sc, cuda, pre, pre_o)
    image, extras, g, img_o, ex_o, gr_o = _render_both(sc, cuda)
    assert np.abs(_np(image) - img_o).max() <= IMG_TOL
    assert int(extras["n_interactions"]) == ex_o["n_interactions"]
    np.testing.assert_array_equal(_np(extras["radii"]), ex_o["radii"])
    np.testing.assert_array_equal(_np(extras["valid_mask"]), ex_o["valid_mask"])
    for f in FIELDS:
        assert _rel(_np(getattr(g, f).grad), gr_o[f]) <= GRAD_TOL, f


def test_cfg0_full_forward(cuda):
    """Configuration 0 at full size: preprocessing + binning bit-exact, image <= 1e-4."""
    sc = scenes.make_scene(0)
    pre, pre_o = _check_preprocess(sc, cuda)
    _check_binning(sc, cuda, pre, pre_o)
    g, cam, _, _ = scenes.to_torch(sc, cuda)
    image, extras = render(g, cam, sh_degree=0)
    img_o, ex_o, _ = oracle.render(sc["params"], sc["cam"], sh_degree=0)
    assert np.abs(_np(image) - img_o).max() <= IMG_TOL
    for k in ("n_interactions", "max_interactions_per_tile", "overflow_tiles", "overflow_interactions",
              "truncated_tiles", "truncated_interactions", "radius_cap_violations"):
        assert int(extras[k]) == int(ex_o[k]), k
    assert float(extras["mean_interactions_per_tile"]) == float(ex_o["mean_interactions_per_tile"])


def test_cfg1_full_fwd_bwd(cuda):
    """Configuration 1 at full size: 200k Gaussians, SH3, 504x378, L1 seed."""
    sc = scenes.make_scene(1)
    pre, pre_o = _check_preprocess(sc, cuda)
    _check_binning(sc, cuda, pre, pre_o)
    image, extras, g, img_o, ex_o, gr_o = _render_both(sc, cuda)
    assert np.abs(_np(image) - img_o).max() <= IMG_TOL
    for f in FIELDS:
        assert _rel(_np(getattr(g, f).grad), gr_o[f]) <= GRAD_TOL, f


@pytest.mark.parametrize("cfg,n,w,h", [(1, 20000, 4400, 2600), (3, 30000, 2100, 2100), (1, 20000, 5200, 5200)])
def test_binning_large_image(cuda, cfg, n, w, h):
    """Images with more than 256 superblocks of 8x8 tiles (two-pass superblock sort); the
    5200x5200 case has more than 1024 (chunk and segment maps filled per superblock)."""
    sc = scenes.make_scene(cfg, n=n, width=w, height=h)
    pre, pre_o = _check_preprocess(sc, cuda)
    b, _ = _check_binning(sc, cuda, pre, pre_o)
    S = (((w + 15) // 16 + 7) // 8) * (((h + 15) // 16 + 7) // 8)
    assert S > 256


def test_cfg3_truncated_tiles(cuda):
    """Clustered scene whose densest tiles exceed the 4096-entry compositing cap."""
    sc = scenes.make_scene(3, n=60000, width=320, height=180)
    pre, pre_o = _check_preprocess(sc, cuda)
    b, _ = _check_binning(sc, cuda, pre, pre_o)
    assert int(_np(b["stats"])[4]) > 0  # truncated tiles present
    image, extras, g, img_o, ex_o, gr_o = _render_both(sc, cuda)
    assert np.abs(_np(image) - img_o).max() <= IMG_TOL
    for f in FIELDS:
        assert _rel(_np(getattr(g, f).grad), gr_o[f]) <= GRAD_TOL, f


@pytest.mark.parametrize("shape,offset", [((96, 128, 3), 0), ((37, 41, 3), 0), ((37, 41, 3), 1)])
def test_l1_loss(cuda, shape, offset):
    """losses.py:4-8: loss and its gradient seed against the oracle (vector path, odd
    sizes, and a misaligned view that takes the scalar path)."""
    from jax_gs_amd.training.losses import l1_loss

    rng = np.random.default_rng(3)
    count = int(np.prod(shape))
    pred_np = rng.uniform(0, 1, count + offset).astype(np.float32)
    tgt_np = rng.uniform(0, 1, count + offset).astype(np.float32)
    tgt_np[offset + 5] = pred_np[offset + 5]  # a zero difference: sign 0
    pred = torch.from_numpy(pred_np).to(cuda)[offset:].view(shape).requires_grad_(True)
    tgt = torch.from_numpy(tgt_np).to(cuda)[offset:].view(shape)
    loss = l1_loss(pred, tgt)
    loss.backward()
    want, seed = oracle.l1_loss_and_grad(pred_np[offset:].reshape(shape), tgt_np[offset:].reshape(shape))
    got = float(loss.detach())
    assert abs(got - float(want)) <= 1e-6 * max(1.0, abs(float(want)))
    np.testing.assert_array_equal(_np(pred.grad), seed)


@pytest.mark.parametrize("kind", ["l1", "mse"])
def test_loss_vjp_with_cotangent(cuda, kind):
    """The loss VJP reads the cotangent on the device: (2.5 * loss).backward() gives
    seed(pred - target) * (2.5 / count), the mean's VJP dividing the cotangent by the
    count first (losses.py:4-14 under jax.grad), bit for bit in float32."""
    from jax_gs_amd.training.losses import l1_loss, mse_loss

    rng = np.random.default_rng(11)
    shape = (45, 67, 3)
    p_np = rng.uniform(0, 1, shape).astype(np.float32)
    t_np = rng.uniform(0, 1, shape).astype(np.float32)
    t_np[3, 4, 1] = p_np[3, 4, 1]
    pred = torch.from_numpy(p_np).to(cuda).requires_grad_(True)
    tgt = torch.from_numpy(t_np).to(cuda)
    loss = (l1_loss if kind == "l1" else mse_loss)(pred, tgt)
    (2.5 * loss).backward()
    d = p_np - t_np
    sc = np.float32(2.5) / np.float32(d.size)
    want = (np.sign(d) if kind == "l1" else np.float32(2.0) * d).astype(np.float32) * sc
    np.testing.assert_array_equal(_np(pred.grad), want.astype(np.float32))


def test_background_forward_and_grad(cuda):
    """A coloured background (rasterizer.py:244, C + T * bg) and its cotangent."""
    sc = scenes.make_scene(1, n=4000, width=200, height=150)
    bg_np = np.array([0.2, 0.5, 0.9], np.float32)
    g, cam, _, _ = scenes.to_torch(sc, cuda)
    for f in FIELDS:
        getattr(g, f).requires_grad_(True)
    bg = torch.from_numpy(bg_np).to(cuda).requires_grad_(True)
    image, _ = render(g, cam, background=bg, sh_degree=sc["sh_degree"])
    img_o, _, res = oracle.render(sc["params"], sc["cam"], background=bg_np, sh_degree=sc["sh_degree"])
    assert np.abs(_np(image) - img_o).max() <= IMG_TOL
    seed = np.random.default_rng(5).normal(0, 1, img_o.shape).astype(np.float32)
    image.backward(torch.from_numpy(seed).to(cuda))
    gr_o = oracle.render_vjp(sc["params"], sc["cam"], res, seed, sh_degree=sc["sh_degree"])
    assert _rel(_np(bg.grad), gr_o["background"]) <= GRAD_TOL
    for f in FIELDS:
        assert _rel(_np(getattr(g, f).grad), gr_o[f]) <= GRAD_TOL, f


def test_cfg4_masked_step_with_densify_accumulators(cuda):
    """Configuration 4's step on a small scene: masked render, backward, then the
    densification statistics (trainer.py:143-159) against the oracle's."""
    from jax_gs_amd.training.trainer import accumulate_from_extras

    sc = scenes.make_scene(4, n=6000, width=160, height=96)
    image, extras, g, img_o, ex_o, gr_o = _render_both(sc, cuda)
    assert np.abs(_np(image) - img_o).max() <= IMG_TOL
    n = sc["params"]["means"].shape[0]
    state = {"grad_accum": torch.full((n,), 0.25, device=cuda), "denom": torch.ones(n, dtype=torch.int32, device=cuda),
             "max_radii": torch.full((n,), 2.0, device=cuda)}
    _, cam, _, m = scenes.to_torch(sc, cuda)
    accumulate_from_extras(state, g.means.grad, g.means.detach(), cam, extras, active=m)
    c = sc["cam"]
    ga, de, mr = oracle.densify(gr_o["means"], sc["params"]["means"], c["W2C"], c["fx"], c["fy"], c["W"], c["H"],
                                ex_o["valid_mask"], ex_o["radii"], np.full(n, 0.25, np.float32),
                                np.ones(n, np.int32), np.full(n, 2.0, np.float32), active=sc["mask"])
    np.testing.assert_array_equal(_np(state["denom"]), de)
    np.testing.assert_array_equal(_np(state["max_radii"]), mr)
    assert _rel(_np(state["grad_accum"]), ga) <= GRAD_TOL


def test_render_backward_twice(cuda):
    """The forward clears the gradient records its backward accumulates into; a second
    backward through a retained graph starts from fresh records, so the parameter
    gradients of two backward calls are twice those of one."""
    sc = scenes.make_scene(1, n=4000, width=200, height=150)
    g, cam, _, m = scenes.to_torch(sc, cuda)
    for f in FIELDS:
        getattr(g, f).requires_grad_(True)
    image, _ = render(g, cam, mask=m, sh_degree=sc["sh_degree"])
    seed = torch.from_numpy(np.random.default_rng(5).normal(0, 1, tuple(image.shape)).astype(np.float32)).to(cuda)
    image.backward(seed, retain_graph=True)
    once = {f: _np(getattr(g, f).grad).copy() for f in FIELDS}
    image.backward(seed)
    for f in FIELDS:
        assert _rel(_np(getattr(g, f).grad), 2.0 * once[f]) <= 1e-5, f


@pytest.mark.parametrize("cfg", [1, 2])
def test_backward_tile_order(cuda, cfg):
    """The forward's tile order (tiles by decreasing walk length) is a permutation of
    the tiles, and the backward launched in that order equals the backward in the fixed
    order up to the order of the gradient additions (one and four waves per tile)."""
    from jax_gs_amd import _lib
    from jax_gs_amd.renderer._buffers import num_tiles

    sc = scenes.make_scene(cfg)
    g, cam, _, mask = scenes.to_torch(sc, cuda)
    W, H = cam.W, cam.H
    with torch.no_grad():
        pre = preprocess(g, cam, mask=mask, sh_degree=sc["sh_degree"])
        b = rasterizer.bin_gaussians(pre["means2d"], pre["radii"], pre["valid"], pre["depths"], H, W,
                                     want_tiles=False)
        bg = torch.zeros(3, device=cuda)
        image, fT, nc, order = rasterizer.composite(pre["records"], b["sorted_gids"], b["ranges"], H, W, bg)
        _, _, T = num_tiles(W, H)
        assert order.shape == (T,)
        assert np.array_equal(np.sort(_np(order)), np.arange(T))
        gimg = torch.from_numpy(np.random.default_rng(7).normal(0, 1, (H, W, 3)).astype(np.float32)).to(cuda)
        n = pre["records"].shape[0]
        out = []
        for o in (order, None):
            grec = torch.empty((n, _lib.GS_REC_STRIDE), device=cuda)
            gbg = torch.empty(3, device=cuda)
            _lib.call("gs_composite_bwd", _lib.stream_handle(cuda), n, _lib.ptr(pre["records"]),
                      _lib.ptr(b["sorted_gids"]), b["sorted_gids"].shape[0], _lib.ptr(b["ranges"]), W, H, _lib.ptr(bg),
                      _lib.ptr(gimg), _lib.ptr(fT), _lib.ptr(nc), _lib.ptr(o), _lib.ptr(grec), _lib.ptr(gbg), 0, None, None)
            out.append((_np(grec), _np(gbg)))
        # records cleared by the forward, then accumulated into (twice: the sum doubles)
        grec = torch.full((n, _lib.GS_REC_STRIDE), float("nan"), device=cuda)
        rasterizer.composite(pre["records"], b["sorted_gids"], b["ranges"], H, W, bg, clear_records=grec)
        assert not torch.isnan(grec).any()
        for rep in range(2):
            _lib.call("gs_composite_bwd", _lib.stream_handle(cuda), n, _lib.ptr(pre["records"]),
                      _lib.ptr(b["sorted_gids"]), b["sorted_gids"].shape[0], _lib.ptr(b["ranges"]), W, H, _lib.ptr(bg),
                      _lib.ptr(gimg), _lib.ptr(fT), _lib.ptr(nc), _lib.ptr(order), _lib.ptr(grec), None, 1, None, None)
            if rep == 0:
                acc1 = _np(grec)
        acc2 = _np(grec)
    assert _rel(out[0][0], out[1][0]) <= 1e-5
    assert _rel(out[0][1], out[1][1]) <= 1e-5
    assert _rel(acc1, out[0][0]) <= 1e-5
    assert _rel(acc2, 2.0 * out[0][0]) <= 1e-5


@pytest.mark.parametrize("w,h", [(504, 378), (1280, 720), (1920, 1080)])
def test_records_beyond_4gib(cuda, w, h):
    """Compositing addresses a walked entry's record by its byte offset in a 32-bit
    register while the records span less than 4 GiB, and by its id beyond.  The same scene
    placed at the end of a 4.3 GB record array (ids shifted, the other builds) must give
    the same image, final T and entry counts bit for bit, and the same gradient records up
    to the order of the atomic additions (one, two and four pixels per lane)."""
    from jax_gs_amd import _lib

    sc = scenes.make_scene(2, n=20000, width=w, height=h)
    g, cam, _, mask = scenes.to_torch(sc, cuda)
    W, H = cam.W, cam.H
    n_big = (2**32 - 64) // (4 * _lib.GS_REC_STRIDE) + 1  # records past 32-bit byte offsets
    with torch.no_grad():
        pre = preprocess(g, cam, mask=mask, sh_degree=sc["sh_degree"])
        b = rasterizer.bin_gaussians(pre["means2d"], pre["radii"], pre["valid"], pre["depths"], H, W,
                                     want_tiles=False)
        rec, gids, ranges = pre["records"], b["sorted_gids"], b["ranges"]
        n = rec.shape[0]
        shift = n_big - n
        rec_big = torch.empty((n_big, _lib.GS_REC_STRIDE), device=cuda)
        rec_big[shift:] = rec
        gids_big = gids + shift
        bg = torch.tensor([0.1, 0.2, 0.3], device=cuda)
        small = rasterizer.composite(rec, gids, ranges, H, W, bg)
        big = rasterizer.composite(rec_big, gids_big, ranges, H, W, bg)
        for a, c in zip(small[:3], big[:3]):
            assert torch.equal(a, c)
        # the tile order within a bucket of equal cost follows the order of LDS atomics
        assert torch.equal(torch.sort(small[3]).values, torch.sort(big[3]).values)
        image, fT, nc, order = small
        gimg = torch.from_numpy(np.random.default_rng(3).normal(0, 1, (H, W, 3)).astype(np.float32)).to(cuda)
        grads = []
        for rr, gg, nn in ((rec, gids, n), (rec_big, gids_big, n_big)):
            grec = torch.empty((nn, _lib.GS_REC_STRIDE), device=cuda)
            _lib.call("gs_composite_bwd", _lib.stream_handle(cuda), nn, _lib.ptr(rr), _lib.ptr(gg), gg.shape[0],
                      _lib.ptr(ranges), W, H, _lib.ptr(bg), _lib.ptr(gimg), _lib.ptr(fT), _lib.ptr(nc),
                      _lib.ptr(order), _lib.ptr(grec), None, 0, None, None)
            grads.append(_np(grec[-n:]))
            assert nn == n or not grec[:shift].any()
        del rec_big, grec
        torch.cuda.empty_cache()
    assert np.abs(grads[0]).max() > 0
    assert _rel(grads[1], grads[0]) <= 1e-5


def _l1_ssim_gpu(cuda, pred_np, tgt_np, gout):
    from jax_gs_amd import _lib

    H, W, C = pred_np.shape
    pred = torch.from_numpy(pred_np).to(cuda)
    tgt = torch.from_numpy(tgt_np).to(cuda)
    nb = _lib.lib().gs_l1_ssim_workspace_size(H, W, C)
    ws = torch.empty((nb,), dtype=torch.uint8, device=cuda)
    out = torch.empty((2,), device=cuda)
    s = _lib.stream_handle(cuda)
    _lib.call("gs_l1_ssim", s, H, W, C, _lib.ptr(pred), _lib.ptr(tgt), _lib.ptr(out), 1, _lib.ptr(ws), nb)
    g = torch.tensor(gout, dtype=torch.float32, device=cuda)
    grad = torch.empty_like(pred)
    _lib.call("gs_l1_ssim_bwd", s, H, W, C, _lib.ptr(pred), _lib.ptr(tgt), _lib.ptr(g), _lib.ptr(ws), nb,
              _lib.ptr(grad))
    return _np(out), _np(grad)


@pytest.mark.parametrize("shape", [(32, 32, 3), (37, 41, 3), (70, 55, 1), (378, 504, 3), (1080, 1920, 3)])
def test_l1_ssim_parity(cuda, shape):
    """losses.py:4-8 and :16-68 in one kernel pair: the L1 and SSIM means against the
    float64 oracle, and the image gradient of a * l1 + b * ssim against the oracle's
    L1 seed and hand-written SSIM VJP (shapes: the reference's test image, odd sizes
    that end inside a tile, one channel, cfg1's and cfg2's frames)."""
    rng = np.random.default_rng(sum(shape))
    tgt = rng.uniform(0, 1, shape).astype(np.float32)
    pred = np.clip(tgt + rng.normal(0, 0.2, shape), 0, 1).astype(np.float32)
    a, b = 0.8, -0.1  # trainer.py:26 weights of l1 and d_ssim = (1 - ssim) / 2
    out, grad = _l1_ssim_gpu(cuda, pred, tgt, [a, b])
    want_l1, seed = oracle.l1_loss_and_grad(pred, tgt)
    want_s = oracle.ssim(pred, tgt)
    assert abs(out[0] - want_l1) <= 1e-6 * want_l1
    assert abs(out[1] - want_s) <= 1e-5
    want_g = a * seed.astype(np.float64) + oracle.ssim_vjp(pred, tgt, b)
    assert _rel(grad, want_g) <= 1e-4
    assert np.abs(grad - want_g).max() <= 1e-3 * np.abs(want_g).max()


@pytest.mark.parametrize("shape,L", [((32, 40, 3), 3), ((33, 29, 3), 4), ((40, 52, 2), 7), ((24, 31, 5), 11),
                                     ((64, 70, 3), 15), ((18, 20, 1), 1)])
def test_l1_ssim_any_window_parity(cuda, shape, L):
    """losses.py:16 ssim(..., window_size) through the module (gs_l1_ssim_window: any
    window, even ones off centre, any channel count): both means against the float64 oracle
    and the image gradient of a * l1 + b * ssim against the oracle's VJP."""
    from jax_gs_amd.training import losses

    rng = np.random.default_rng(7 * L + shape[2])
    tgt = rng.uniform(0, 1, shape).astype(np.float32)
    pred = np.clip(tgt + rng.normal(0, 0.2, shape), 0, 1).astype(np.float32)
    p = torch.from_numpy(pred).to(cuda).requires_grad_(True)
    l1, ss = losses.l1_and_ssim(p, torch.from_numpy(tgt).to(cuda), window_size=L)
    want_l1, seed = oracle.l1_loss_and_grad(pred, tgt)
    want_s = oracle.ssim(pred, tgt, window_size=L)
    assert abs(float(l1.detach()) - want_l1) <= 1e-6 * want_l1
    assert abs(float(ss.detach()) - want_s) <= 1e-5
    a, b = 0.8, -0.1
    (a * l1 + b * ss).backward()
    want_g = a * seed.astype(np.float64) + oracle.ssim_vjp(pred, tgt, b, window_size=L)
    assert _rel(_np(p.grad), want_g) <= 1e-4
    assert abs(float(losses.ssim(p.detach(), p.detach(), window_size=L)) - 1.0) <= 1e-5


def test_ssim_identical_images_and_losses_module(cuda):
    """test_training.py:21-38 through the host module: ssim(t, t) = 1, d_ssim(t, t) = 0,
    bounds, d_ssim = (1 - ssim) / 2, and l1_ssim_loss's total and gradient."""
    from jax_gs_amd.training import losses

    rng = np.random.default_rng(0)
    t_np = rng.uniform(0, 1, (32, 32, 3)).astype(np.float32)
    p_np = (t_np + 0.1 * rng.uniform(0, 1, t_np.shape)).astype(np.float32)
    t = torch.from_numpy(t_np).to(cuda)
    assert abs(float(losses.ssim(t, t)) - 1.0) <= 1e-6
    assert abs(float(losses.d_ssim_loss(t, t))) <= 1e-6
    p = torch.from_numpy(p_np).to(cuda).requires_grad_(True)
    s = float(losses.ssim(p, t).detach())
    d = float(losses.d_ssim_loss(p, t).detach())
    assert 0.0 <= s <= 1.0 and 0.0 <= d <= 1.0 and abs(d - (1.0 - s) / 2.0) <= 1e-7
    total, l1, dss = losses.l1_ssim_loss(p, t, 0.2)
    total.backward()
    want_l1, seed = oracle.l1_loss_and_grad(p_np, t_np)
    want_total = 0.8 * want_l1 + 0.2 * oracle.d_ssim_loss(p_np, t_np)
    assert abs(float(total.detach()) - want_total) <= 1e-6
    want_g = 0.8 * seed.astype(np.float64) + 0.2 * oracle.d_ssim_vjp(p_np, t_np, 1.0)
    assert _rel(_np(p.grad), want_g) <= 1e-4


def test_mse_loss(cuda):
    """losses.py:10-14 and its seed, through the host module."""
    from jax_gs_amd.training import losses

    rng = np.random.default_rng(4)
    p_np = rng.uniform(0, 1, (37, 41, 3)).astype(np.float32)
    t_np = rng.uniform(0, 1, p_np.shape).astype(np.float32)
    p = torch.from_numpy(p_np).to(cuda).requires_grad_(True)
    loss = losses.mse_loss(p, torch.from_numpy(t_np).to(cuda))
    loss.backward()
    want, seed = oracle.mse_loss_and_grad(p_np, t_np)
    assert abs(float(loss.detach()) - float(want)) <= 1e-6 * float(want)
    np.testing.assert_allclose(_np(p.grad), seed, rtol=1e-6, atol=1e-12)


def test_adam_step_parity(cuda):
    """train.py:127-155 / trainer.py:44-53 / optax.apply_updates: three masked Adam steps of
    the five arrays (one launch each) against the oracle's optax restatement, with the
    means on the exponential-decay schedule and sizes that end mid-vector."""
    from jax_gs_amd.core.gaussians import Gaussians
    from jax_gs_amd.training.optimizer import FIELDS, make_optimizer

    n, K = 5003, 16
    rng = np.random.default_rng(11)
    shapes = {"means": (n, 3), "scales": (n, 3), "quaternions": (n, 4), "opacities": (n, 1), "sh_coeffs": (n, K, 3)}
    p_np = {f: rng.normal(size=s).astype(np.float32) for f, s in shapes.items()}
    params = Gaussians(**{f: torch.from_numpy(p_np[f].copy()).to(cuda) for f in FIELDS})
    opt = make_optimizer(extent=2.5, num_iterations=30000)
    state = opt.init(params)
    mu = {f: np.zeros_like(p_np[f]) for f in FIELDS}
    nu = {f: np.zeros_like(p_np[f]) for f in FIELDS}
    active = rng.uniform(size=n) < 0.7
    for step in range(3):
        g_np = {f: (rng.normal(size=s) * 10.0 ** rng.integers(-4, 1)).astype(np.float32) for f, s in shapes.items()}
        grads = Gaussians(**{f: torch.from_numpy(g_np[f]).to(cuda) for f in FIELDS})
        opt.step(params, grads, state, torch.from_numpy(active).to(cuda))
        for f in FIELDS:
            lr = opt.lr_at(f, step)
            p_np[f], mu[f], nu[f] = oracle.adam_step(p_np[f], g_np[f], mu[f], nu[f], step, lr, active)
    assert state.count == 3
    for f in FIELDS:
        got = _np(getattr(params, f))
        np.testing.assert_allclose(got, p_np[f], rtol=0, atol=4e-7 * max(1.0, float(np.abs(p_np[f]).max())))
        np.testing.assert_array_equal(got[~active], p_np[f][~active])
        np.testing.assert_allclose(_np(state.mu[f]), mu[f], rtol=1e-6, atol=1e-30)
        np.testing.assert_allclose(_np(state.nu[f]), nu[f], rtol=1e-6, atol=1e-30)


@pytest.mark.parametrize("enabled", [True, False])
def test_densify_and_prune_parity(cuda, enabled):
    """density.py:98-211 with the optimizer moments moving along: every array, the mask,
    the cleared statistics and the counts bit-identical to the oracle (same noise)."""
    from jax_gs_amd.core.gaussians import Gaussians
    from jax_gs_amd.training import density
    from jax_gs_amd.training.optimizer import FIELDS, AdamState

    rng = np.random.default_rng(21)
    M, K = 6007, 16
    f = np.float32
    s = {"means": rng.normal(size=(M, 3)).astype(f), "scales": np.log(rng.uniform(0.002, 0.08, (M, 3))).astype(f),
         "quaternions": rng.normal(size=(M, 4)).astype(f), "opacities": rng.normal(0, 3, (M, 1)).astype(f),
         "sh_coeffs": rng.normal(size=(M, K, 3)).astype(f), "active": rng.uniform(size=M) < 0.7,
         "grad_accum": rng.uniform(0, 0.0004, M).astype(f), "denom": rng.integers(0, 5, M).astype(np.int32),
         "max_radii": rng.uniform(0, 600, M).astype(f)}
    s["moments"] = {f"{k}_{fl}": rng.normal(size=s[fl].shape).astype(f) for k in ("mu", "nu") for fl in FIELDS}
    noise = rng.normal(size=(M, 3)).astype(f)
    want, c = oracle.densify_and_prune(s, noise, densify_enabled=enabled, extent=5.0)
    if enabled:
        assert c["clones"] > 0 and c["splits"] > 0

    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    st = density.DensityState(
        gaussians=Gaussians(*[T(s[fl]) for fl in FIELDS]),
        opt_state=AdamState(mu={fl: T(s["moments"][f"mu_{fl}"]) for fl in FIELDS},
                            nu={fl: T(s["moments"][f"nu_{fl}"]) for fl in FIELDS}, count=3),
        active_mask=T(s["active"].astype(np.uint8)), num_active=int(s["active"].sum()),
        grad_accum=T(s["grad_accum"]), denom=T(s["denom"]), max_radii=T(s["max_radii"]))
    density.densify_and_prune(st, densify_enabled=enabled, extent=5.0, noise=T(noise))
    got_counts = _np(st.last_counts)
    assert list(got_counts) == [c["clones"], c["splits"], c["pruned"], c["available"], int(enabled)]
    for fl in FIELDS:
        np.testing.assert_array_equal(_np(getattr(st.gaussians, fl)), want[fl], err_msg=fl)
        np.testing.assert_array_equal(_np(st.opt_state.mu[fl]), want["moments"][f"mu_{fl}"], err_msg=fl)
        np.testing.assert_array_equal(_np(st.opt_state.nu[fl]), want["moments"][f"nu_{fl}"], err_msg=fl)
    np.testing.assert_array_equal(_np(st.active_mask).astype(bool), want["active"])
    assert not _np(st.grad_accum).any() and not _np(st.denom).any()
    np.testing.assert_array_equal(_np(st.max_radii), s["max_radii"])
    # reset_opacities (density.py:69-93) on the new mask
    density.reset_opacities(st, 0.01)
    op = _np(st.gaussians.opacities)[:, 0]
    a = want["active"]
    np.testing.assert_array_equal(op[a], np.full(a.sum(), np.float32(np.log(0.01 / 0.99)), np.float32))
    np.testing.assert_array_equal(op[~a], want["opacities"][~a, 0])


def test_ply_save_load(cuda, tmp_path):
    """ply.py:6-123: the file save_ply writes is byte-identical to the oracle's
    restatement of the reference writer, and load_ply returns the arrays exactly
    (test_io.py:9-40 with more points and degree-3 SH)."""
    from jax_gs_amd.core.gaussians import Gaussians
    from jax_gs_amd.io.ply import load_ply, save_ply

    rng = np.random.default_rng(31)
    n = 5003
    arr = {"means": rng.uniform(-1, 1, (n, 3)), "scales": rng.uniform(-2, 0, (n, 3)),
           "quaternions": rng.uniform(-1, 1, (n, 4)), "opacities": rng.uniform(0, 1, (n, 1)),
           "sh_coeffs": rng.normal(size=(n, 16, 3))}
    arr = {k: v.astype(np.float32) for k, v in arr.items()}
    g = Gaussians(*[torch.from_numpy(arr[k]).to(cuda) for k in FIELDS])
    path = str(tmp_path / "g.ply")
    save_ply(path, g)
    got = open(path, "rb").read()
    want = oracle.ply_bytes(arr["means"], arr["scales"], arr["quaternions"], arr["opacities"], arr["sh_coeffs"])
    assert got == want
    back = load_ply(path, device=cuda)
    for k in FIELDS:
        np.testing.assert_array_equal(_np(getattr(back, k)), arr[k], err_msg=k)


def test_train_step_composition(cuda):
    """trainer.py:55-169 on the GPU: the rendered loss (0.8 L1 + 0.2 D-SSIM), the
    gradients of the five arrays, the densification statistics and the masked Adam step
    against the oracle's render, losses, VJP, statistics and optimizer (the optimizer is
    fed the GPU's gradients, whose own parity is checked first: near-zero gradient
    components decide Adam's first-step sign)."""
    from jax_gs_amd.core.gaussians import Gaussians
    from jax_gs_amd.training import density
    from jax_gs_amd.training.optimizer import make_optimizer
    from jax_gs_amd.training.trainer import train_step

    sc = scenes.make_scene(4, n=3000, width=96, height=64)
    g, cam, tgt, mask = scenes.to_torch(sc, cuda)
    opt = make_optimizer(extent=3.0, num_iterations=1000)
    st = density.init_density_state(g, opt, 3000)
    st.active_mask.copy_(torch.from_numpy(sc["mask"].astype(np.uint8)).to(cuda))
    p0 = {f: _np(getattr(st.gaussians, f)).copy() for f in FIELDS}
    cs = (cam.W, cam.H, cam.fx, cam.fy, cam.cx, cam.cy)
    state, loss, metrics = train_step(st, tgt, cam.W2C, cs, opt, sh_degree=sc["sh_degree"])
    # oracle forward, loss and VJP at the pre-step parameters
    params_o = {**sc["params"], **{f: p0[f] for f in FIELDS}}
    img_o, ex_o, res = oracle.render(params_o, sc["cam"], mask=sc["mask"], sh_degree=sc["sh_degree"])
    t_np = _np(tgt)
    l1_o, seed_l1 = oracle.l1_loss_and_grad(img_o, t_np)
    want_loss = 0.8 * float(l1_o) + 0.2 * oracle.d_ssim_loss(img_o, t_np)
    assert abs(float(loss) - want_loss) <= 1e-5
    assert abs(float(metrics["ssim"]) - oracle.ssim(img_o, t_np)) <= 1e-5
    g_img = (0.8 * seed_l1.astype(np.float64) + 0.2 * oracle.d_ssim_vjp(img_o, t_np, 1.0)).astype(np.float32)
    gr_o = oracle.render_vjp(params_o, sc["cam"], res, g_img, sh_degree=sc["sh_degree"])
    # reconstruct the GPU gradients from the Adam update of the first step: with zero
    # moments mu = 0.1 g exactly, so compare the moments instead
    for f in FIELDS:
        g_gpu = _np(state.opt_state.mu[f]) / np.float32(0.1)
        assert _rel(g_gpu, gr_o[f]) <= GRAD_TOL, f
        want_p, _, _ = oracle.adam_step(p0[f], g_gpu.astype(np.float32), np.zeros_like(p0[f]), np.zeros_like(p0[f]),
                                        0, opt.lr_at(f, 0), sc["mask"])
        np.testing.assert_allclose(_np(getattr(state.gaussians, f)), want_p, rtol=0, atol=1e-6, err_msg=f)
    ga, de, mr = oracle.densify(gr_o["means"], p0["means"], sc["cam"]["W2C"], sc["cam"]["fx"], sc["cam"]["fy"],
                                sc["cam"]["W"], sc["cam"]["H"], ex_o["valid_mask"], ex_o["radii"],
                                np.zeros(3000, np.float32), np.zeros(3000, np.int32), np.zeros(3000, np.float32),
                                active=sc["mask"])
    np.testing.assert_array_equal(_np(state.denom), de)
    np.testing.assert_array_equal(_np(state.max_radii), mr)
    assert _rel(_np(state.grad_accum), ga) <= GRAD_TOL


def _subscene(sc, idx):
    """The Gaussians idx of scene sc (same camera)."""
    out = dict(sc)
    out["params"] = {k: np.ascontiguousarray(v[idx]) for k, v in sc["params"].items()}
    out["mask"] = None if sc["mask"] is None else np.ascontiguousarray(sc["mask"][idx])
    return out


@pytest.mark.parametrize("case", ["empty", "one", "behind", "mixed_behind"])
def test_degenerate_scenes(cuda, case):
    """No Gaussians, a single one, all behind the camera (depth sign bit set: the
    reference's tile -1 slots), and a scene with a quarter of them behind: image,
    extras and gradients against the oracle."""
    sc = scenes.make_scene(1, n=400, width=96, height=80)
    n = 400
    if case == "empty":
        sc = _subscene(sc, np.arange(0))
    elif case == "one":
        sc = _subscene(sc, np.arange(1))
        sc["params"]["means"][0] = [0.0, 0.0, 3.0]
        sc["params"]["scales"][0] = np.log([0.05, 0.08, 0.05])
    elif case == "behind":
        sc["params"]["means"][:, 2] = -np.abs(sc["params"]["means"][:, 2])
    else:
        sc["params"]["means"][: n // 4, 2] = -np.abs(sc["params"]["means"][: n // 4, 2])
    if sc["target"] is None:
        sc["target"] = np.random.default_rng(1).uniform(0, 1, (80, 96, 3)).astype(np.float32)
    image, extras, g, img_o, ex_o, gr_o = _render_both(sc, cuda)
    assert np.abs(_np(image) - img_o).max() <= IMG_TOL
    for k in ("n_interactions", "max_interactions_per_tile", "overflow_tiles", "truncated_tiles",
              "radius_cap_violations"):
        assert int(extras[k]) == int(ex_o[k]), k
    np.testing.assert_array_equal(_np(extras["valid_mask"]), ex_o["valid_mask"])
    for f in FIELDS:
        got = _np(getattr(g, f).grad)
        assert got.shape == gr_o[f].shape
        if np.linalg.norm(gr_o[f]) == 0.0:
            assert not got.any(), f
        else:
            assert _rel(got, gr_o[f]) <= GRAD_TOL, f


def test_capacity_exceeded_is_flagged(cuda):
    """An entry capacity below the scene's count: the binning flags it, keeps the first
    `capacity` entries of the reference order, and compositing stays inside them."""
    from jax_gs_amd import _lib

    sc = scenes.make_scene(1, n=3000, width=160, height=120)
    g, cam, _, _ = scenes.to_torch(sc, cuda)
    with torch.no_grad():
        pre = preprocess(g, cam, sh_degree=sc["sh_degree"])
        full = rasterizer.bin_gaussians(pre["means2d"], pre["radii"], pre["valid"], pre["depths"], cam.H, cam.W)
        n_int = int(full["n_interactions"])
        cap = n_int // 2
        part = rasterizer.bin_gaussians(pre["means2d"], pre["radii"], pre["valid"], pre["depths"], cam.H, cam.W,
                                        capacity=cap)
        st = _np(part["stats"])
        assert st[_lib.STAT["capacity_exceeded"]] == 1 and st[_lib.STAT["n_interactions"]] == n_int
        np.testing.assert_array_equal(_np(part["sorted_gids"])[:cap], _np(full["sorted_gids"])[:cap])
        image, _, _, _ = rasterizer.composite(pre["records"], part["sorted_gids"], part["ranges"], cam.H, cam.W,
                                              torch.zeros(3, device=cuda))
        assert torch.isfinite(image).all()


@pytest.mark.gpu
def test_l1_ssim_terms(cuda):
    """gs_l1_ssim_terms against the loss composition of trainer.py:18-30 in float32, over
    SSIM values above, at and below the max's tie (1) and outside [0, 1]."""
    from jax_gs_amd import _lib

    lam = 0.2
    s = _lib.stream_handle(cuda)
    for l1, ssim_v in ((0.125, 0.6), (0.3, 1.0), (0.01, 1.25), (0.5, -0.3), (0.0, 0.9999999)):
        out = torch.tensor([l1, ssim_v], dtype=torch.float32, device=cuda)
        terms = torch.full((5,), float("nan"), dtype=torch.float32, device=cuda)
        _lib.call("gs_l1_ssim_terms", s, _lib.ptr(out), lam, _lib.ptr(terms))
        t = _np(terms)
        f = np.float32
        half = (f(1.0) - f(ssim_v)) / f(2.0)
        d = max(f(0.0), half)
        assert t[0] == d
        assert t[1] == f(1.0 - lam) * f(l1) + f(lam) * d
        assert t[2] == f(1.0 - lam)
        assert t[3] == f(-(lam * 0.5)) * f(oracle._tie_grad(np.float64(half)))
        assert t[4] == f(1.0) - d * f(2.0)


@pytest.mark.gpu
def test_fused_train_step_matches_autograd_step(cuda):
    """The fused step (one kernel for the preprocessing VJP, statistics and Adam) against
    the autograd step (render's backward, accumulate_from_extras, Adam.step) over two steps
    from the same state.  The rasterizer's VJP sums with atomics, so the two see gradients
    equal up to float summation order: moments and statistics within 1e-4 relative."""
    from jax_gs_amd.training import density
    from jax_gs_amd.training.optimizer import make_optimizer
    from jax_gs_amd.training.trainer import train_step

    sc = scenes.make_scene(4, n=3000, width=96, height=64)
    g, cam, tgt, _ = scenes.to_torch(sc, cuda)
    states = []
    for _ in range(2):
        st = density.init_density_state(g, make_optimizer(extent=3.0, num_iterations=1000), 3000)
        st.active_mask.copy_(torch.from_numpy(sc["mask"].astype(np.uint8)).to(cuda))
        states.append(st)
    opt = make_optimizer(extent=3.0, num_iterations=1000)
    cs = (cam.W, cam.H, cam.fx, cam.fy, cam.cx, cam.cy)
    for step in range(2):
        _, loss_f, met_f = train_step(states[0], tgt, cam.W2C, cs, opt, sh_degree=sc["sh_degree"], fused=True)
        _, loss_a, met_a = train_step(states[1], tgt, cam.W2C, cs, opt, sh_degree=sc["sh_degree"], fused=False)
        assert abs(float(loss_f) - float(loss_a)) <= 1e-6
        assert abs(float(met_f["ssim"]) - float(met_a["ssim"])) <= 1e-6
        assert float(met_f["n_interactions"]) == float(met_a["n_interactions"])
        f, a = states
        assert f.opt_state.count == a.opt_state.count == step + 1
        for fl in FIELDS:
            assert _rel(_np(f.opt_state.mu[fl]), _np(a.opt_state.mu[fl])) <= 1e-4, fl
            assert _rel(_np(f.opt_state.nu[fl]), _np(a.opt_state.nu[fl])) <= 1e-4, fl
            pf, pa = _np(getattr(f.gaussians, fl)), _np(getattr(a.gaussians, fl))
            # Adam's early updates are about -lr sign(g): a few near-zero gradients may
            # differ in sign between summation orders
            assert np.mean(np.abs(pf - pa) > 1e-6) <= 1e-3, fl
        np.testing.assert_array_equal(_np(f.denom), _np(a.denom))
        np.testing.assert_array_equal(_np(f.max_radii), _np(a.max_radii))
        assert _rel(_np(f.grad_accum), _np(a.grad_accum)) <= 1e-4
