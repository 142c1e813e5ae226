"""GPU parity at the sizes the benchmarks run: every compositing build the dispatcher
picks (by tile count), and configurations 2, 3 and 4 of BASELINE.json at their
configured sizes, against the CPU oracle (same bars as gpu_helpers.py).

Kernel builds by tile count T (gs_composite.hip dispatch):
  T < 2048          forward and backward with four waves per tile (one pixel per lane)
  2048 <= T < 6144  two waves per tile forward (composite_fwd_kernel<2>), one wave per
                    tile backward (composite_bwd_wide_kernel, with the path for entries
                    no pixel of the wave sees at the 0.99 alpha cap)
  T >= 6144         one wave per tile forward (composite_fwd_kernel<4>) and the same
                    backward: the builds behind the headline numbers.
The dense scenes saturate many pixels (T <= 1e-4), so the wave-wide early exit, the
per-pixel n_contrib < count and the backward's replay from saturated pixels are compared,
not only the open-pixel paths.
"""
import time

import numpy as np
import pytest
import torch

import oracle
from gpu_helpers import FIELDS, GRAD_TOL, IMG_TOL, l1_seed, log, np_, ref_valid_sublist, rel
from jax_gs_amd import _lib, render, scenes
from jax_gs_amd.renderer import rasterizer
from jax_gs_amd.renderer.projection import preprocess

pytestmark = pytest.mark.gpu


def _tiles(W, H):
    return ((W + 15) // 16) * ((H + 15) // 16)


def _full_check(sc, cuda, seed_kind="l1", min_saturated=0.0):
    """Preprocessing and binning bit-exact, image (and per-pixel residuals), gradients of
    the five arrays, all from one oracle forward and one oracle VJP."""
    c = sc["cam"]
    W, H = c["W"], c["H"]
    log(f"{sc['name']}: N={sc['params']['means'].shape[0]} {W}x{H} T={_tiles(W, H)}; oracle forward "
        f"({oracle.threads()} threads)")
    t0 = time.time()
    img_o, ex_o, res = oracle.render(sc["params"], c, mask=sc["mask"], sh_degree=sc["sh_degree"])
    log(f"oracle forward {time.time() - t0:.1f} s, {ex_o['n_interactions']} entries")
    pre_o, st, sg = res["pre"], res["sorted_tiles"], res["sorted_gids"]
    n_int = int(ex_o["n_interactions"])
    g, cam, _, m = scenes.to_torch(sc, cuda)
    D = sc["sh_degree"]
    with torch.no_grad():
        pre = preprocess(g, cam, mask=m, sh_degree=D)
        for k in ("means2d", "cov2d", "radii", "depths", "colors"):
            np.testing.assert_array_equal(np_(pre[k]), pre_o[k], err_msg=k)
        np.testing.assert_array_equal(np_(pre["valid"]).astype(bool), pre_o["valid"])
        b = rasterizer.bin_gaussians(pre["means2d"], pre["radii"], pre["valid"], pre["depths"], H, W)
        stats = np_(b["stats"])
        n_neg = int(np.signbit(pre_o["depths"]).sum())
        assert stats[_lib.STAT["n_interactions"]] == n_int and stats[_lib.STAT["negative_depth"]] == n_neg
        assert stats[_lib.STAT["capacity_exceeded"]] == 0
        st_v, sg_v = ref_valid_sublist(st, sg, n_neg, n_int)
        np.testing.assert_array_equal(np_(b["sorted_tiles"][:n_int]), st_v)
        np.testing.assert_array_equal(np_(b["sorted_gids"][:n_int]), sg_v)
        np.testing.assert_array_equal(np_(b["ranges"]).astype(np.int64) + 256 * n_neg,
                                      ex_o["tile_boundaries"])
        for k in ("max_interactions_per_tile", "overflow_tiles", "overflow_interactions", "truncated_tiles",
                  "truncated_interactions", "radius_cap_violations"):
            assert stats[_lib.STAT[k]] == int(ex_o[k]), k
        log("preprocessing and binning bit-exact")
        # the per-pixel residuals of the same launch the renderer makes
        _, fT, nc, _ = rasterizer.composite(pre["records"], b["sorted_gids"], b["ranges"], H, W,
                                            torch.zeros(3, device=cuda))
        del b
    sat = float((res["final_T"] <= 1e-4).mean())
    assert sat >= min_saturated, f"scene saturates only {sat:.3f} of its pixels"
    same_nc = float((np_(nc) == res["n_contrib"]).mean())
    assert same_nc >= 0.999, f"n_contrib equal at only {same_nc:.5f} of the pixels"
    assert np.abs(np_(fT) - res["final_T"]).max() <= IMG_TOL
    for f in FIELDS:
        getattr(g, f).requires_grad_(True)
    image, extras = render(g, cam, mask=m, sh_degree=D)
    err = float(np.abs(np_(image) - img_o).max())
    log(f"image max-abs {err:.2e}; saturated {sat:.3f}; n_contrib equal {same_nc:.5f}")
    assert err <= IMG_TOL
    np.testing.assert_array_equal(np_(extras["radii"]), ex_o["radii"])
    np.testing.assert_array_equal(np_(extras["valid_mask"]), ex_o["valid_mask"])
    if seed_kind == "l1":
        seed = l1_seed(sc, img_o)
    else:
        seed = np.random.default_rng(11).normal(0, 1, img_o.shape).astype(np.float32)
    image.backward(torch.from_numpy(seed).to(cuda))
    t0 = time.time()
    gr_o = oracle.render_vjp(sc["params"], c, res, seed, sh_degree=D)
    log(f"oracle backward {time.time() - t0:.1f} s")
    errs = {f: rel(np_(getattr(g, f).grad), gr_o[f]) for f in FIELDS}
    log("gradient relative L2: " + ", ".join(f"{f} {e:.1e}" for f, e in errs.items()))
    for f in FIELDS:
        assert errs[f] <= GRAD_TOL, f
    return dict(g=g, cam=cam, mask=m, extras=extras, ex_o=ex_o, gr_o=gr_o, res=res)


@pytest.mark.parametrize("n,w,h,build", [(100000, 1024, 768, "fwd<2>/bwd_wide"), (100000, 1920, 832, "fwd<4>/bwd_wide")])
def test_dense_scene_per_kernel_build(cuda, n, w, h, build):
    """The configuration-2 family, dense enough that 40 % of the pixels saturate, at a
    tile count of each large-image build."""
    T = _tiles(w, h)
    assert (2048 <= T < 6144) if build.startswith("fwd<2>") else T >= 6144
    sc = scenes.make_scene(2, n=n, width=w, height=h)
    _full_check(sc, cuda, min_saturated=0.3)


@pytest.mark.parametrize("w,h", [(1024, 768), (1920, 832)])
def test_alpha_cap_in_large_image_builds(cuda, w, h):
    """Near-opaque Gaussians (opacity logits 4.6 to 9: sigmoid >= 0.99 for most) on both
    large-image builds, so that many entries reach the 0.99 alpha cap (rasterizer.py:211)
    and the backward takes its general body for them (the cap's zero derivative, the tie's
    half) beside the no-cap path for the rest."""
    sc = scenes.make_scene(1, n=30000, width=w, height=h)
    rng = np.random.default_rng(5)
    op = sc["params"]["opacities"]
    sel = rng.random(op.shape[0]) < 0.5
    op[sel, 0] = rng.uniform(4.6, 9.0, int(sel.sum())).astype(np.float32)
    # a third of the Gaussians at opacity >= 0.99: their alpha reaches the cap near their centres
    assert float((1.0 / (1.0 + np.exp(-op[:, 0].astype(np.float64))) >= 0.99).mean()) > 0.3
    _full_check(sc, cuda, seed_kind="normal")


def test_cfg2_full_frame(cuda):
    """Configuration 2 (the headline: 1M Gaussians, SH3, 1920x1080, L1 seed) over the
    whole frame: the 8160-tile builds of both compositing kernels."""
    sc = scenes.make_scene(2)
    assert _tiles(sc["cam"]["W"], sc["cam"]["H"]) >= 6144
    _full_check(sc, cuda, min_saturated=0.9)


def test_cfg2_full_frame_oblique_camera(cuda):
    """Configuration 2 at full size under a rotated, translated camera whose W2C requires
    grad: the whole-frame image, the five cotangents and dL/dW2C against the oracle's VJP.
    The camera cotangent is the sum of 1M per-Gaussian shares, reduced in one partial per
    workgroup of the preprocessing VJP (977 of 1024 Gaussians) and one finishing workgroup
    (gs_preprocess_bwd_w2c), where float32 cancellation in the twelve sums is the risk."""
    sc = scenes.make_scene(2)
    ax = np.array([0.3, -0.5, 0.8])
    ax /= np.linalg.norm(ax)
    K = np.array([[0, -ax[2], ax[1]], [ax[2], 0, -ax[0]], [-ax[1], ax[0], 0]])
    w = np.eye(4)
    w[:3, :3] = np.eye(3) + np.sin(0.15) * K + (1 - np.cos(0.15)) * K @ K
    w[:3, 3] = [0.05, -0.03, 0.2]
    sc["cam"]["W2C"] = w.astype(np.float32)
    c = sc["cam"]
    log(f"cfg2 oblique camera: oracle forward ({oracle.threads()} threads)")
    img_o, ex_o, res = oracle.render(sc["params"], c, sh_degree=sc["sh_degree"])
    g, cam, _, _ = scenes.to_torch(sc, cuda)
    for f in FIELDS:
        getattr(g, f).requires_grad_(True)
    cam = cam._replace(W2C=cam.W2C.clone().requires_grad_(True))
    image, extras = render(g, cam, sh_degree=sc["sh_degree"])
    assert int(np_(extras["n_interactions"])) == int(ex_o["n_interactions"])
    err = float(np.abs(np_(image) - img_o).max())
    log(f"image max-abs {err:.2e}, {int(ex_o['n_interactions'])} entries")
    assert err <= IMG_TOL
    seed = l1_seed(sc, img_o)
    image.backward(torch.from_numpy(seed).to(cuda))
    gr_o = oracle.render_vjp(sc["params"], c, res, seed, sh_degree=sc["sh_degree"])
    errs = {f: rel(np_(getattr(g, f).grad), gr_o[f]) for f in FIELDS}
    gw = np_(cam.W2C.grad)
    errs["W2C"] = rel(gw, gr_o["W2C"])
    log("gradient relative L2: " + ", ".join(f"{f} {e:.1e}" for f, e in errs.items()))
    assert np.all(gw[3] == 0)
    for f, e in errs.items():
        assert e <= GRAD_TOL, f


def test_cfg3_full_size(cuda):
    """Configuration 3 (3M Gaussians, SH1, 1280x720, 70 % in four tight clusters): 65M
    entries, tiles past 10k entries composited to 4096, the whole frame forward and
    backward (a normal image cotangent; the benchmark runs it forward only)."""
    sc = scenes.make_scene(3)
    out = _full_check(sc, cuda, seed_kind="normal", min_saturated=0.5)
    assert int(out["ex_o"]["max_interactions_per_tile"]) > 10000
    assert int(out["ex_o"]["truncated_tiles"]) > 0


def test_cfg4_full_size_with_accumulators(cuda):
    """Configuration 4 (capacity 2,097,152 with a 60 % active mask, SH3, 1280x720):
    masked forward and backward, then the densification statistics (trainer.py:143-159)
    against the oracle's."""
    from jax_gs_amd.training.trainer import accumulate_from_extras

    sc = scenes.make_scene(4)
    n = sc["params"]["means"].shape[0]
    assert n == 2097152 and sc["mask"] is not None and 0.55 < sc["mask"].mean() < 0.65
    out = _full_check(sc, cuda, min_saturated=0.5)
    g, cam, m, extras, ex_o, gr_o = (out[k] for k in ("g", "cam", "mask", "extras", "ex_o", "gr_o"))
    rng = np.random.default_rng(3)
    ga0 = rng.uniform(0, 1e-3, n).astype(np.float32)
    de0 = rng.integers(0, 5, n).astype(np.int32)
    mr0 = rng.uniform(0, 40, n).astype(np.float32)
    state = {"grad_accum": torch.from_numpy(ga0).to(cuda), "denom": torch.from_numpy(de0).to(cuda),
             "max_radii": torch.from_numpy(mr0).to(cuda)}
    accumulate_from_extras(state, g.means.grad, g.means.detach(), cam, extras, active=m)
    c = sc["cam"]
    ga, de, mr = oracle.densify(gr_o["means"], sc["params"]["means"], c["W2C"], c["fx"], c["fy"], c["W"], c["H"],
                                ex_o["valid_mask"], ex_o["radii"], ga0, de0, mr0, active=sc["mask"])
    np.testing.assert_array_equal(np_(state["denom"]), de)
    np.testing.assert_array_equal(np_(state["max_radii"]), mr)
    assert rel(np_(state["grad_accum"]) - ga0, ga - ga0) <= GRAD_TOL
