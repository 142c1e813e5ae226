"""Shared checks of the GPU parity tests: the HIP path (through the C ABI) against the
CPU oracle.

Bars:
  * integer outputs bit-exact: per-Gaussian tile rectangles/counts (via the entry
    list), the sorted entry list (tile, Gaussian id) and the tile ranges;
  * image max-abs error <= 1e-4;
  * gradients: relative L2 error <= 1e-3 per parameter tensor.
The per-Gaussian preprocessing is compared bit-for-bit (same float32 operation
order, no FMA contraction, same exp on both sides).

Reference-order note: the reference's arrays carry 256 slots of every Gaussian whose
depth has its sign bit set in front of the valid entries (tile -1); the renderer's
GPU list holds only the valid entries, so its boundaries are compared after that shift
and its entries against the reference's valid sub-list.
"""
import time

import numpy as np
import torch

import oracle
from jax_gs_amd import render, scenes
from jax_gs_amd.renderer import rasterizer
from jax_gs_amd.renderer.projection import preprocess

IMG_TOL = 1e-4
GRAD_TOL = 1e-3
FIELDS = ("means", "scales", "quaternions", "opacities", "sh_coeffs")


def np_(t):
    return t.detach().cpu().numpy()


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)


def log(msg):
    print(f"[{time.strftime('%H:%M:%S')}] {msg}", flush=True)


def ref_valid_sublist(st, sg, n_neg, n_int):
    off = 256 * n_neg
    return st[off:off + n_int], sg[off:off + n_int]


def oracle_preprocess(sc):
    c = sc["cam"]
    f32 = np.float32
    return oracle.preprocess(sc["params"]["means"], sc["params"]["scales"], sc["params"]["quaternions"],
                             sc["params"]["sh_coeffs"], c["W2C"], c["W"], c["H"], f32(c["fx"]), f32(c["fy"]),
                             f32(c["cx"]), f32(c["cy"]), sc["sh_degree"], mask=sc["mask"])


def check_preprocess(sc, cuda, pre_o=None):
    """GPU preprocessing bit-identical to the oracle's (all outputs, both output modes)."""
    g, cam, _, m = scenes.to_torch(sc, cuda)
    pre = preprocess(g, cam, mask=m, sh_degree=sc["sh_degree"])
    o = oracle_preprocess(sc) if pre_o is None else pre_o
    for k in ("means2d", "cov2d", "radii", "depths", "colors"):
        np.testing.assert_array_equal(np_(pre[k]), o[k], err_msg=k)
    np.testing.assert_array_equal(np_(pre["valid"]).astype(bool), o["valid"])
    # the renderer's call writes no cov2d / colour arrays; everything else is identical,
    # except the colour slots (6-8) of masked-out Gaussians' records: their SH rows are not
    # read (never an entry)
    lean = preprocess(g, cam, mask=m, sh_degree=sc["sh_degree"], projected=False)
    assert lean["cov2d"] is None and lean["colors"] is None
    for k in ("means2d", "radii", "valid", "depths"):
        assert torch.equal(lean[k], pre[k]), k
    rl, rf = lean["records"].clone(), pre["records"]
    if m is not None:
        off = ~m.to(torch.bool)
        rl[off, 6:9] = rf[off, 6:9]
    assert torch.equal(rl, rf)
    return pre, o


def check_binning(sc, cuda, pre_gpu, pre_o, ref=None):
    """GPU entry list, ranges and health statistics bit-exact against the oracle.
    ref: (sorted_tiles, sorted_gids, n_interactions) of the oracle when already computed."""
    c = sc["cam"]
    W, H = c["W"], c["H"]
    b = rasterizer.bin_gaussians(pre_gpu["means2d"], pre_gpu["radii"], pre_gpu["valid"], pre_gpu["depths"], H, W)
    if ref is None:
        ref = oracle.tile_interactions(pre_o["means2d"], pre_o["radii"], pre_o["valid"], pre_o["depths"], H, W)
    st, sg, n_int = ref
    stats = np_(b["stats"])
    n_neg = int((np.signbit(pre_o["depths"])).sum())
    assert stats[7] == n_neg
    assert stats[0] == n_int
    assert stats[8] == 0
    st_v, sg_v = ref_valid_sublist(st, sg, n_neg, n_int)
    np.testing.assert_array_equal(np_(b["sorted_tiles"][:n_int]), st_v)
    np.testing.assert_array_equal(np_(b["sorted_gids"][:n_int]), sg_v)
    T = ((W + 15) // 16) * ((H + 15) // 16)
    b_ref = oracle.tile_boundaries(st, T)
    np.testing.assert_array_equal(np_(b["ranges"]).astype(np.int64) + 256 * n_neg, b_ref)
    ex = oracle.extras_from(pre_o, st, n_int, H, W)
    for k, idx in (("max_interactions_per_tile", 1), ("overflow_tiles", 2), ("overflow_interactions", 3),
                   ("truncated_tiles", 4), ("truncated_interactions", 5), ("radius_cap_violations", 6)):
        assert stats[idx] == ex[k], k
    return b, (st, sg, n_int)


def l1_seed(sc, img_o):
    target = sc["target"] if sc["target"] is not None else np.random.default_rng(7).uniform(
        0, 1, img_o.shape).astype(np.float32)
    # one seed for both sides (the L1 sign must not flip between them)
    return oracle.l1_loss_and_grad(img_o, target)[1]


def render_both(sc, cuda, seed_kind="l1"):
    g, cam, tgt, m = scenes.to_torch(sc, cuda)
    for f in FIELDS:
        getattr(g, f).requires_grad_(True)
    image, extras = render(g, cam, mask=m, sh_degree=sc["sh_degree"])
    img_o, ex_o, res = oracle.render(sc["params"], sc["cam"], mask=sc["mask"], sh_degree=sc["sh_degree"])
    if seed_kind == "l1":
        seed = l1_seed(sc, img_o)
    else:
        seed = np.random.default_rng(11).normal(0, 1, img_o.shape).astype(np.float32)
    image.backward(torch.from_numpy(seed).to(cuda))
    gr_o = oracle.render_vjp(sc["params"], sc["cam"], res, seed, sh_degree=sc["sh_degree"])
    return image, extras, g, img_o, ex_o, gr_o
