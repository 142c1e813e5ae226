"""The L1 loss fused into the compositing launches (render_l1: gs_composite_fwd_deferred_l1,
gs_composite_bwd_l1) against render followed by l1_loss (the separate loss kernels) and
against the oracle (losses.py:4-8 applied to the rendered image, trainer.py's
l1_loss(render(...)) under jax.grad).

The fused forward writes the same image bit for bit (the same kernel); the loss is the same
sum in another order (within float32 rounding).  The fused backward forms the image
cotangent sign(image - target) * g / count per pixel exactly as gs_l1_loss_bwd does, so the
gradients agree with the unfused path's up to the order of the backward's float atomics.
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_helpers import FIELDS, GRAD_TOL, log
from gpu_helpers import np_ as _np
from gpu_helpers import rel as _rel
from jax_gs_amd import render, render_l1, scenes
from jax_gs_amd.training.losses import l1_loss

pytestmark = pytest.mark.gpu

# the two paths' gradients differ only in the order of the compositing VJP's float atomics
ATOMIC_ORDER_TOL = 2e-5
# the loss: the same |image - target| terms summed in two orders
LOSS_TOL = 2e-6


def _target(sc, cuda, H, W):
    if sc["target"] is not None:
        return torch.from_numpy(sc["target"]).to(cuda)
    rng = np.random.default_rng(17)
    return torch.from_numpy(rng.uniform(0, 1, (H, W, 3)).astype(np.float32)).to(cuda)


def _grads(g):
    out = {f: getattr(g, f).grad.detach().clone() for f in FIELDS}
    for f in FIELDS:
        getattr(g, f).grad = None
    return out


def _both(sc, cuda, bg=None, scale=1.0, image_weight=None):
    """(fused image, loss, extras, grads, gbg), (unfused ...) on the same inputs."""
    g, cam, _, m = scenes.to_torch(sc, cuda)
    tgt = _target(sc, cuda, cam.H, cam.W)
    for f in FIELDS:
        getattr(g, f).requires_grad_(True)
    res = []
    for fused in (True, False):
        bgt = None if bg is None else torch.tensor(bg, device=cuda, requires_grad=True)
        if fused:
            image, loss, extras = render_l1(g, cam, tgt, background=bgt, mask=m, sh_degree=sc["sh_degree"])
        else:
            image, extras = render(g, cam, background=bgt, mask=m, sh_degree=sc["sh_degree"])
            loss = l1_loss(image, tgt)
        total = scale * loss
        if image_weight is not None:
            total = total + (image * image_weight).sum()
        total.backward()
        torch.cuda.synchronize()
        res.append((image.detach(), loss.detach(), extras, _grads(g), None if bgt is None else bgt.grad.clone()))
    return res, g, cam, tgt


@pytest.mark.parametrize("cfg,n,w,h", [(1, 4000, 200, 150), (2, 20000, 1024, 768), (4, 30000, 640, 400),
                                       (0, 3000, 128, 96)])
def test_render_l1_matches_render_then_l1_loss(cuda, cfg, n, w, h):
    sc = scenes.make_scene(cfg, n=n, width=w, height=h)
    log(f"render_l1 vs render + l1_loss: cfg{cfg} n={n} {w}x{h}")
    (a, b), g, cam, tgt = _both(sc, cuda)
    assert torch.equal(a[0], b[0])  # the same compositing kernel writes the image
    la, lb = float(a[1]), float(b[1])
    want = float(np.abs(_np(a[0]).astype(np.float64) - _np(tgt).astype(np.float64)).mean())
    assert abs(la - want) <= LOSS_TOL * want
    assert abs(lb - want) <= LOSS_TOL * want
    for k in ("n_interactions", "max_interactions_per_tile", "overflow_tiles", "truncated_tiles"):
        assert int(a[2][k]) == int(b[2][k]), k
    for f in FIELDS:
        assert _rel(_np(a[3][f]), _np(b[3][f])) <= ATOMIC_ORDER_TOL, f


def test_render_l1_gradients_against_the_oracle(cuda):
    """The fused VJP against the oracle's render VJP seeded with the L1 seed of the GPU
    image (sign(image - target) / count: the seed must not flip between the two sides)."""
    sc = scenes.make_scene(1, n=5000, width=240, height=160)
    g, cam, _, m = scenes.to_torch(sc, cuda)
    tgt = _target(sc, cuda, cam.H, cam.W)
    for f in FIELDS:
        getattr(g, f).requires_grad_(True)
    image, loss, _ = render_l1(g, cam, tgt, mask=m, sh_degree=sc["sh_degree"])
    loss.backward()
    img_o, _, res = oracle.render(sc["params"], sc["cam"], mask=sc["mask"], sh_degree=sc["sh_degree"])
    assert np.abs(_np(image) - img_o).max() <= 1e-4
    want, seed = oracle.l1_loss_and_grad(_np(image), _np(tgt))
    assert abs(float(loss.detach()) - float(want)) <= LOSS_TOL * float(want)
    gr_o = oracle.render_vjp(sc["params"], sc["cam"], res, seed, sh_degree=sc["sh_degree"])
    for f in FIELDS:
        assert _rel(_np(getattr(g, f).grad), gr_o[f]) <= GRAD_TOL, f


def test_render_l1_loss_cotangent_image_cotangent_and_background(cuda):
    """A scaled loss, the image used elsewhere in the objective as well, and a differentiated
    coloured background: the fused backward adds the L1 seed to the image's own cotangent
    (the unfused path's autograd sums the same two terms) and the background cotangent
    sees their sum."""
    sc = scenes.make_scene(2, n=8000, width=512, height=320)
    H, W = 320, 512
    w = torch.from_numpy(np.random.default_rng(5).normal(0, 1e-6, (H, W, 3)).astype(np.float32)).to(cuda)
    (a, b), _, _, _ = _both(sc, cuda, bg=[0.2, 0.5, 0.9], scale=2.5, image_weight=w)
    assert torch.equal(a[0], b[0])
    for f in FIELDS:
        assert _rel(_np(a[3][f]), _np(b[3][f])) <= ATOMIC_ORDER_TOL, f
    assert _rel(_np(a[4]), _np(b[4])) <= 1e-5


def test_render_l1_image_cotangent_only(cuda):
    """render_l1 whose loss is not used: the backward takes the image cotangent alone."""
    sc = scenes.make_scene(1, n=3000, width=160, height=120)
    g, cam, _, m = scenes.to_torch(sc, cuda)
    tgt = _target(sc, cuda, cam.H, cam.W)
    for f in FIELDS:
        getattr(g, f).requires_grad_(True)
    seed = torch.from_numpy(np.random.default_rng(9).normal(0, 1, (cam.H, cam.W, 3)).astype(np.float32)).to(cuda)
    image, _, _ = render_l1(g, cam, tgt, mask=m, sh_degree=sc["sh_degree"])
    image.backward(seed)
    ga = _grads(g)
    image2, _ = render(g, cam, mask=m, sh_degree=sc["sh_degree"])
    image2.backward(seed)
    gb = _grads(g)
    for f in FIELDS:
        assert _rel(_np(ga[f]), _np(gb[f])) <= ATOMIC_ORDER_TOL, f


@pytest.mark.parametrize("cfg", [2, 1])
def test_render_l1_full_size(cuda, cfg):
    """The bench's step (cfg2: 1M Gaussians, 1080p, SH3; cfg1: 200k at 504x378, the whole
    list written) fused against unfused: image bit-identical, loss and gradients within
    float32 reordering."""
    sc = scenes.make_scene(cfg)
    log(f"render_l1 full size cfg{cfg}")
    (a, b), _, _, tgt = _both(sc, cuda)
    assert torch.equal(a[0], b[0])
    want = float(np.abs(_np(a[0]).astype(np.float64) - _np(tgt).astype(np.float64)).mean())
    assert abs(float(a[1]) - want) <= LOSS_TOL * want
    for f in FIELDS:
        assert _rel(_np(a[3][f]), _np(b[3][f])) <= ATOMIC_ORDER_TOL, f


def test_render_l1_rejects_a_differentiated_target(cuda):
    sc = scenes.make_scene(1, n=100, width=64, height=48)
    g, cam, _, _ = scenes.to_torch(sc, cuda)
    tgt = torch.zeros((48, 64, 3), device=cuda, requires_grad=True)
    with pytest.raises(ValueError):
        render_l1(g, cam, tgt, sh_degree=sc["sh_degree"])
