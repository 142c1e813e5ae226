"""render(): the drop-in for jax_gs/renderer/renderer.py:15-107.

Same call signature and outputs: ``render(gaussians, camera, background=None,
fast_tpu_rasterizer=False, mask=None, sh_degree=0) -> (image [H,W,3], extras)``.
The reference differentiates render with JAX autodiff; here a
``torch.autograd.Function`` plays the role of a ``jax.custom_vjp``: its forward runs
the preprocessing, binning and compositing kernels and keeps the per-Gaussian
records, the sorted entry list, the tile ranges, per-pixel (final T, entry count)
and the backward's tile order as residuals; its backward runs the compositing VJP and the preprocessing VJP and
returns cotangents of the five Gaussian arrays (equal to JAX autodiff of the
reference forward, with its tie conventions), of the background, and of the camera's
W2C when it requires grad (through the camera-space means, W_rot and the view
directions' camera centre); mask gets None.
``fast_tpu_rasterizer`` selects the reference's compositing path: True reads each tile's
own entries (rasterizer_tpu.py:90-97); False (the default) slices 512-entry chunk windows
clamped to the end of the reference's max(256*N, 512)-slot arrays (rasterizer.py:184-190),
which reads other slots when a chunk starts within 512 slots of that end (one or two
Gaussians, or every Gaussian covering nearly 16x16 tiles).  Both run the same kernels: the
binning writes the clamped window (gs_window_from_bins) and the compositing kernels read
it for the chunks past its threshold.
"""
from __future__ import annotations

import ctypes

import torch

from .. import _lib
from ..core.camera import Camera
from ..core.gaussians import Gaussians
from ._buffers import as_mask, background_tensor, check_f32, num_tiles
from .projection import preprocess
from .rasterizer import bin_gaussians, check_capacity, composite


def _render_forward(ctx, means, scales, quats, opac, sh, w2c, bg, mask, static, target=None):
    """The forward of _Render and _RenderL1: (image, radii, valid, stats[, loss])."""
    W, H, fx, fy, cx, cy, sh_degree, capacity, tpu = static
    g = Gaussians(means, scales, quats, opac, sh)
    cam = Camera(W, H, fx, fy, cx, cy, w2c, None)
    pre = preprocess(g, cam, mask=mask, sh_degree=sh_degree, records=True, projected=False)
    b = bin_gaussians(pre["means2d"], pre["radii"], pre["valid"], pre["depths"], H, W, capacity=capacity,
                      want_tiles=False, window=not tpu, deferred=True)
    # the gradient records the backward accumulates into, cleared by the forward's
    # compositing launch (its waves are arithmetic-bound: the stores are free)
    n = means.shape[0]
    grec = (torch.empty((n, _lib.GS_REC_STRIDE), dtype=torch.float32, device=means.device)
            if any(ctx.needs_input_grad[:5]) else None)
    win = b["window"]
    out = composite(pre["records"], b["sorted_gids"], b["ranges"], H, W, bg, residuals=True, clear_records=grec,
                    window=win, bins=b, l1_target=target)
    image, fT, nc, order = out[:4]
    ctx.static = static
    ctx.grec_fresh = grec is not None
    # radii, valid and stats carry no gradient: no zero cotangents for them
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(means, scales, quats, opac, sh, w2c, bg, pre["records"], b["sorted_gids"], b["ranges"],
                          fT, nc, order, grec, win, image if target is not None else None, target)
    radii = pre["radii"]
    valid = pre["valid"].view(torch.bool)  # the kernel writes 0/1 bytes
    stats = b["stats"]
    ctx.mark_non_differentiable(radii, valid, stats)
    return (image, radii, valid, stats) + tuple(out[4:])


def _render_backward(ctx, g_image, g_loss=None):
    """Cotangents of (means, scales, quats, opacities, sh, W2C, background)."""
    W, H, fx, fy, cx, cy, sh_degree, _, _ = ctx.static
    if g_image is None and g_loss is None:
        return (None,) * 7
    (means, scales, quats, opac, sh, w2c, bg, rec, gids, ranges, fT, nc, order, grec, win, image,
     target) = ctx.saved_tensors
    dev = means.device
    n = means.shape[0]
    s = _lib.stream_handle(dev)
    # the forward cleared grec: accumulate into it once; a repeated backward
    # (retain_graph) starts from a fresh, cleared buffer
    accumulate = 1 if ctx.grec_fresh else 0
    ctx.grec_fresh = False
    if not accumulate:
        grec = torch.empty((n, _lib.GS_REC_STRIDE), dtype=torch.float32, device=dev)
    # dL/dbackground only when the background is differentiated (the trainer's is not)
    gbg = torch.empty((3,), dtype=torch.float32, device=dev) if ctx.needs_input_grad[6] else None
    gi = None if g_image is None else g_image.contiguous()
    # the five cotangent arrays are set to zero by the compositing VJP's arithmetic-bound waves
    # (its clear list), so the preprocessing VJP writes only the rows of the Gaussians some
    # pixel reached (zeroed = 1)
    gm = torch.empty_like(means)
    gs_ = torch.empty_like(scales)
    gq = torch.empty_like(quats)
    go = torch.empty_like(opac)
    gsh = torch.empty_like(sh)
    cl = _lib.clear_list(gm, gs_, gq, go, gsh)
    head = (s, n, _lib.ptr(rec), _lib.ptr(gids), gids.shape[0], _lib.ptr(ranges), int(W), int(H), _lib.ptr(bg))
    tail = (_lib.ptr(fT), _lib.ptr(nc), _lib.ptr(order), _lib.ptr(grec), _lib.ptr(gbg), accumulate, _lib.ptr(win),
            ctypes.byref(cl))
    if g_loss is not None:
        # the fused L1 loss: its VJP is formed per pixel inside the compositing VJP
        gl = g_loss.to(device=dev, dtype=torch.float32).contiguous()
        _lib.call("gs_composite_bwd_l1", *head, _lib.ptr(gi), _lib.ptr(image), _lib.ptr(target), _lib.ptr(gl), *tail)
    else:
        _lib.call("gs_composite_bwd", *head, _lib.ptr(gi), *tail)
    args = (s, n, sh.shape[1], int(sh_degree), _lib.ptr(means), _lib.ptr(scales), _lib.ptr(quats), _lib.ptr(opac),
            _lib.ptr(sh), _lib.ptr(w2c), int(W), int(H), float(fx), float(fy), float(cx), float(cy), _lib.ptr(grec),
            _lib.ptr(gm), _lib.ptr(gs_), _lib.ptr(gq), _lib.ptr(go), _lib.ptr(gsh))
    gw = None
    if ctx.needs_input_grad[5]:
        # the camera's cotangent (the reference differentiates W2C like any input)
        gw = torch.empty((4, 4), dtype=torch.float32, device=dev)
        nb = _lib.lib().gs_preprocess_bwd_w2c_workspace_size(n)
        ws = torch.empty((nb,), dtype=torch.uint8, device=dev)
        _lib.call("gs_preprocess_bwd_w2c", *args, _lib.ptr(gw), _lib.ptr(ws), nb, 1)
    else:
        _lib.call("gs_preprocess_bwd", *args, 1)
    return gm, gs_, gq, go, gsh, gw, gbg


class _Render(torch.autograd.Function):
    @staticmethod
    def forward(ctx, means, scales, quats, opac, sh, w2c, bg, mask, static):
        return _render_forward(ctx, means, scales, quats, opac, sh, w2c, bg, mask, static)

    @staticmethod
    def backward(ctx, g_image, _g_radii, _g_valid, _g_stats):
        return _render_backward(ctx, g_image) + (None, None)


class _RenderL1(torch.autograd.Function):
    """render followed by l1_loss(image, target), the loss computed by the compositing
    launches and its VJP formed inside the compositing VJP (no loss kernels, no image
    gradient array)."""

    @staticmethod
    def forward(ctx, means, scales, quats, opac, sh, w2c, bg, mask, target, static):
        return _render_forward(ctx, means, scales, quats, opac, sh, w2c, bg, mask, static, target=target)

    @staticmethod
    def backward(ctx, g_image, _g_radii, _g_valid, _g_stats, g_loss):
        return _render_backward(ctx, g_image, g_loss) + (None, None, None)


def _prepare(gaussians: Gaussians, camera: Camera, background, fast_tpu_rasterizer, mask, sh_degree, capacity):
    means = gaussians.means
    dev = means.device
    n = means.shape[0]
    means = check_f32("means", means, (n, 3), dev)
    w2c = torch.as_tensor(camera.W2C, dtype=torch.float32, device=dev).contiguous()
    bg = background_tensor(background, dev)
    m = as_mask(mask, n, dev)
    cap = check_capacity(capacity, n)
    static = (int(camera.W), int(camera.H), float(camera.fx), float(camera.fy), float(camera.cx), float(camera.cy),
              int(sh_degree), cap, bool(fast_tpu_rasterizer))
    return (means, gaussians.scales.contiguous(), gaussians.quaternions.contiguous(),
            gaussians.opacities.contiguous(), gaussians.sh_coeffs.contiguous(), w2c, bg, m), static


def render(gaussians: Gaussians, camera: Camera, background=None, fast_tpu_rasterizer: bool = False, mask=None,
           sh_degree: int = 0, capacity: int | None = None):
    """Render one view; returns (image [H,W,3] float32, extras dict) like renderer.py:15-107.

    capacity bounds the number of (Gaussian, tile) entries; the default is the
    reference's static bound 256*N (every Gaussian may touch 16x16 tiles), limited to the
    2^31 - 1 entries int32 indices address (N >= 8,388,608)."""
    inputs, static = _prepare(gaussians, camera, background, fast_tpu_rasterizer, mask, sh_degree, capacity)
    image, radii, valid, stats = _Render.apply(*inputs, static)
    _, _, T = num_tiles(camera.W, camera.H)
    extras = extras_from_stats(stats, radii, valid, T)
    return image, extras


def render_l1(gaussians: Gaussians, camera: Camera, target: torch.Tensor, background=None,
              fast_tpu_rasterizer: bool = False, mask=None, sh_degree: int = 0, capacity: int | None = None):
    """render(...) and l1_loss(image, target) (losses.py:4-8) in one: returns (image, loss,
    extras) with the same values as ``render`` followed by ``training.losses.l1_loss``
    (the loss summed in another order: within float32 rounding), differentiable through
    both the image and the loss.  The loss is computed by the compositing launches as
    they write the image and its VJP inside the compositing VJP, which saves the loss's own
    launches and the image-gradient round trip (the step the reference's trainer
    differentiates, trainer.py:18-26 with lambda_ssim = 0).  target is not differentiated."""
    inputs, static = _prepare(gaussians, camera, background, fast_tpu_rasterizer, mask, sh_degree, capacity)
    dev = inputs[0].device
    if target.requires_grad:
        raise ValueError("render_l1: the target is not differentiated (detach it)")
    tgt = check_f32("target", target, (int(camera.H), int(camera.W), 3), dev)
    image, radii, valid, stats, loss = _RenderL1.apply(*inputs, tgt, static)
    _, _, T = num_tiles(camera.W, camera.H)
    extras = extras_from_stats(stats, radii, valid, T)
    return image, loss, extras


def extras_from_stats(stats: torch.Tensor, radii: torch.Tensor, valid: torch.Tensor, num_tiles_total: int) -> dict:
    """renderer.py:79-90 from the binning kernel's stats (device tensors, no sync)."""
    S = _lib.STAT
    n = stats[S["n_interactions"]]
    return {
        "radii": radii,
        "valid_mask": valid,
        "n_interactions": n,
        # float32(n) / num_tiles, computed by the binning kernel (stats holds its bits)
        "mean_interactions_per_tile": stats.view(torch.float32)[S["mean_per_tile"]],
        "max_interactions_per_tile": stats[S["max_interactions_per_tile"]],
        "overflow_tiles": stats[S["overflow_tiles"]],
        "overflow_interactions": stats[S["overflow_interactions"]],
        "truncated_tiles": stats[S["truncated_tiles"]],
        "truncated_interactions": stats[S["truncated_interactions"]],
        "radius_cap_violations": stats[S["radius_cap_violations"]],
    }
