"""The training step (jax_gs/training/trainer.py:11-169) on the GPU path.

``train_step`` renders the active Gaussians, takes the trainer's loss
(0.8 L1 + 0.2 D-SSIM, one forward and one backward kernel), backpropagates through the
rasterizer, accumulates the densification statistics from the pre-update means and
applies the masked Adam step -- the same sequence as the reference's jitted step, with the
state's tensors updated in place.  ``accumulate_from_extras`` is the statistics part
(trainer.py:143-159) on its own.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from .. import _lib
from ..core.camera import Camera
from ..core.gaussians import Gaussians
from ..renderer._buffers import as_bytes


def accumulate_from_extras(state: dict, grad_means: torch.Tensor, means: torch.Tensor, camera, extras: dict,
                           active=None) -> None:
    """Update state['grad_accum'] (f32 [N]), state['denom'] (i32 [N]), state['max_radii'] (f32 [N]) in place."""
    dev = means.device
    n = means.shape[0]
    focal = float(np.float32((camera.fx + camera.fy) / 2.0))
    pixel_scale = float(np.float32(float(camera.W) * float(camera.H) * 3.0))
    w2c = torch.as_tensor(camera.W2C, dtype=torch.float32, device=dev).contiguous()
    valid = as_bytes(extras["valid_mask"])
    act = None if active is None else as_bytes(torch.as_tensor(active, device=dev))
    radii = extras["radii"].contiguous()
    for k, dt in (("grad_accum", torch.float32), ("denom", torch.int32), ("max_radii", torch.float32)):
        t = state[k]
        if t.dtype != dt or tuple(t.shape) != (n,) or not t.is_contiguous():
            raise ValueError(f"state[{k!r}] must be a contiguous {dt} tensor of shape ({n},)")
    _lib.call("gs_densify_accumulate", _lib.stream_handle(dev), n, _lib.ptr(grad_means.contiguous()),
              _lib.ptr(means.contiguous()), _lib.ptr(w2c), focal, pixel_scale, _lib.ptr(valid), _lib.ptr(act),
              _lib.ptr(radii), _lib.ptr(state["grad_accum"]), _lib.ptr(state["denom"]), _lib.ptr(state["max_radii"]))


def compute_loss_and_metrics(params: Gaussians, target_image, camera: Camera, active_mask=None, sh_degree: int = 0,
                             fast_tpu_rasterizer: bool = False, lambda_ssim: float = 0.2):
    """trainer.py:11-43: (total loss, metrics, image, extras); metrics are device scalars."""
    from ..renderer.renderer import render
    from .losses import l1_ssim_loss

    image, extras = render(params, camera, fast_tpu_rasterizer=fast_tpu_rasterizer, mask=active_mask,
                           sh_degree=sh_degree)
    total, l1, d_ssim = l1_ssim_loss(image, target_image, lambda_ssim)
    metrics = {"l1": l1.detach(), "ssim": (1.0 - d_ssim * 2.0).detach()}
    for k in _EXTRA_KEYS:
        metrics[k] = extras[k].to(torch.float32)
    return total, metrics, image, extras


def train_step(state, target_image, w2c, camera_static, optimizer, fast_tpu_rasterizer: bool = False,
               sh_degree: int = 0, fused: bool = True):
    """trainer.py:55-169 (single device): returns (state, loss, metrics) with the state's
    Gaussians, optimizer moments and statistics updated in place.

    fused=True runs the step without autograd: forward kernels, the loss pair, the
    rasterizer's VJP, then one kernel for the preprocessing VJP, the statistics and the
    Adam update (no parameter gradient reaches memory).  fused=False builds the same
    step from ``render``'s autograd, ``accumulate_from_extras`` and ``Adam.step``."""
    W, H, fx, fy, cx, cy = camera_static
    params = state.gaussians
    dev = params.means.device
    camera = Camera(int(W), int(H), float(fx), float(fy), float(cx), float(cy),
                    torch.as_tensor(w2c, dtype=torch.float32, device=dev), None)
    if not fused:
        return _train_step_autograd(state, target_image, camera, optimizer, fast_tpu_rasterizer, sh_degree)
    return _train_step_fused(state, target_image, camera, optimizer, sh_degree, fast_tpu_rasterizer)


_FIELDS = ("means", "scales", "quaternions", "opacities", "sh_coeffs")
_EXTRA_KEYS = ("n_interactions", "mean_interactions_per_tile", "max_interactions_per_tile", "overflow_tiles",
               "overflow_interactions", "truncated_tiles", "truncated_interactions", "radius_cap_violations")


def _train_step_autograd(state, target_image, camera, optimizer, fast_tpu_rasterizer, sh_degree):
    params = state.gaussians
    # leaves sharing the state's storage: the optimizer updates them in place afterwards
    leaves = [getattr(params, f).detach().requires_grad_(True) for f in _FIELDS]
    active = state.active_mask.to(torch.bool)
    total, metrics, _, extras = compute_loss_and_metrics(Gaussians(*leaves), target_image, camera, active,
                                                         sh_degree, fast_tpu_rasterizer)
    total.backward()
    grads = Gaussians(*[l.grad if l.grad is not None else torch.zeros_like(l) for l in leaves])
    # statistics from the means before the update (trainer.py:79-103)
    accumulate_from_extras({"grad_accum": state.grad_accum, "denom": state.denom, "max_radii": state.max_radii},
                           grads.means, params.means, camera, extras, active=state.active_mask)
    optimizer.step(params, grads, state.opt_state, state.active_mask)
    return state, total.detach(), metrics


def _train_step_fused(state, target_image, camera, optimizer, sh_degree, fast_tpu_rasterizer: bool = False,
                      lambda_ssim: float = 0.2):
    from ..renderer.rasterizer import bin_gaussians, composite
    from ..renderer.projection import preprocess
    from ..renderer._buffers import background_tensor

    params = state.gaussians
    dev = params.means.device
    s = _lib.stream_handle(dev)
    W, H = camera.W, camera.H
    n = params.means.shape[0]
    fields = [getattr(params, f) for f in _FIELDS]
    with torch.no_grad():
        active = state.active_mask.view(torch.bool)  # 0/1 bytes
        pre = preprocess(params, camera, mask=active, sh_degree=sh_degree, records=True, projected=False)
        # the default rasterizer's clamped chunk windows unless fast_tpu_rasterizer
        b = bin_gaussians(pre["means2d"], pre["radii"], pre["valid"], pre["depths"], H, W, want_tiles=False,
                          window=not fast_tpu_rasterizer, deferred=True)
        bg = background_tensor(None, dev)
        grec = torch.empty((n, _lib.GS_REC_STRIDE), dtype=torch.float32, device=dev)  # cleared by the forward
        image, fT, nc, order = composite(pre["records"], b["sorted_gids"], b["ranges"], H, W, bg, residuals=True,
                                         clear_records=grec, window=b["window"], bins=b)
        # loss (trainer.py:18-26): one kernel for the L1 and SSIM means
        tgt = target_image.to(device=dev, dtype=torch.float32).contiguous()
        Hh, Ww, C = image.shape
        nbytes = _lib.lib().gs_l1_ssim_workspace_size(Hh, Ww, C)
        ws = torch.empty((nbytes,), dtype=torch.uint8, device=dev)
        out = torch.empty((2,), dtype=torch.float32, device=dev)
        _lib.call("gs_l1_ssim", s, Hh, Ww, C, _lib.ptr(image), _lib.ptr(tgt), _lib.ptr(out), 1, _lib.ptr(ws), nbytes)
        # d_ssim, the total and the cotangents of (l1, ssim) in one launch
        terms = torch.empty((5,), dtype=torch.float32, device=dev)
        _lib.call("gs_l1_ssim_terms", s, _lib.ptr(out), float(lambda_ssim), _lib.ptr(terms))
        l1, total, gout = out[0], terms[1], terms[2:4]
        gimg = torch.empty_like(image)
        _lib.call("gs_l1_ssim_bwd", s, Hh, Ww, C, _lib.ptr(image), _lib.ptr(tgt), _lib.ptr(gout), _lib.ptr(ws), nbytes,
                  _lib.ptr(gimg))
        _lib.call("gs_composite_bwd", s, n, _lib.ptr(pre["records"]), _lib.ptr(b["sorted_gids"]),
                  b["sorted_gids"].shape[0], _lib.ptr(b["ranges"]), int(W), int(H), _lib.ptr(bg), _lib.ptr(gimg),
                  _lib.ptr(fT), _lib.ptr(nc), _lib.ptr(order), _lib.ptr(grec), None, 1, _lib.ptr(b["window"]),
                  None)
        # preprocessing VJP + statistics + masked Adam, in place
        ost = state.opt_state
        moments = [ost.mu[f] for f in _FIELDS] + [ost.nu[f] for f in _FIELDS]
        P = ctypes.c_void_p * 10
        lrs = (ctypes.c_double * 5)(*[optimizer.lr_at(f, ost.count) for f in _FIELDS])
        focal = float(np.float32((camera.fx + camera.fy) / 2.0))
        pixel_scale = float(np.float32(float(W) * float(H) * 3.0))
        w2c = torch.as_tensor(camera.W2C, dtype=torch.float32, device=dev).contiguous()
        valid = pre["valid"]
        _lib.call("gs_preprocess_bwd_adam", s, n, params.sh_coeffs.shape[1], int(sh_degree),
                  *[_lib.ptr(t) for t in fields], _lib.ptr(w2c), int(W), int(H), float(camera.fx),
                  float(camera.fy), float(camera.cx), float(camera.cy), _lib.ptr(grec),
                  P(*[m.data_ptr() for m in moments]), lrs, ost.count + 1, optimizer.b1, optimizer.b2,
                  optimizer.eps, _lib.ptr(state.active_mask), _lib.ptr(valid), _lib.ptr(pre["radii"]), focal,
                  pixel_scale, _lib.ptr(state.grad_accum), _lib.ptr(state.denom), _lib.ptr(state.max_radii))
        ost.count += 1
        metrics = {"l1": l1, "ssim": terms[4]}
        metrics.update(_stats_metrics(b["stats"]))
    return state, total, metrics


def _stats_metrics(stats: torch.Tensor) -> dict:
    """The renderer-health metrics of trainer.py:28-39 as float32 device scalars, from
    one conversion of the binning stats."""
    S = _lib.STAT
    f = stats.to(torch.float32)
    out = {k: f[S[k]] for k in _EXTRA_KEYS if k != "mean_interactions_per_tile"}
    out["mean_interactions_per_tile"] = stats.view(torch.float32)[S["mean_per_tile"]]
    return out
