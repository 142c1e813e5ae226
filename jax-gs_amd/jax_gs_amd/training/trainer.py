"""The training step (jax_gs/training/trainer.py:11-169) on the GPU path.

``train_step`` renders the active Gaussians, takes the trainer's loss
(0.8 L1 + 0.2 D-SSIM, one forward and one backward kernel), backpropagates through the
rasterizer, accumulates the densification statistics from the pre-update means and
applies the masked Adam step -- the same sequence as the reference's jitted step, with the
state's tensors updated in place.  ``accumulate_from_extras`` is the statistics part
(trainer.py:278-294) on its own.
"""
from __future__ import annotations

import numpy as np
import torch

from .. import _lib
from ..core.camera import Camera
from ..core.gaussians import Gaussians


def accumulate_from_extras(state: dict, grad_means: torch.Tensor, means: torch.Tensor, camera, extras: dict,
                           active=None) -> None:
    """Update state['grad_accum'] (f32 [N]), state['denom'] (i32 [N]), state['max_radii'] (f32 [N]) in place."""
    dev = means.device
    n = means.shape[0]
    focal = float(np.float32((camera.fx + camera.fy) / 2.0))
    pixel_scale = float(np.float32(float(camera.W) * float(camera.H) * 3.0))
    w2c = torch.as_tensor(camera.W2C, dtype=torch.float32, device=dev).contiguous()
    valid = extras["valid_mask"].to(torch.uint8).contiguous()
    act = None if active is None else torch.as_tensor(active, device=dev).to(torch.uint8).contiguous()
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
    for k in ("n_interactions", "mean_interactions_per_tile", "max_interactions_per_tile", "overflow_tiles",
              "overflow_interactions", "truncated_tiles", "truncated_interactions", "radius_cap_violations"):
        metrics[k] = extras[k].to(torch.float32)
    return total, metrics, image, extras


def train_step(state, target_image, w2c, camera_static, optimizer, fast_tpu_rasterizer: bool = False,
               sh_degree: int = 0):
    """trainer.py:55-169 (single device): returns (state, loss, metrics) with the state's
    Gaussians, optimizer moments and statistics updated in place."""
    W, H, fx, fy, cx, cy = camera_static
    params = state.gaussians
    dev = params.means.device
    camera = Camera(int(W), int(H), float(fx), float(fy), float(cx), float(cy),
                    torch.as_tensor(w2c, dtype=torch.float32, device=dev), None)
    fields = ("means", "scales", "quaternions", "opacities", "sh_coeffs")
    # leaves sharing the state's storage: the optimizer updates them in place afterwards
    leaves = [getattr(params, f).detach().requires_grad_(True) for f in fields]
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
