"""Densification statistics of a training step (jax_gs/training/trainer.py:278-294)."""
from __future__ import annotations

import numpy as np
import torch

from .. import _lib


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
