"""Static-capacity density control on the GPU (jax_gs/training/density.py).

``DensityState`` holds the Gaussians padded to a fixed capacity, the optimizer state,
the active mask and the densification statistics, like the reference's.
``densify_and_prune`` and ``reset_opacities`` run as device kernels
(``gs_densify_and_prune``, ``gs_reset_opacities``) and update the state's tensors in
place (the reference returns a new state; here the same state object comes back).
The split jitter uses standard normal draws from torch's generator on the device where
the reference uses ``jax.random.normal``: the draws differ, their use is the same.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import torch

from .. import _lib
from ..core.gaussians import Gaussians
from .optimizer import FIELDS, Adam, AdamState


@dataclass
class DensityState:
    gaussians: Gaussians
    opt_state: Optional[AdamState]
    active_mask: torch.Tensor  # uint8 [M] (0/1)
    num_active: int
    grad_accum: torch.Tensor   # float32 [M]
    denom: torch.Tensor        # int32 [M]
    max_radii: torch.Tensor    # float32 [M]


def init_density_state(gaussians: Gaussians, optimizer: Optional[Adam], max_gaussians: int) -> DensityState:
    """density.py:19-61: pad every array to max_gaussians (padded quaternions are
    (1, 0, 0, 0)), the first N active, zero statistics, the optimizer initialised on the
    padded arrays."""
    n = gaussians.means.shape[0]
    if max_gaussians < n:
        raise ValueError(f"init_density_state: capacity {max_gaussians} < {n} Gaussians")
    dev = gaussians.means.device

    def pad(x):
        out = torch.zeros((max_gaussians,) + tuple(x.shape[1:]), dtype=torch.float32, device=dev)
        out[:n] = x
        return out

    quats = pad(gaussians.quaternions)
    quats[n:, 0] = 1.0
    padded = Gaussians(pad(gaussians.means), pad(gaussians.scales), quats, pad(gaussians.opacities),
                       pad(gaussians.sh_coeffs))
    active = torch.zeros((max_gaussians,), dtype=torch.uint8, device=dev)
    active[:n] = 1
    return DensityState(gaussians=padded, opt_state=optimizer.init(padded) if optimizer is not None else None,
                        active_mask=active, num_active=n,
                        grad_accum=torch.zeros((max_gaussians,), dtype=torch.float32, device=dev),
                        denom=torch.zeros((max_gaussians,), dtype=torch.int32, device=dev),
                        max_radii=torch.zeros((max_gaussians,), dtype=torch.float32, device=dev))


def densify_and_prune(state: DensityState, generator: Optional[torch.Generator] = None, densify_enabled: bool = True,
                      grad_threshold: float = 0.0002, min_opacity: float = 0.005, extent: float = 5.0,
                      max_screen_size: int = 512, noise: Optional[torch.Tensor] = None) -> DensityState:
    """density.py:98-211 in place; returns the state.  ``noise`` ([M, 3] standard normal)
    overrides the draws from ``generator``.  state.last_counts (int32 [5] on the device):
    clones, splits, pruned, available slots, densified."""
    g = state.gaussians
    M = g.means.shape[0]
    dev = g.means.device
    if noise is None:
        noise = torch.randn((M, 3), generator=generator, device=dev, dtype=torch.float32)
    noise = noise.to(device=dev, dtype=torch.float32).contiguous()
    if tuple(noise.shape) != (M, 3):
        raise ValueError(f"densify_and_prune: noise must be [{M}, 3]")
    moments = []
    if state.opt_state is not None:
        moments = [state.opt_state.mu[f] for f in FIELDS] + [state.opt_state.nu[f] for f in FIELDS]
    for t in [getattr(g, f) for f in FIELDS] + moments:
        if t.dtype != torch.float32 or not t.is_contiguous() or t.shape[0] != M:
            raise ValueError("densify_and_prune: every array must be contiguous float32 with the capacity rows")
    nbytes = _lib.lib().gs_densify_workspace_size(M)
    ws = torch.empty((nbytes,), dtype=torch.uint8, device=dev)
    counts = torch.empty((5,), dtype=torch.int32, device=dev)
    P = ctypes.c_void_p * max(len(moments), 1)
    mptr = P(*[m.data_ptr() for m in moments]) if moments else None
    _lib.call("gs_densify_and_prune", _lib.stream_handle(dev), M, g.sh_coeffs.shape[1], _lib.ptr(g.means),
              _lib.ptr(g.scales), _lib.ptr(g.quaternions), _lib.ptr(g.opacities), _lib.ptr(g.sh_coeffs),
              len(moments), mptr, _lib.ptr(state.active_mask), _lib.ptr(state.grad_accum), _lib.ptr(state.denom),
              _lib.ptr(state.max_radii), _lib.ptr(noise), int(bool(densify_enabled)), float(grad_threshold),
              float(min_opacity), float(extent), float(max_screen_size), _lib.ptr(ws), nbytes, _lib.ptr(counts))
    state.last_counts = counts
    return state


def reset_opacities(state: DensityState, reset_val: float = 0.01) -> DensityState:
    """density.py:69-93: active Gaussians' opacity logits set to logit(reset_val)."""
    g = state.gaussians
    _lib.call("gs_reset_opacities", _lib.stream_handle(g.means.device), g.opacities.shape[0],
              _lib.ptr(state.active_mask), float(reset_val), _lib.ptr(g.opacities))
    return state
