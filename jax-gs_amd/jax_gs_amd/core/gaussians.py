"""Gaussian parameter container, as jax_gs/core/gaussians.py:5-11.

Arrays (float32, row-major, on the GPU for rendering):
  means [N,3], scales [N,3] (log), quaternions [N,4] (w,x,y,z, unnormalised),
  opacities [N,1] (logit), sh_coeffs [N,K,3] (K = (degree+1)^2 used, 16 stored by
  the reference's initialiser).
"""
from __future__ import annotations

import dataclasses

import torch

SH_C0 = 0.28209479177387814


@dataclasses.dataclass
class Gaussians:
    means: torch.Tensor
    scales: torch.Tensor
    quaternions: torch.Tensor
    opacities: torch.Tensor
    sh_coeffs: torch.Tensor

    def replace(self, **kw) -> "Gaussians":
        """Functional update, like chex.dataclass.replace."""
        return dataclasses.replace(self, **kw)

    def to(self, device) -> "Gaussians":
        return Gaussians(*(getattr(self, f.name).to(device) for f in dataclasses.fields(self)))


def init_gaussians_from_pcd(points: torch.Tensor, colors: torch.Tensor) -> Gaussians:
    """Point-cloud initialiser with the reference's conventions (gaussians.py:13-56):
    log-scale -3, identity rotation, opacity logit 0, SH DC = (c - 0.5) / C0, 16 coefficients.
    A cloud whose largest colour value is below 1e-3 gets uniform random colours in
    [0.1, 0.9) (gaussians.py:40-42), decided on the device; the draw comes from torch's
    generator seeded 42 where the reference uses jax.random with PRNGKey(42), so the
    distribution matches and the values do not."""
    points = torch.as_tensor(points, dtype=torch.float32)
    colors = torch.as_tensor(colors, dtype=torch.float32, device=points.device)
    n = points.shape[0]
    dev = points.device
    gen = torch.Generator(device=dev)
    gen.manual_seed(42)
    rand = torch.rand(colors.shape, generator=gen, device=dev, dtype=torch.float32) * 0.8 + 0.1
    colors = torch.where(colors.max() < 1e-3, rand, colors) if colors.numel() else colors
    sh = torch.zeros((n, 16, 3), dtype=torch.float32, device=dev)
    sh[:, 0, :] = (colors - 0.5) / SH_C0
    quats = torch.zeros((n, 4), dtype=torch.float32, device=dev)
    quats[:, 0] = 1.0
    return Gaussians(means=points.clone(), scales=torch.full((n, 3), -3.0, device=dev), quaternions=quats,
                     opacities=torch.zeros((n, 1), device=dev), sh_coeffs=sh)
