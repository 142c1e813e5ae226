"""Pinhole camera, as jax_gs/core/camera.py:4-21 (a NamedTuple of intrinsics + W2C)."""
from __future__ import annotations

from typing import NamedTuple

import torch


class Camera(NamedTuple):
    W: int  # image width
    H: int  # image height
    fx: float
    fy: float
    cx: float
    cy: float
    W2C: torch.Tensor  # [4,4] world-to-camera
    full_proj: torch.Tensor  # unused by the renderer (kept for signature parity)

    @property
    def center(self) -> torch.Tensor:
        """Optical centre in world coordinates, -R^T t (camera.py:15-21)."""
        R = self.W2C[:3, :3]
        t = self.W2C[:3, 3]
        return -R.T @ t
