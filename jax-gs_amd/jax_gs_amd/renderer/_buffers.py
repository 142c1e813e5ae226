"""Argument checking and output allocation shared by the renderer entry points."""
from __future__ import annotations

import torch


def check_f32(name: str, t: torch.Tensor, shape: tuple, device=None) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.dtype != torch.float32:
        raise TypeError(f"{name} must be float32 (got {t.dtype})")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    if device is not None and t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must live on the GPU (the renderer has no CPU path)")
    return t.contiguous()


def as_mask(mask, n: int, device) -> torch.Tensor | None:
    if mask is None:
        return None
    m = torch.as_tensor(mask, device=device)
    if tuple(m.shape) != (n,):
        raise ValueError(f"mask has shape {tuple(m.shape)}, expected ({n},)")
    return as_bytes(m)


def as_bytes(m: torch.Tensor) -> torch.Tensor:
    """A 0/1 byte view of a bool tensor (no cast kernel: torch stores bools as bytes), else
    the tensor cast to uint8; contiguous."""
    m = m.contiguous()
    return m.view(torch.uint8) if m.dtype == torch.bool else m.to(torch.uint8)


_BLACK: dict = {}


def background_tensor(background, device) -> torch.Tensor:
    if background is None:
        # one read-only black background per device (no fill kernel per call)
        key = str(torch.device(device))
        if key not in _BLACK:
            _BLACK[key] = torch.zeros(3, dtype=torch.float32, device=device)
        return _BLACK[key]
    b = torch.as_tensor(background, dtype=torch.float32, device=device).reshape(3)
    return b.contiguous()


def num_tiles(W: int, H: int, tile: int = 16) -> tuple[int, int, int]:
    tx = (W + tile - 1) // tile
    ty = (H + tile - 1) // tile
    return tx, ty, tx * ty
