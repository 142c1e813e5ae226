"""Photometric losses on the GPU (jax_gs/training/losses.py:4-75) with their VJPs.

``l1_loss`` and ``mse_loss`` run one reduction kernel that also writes the gradient
seed; ``ssim``, ``d_ssim_loss`` and ``l1_ssim_loss`` (the trainer's
``(1 - lambda) l1 + lambda d_ssim``, trainer.py:18-26) share one forward kernel that
computes the L1 and SSIM means together and one backward kernel that writes the
combined gradient of the image.
"""
from __future__ import annotations

import torch

from .. import _lib


class _MeanLoss(torch.autograd.Function):
    """Forward: the mean only.  Backward: one kernel writes seed(pred - target) * (g / count)
    with the loss cotangent g read on the device (no host sync, no separate scaling pass)."""

    @staticmethod
    def forward(ctx, pred, target, entry):
        pred = pred.contiguous()
        target = target.contiguous()
        loss = torch.empty((), dtype=torch.float32, device=pred.device)
        _lib.call(entry, _lib.stream_handle(pred.device), pred.numel(), _lib.ptr(pred), _lib.ptr(target),
                  _lib.ptr(loss), None)
        ctx.save_for_backward(pred, target)
        ctx.entry = entry
        return loss

    @staticmethod
    def backward(ctx, g):
        pred, target = ctx.saved_tensors
        g = g.to(device=pred.device, dtype=torch.float32).contiguous()
        grad = torch.empty_like(pred)
        _lib.call(ctx.entry + "_bwd", _lib.stream_handle(pred.device), pred.numel(), _lib.ptr(pred),
                  _lib.ptr(target), _lib.ptr(g), _lib.ptr(grad))
        return grad, None, None


def _check(name, pred, target):
    if pred.shape != target.shape:
        raise ValueError(f"{name}: shapes {tuple(pred.shape)} and {tuple(target.shape)} differ")


def l1_loss(pred: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
    """mean(|pred - target|); backward seeds sign(pred - target) / count (sign(0) = 0)."""
    _check("l1_loss", pred, target)
    return _MeanLoss.apply(pred, target, "gs_l1_loss")


def mse_loss(pred: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
    """mean((pred - target)^2) (losses.py:10-14); backward seeds 2 (pred - target) / count."""
    _check("mse_loss", pred, target)
    return _MeanLoss.apply(pred, target, "gs_mse_loss")


class _L1SSIM(torch.autograd.Function):
    """window 11 with at most 4 channels: the tiled kernels (gs_l1_ssim); any other window
    size or channel count: gs_l1_ssim_window."""

    @staticmethod
    def forward(ctx, pred, target, window_size):
        pred = pred.contiguous()
        target = target.contiguous()
        H, W, C = pred.shape
        dev = pred.device
        fast = window_size == 11 and C <= 4
        if fast:
            nbytes = _lib.lib().gs_l1_ssim_workspace_size(H, W, C)
        else:
            nbytes = _lib.lib().gs_l1_ssim_window_workspace_size(H, W, C, window_size)
        ws = torch.empty((nbytes,), dtype=torch.uint8, device=dev)
        out = torch.empty((2,), dtype=torch.float32, device=dev)
        grad_needed = ctx.needs_input_grad[0]
        if fast:
            _lib.call("gs_l1_ssim", _lib.stream_handle(dev), H, W, C, _lib.ptr(pred), _lib.ptr(target),
                      _lib.ptr(out), int(grad_needed), _lib.ptr(ws), nbytes)
        else:
            _lib.call("gs_l1_ssim_window", _lib.stream_handle(dev), H, W, C, int(window_size), _lib.ptr(pred),
                      _lib.ptr(target), _lib.ptr(out), int(grad_needed), _lib.ptr(ws), nbytes)
        ctx.set_materialize_grads(False)
        ctx.window = None if fast else int(window_size)
        if grad_needed:
            ctx.save_for_backward(pred, target, ws)
        return out[0], out[1]

    @staticmethod
    def backward(ctx, g_l1, g_ssim):
        pred, target, ws = ctx.saved_tensors
        dev = pred.device
        zero = torch.zeros((), dtype=torch.float32, device=dev)
        gout = torch.stack([zero if g_l1 is None else g_l1.to(torch.float32),
                            zero if g_ssim is None else g_ssim.to(torch.float32)])
        H, W, C = pred.shape
        grad = torch.empty_like(pred)
        if ctx.window is None:
            _lib.call("gs_l1_ssim_bwd", _lib.stream_handle(dev), H, W, C, _lib.ptr(pred), _lib.ptr(target),
                      _lib.ptr(gout), _lib.ptr(ws), ws.numel(), _lib.ptr(grad))
        else:
            _lib.call("gs_l1_ssim_window_bwd", _lib.stream_handle(dev), H, W, C, ctx.window, _lib.ptr(pred),
                      _lib.ptr(target), _lib.ptr(gout), _lib.ptr(ws), ws.numel(), _lib.ptr(grad))
        return grad, None, None


def l1_and_ssim(pred: torch.Tensor, target: torch.Tensor, window_size: int = 11):
    """(mean |pred - target|, mean SSIM) of [H, W, C] images from one forward kernel;
    window_size in [1, 63] (losses.py:16)."""
    _check("ssim", pred, target)
    if pred.dim() != 3:
        raise ValueError("ssim: images must be [H, W, C]")
    if not 1 <= int(window_size) <= 63:
        raise ValueError(f"ssim: window_size must be in [1, 63] (got {window_size})")
    return _L1SSIM.apply(pred, target, int(window_size))


def ssim(img1: torch.Tensor, img2: torch.Tensor, window_size: int = 11, size_average: bool = True) -> torch.Tensor:
    """losses.py:16-68: mean SSIM with a window_size-tap Gaussian window (sigma 1.5).  The
    reference's size_average=False also reduces over every axis of an [H, W, C] map."""
    del size_average
    return l1_and_ssim(img1, img2, window_size)[1]


def _d_ssim(s: torch.Tensor) -> torch.Tensor:
    # max(0, (1 - ssim) / 2); torch.maximum passes half the cotangent at a tie, as lax.max
    return torch.maximum(torch.zeros_like(s), (1.0 - s) / 2.0)


def d_ssim_loss(pred: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
    """losses.py:70-75: max(0, (1 - ssim(pred, target)) / 2)."""
    return _d_ssim(ssim(pred, target))


def l1_ssim_loss(pred: torch.Tensor, target: torch.Tensor, lambda_ssim: float = 0.2):
    """trainer.py:18-26: ((1 - lambda) l1 + lambda d_ssim, l1, d_ssim), all three from one
    forward kernel; the backward writes the image gradient of the total in one kernel."""
    l1, s = l1_and_ssim(pred, target)
    d = _d_ssim(s)
    return (1.0 - lambda_ssim) * l1 + lambda_ssim * d, l1, d
