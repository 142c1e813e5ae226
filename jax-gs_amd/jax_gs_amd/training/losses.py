"""L1 loss on the GPU (jax_gs/training/losses.py:4-8) with its gradient seed."""
from __future__ import annotations

import torch

from .. import _lib


class _L1(torch.autograd.Function):
    @staticmethod
    def forward(ctx, pred, target):
        pred = pred.contiguous()
        target = target.contiguous()
        loss = torch.empty((), dtype=torch.float32, device=pred.device)
        grad = torch.empty_like(pred)
        _lib.call("gs_l1_loss", _lib.stream_handle(pred.device), pred.numel(), _lib.ptr(pred), _lib.ptr(target),
                  _lib.ptr(loss), _lib.ptr(grad))
        ctx.save_for_backward(grad)
        return loss

    @staticmethod
    def backward(ctx, g):
        (grad,) = ctx.saved_tensors
        return grad * g, None


def l1_loss(pred: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
    """mean(|pred - target|); backward seeds sign(pred - target) / count (sign(0) = 0)."""
    if pred.shape != target.shape:
        raise ValueError(f"l1_loss: shapes {tuple(pred.shape)} and {tuple(target.shape)} differ")
    return _L1.apply(pred, target)
