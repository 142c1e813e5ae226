"""Spherical harmonics of jax_gs/renderer/sh.py: the constants and eval_sh.

The renderer evaluates SH inside the fused preprocessing kernel (gs_preprocess_fwd);
``eval_sh`` is the module function on its own (gs_eval_sh, with its VJP gs_eval_sh_bwd
for autograd), for callers that colour Gaussians outside the render path.
"""
from __future__ import annotations

import torch

from .. import _lib
from ._buffers import check_f32

C0 = 0.28209479177387814
C1 = 0.4886025119029199
C2 = [1.0925484305920792, -1.0925484305920792, 0.31539156525252005, -1.0925484305920792, 0.5462742152960396]
C3 = [-0.5900435899266435, 2.890611442640554, -0.4570457994644658, 0.3731763325901154, -0.4570457994644658,
      1.445305721320277, -0.5900435899266435]


class _EvalSH(torch.autograd.Function):
    @staticmethod
    def forward(ctx, sh, dirs, deg):
        n, K = sh.shape[0], sh.shape[1]
        out = torch.empty((n, 3), dtype=torch.float32, device=sh.device)
        _lib.call("gs_eval_sh", _lib.stream_handle(sh.device), n, K, deg, _lib.ptr(sh), _lib.ptr(dirs), _lib.ptr(out))
        ctx.deg = deg
        ctx.save_for_backward(sh, dirs)
        return out

    @staticmethod
    def backward(ctx, g):
        sh, dirs = ctx.saved_tensors
        n, K = sh.shape[0], sh.shape[1]
        g = g.contiguous()
        g_sh = torch.empty_like(sh)
        g_dirs = torch.empty_like(dirs) if ctx.needs_input_grad[1] else None
        _lib.call("gs_eval_sh_bwd", _lib.stream_handle(sh.device), n, K, ctx.deg, _lib.ptr(sh), _lib.ptr(dirs),
                  _lib.ptr(g), _lib.ptr(g_sh), _lib.ptr(g_dirs))
        return (g_sh if ctx.needs_input_grad[0] else None), g_dirs, None


def eval_sh(sh_degree: int, sh_coeffs: torch.Tensor, view_dirs: torch.Tensor) -> torch.Tensor:
    """sh.py:25-74: view-dependent colours [N, 3] of degree sh_degree (0..3) from
    sh_coeffs [N, K, 3] (K >= (sh_degree+1)^2) and view_dirs [N, 3] (used as given; the
    renderer normalises them), without the renderer's +0.5 and clip.  Differentiable with
    respect to both arrays."""
    deg = int(sh_degree)
    if not 0 <= deg <= 3:
        raise ValueError(f"sh_degree must be in 0..3 (got {deg})")
    dev = sh_coeffs.device
    n = sh_coeffs.shape[0]
    if sh_coeffs.dim() != 3 or sh_coeffs.shape[2] != 3 or sh_coeffs.shape[1] < (deg + 1) ** 2:
        raise ValueError(f"sh_coeffs must be [N, K >= {(deg + 1) ** 2}, 3] (got {tuple(sh_coeffs.shape)})")
    sh = check_f32("sh_coeffs", sh_coeffs, tuple(sh_coeffs.shape), dev)
    dirs = check_f32("view_dirs", view_dirs, (n, 3), dev)
    return _EvalSH.apply(sh, dirs, deg)
