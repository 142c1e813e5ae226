"""project_gaussians on the GPU (jax_gs/renderer/projection.py:6-79)."""
from __future__ import annotations

import torch

from .. import _lib
from ..core.camera import Camera
from ..core.gaussians import Gaussians
from ._buffers import as_mask, check_f32


def preprocess(gaussians: Gaussians, camera: Camera, mask=None, sh_degree: int = 0, records: bool = True,
               projected: bool = True) -> dict:
    """Fused projection + covariance + SH colour (+ compositing records) for every Gaussian.

    Returns a dict of device tensors: means2d [N,2], cov2d [N,2,2], radii [N] (float,
    integer-valued), valid [N] (bool), depths [N], colors [N,3] and records [N,12].
    projected=False (with records) leaves cov2d and colors out (None): the records hold
    the conic and colour compositing reads, and the renderer needs nothing else of them."""
    if not projected and not records:
        raise ValueError("preprocess: projected=False needs records=True")
    means = gaussians.means
    dev = means.device
    n = means.shape[0]
    means = check_f32("means", means, (n, 3), dev)
    scales = check_f32("scales", gaussians.scales, (n, 3), dev)
    quats = check_f32("quaternions", gaussians.quaternions, (n, 4), dev)
    opac = check_f32("opacities", gaussians.opacities, (n, 1), dev)
    sh = gaussians.sh_coeffs
    if sh.ndim != 3 or sh.shape[0] != n or sh.shape[2] != 3:
        raise ValueError(f"sh_coeffs has shape {tuple(sh.shape)}, expected ({n}, K, 3)")
    sh = check_f32("sh_coeffs", sh, tuple(sh.shape), dev)
    w2c = check_f32("W2C", torch.as_tensor(camera.W2C, dtype=torch.float32, device=dev), (4, 4), dev)
    m = as_mask(mask, n, dev)
    out = dict(
        means2d=torch.empty((n, 2), dtype=torch.float32, device=dev),
        cov2d=torch.empty((n, 2, 2), dtype=torch.float32, device=dev) if projected else None,
        radii=torch.empty((n,), dtype=torch.float32, device=dev),
        valid=torch.empty((n,), dtype=torch.uint8, device=dev),
        depths=torch.empty((n,), dtype=torch.float32, device=dev),
        colors=torch.empty((n, 3), dtype=torch.float32, device=dev) if projected else None,
        records=torch.empty((n, _lib.GS_REC_STRIDE), dtype=torch.float32, device=dev) if records else None,
    )
    _lib.call("gs_preprocess_fwd", _lib.stream_handle(dev), n, sh.shape[1], int(sh_degree), _lib.ptr(means),
              _lib.ptr(scales), _lib.ptr(quats), _lib.ptr(opac), _lib.ptr(sh), _lib.ptr(m), _lib.ptr(w2c),
              int(camera.W), int(camera.H), float(camera.fx), float(camera.fy), float(camera.cx), float(camera.cy),
              _lib.ptr(out["means2d"]), _lib.ptr(out["cov2d"]), _lib.ptr(out["radii"]), _lib.ptr(out["valid"]),
              _lib.ptr(out["depths"]), _lib.ptr(out["colors"]), _lib.ptr(out["records"]))
    return out


class _ProjectGaussians(torch.autograd.Function):
    """project_gaussians with its VJP (JAX autodiff of projection.py:6-79): cotangents of
    means2D, cov2D (all four entries) and z flow to the means, scales, quaternions and the
    camera's W2C; radii and valid_mask are not differentiable; opacities, SH and mask get none."""

    @staticmethod
    def forward(ctx, means, scales, quats, w2c, opac, sh, mask, static):
        W, H, fx, fy, cx, cy = static
        dev = means.device
        n = means.shape[0]
        out = dict(means2d=torch.empty((n, 2), dtype=torch.float32, device=dev),
                   cov2d=torch.empty((n, 2, 2), dtype=torch.float32, device=dev),
                   radii=torch.empty((n,), dtype=torch.float32, device=dev),
                   valid=torch.empty((n,), dtype=torch.uint8, device=dev),
                   depths=torch.empty((n,), dtype=torch.float32, device=dev),
                   colors=torch.empty((n, 3), dtype=torch.float32, device=dev))  # degree 0, not returned
        _lib.call("gs_preprocess_fwd", _lib.stream_handle(dev), n, sh.shape[1], 0, _lib.ptr(means), _lib.ptr(scales),
                  _lib.ptr(quats), _lib.ptr(opac), _lib.ptr(sh), _lib.ptr(mask), _lib.ptr(w2c), int(W), int(H),
                  float(fx), float(fy), float(cx), float(cy), _lib.ptr(out["means2d"]), _lib.ptr(out["cov2d"]),
                  _lib.ptr(out["radii"]), _lib.ptr(out["valid"]), _lib.ptr(out["depths"]), _lib.ptr(out["colors"]),
                  None)
        ctx.static = static
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(means, scales, quats, w2c)
        valid = out["valid"].view(torch.bool)  # the kernel writes 0/1 bytes
        ctx.mark_non_differentiable(out["radii"], valid)
        return out["means2d"], out["cov2d"], out["radii"], valid, out["depths"]

    @staticmethod
    def backward(ctx, g_m2, g_cov, _g_radii, _g_valid, g_z):
        none = (None,) * 4
        if g_m2 is None and g_cov is None and g_z is None:
            return (None,) * 8
        W, H, fx, fy, cx, cy = ctx.static
        means, scales, quats, w2c = ctx.saved_tensors
        dev = means.device
        n = means.shape[0]
        g_m2 = torch.zeros((n, 2), dtype=torch.float32, device=dev) if g_m2 is None else g_m2.contiguous()
        g_cov = torch.zeros((n, 2, 2), dtype=torch.float32, device=dev) if g_cov is None else g_cov.contiguous()
        g_z = None if g_z is None else g_z.contiguous()
        gm, gs_, gq = torch.empty_like(means), torch.empty_like(scales), torch.empty_like(quats)
        gw = ws = None
        nb = 0
        if ctx.needs_input_grad[3]:
            gw = torch.empty((4, 4), dtype=torch.float32, device=dev)
            nb = _lib.lib().gs_preprocess_bwd_w2c_workspace_size(n)
            ws = torch.empty((nb,), dtype=torch.uint8, device=dev)
        _lib.call("gs_project_bwd", _lib.stream_handle(dev), n, _lib.ptr(means), _lib.ptr(scales), _lib.ptr(quats),
                  _lib.ptr(w2c), float(fx), float(fy), _lib.ptr(g_m2), _lib.ptr(g_cov), _lib.ptr(g_z), _lib.ptr(gm),
                  _lib.ptr(gs_), _lib.ptr(gq), _lib.ptr(gw), _lib.ptr(ws), nb)
        return (gm, gs_, gq, gw) + none


def project_gaussians(gaussians: Gaussians, camera: Camera, mask=None):
    """(means2D [N,2], cov2D [N,2,2], radii [N], valid_mask [N] bool, depths [N]).

    The reference's project_gaussians (projection.py:6-79), computed by the fused
    preprocessing kernel and differentiable like it: means2D, cov2D and depths carry
    gradients to gaussians.means / scales / quaternions and to camera.W2C (gs_project_bwd)."""
    means = gaussians.means
    dev = means.device
    n = means.shape[0]
    means = check_f32("means", means, (n, 3), dev)
    scales = check_f32("scales", gaussians.scales, (n, 3), dev)
    quats = check_f32("quaternions", gaussians.quaternions, (n, 4), dev)
    opac = check_f32("opacities", gaussians.opacities, (n, 1), dev).detach()
    sh = gaussians.sh_coeffs
    if sh.ndim != 3 or sh.shape[0] != n or sh.shape[2] != 3:
        raise ValueError(f"sh_coeffs has shape {tuple(sh.shape)}, expected ({n}, K, 3)")
    sh = check_f32("sh_coeffs", sh, tuple(sh.shape), dev).detach()
    w2c = check_f32("W2C", torch.as_tensor(camera.W2C, dtype=torch.float32, device=dev), (4, 4), dev)
    m = as_mask(mask, n, dev)
    static = (int(camera.W), int(camera.H), float(camera.fx), float(camera.fy), float(camera.cx), float(camera.cy))
    return _ProjectGaussians.apply(means, scales, quats, w2c, opac, sh, m, static)
