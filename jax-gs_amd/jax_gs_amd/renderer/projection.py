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


def project_gaussians(gaussians: Gaussians, camera: Camera, mask=None):
    """(means2D [N,2], cov2D [N,2,2], radii [N], valid_mask [N] bool, depths [N]).

    Same outputs as the reference's project_gaussians; computed by the fused
    preprocessing kernel (not differentiable through this entry point; use render)."""
    out = preprocess(gaussians, camera, mask=mask, sh_degree=0, records=False)
    return out["means2d"], out["cov2d"], out["radii"], out["valid"].bool(), out["depths"]
