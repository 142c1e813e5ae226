"""jax_gs_amd -- MI355X (gfx950) tiled Gaussian-splatting rasterizer.

Drop-in for the renderer of ghif/jax-gs (jax_gs/renderer/*): the same ``render``
signature and ``extras``, backed by hand-written HIP kernels in libgsraster.so
(include/gs_raster.h) called through ctypes with torch-ROCm device tensors.
"""
from .core.camera import Camera
from .core.gaussians import Gaussians, init_gaussians_from_pcd
from .renderer.renderer import render, render_l1

__all__ = ["Camera", "Gaussians", "init_gaussians_from_pcd", "render", "render_l1"]
