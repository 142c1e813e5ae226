"""jax_gs/renderer/rasterizer_tpu.py on the GPU: the compositing variant that gathers
each tile's entries one by one (rasterizer_tpu.py:90-97).

It computes the same image as rasterizer.render_tiles except where a 512-entry chunk of a
tile starts within 512 entries of the end of the sorted arrays: rasterizer.py:184-190
clamps that chunk's slice to the arrays' last 512 entries, while this variant reads the
tile's own entries.  Both run the same kernels: the compositing launch takes no chunk
window here (gs_composite_fwd/bwd with window = NULL).  Differentiable like the
reference's (JAX autodiff of rasterizer_tpu.py:13-135): the image's cotangent reaches
means2D, cov2D, opacities, colors and a tensor background.
"""
from __future__ import annotations

from .rasterizer import BLOCK_SIZE, MAX_TILE_CHUNKS, MAX_TILE_INTERACTIONS, TILE_SIZE, _render_tiles

__all__ = ["render_tiles_tpu", "TILE_SIZE", "BLOCK_SIZE", "MAX_TILE_CHUNKS", "MAX_TILE_INTERACTIONS"]


def render_tiles_tpu(means2D, cov2D, opacities, colors, sorted_tile_ids, sorted_gaussian_ids, H, W, background=None):
    """rasterizer_tpu.py:13-135: (image [H, W, 3]) from the caller's sorted arrays in the
    reference's layout (get_tile_interactions); every entry of a tile (capped at 4096) is
    read from the tile's own positions of sorted_gaussian_ids."""
    return _render_tiles(means2D, cov2D, opacities, colors, sorted_tile_ids, sorted_gaussian_ids, H, W, background,
                         clamped_windows=False)
