"""jax_gs/renderer/rasterizer_tpu.py on the GPU: the compositing variant that gathers
each tile's entries one by one (rasterizer_tpu.py:90-97).  It computes the same image as
rasterizer.render_tiles except where a 512-entry chunk of a tile starts within 512
entries of the end of the sorted arrays (rasterizer.py:184-190 clamps that chunk's
slice; this variant reads the tile's own entries)."""
from .rasterizer import BLOCK_SIZE, MAX_TILE_CHUNKS, MAX_TILE_INTERACTIONS, TILE_SIZE, render_tiles_tpu

__all__ = ["render_tiles_tpu", "TILE_SIZE", "BLOCK_SIZE", "MAX_TILE_CHUNKS", "MAX_TILE_INTERACTIONS"]
