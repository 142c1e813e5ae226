"""Tile binning and compositing on the GPU (jax_gs/renderer/rasterizer.py).

Constants and function names follow the reference module so that callers (and the
2DGS family's ``from ...rasterizer import get_tile_interactions, TILE_SIZE``) keep
working.  Arrays are torch tensors on the GPU.
"""
from __future__ import annotations

import torch

from .. import _lib
from ._buffers import as_bytes, background_tensor, check_f32, num_tiles

TILE_SIZE = 16  # rasterizer.py:6
OFFSET_SIZE = 16  # rasterizer.py:7
BLOCK_SIZE = 512  # rasterizer.py:8
MAX_TILE_CHUNKS = 8  # rasterizer.py:9
MAX_TILE_INTERACTIONS = BLOCK_SIZE * MAX_TILE_CHUNKS  # rasterizer.py:10
# entries are indexed with int32 (ranges, ids): the largest entry list the kernels take
MAX_ENTRIES = 2 ** 31 - 1


def default_capacity(n: int) -> int:
    """The reference's static entry bound max(256 n, 512) (rasterizer.py:56-69, 107-110),
    limited to what int32 indices address (n >= 8,388,608 reaches that limit; a count above
    it is flagged in the binning stats, GS_STAT_CAPACITY_EXCEEDED, and the first entries of
    the reference order are kept)."""
    return min(max(256 * int(n), BLOCK_SIZE), MAX_ENTRIES)


def check_capacity(capacity: int | None, n: int) -> int:
    cap = default_capacity(n) if not capacity else int(capacity)
    if not 0 < cap <= MAX_ENTRIES:
        raise ValueError(f"capacity {cap} outside [1, {MAX_ENTRIES}] (entries are indexed with int32)")
    return cap


class BinResult(dict):
    """Outputs of the binning kernels (all device tensors).

    sorted_gids / sorted_tiles: [capacity] int32, the first n entries valid;
    ranges: [T+1] int32 (searchsorted-left boundaries); stats: [16] int32;
    n_interactions: 0-d int32 view of stats; window: the default path's chunk window
    (gs_window_t bytes) when asked for, else None; deferred: the entry list is left to
    the compositing forward (composite(..., bins=this)), which reads the superblock lists
    in workspace."""


def new_window(dev) -> torch.Tensor:
    """Device storage for one gs_window_t (8-byte aligned: torch allocations are)."""
    return torch.empty((_lib.GS_WINDOW_BYTES,), dtype=torch.uint8, device=dev)


def window_from_list(sorted_gids: torch.Tensor) -> torch.Tensor:
    """The clamped chunk window of a list in the reference's layout (rasterizer.py:187):
    thr = len - 512 and its last 512 ids."""
    g = sorted_gids.to(torch.int32).contiguous()
    win = new_window(g.device)
    _lib.call("gs_window_from_list", _lib.stream_handle(g.device), _lib.ptr(g), g.shape[0], _lib.ptr(win))
    return win


def bin_gaussians(means2d: torch.Tensor, radii: torch.Tensor, valid: torch.Tensor, depths: torch.Tensor, H: int,
                  W: int, capacity: int | None = None, want_tiles: bool = True, window: bool = False,
                  deferred: bool = False) -> BinResult:
    """gs_bin: the entries in the reference's (tile, depth quantum, id) order, compact.
    window=True also builds the default path's chunk window of that list (the reference's
    rasterizer.py:184-190 clamp; the binning's last launch writes it, as gs_window_from_bins
    would).  deferred=True (gs_bin_deferred, no
    sorted_tiles) leaves the entry list to composite(..., bins=result), which writes the
    entries its walk meets: the part gs_composite_bwd reads."""
    if deferred and want_tiles:
        raise ValueError("bin_gaussians: deferred binning writes no sorted_tiles (want_tiles=False)")
    dev = means2d.device
    n = means2d.shape[0]
    means2d = check_f32("means2D", means2d, (n, 2), dev)
    radii = check_f32("radii", radii.to(torch.float32), (n,), dev)
    depths = check_f32("depths", depths, (n,), dev)
    v = valid.to(device=dev, dtype=torch.uint8).contiguous()
    cap = check_capacity(capacity, n)
    ws_bytes = (_lib.lib().gs_bin_deferred_workspace_size if deferred else _lib.lib().gs_bin_workspace_size)(
        n, int(W), int(H), cap)
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
    _, _, T = num_tiles(W, H)
    gids = torch.empty((cap,), dtype=torch.int32, device=dev)
    tiles = torch.empty((cap,), dtype=torch.int32, device=dev) if want_tiles else None
    ranges = torch.empty((T + 1,), dtype=torch.int32, device=dev)
    stats = torch.empty((_lib.GS_NUM_STATS,), dtype=torch.int32, device=dev)
    win = new_window(dev) if window else None  # built by the binning's last launch
    if deferred:
        _lib.call("gs_bin_deferred", _lib.stream_handle(dev), n, _lib.ptr(means2d), _lib.ptr(radii), _lib.ptr(v),
                  _lib.ptr(depths), int(W), int(H), cap, _lib.ptr(ws), ws_bytes, _lib.ptr(gids), _lib.ptr(ranges),
                  _lib.ptr(stats), _lib.ptr(win))
    else:
        _lib.call("gs_bin", _lib.stream_handle(dev), n, _lib.ptr(means2d), _lib.ptr(radii), _lib.ptr(v),
                  _lib.ptr(depths), int(W), int(H), cap, _lib.ptr(ws), ws_bytes, _lib.ptr(gids), _lib.ptr(tiles),
                  _lib.ptr(ranges), _lib.ptr(stats), _lib.ptr(win))
    return BinResult(sorted_gids=gids, sorted_tiles=tiles, ranges=ranges, stats=stats,
                     n_interactions=stats[_lib.STAT["n_interactions"]], capacity=cap, num_tiles=T, window=win,
                     deferred=deferred, workspace=ws if deferred else None, n=n)


def get_tile_interactions(means2D, radii, valid_mask, depths, H, W, tile_size: int = TILE_SIZE):
    """rasterizer.py:12-116 -> (sorted_tile_ids [L], sorted_gaussian_ids [L], n_interactions),
    L = max(256 N, 512): the reference's own arrays, slot for slot -- the 256 slots of each
    Gaussian whose depth has its sign bit set (tile -1), the entries in (tile, depth
    quantum, id) order, the other Gaussians' empty slots (tile T), padding (tile T, id 0)."""
    if tile_size != TILE_SIZE:
        raise ValueError("only 16x16 tiles are supported (rasterizer.py:6)")
    dev = means2D.device
    n = means2D.shape[0]
    if 256 * n >= 2 ** 31:
        raise ValueError(f"get_tile_interactions: 256 * {n} slots exceed int32 indexing")
    m2 = check_f32("means2D", means2D, (n, 2), dev)
    r = check_f32("radii", torch.as_tensor(radii, device=dev).to(torch.float32), (n,), dev)
    z = check_f32("depths", depths, (n,), dev)
    v = as_bytes(torch.as_tensor(valid_mask, device=dev))
    L = max(256 * n, BLOCK_SIZE)
    _, _, T = num_tiles(W, H)
    nb = _lib.lib().gs_bin_reference_workspace_size(n, int(W), int(H))
    ws = torch.empty((nb,), dtype=torch.uint8, device=dev)
    tiles = torch.empty((L,), dtype=torch.int32, device=dev)
    gids = torch.empty((L,), dtype=torch.int32, device=dev)
    ranges = torch.empty((T + 1,), dtype=torch.int32, device=dev)
    stats = torch.empty((_lib.GS_NUM_STATS,), dtype=torch.int32, device=dev)
    _lib.call("gs_bin_reference", _lib.stream_handle(dev), n, _lib.ptr(m2), _lib.ptr(r), _lib.ptr(v), _lib.ptr(z),
              int(W), int(H), _lib.ptr(ws), nb, _lib.ptr(tiles), _lib.ptr(gids), _lib.ptr(ranges), _lib.ptr(stats))
    return tiles, gids, stats[_lib.STAT["n_interactions"]]


def tile_ranges(sorted_tile_ids: torch.Tensor, num_tiles_total: int) -> torch.Tensor:
    """jnp.searchsorted(sorted_tile_ids, arange(T+1)) on the GPU (renderer.py:60)."""
    st = sorted_tile_ids.to(torch.int32).contiguous()
    out = torch.empty((num_tiles_total + 1,), dtype=torch.int32, device=st.device)
    _lib.call("gs_tile_ranges", _lib.stream_handle(st.device), _lib.ptr(st), st.shape[0], int(num_tiles_total),
              _lib.ptr(out))
    return out


def composite_records(means2D, cov2D, opacities, colors) -> torch.Tensor:
    """Per-Gaussian compositing records (det clamp, inverse covariance, sigmoid)."""
    dev = means2D.device
    n = means2D.shape[0]
    m = check_f32("means2D", means2D, (n, 2), dev)
    c = check_f32("cov2D", cov2D, (n, 2, 2), dev)
    o = check_f32("opacities", opacities, (n, 1), dev)
    col = check_f32("colors", colors, (n, 3), dev)
    rec = torch.empty((n, _lib.GS_REC_STRIDE), dtype=torch.float32, device=dev)
    _lib.call("gs_composite_prep", _lib.stream_handle(dev), n, _lib.ptr(m), _lib.ptr(c), _lib.ptr(o), _lib.ptr(col),
              _lib.ptr(rec))
    return rec


def composite(records: torch.Tensor, sorted_gids: torch.Tensor, ranges: torch.Tensor, H: int, W: int,
              background: torch.Tensor, residuals: bool = True, clear_records: torch.Tensor | None = None,
              window: torch.Tensor | None = None, bins: BinResult | None = None,
              l1_target: torch.Tensor | None = None):
    """Front-to-back compositing; returns (image [H,W,3], final_T [H,W], n_contrib [H,W],
    tile_order [T]), the last three the backward's residuals (None unless residuals):
    tile_order lists the tiles longest walk first, the backward's launch order.
    clear_records ([n, GS_REC_STRIDE] float32), when given, is set to zero by the same launch
    (for a backward that accumulates into it).  window None reads each tile's own entries
    (rasterizer_tpu.py:90-97); a window (window_from_list, bin_gaussians(window=True))
    reads the default path's clamped 512-entry chunk windows (rasterizer.py:184-190),
    which differ only for chunks that start within 512 slots of the end of the
    reference's arrays.  bins: the BinResult of a deferred binning whose sorted_gids and
    ranges these are (gs_composite_fwd_deferred); the results are the same as with the
    full list.  l1_target ([H,W,3], with a deferred binning's bins): the L1 loss
    mean |image - target| (losses.py:4-8) is computed by the same launches
    (gs_composite_fwd_deferred_l1) and returned as a fifth value, a 0-d tensor."""
    dev = records.device
    _, _, T = num_tiles(W, H)
    image = torch.empty((H, W, 3), dtype=torch.float32, device=dev)
    fT = torch.empty((H, W), dtype=torch.float32, device=dev) if residuals else None
    nc = torch.empty((H, W), dtype=torch.int32, device=dev) if residuals else None
    order = torch.empty((T,), dtype=torch.int32, device=dev) if residuals else None
    if bins is not None and bins["deferred"]:
        if sorted_gids is not bins["sorted_gids"] or ranges is not bins["ranges"] or records.shape[0] != bins["n"]:
            raise ValueError("composite: bins must be the deferred binning of these entries and records")
        ws = bins["workspace"]
        args = (_lib.stream_handle(dev), records.shape[0], _lib.ptr(records), _lib.ptr(sorted_gids), bins["capacity"],
                _lib.ptr(ranges), _lib.ptr(bins["stats"]), _lib.ptr(ws), ws.shape[0], int(W), int(H),
                _lib.ptr(background), _lib.ptr(image), _lib.ptr(fT), _lib.ptr(nc), _lib.ptr(order),
                _lib.ptr(clear_records), _lib.ptr(window))
        if l1_target is not None:
            tgt = check_f32("l1_target", l1_target, (H, W, 3), dev)
            l1_out = torch.empty((_lib.lib().gs_composite_l1_out_size(int(W), int(H)),), dtype=torch.float32,
                                 device=dev)
            _lib.call("gs_composite_fwd_deferred_l1", *args, _lib.ptr(tgt), _lib.ptr(l1_out))
            return image, fT, nc, order, l1_out[0]
        _lib.call("gs_composite_fwd_deferred", *args)
    elif l1_target is not None:
        raise ValueError("composite: the fused L1 loss needs a deferred binning's bins")
    else:
        _lib.call("gs_composite_fwd", _lib.stream_handle(dev), records.shape[0], _lib.ptr(records),
                  _lib.ptr(sorted_gids), sorted_gids.shape[0], _lib.ptr(ranges), int(W), int(H),
                  _lib.ptr(background), _lib.ptr(image), _lib.ptr(fT), _lib.ptr(nc), _lib.ptr(order),
                  _lib.ptr(clear_records), _lib.ptr(window))
    return image, fT, nc, order


class _RenderTiles(torch.autograd.Function):
    """render_tiles with its VJP (JAX autodiff of rasterizer.py:119-248): the image's
    cotangent reaches means2D, cov2D ([1,0] gets 0: render_tiles reads cov2D[0,1] only),
    the opacity logits, the colours and the background through gs_composite_bwd (the
    compositing replay, gradient records) and gs_composite_prep_bwd (the prologue)."""

    @staticmethod
    def forward(ctx, means2D, cov2D, opacities, colors, bg, gids, ranges, win, static):
        H, W = static
        rec = composite_records(means2D, cov2D, opacities, colors)
        image, fT, nc, order = composite(rec, gids, ranges, H, W, bg, residuals=True, window=win)
        ctx.static = static
        ctx.save_for_backward(cov2D, opacities, bg, rec, gids, ranges, win, fT, nc, order)
        return image

    @staticmethod
    def backward(ctx, g_image):
        H, W = ctx.static
        cov2D, opacities, bg, rec, gids, ranges, win, fT, nc, order = ctx.saved_tensors
        dev = rec.device
        n = rec.shape[0]
        s = _lib.stream_handle(dev)
        g_image = g_image.contiguous()
        grec = torch.empty((n, _lib.GS_REC_STRIDE), dtype=torch.float32, device=dev)
        gbg = torch.empty((3,), dtype=torch.float32, device=dev) if ctx.needs_input_grad[4] else None
        _lib.call("gs_composite_bwd", s, n, _lib.ptr(rec), _lib.ptr(gids), gids.shape[0], _lib.ptr(ranges), int(W),
                  int(H), _lib.ptr(bg), _lib.ptr(g_image), _lib.ptr(fT), _lib.ptr(nc), _lib.ptr(order),
                  _lib.ptr(grec), _lib.ptr(gbg), 0, _lib.ptr(win), None)
        gm = torch.empty((n, 2), dtype=torch.float32, device=dev)
        gc = torch.empty((n, 2, 2), dtype=torch.float32, device=dev)
        go = torch.empty((n, 1), dtype=torch.float32, device=dev)
        gcol = torch.empty((n, 3), dtype=torch.float32, device=dev)
        _lib.call("gs_composite_prep_bwd", s, n, _lib.ptr(cov2D), _lib.ptr(opacities), _lib.ptr(grec), _lib.ptr(gm),
                  _lib.ptr(gc), _lib.ptr(go), _lib.ptr(gcol))
        return gm, gc, go, gcol, gbg, None, None, None, None


def _render_tiles(means2D, cov2D, opacities, colors, sorted_tile_ids, sorted_gaussian_ids, H, W, background,
                  clamped_windows):
    """Both reference compositing paths on caller arrays in the reference's layout,
    differentiable in means2D, cov2D, opacities, colors and a tensor background."""
    dev = means2D.device
    n = means2D.shape[0]
    _, _, T = num_tiles(W, H)
    m = check_f32("means2D", means2D, (n, 2), dev)
    c = check_f32("cov2D", cov2D, (n, 2, 2), dev)
    o = check_f32("opacities", opacities, (n, 1), dev)
    col = check_f32("colors", colors, (n, 3), dev)
    ranges = tile_ranges(sorted_tile_ids, T)
    bg = background_tensor(background, dev)
    gids = sorted_gaussian_ids.to(torch.int32).contiguous()
    win = window_from_list(gids) if clamped_windows else None
    return _RenderTiles.apply(m, c, o, col, bg, gids, ranges, win, (int(H), int(W)))


def render_tiles(means2D, cov2D, opacities, colors, sorted_tile_ids, sorted_gaussian_ids, H, W,
                 tile_size: int = TILE_SIZE, background=None):
    """rasterizer.py:119-248.  Entries of tile t are the ones whose sorted tile id equals t
    (searchsorted ranges), capped at 4096 per tile, read through the reference's 512-entry
    chunk windows: a chunk that starts within 512 entries of the end of the arrays reads
    their last 512 entries (rasterizer.py:184-190).  Differentiable like the reference's:
    the image's cotangent reaches means2D, cov2D, opacities, colors and a tensor background."""
    if tile_size != TILE_SIZE:
        raise ValueError("only 16x16 tiles are supported (rasterizer.py:6)")
    return _render_tiles(means2D, cov2D, opacities, colors, sorted_tile_ids, sorted_gaussian_ids, H, W, background,
                         clamped_windows=True)


def render_tiles_tpu(*args, **kwargs):
    """rasterizer_tpu.py:13-135 (defined in rasterizer_tpu.py)."""
    from .rasterizer_tpu import render_tiles_tpu as impl

    return impl(*args, **kwargs)
