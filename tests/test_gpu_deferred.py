"""The deferred binning (gs_bin_deferred + gs_composite_fwd_deferred) against the full one.

The deferred binning leaves the entry list unwritten; the compositing forward walks each
tile's 8x8-tile superblock list (words whose tile rectangle holds the tile are the tile's
entries, in the list's order) and writes the entries it meets.  Against gs_bin +
gs_composite_fwd on the same inputs:
  * ranges and stats bit-identical; image, final T and n_contrib bit-identical (the
    same entries blended in the same order);
  * every entry below the tile's largest n_contrib -- all that gs_composite_bwd reads --
    written and equal to the full list's;
  * gs_composite_bwd on the deferred list equals it on the full list (up to the order of
    its float atomics: relative L2 1e-6 for the records, 1e-4 for the background, a sum
    over every pixel);
  * where the entry list must exist in full -- the default path's clamped chunk window, or
    more entries than the capacity -- the binning writes it all and the forward reads it.
Cases: the compositing builds by tile count (four, two and one waves per tile), BASELINE
configurations 2, 3 and 4 at full size (3: tiles beyond 4096 entries, the walk's cap),
both rasterizer paths (window / own entries), Gaussians behind the camera, masked ones.
"""
import numpy as np
import pytest
import torch

from gpu_helpers import log, np_, rel
from jax_gs_amd import _lib, scenes
from jax_gs_amd.renderer import rasterizer
from jax_gs_amd.renderer.projection import preprocess

pytestmark = pytest.mark.gpu
F32 = np.float32


def _tile_max(nc, W, H):
    TX, TY = (W + 15) // 16, (H + 15) // 16
    pad = np.zeros((TY * 16, TX * 16), np.int64)
    pad[:H, :W] = nc
    return pad.reshape(TY, 16, TX, 16).max(axis=(1, 3)).reshape(-1)


def _prefix_positions(ranges, kmax):
    """Positions ranges[t] + k, k < kmax[t], of every tile."""
    kmax = np.asarray(kmax, np.int64)
    total = int(kmax.sum())
    starts = np.repeat(np.asarray(ranges[:-1], np.int64), kmax)
    first = np.repeat(np.cumsum(kmax) - kmax, kmax)
    return starts + (np.arange(total, dtype=np.int64) - first)


def _compare(sc, cuda, window, capacity=None, expect_deferred=True):
    c = sc["cam"]
    W, H = c["W"], c["H"]
    # images under 2048 tiles (four waves per tile) get the whole list from the binning
    expect_deferred = expect_deferred and ((W + 15) // 16) * ((H + 15) // 16) >= 2048
    g, cam, _, m = scenes.to_torch(sc, cuda)
    n = g.means.shape[0]
    bg = torch.tensor([0.1, 0.3, 0.2], device=cuda)
    with torch.no_grad():
        pre = preprocess(g, cam, mask=m, sh_degree=sc["sh_degree"], projected=False)
        args = (pre["means2d"], pre["radii"], pre["valid"], pre["depths"], H, W)
        full = rasterizer.bin_gaussians(*args, capacity=capacity, want_tiles=False, window=window)
        out_f = rasterizer.composite(pre["records"], full["sorted_gids"], full["ranges"], H, W, bg,
                                     window=full["window"])
        defer = rasterizer.bin_gaussians(*args, capacity=capacity, want_tiles=False, window=window, deferred=True)
        stats = np_(defer["stats"])
        m_ent = int(stats[_lib.STAT["tile_entries"]])
        deferred = bool(stats[_lib.STAT["entries_deferred"]])
        # the binning's decision, as documented: >= 2048 tiles, within the capacity, not clamped
        assert deferred == (stats[_lib.STAT["window_clamped"]] == 0 and 0 <= m_ent <= defer["capacity"] and
                            defer["num_tiles"] >= 2048)
        assert deferred == expect_deferred
        if deferred:
            # the binning wrote no entry: every entry the forward and backward read must be
            # written by the forward (an id no entry has marks the rest)
            defer["sorted_gids"].fill_(-7)
        out_d = rasterizer.composite(pre["records"], defer["sorted_gids"], defer["ranges"], H, W, bg,
                                     window=defer["window"], bins=defer)
    sf = np_(full["stats"])
    assert sf[_lib.STAT["entries_deferred"]] == 0  # gs_bin writes the list whole
    sf[_lib.STAT["entries_deferred"]] = stats[_lib.STAT["entries_deferred"]]
    np.testing.assert_array_equal(stats, sf)
    np.testing.assert_array_equal(np_(defer["ranges"]), np_(full["ranges"]))
    if window:  # the window's ids are written only when a chunk reads them (clamped)
        k = None if stats[_lib.STAT["window_clamped"]] else 16
        np.testing.assert_array_equal(np_(defer["window"])[:k], np_(full["window"])[:k])
    for name, a, b in zip(("image", "final_T", "n_contrib"), out_d, out_f):
        np.testing.assert_array_equal(np_(a), np_(b), err_msg=name)
    # the tile order (the backward's launch order) ranks the tiles by walk length, which
    # depends on where the wave's exit test falls (once per 8 walked entries, restarted
    # per batch); it is a permutation of the tiles either way
    np.testing.assert_array_equal(np.sort(np_(out_d[3])), np.arange(out_d[3].shape[0]))
    ranges = np_(full["ranges"]).astype(np.int64)
    gids_f, gids_d = np_(full["sorted_gids"]), np_(defer["sorted_gids"])
    cnt = np.minimum(np.diff(ranges), 4096)
    kmax = np.minimum(_tile_max(np_(out_f[2]), W, H), cnt)
    pos = _prefix_positions(ranges, kmax)
    pos = pos[pos < gids_f.shape[0]]  # entries beyond the capacity are dropped (tile lists clamped)
    np.testing.assert_array_equal(gids_d[pos], gids_f[pos])
    written = int(kmax.sum())
    if deferred:
        assert np.all(gids_d[m_ent:] == -7)  # nothing written past the entries
    else:
        # written in full by the binning
        k = min(m_ent, full["capacity"])
        np.testing.assert_array_equal(gids_d[:k], gids_f[:k])
    log(f"{sc.get('name', 'scene')}: N={n} {W}x{H} window={window} deferred={deferred}: "
        f"{m_ent} entries, {written} below the tiles' n_contrib ({written / max(m_ent, 1):.3f})")
    # the backward on the deferred list
    seed = torch.from_numpy(np.random.default_rng(5).normal(0, 1, (H, W, 3)).astype(F32)).to(cuda)
    grads = []
    for b in (full, defer):
        grec = torch.empty((n, _lib.GS_REC_STRIDE), dtype=torch.float32, device=cuda)
        gbg = torch.empty((3,), dtype=torch.float32, device=cuda)
        _lib.call("gs_composite_bwd", _lib.stream_handle(cuda), n, _lib.ptr(pre["records"]),
                  _lib.ptr(b["sorted_gids"]), b["sorted_gids"].shape[0], _lib.ptr(b["ranges"]), W, H, _lib.ptr(bg),
                  _lib.ptr(seed), _lib.ptr(out_f[1]), _lib.ptr(out_f[2]), _lib.ptr(out_f[3]), _lib.ptr(grec),
                  _lib.ptr(gbg), 0, _lib.ptr(b["window"]), None)
        grads.append((np_(grec), np_(gbg)))
    e, e_bg = rel(grads[1][0], grads[0][0]), rel(grads[1][1], grads[0][1])
    log(f"backward on the deferred list vs the full one: records {e:.1e}, background {e_bg:.1e}")
    # the same terms added in another order (float atomics); the background sums every pixel,
    # with cancellation (1.0e-5 seen on the 304-Gaussian window scene)
    assert e <= 1e-6 and e_bg <= 1e-4, (e, e_bg)
    return written, m_ent


@pytest.mark.parametrize("window", [True, False])
@pytest.mark.parametrize("cfg,n,w,h", [(1, 20000, 256, 192), (2, 60000, 1024, 768), (2, 100000, 1920, 832)])
def test_deferred_equals_full_per_build(cuda, window, cfg, n, w, h):
    """Four (T < 2048: the binning writes the whole list), two (2048 <= T < 6144) and one
    (T >= 6144) forward waves per tile."""
    sc = scenes.make_scene(cfg, n=n, width=w, height=h)
    sc["name"] = f"cfg{cfg}-family"
    _compare(sc, cuda, window)


@pytest.mark.parametrize("cfg", [2, 3, 4])
def test_deferred_equals_full_at_full_size(cuda, cfg):
    """BASELINE configurations 2-4 as configured; configuration 3's tiles hold more than
    4096 entries (the walk stops at the reference's cap)."""
    sc = scenes.make_scene(cfg)
    sc["name"] = f"cfg{cfg}"
    written, m_ent = _compare(sc, cuda, window=True)
    assert written < m_ent  # tiles turn opaque: the walk meets a prefix only


def test_deferred_with_gaussians_behind_the_camera_and_masked(cuda):
    sc = scenes.make_scene(1, n=60000, width=1024, height=768, seed=9)
    p = sc["params"]
    p["means"][:50, 2] = -np.abs(p["means"][:50, 2])
    mask = np.ones(p["means"].shape[0], bool)
    mask[100:400] = False
    sc["mask"] = mask
    sc["name"] = "behind+masked"
    _compare(sc, cuda, window=True)


def test_deferred_falls_back_beyond_the_capacity(cuda):
    """A capacity below the entry count: the binning writes the first entries in full and
    the forward reads them (both binnings keep the same entries)."""
    sc = scenes.make_scene(1, n=40000, width=1024, height=768)
    g, cam, _, m = scenes.to_torch(sc, cuda)
    with torch.no_grad():
        pre = preprocess(g, cam, mask=m, sh_degree=sc["sh_degree"], projected=False)
        b = rasterizer.bin_gaussians(pre["means2d"], pre["radii"], pre["valid"], pre["depths"], 768, 1024,
                                     want_tiles=False)
    m_ent = int(np_(b["stats"])[_lib.STAT["tile_entries"]])
    sc["name"] = "capacity"
    _compare(sc, cuda, window=True, capacity=m_ent // 2, expect_deferred=False)


def test_deferred_falls_back_for_clamped_windows(cuda):
    """The default path's clamped chunk window reads the entry list: written in full.  Small
    images (the window tests' scenes) and 300 Gaussians spanning 16 x 16 tiles of a 1024 x 768
    image (3072 tiles: no empty slot, so the last tiles' chunks are clamped)."""
    from test_gpu_windows import CASES, _scene

    rng = np.random.default_rng(5)
    m = np.zeros((300, 3), F32)
    m[:, :2] = rng.uniform(-0.05, 0.05, (300, 2))
    m[:, 2] = rng.uniform(4.8, 5.2, 300)
    wide = _scene(m, np.zeros(300), rng.uniform(-4.5, -3.5, 300), rng.uniform(0.0, 1.0, (300, 3)), 1024, 768,
                  400.0)
    for name, sc in (("two", CASES["two"]()), ("big", CASES["big"]()), ("wide", wide)):
        sc["name"] = f"window-{name}"
        _compare(sc, cuda, window=True, expect_deferred=False)
