"""gs_bin_static, the binning entry point that allocates nothing (its workspace is the
library's static device array), against gs_bin with a caller workspace: outputs
bit-identical on two calls in a row on the same array, the second with a smaller
scene, and sizes past the array rejected before any launch."""
import numpy as np
import pytest
import torch

from gpu_helpers import log
from jax_gs_amd import _lib, scenes
from jax_gs_amd.renderer._buffers import num_tiles
from jax_gs_amd.renderer.projection import preprocess

pytestmark = pytest.mark.gpu


def _inputs(cfg, n, w, h, cuda):
    sc = scenes.make_scene(cfg, n=n, width=w, height=h)
    g, cam, _, m = scenes.to_torch(sc, cuda)
    with torch.no_grad():
        pre = preprocess(g, cam, mask=m, sh_degree=sc["sh_degree"], projected=False)
    return pre, cam.W, cam.H


def _outputs(cap, T, cuda):
    # the same fill on both sides, so entries neither call writes compare equal too
    return [torch.full((cap,), -7, dtype=torch.int32, device=cuda), torch.full((cap,), -7, dtype=torch.int32, device=cuda),
            torch.full((T + 1,), -7, dtype=torch.int32, device=cuda),
            torch.full((_lib.GS_NUM_STATS,), -7, dtype=torch.int32, device=cuda)]


def _bin(pre, W, H, cuda, static):
    n = pre["means2d"].shape[0]
    cap = 256 * n
    _, _, T = num_tiles(W, H)
    out = _outputs(cap, T, cuda)
    s = _lib.stream_handle(cuda)
    args = [n, _lib.ptr(pre["means2d"]), _lib.ptr(pre["radii"]), _lib.ptr(pre["valid"]), _lib.ptr(pre["depths"]), W, H,
            cap]
    if static:
        _lib.call("gs_bin_static", s, *args, *[_lib.ptr(o) for o in out])
    else:
        nb = _lib.lib().gs_bin_workspace_size(n, W, H, cap)
        ws = torch.empty((nb,), dtype=torch.uint8, device=cuda)
        _lib.call("gs_bin", s, *args, _lib.ptr(ws), nb, *[_lib.ptr(o) for o in out], None)
    torch.cuda.synchronize()
    return [o.cpu().numpy() for o in out]


def test_bin_static_matches_bin_two_calls(cuda):
    # the headline scene (1M Gaussians, 1080p: 117 MiB of the 128 MiB array), then a
    # smaller one on the array the first call left behind
    for cfg, n, w, h in ((2, None, 1920, 1080), (1, 20000, 504, 378)):
        pre, W, H = _inputs(cfg, n, w, h, cuda)
        want = _bin(pre, W, H, cuda, static=False)
        got = _bin(pre, W, H, cuda, static=True)
        n_int = int(want[3][_lib.STAT["n_interactions"]])
        log(f"cfg{cfg} n={pre['means2d'].shape[0]}: {n_int} entries")
        assert n_int > 0
        for a, b, name in zip(got, want, ("sorted_gids", "sorted_tiles", "ranges", "stats")):
            np.testing.assert_array_equal(a, b, err_msg=name)


def test_bin_static_rejects_sizes_past_its_array(cuda):
    # valid = 0 everywhere and a capacity equal to the outputs' length: even a call that
    # went through would stay inside the buffers
    n, W, H, cap = 1500000, 1920, 1080, 16
    assert _lib.lib().gs_bin_workspace_size(n, W, H, cap) > (128 << 20)
    z = torch.zeros((n, 2), device=cuda)
    one = torch.zeros((n,), device=cuda)
    v = torch.zeros((n,), dtype=torch.uint8, device=cuda)
    _, _, T = num_tiles(W, H)
    out = _outputs(cap, T, cuda)
    with pytest.raises(ValueError, match="static scratch"):
        _lib.call("gs_bin_static", _lib.stream_handle(cuda), n, _lib.ptr(z), _lib.ptr(one), _lib.ptr(v), _lib.ptr(one),
                  W, H, cap, *[_lib.ptr(o) for o in out])
    assert int(out[2][0]) == -7  # nothing launched
