"""The C ABI library loads on the CPU and exports every entry point include/gs_raster.h declares."""
import ctypes
import os
import re

import pytest
import torch

from jax_gs_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "gs_raster.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?(?:int64_t|int|size_t|char\s*\*|void)\s*\*?\s*(gs_\w+)\s*\(", src, re.M)))


def test_header_declares_entry_points():
    names = declared_functions()
    for must in ("gs_preprocess_fwd", "gs_bin", "gs_composite_fwd", "gs_composite_bwd", "gs_preprocess_bwd"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIBPATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_every_declared_symbol():
    assert set(declared_functions()) <= set(_lib._SIGS)


def test_abi_version_and_workspace_query_without_gpu():
    L = _lib.lib()
    assert L.gs_abi_version() == _lib.ABI_VERSION == 14
    # size query: pure host arithmetic, grows with the number of Gaussians
    a = L.gs_bin_workspace_size(1000, 64, 64, 0)
    b = L.gs_bin_workspace_size(100000, 64, 64, 0)
    assert 0 < a < b
    assert L.gs_bin_workspace_size(-1, 64, 64, 0) == 0


def test_argument_errors_are_reported_without_launching():
    L = _lib.lib()
    rc = L.gs_preprocess_fwd(None, 10, 4, 3, *([None] * 7), 64, 64, 1.0, 1.0, 0.0, 0.0, *([None] * 7))
    assert rc == 1
    assert b"sh_coeffs has 4 coefficients" in L.gs_last_error()
    rc = L.gs_bin(None, 10, None, None, None, None, 64, 64, 0, None, 0, None, None, None, None, None)
    assert rc == 1
    assert b"workspace" in L.gs_last_error()


def test_argument_errors_of_the_window_sh_ssim_and_camera_entry_points():
    """The entry points added for the default path's chunk windows, eval_sh, SSIM window
    sizes and the camera cotangent reject bad arguments before launching anything."""
    L = _lib.lib()
    assert L.gs_window_from_list(None, None, 600, None) == 1
    assert b"gs_window_from_list" in L.gs_last_error()
    assert L.gs_window_from_bins(None, -1, None, None, None, None, 64, 64, None, 0, None, None) == 1
    assert b"gs_window_from_bins" in L.gs_last_error()
    assert L.gs_eval_sh(None, 10, 4, 3, None, None, None) == 1
    assert b"needs 16" in L.gs_last_error()
    assert L.gs_eval_sh_bwd(None, 10, 16, 4, None, None, None, None, None) == 1
    assert b"sh_degree" in L.gs_last_error()
    assert L.gs_l1_ssim_window_workspace_size(8, 8, 3, 0) == 0
    assert L.gs_l1_ssim_window_workspace_size(8, 8, 3, 64) == 0
    assert L.gs_l1_ssim_window_workspace_size(8, 8, 5, 63) > 0
    assert L.gs_l1_ssim_window(None, 8, 8, 3, 64, None, None, None, 1, None, 0) == 1
    assert b"window_size" in L.gs_last_error()
    nb = L.gs_preprocess_bwd_w2c_workspace_size(1000)
    assert nb == 16 * 16 * 4
    rc = L.gs_preprocess_bwd_w2c(None, 1000, 16, 3, *([None] * 6), 64, 64, 1.0, 1.0, 0.0, 0.0, *([None] * 7), None, 0,
                                 0)
    assert rc == 1 and b"gs_preprocess_bwd_w2c" in L.gs_last_error()
    # the module VJPs: a camera cotangent needs its workspace; NULL arrays are rejected
    rc = L.gs_project_bwd(None, 1000, None, None, None, ctypes.c_void_p(8), 1.0, 1.0, *([None] * 6),
                          ctypes.c_void_p(8), None, 0)
    assert rc == 1 and b"workspace" in L.gs_last_error()
    assert L.gs_project_bwd(None, 1000, *([None] * 3), ctypes.c_void_p(8), 1.0, 1.0, *([None] * 7), None, 0) == 1
    assert b"gs_project_bwd" in L.gs_last_error()
    assert L.gs_composite_prep_bwd(None, 10, *([None] * 7)) == 1
    assert b"gs_composite_prep_bwd" in L.gs_last_error()
    assert L.gs_composite_prep_bwd(None, 0, *([None] * 7)) == 0


def test_argument_errors_of_the_deferred_binning():
    """gs_bin_deferred and gs_composite_fwd_deferred check their sizes, the capacity and the
    binning workspace (the superblock lists are found in it) before launching anything."""
    L = _lib.lib()
    fake = ctypes.c_void_p(256)
    assert L.gs_bin_deferred(None, 10, *([None] * 4), 64, 64, 1000, None, 0, None, None, None, None) == 1
    assert b"workspace" in L.gs_last_error()
    args = (fake, 1000, fake, fake)  # sorted_gids, capacity, ranges, stats
    rc = L.gs_composite_fwd_deferred(None, 10, fake, fake, 0, fake, fake, fake, 1 << 20, 64, 64, *([fake] * 2),
                                     *([None] * 5))
    assert rc == 1 and b"capacity" in L.gs_last_error()
    need = L.gs_bin_deferred_workspace_size(10, 64, 64, 1000)
    assert need > L.gs_bin_workspace_size(10, 64, 64, 1000)
    rc = L.gs_composite_fwd_deferred(None, 10, fake, *args[:3], args[3], fake, need - 1, 64, 64, *([fake] * 2),
                                     *([None] * 5))
    assert rc == 1 and b"smaller than the binning" in L.gs_last_error()
    rc = L.gs_composite_fwd_deferred(None, 10, fake, *args[:3], None, fake, need, 64, 64, *([fake] * 2),
                                     *([None] * 5))
    assert rc == 1 and b"NULL" in L.gs_last_error()
    rc = L.gs_composite_fwd_deferred(None, 10, fake, *args, fake, need, 0, 64, *([fake] * 2), *([None] * 5))
    assert rc == 1 and b"bad sizes" in L.gs_last_error()


def test_argument_errors_of_the_fused_l1_loss():
    """gs_composite_fwd_deferred_l1 / gs_composite_bwd_l1 need their target, loss and
    cotangent arrays; the loss array holds the loss and one partial per compositing
    workgroup (at most four per tile)."""
    L = _lib.lib()
    fake = ctypes.c_void_p(256)
    assert L.gs_composite_l1_out_size(0, 64) == 0
    T = ((1920 + 15) // 16) * ((1080 + 15) // 16)
    assert L.gs_composite_l1_out_size(1920, 1080) >= 1 + T
    rc = L.gs_composite_fwd_deferred_l1(None, 10, fake, fake, 1000, fake, fake, fake, 1 << 20, 64, 64,
                                        *([fake] * 2), *([None] * 5), None, fake)
    assert rc == 1 and b"l1_target" in L.gs_last_error()
    rc = L.gs_composite_bwd_l1(None, 10, fake, fake, 100, fake, 64, 64, fake, None, None, fake, fake, fake, fake,
                               fake, fake, None, 1, None, None)
    assert rc == 1 and b"gs_composite_bwd_l1" in L.gs_last_error()
    # the unfused backward still needs its image cotangent
    rc = L.gs_composite_bwd(None, 10, fake, fake, 100, fake, 64, 64, fake, None, fake, fake, fake, fake, None, 1,
                            None, None)
    assert rc == 1 and b"image cotangent" in L.gs_last_error()


def test_clear_list_and_zeroed_arguments():
    """gs_composite_bwd rejects a clear list with a negative count or a NULL array with a
    count, before launching anything; clear_list() builds the gs_clear_list_t layout."""
    L = _lib.lib()
    fake = ctypes.c_void_p(256)
    assert ctypes.sizeof(_lib.ClearList) == _lib.GS_CLEAR_MAX * 16
    for k, count, ptr, msg in ((3, -1, None, b"negative count"), (7, 10, None, b"is NULL")):
        cl = _lib.ClearList()
        cl.count[k] = count
        cl.ptr[k] = ptr
        rc = L.gs_composite_bwd(None, 10, fake, fake, 100, fake, 64, 64, fake, fake, fake, fake, fake, fake, None, 1,
                                None, ctypes.byref(cl))
        assert rc == 1 and msg in L.gs_last_error() and f"entry {k}".encode() in L.gs_last_error()
    with pytest.raises(ValueError):
        _lib.clear_list(*([torch.zeros(4)] * (_lib.GS_CLEAR_MAX + 1)))
    with pytest.raises(ValueError):
        _lib.clear_list(torch.zeros(4, dtype=torch.float64))
    cl = _lib.clear_list(torch.zeros(7), torch.zeros(3, 5))
    assert list(cl.count) == [7, 15] + [0] * (_lib.GS_CLEAR_MAX - 2)


def test_load_ply_missing_file():
    """test_io.py:42-44: a missing path raises FileNotFoundError (before any GPU work)."""
    import pytest

    from jax_gs_amd.io.ply import load_ply

    with pytest.raises(FileNotFoundError):
        load_ply("non_existent_file.ply")


def test_init_from_pcd_conventions_and_black_cloud_recolour():
    """gaussians.py:13-56 on the CPU (host logic): log-scale -3, identity rotation, logit 0,
    SH DC (c - 0.5) / C0 and zeros elsewhere; a cloud whose colours are all below 1e-3 gets
    uniform colours in [0.1, 0.9) (gaussians.py:40-42), the same draw on every call, and a
    coloured cloud keeps its colours."""
    import torch

    from jax_gs_amd import init_gaussians_from_pcd

    pts = torch.arange(30, dtype=torch.float32).reshape(10, 3)
    col = torch.linspace(0.0, 1.0, 30).reshape(10, 3)
    g = init_gaussians_from_pcd(pts, col)
    assert torch.equal(g.means, pts) and torch.all(g.scales == -3.0) and torch.all(g.opacities == 0.0)
    assert torch.all(g.quaternions[:, 0] == 1.0) and torch.all(g.quaternions[:, 1:] == 0.0)
    assert torch.allclose(g.sh_coeffs[:, 0, :], (col - 0.5) / 0.28209479177387814)
    assert g.sh_coeffs.shape == (10, 16, 3) and torch.all(g.sh_coeffs[:, 1:] == 0.0)
    black = torch.full((1000, 3), 5e-4)
    g1 = init_gaussians_from_pcd(torch.zeros(1000, 3), black)
    g2 = init_gaussians_from_pcd(torch.zeros(1000, 3), black)
    c = g1.sh_coeffs[:, 0, :] * 0.28209479177387814 + 0.5
    assert float(c.min()) >= 0.1 - 1e-6 and float(c.max()) < 0.9 + 1e-6
    assert 0.45 < float(c.mean()) < 0.55 and float(c.std()) > 0.2
    assert torch.equal(g1.sh_coeffs, g2.sh_coeffs)
