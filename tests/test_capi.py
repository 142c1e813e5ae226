"""The C ABI library loads on the CPU and exports every entry point include/gs_raster.h declares."""
import ctypes
import os
import re

from jax_gs_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "gs_raster.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?(?:int|size_t|char\s*\*|void)\s*\*?\s*(gs_\w+)\s*\(", src, re.M)))


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
    assert L.gs_abi_version() == _lib.ABI_VERSION == 7
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
    rc = L.gs_bin(None, 10, None, None, None, None, 64, 64, 0, None, 0, None, None, None, None)
    assert rc == 1
    assert b"workspace" in L.gs_last_error()


def test_load_ply_missing_file():
    """test_io.py:42-44: a missing path raises FileNotFoundError (before any GPU work)."""
    import pytest

    from jax_gs_amd.io.ply import load_ply

    with pytest.raises(FileNotFoundError):
        load_ply("non_existent_file.ply")
