"""ctypes binding of libgsraster.so, the gfx950 HIP kernels behind include/gs_raster.h.

The library is built in-tree by ``jax_gs_amd._build.build_library()`` (called from
``__graft_entry__.build()``).  Loading fails loudly when it is missing: the renderer
has no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIBPATH = os.path.join(_HERE, "libgsraster.so")

GS_OK = 0
GS_REC_STRIDE = 12
GS_NUM_STATS = 16
GS_WINDOW_BYTES = 16 + 4 * 512  # sizeof(gs_window_t): int64 thr, 2 reserved int32, 512 ids
GS_CLEAR_MAX = 8


class ClearList(ctypes.Structure):
    """gs_clear_list_t: float arrays a compositing backward launch sets to zero."""
    _fields_ = [("ptr", ctypes.c_void_p * GS_CLEAR_MAX), ("count", ctypes.c_int64 * GS_CLEAR_MAX)]


def clear_list(*tensors) -> ClearList:
    """A gs_clear_list_t of contiguous float32 device tensors (kept alive by the caller)."""
    if len(tensors) > GS_CLEAR_MAX:
        raise ValueError(f"clear_list: at most {GS_CLEAR_MAX} arrays")
    cl = ClearList()
    for i, t in enumerate(tensors):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError("clear_list: contiguous float32 tensors only")
        cl.ptr[i] = t.data_ptr()
        cl.count[i] = t.numel()
    return cl
STAT = dict(n_interactions=0, max_interactions_per_tile=1, overflow_tiles=2, overflow_interactions=3,
            truncated_tiles=4, truncated_interactions=5, radius_cap_violations=6, negative_depth=7,
            capacity_exceeded=8, mean_per_tile=9, tile_entries=10, window_clamped=11, entries_deferred=12)

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t

# name -> argtypes (all entry points return int status unless listed in _RESTYPE)
_SIGS = {
    "gs_last_error": [],
    "gs_abi_version": [],
    "gs_preprocess_fwd": [_P, _I64, _I, _I, _P, _P, _P, _P, _P, _P, _P, _I, _I, _F, _F, _F, _F, _P, _P, _P, _P, _P,
                          _P, _P],
    "gs_composite_prep": [_P, _I64, _P, _P, _P, _P, _P],
    "gs_bin_workspace_size": [_I64, _I, _I, _I64],
    "gs_bin_deferred_workspace_size": [_I64, _I, _I, _I64],
    "gs_bin": [_P, _I64, _P, _P, _P, _P, _I, _I, _I64, _P, _SZ, _P, _P, _P, _P, _P],
    "gs_bin_deferred": [_P, _I64, _P, _P, _P, _P, _I, _I, _I64, _P, _SZ, _P, _P, _P, _P],
    "gs_bin_static": [_P, _I64, _P, _P, _P, _P, _I, _I, _I64, _P, _P, _P, _P],
    "gs_bin_reference_workspace_size": [_I64, _I, _I],
    "gs_bin_reference": [_P, _I64, _P, _P, _P, _P, _I, _I, _P, _SZ, _P, _P, _P, _P],
    "gs_tile_ranges": [_P, _P, _I64, _I, _P],
    "gs_window_from_list": [_P, _P, _I64, _P],
    "gs_window_from_bins": [_P, _I64, _P, _P, _P, _P, _I, _I, _P, _I64, _P, _P],
    "gs_composite_fwd": [_P, _I64, _P, _P, _I64, _P, _I, _I, _P, _P, _P, _P, _P, _P, _P],
    "gs_composite_fwd_deferred": [_P, _I64, _P, _P, _I64, _P, _P, _P, _SZ, _I, _I, _P, _P, _P, _P, _P, _P, _P],
    "gs_composite_bwd": [_P, _I64, _P, _P, _I64, _P, _I, _I, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P],
    "gs_composite_l1_out_size": [_I, _I],
    "gs_composite_fwd_deferred_l1": [_P, _I64, _P, _P, _I64, _P, _P, _P, _SZ, _I, _I, _P, _P, _P, _P, _P, _P, _P,
                                     _P, _P],
    "gs_composite_bwd_l1": [_P, _I64, _P, _P, _I64, _P, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _P,
                            _P],
    "gs_preprocess_bwd": [_P, _I64, _I, _I, _P, _P, _P, _P, _P, _P, _I, _I, _F, _F, _F, _F, _P, _P, _P, _P, _P, _P,
                          _I],
    "gs_preprocess_bwd_w2c_workspace_size": [_I64],
    "gs_preprocess_bwd_w2c": [_P, _I64, _I, _I, _P, _P, _P, _P, _P, _P, _I, _I, _F, _F, _F, _F, _P, _P, _P, _P, _P,
                              _P, _P, _P, _SZ, _I],
    "gs_composite_prep_bwd": [_P, _I64, _P, _P, _P, _P, _P, _P, _P],
    "gs_project_bwd": [_P, _I64, _P, _P, _P, _P, _F, _F, _P, _P, _P, _P, _P, _P, _P, _P, _SZ],
    "gs_eval_sh": [_P, _I64, _I, _I, _P, _P, _P],
    "gs_eval_sh_bwd": [_P, _I64, _I, _I, _P, _P, _P, _P, _P],
    "gs_l1_loss": [_P, _I64, _P, _P, _P, _P],
    "gs_mse_loss": [_P, _I64, _P, _P, _P, _P],
    "gs_l1_loss_bwd": [_P, _I64, _P, _P, _P, _P],
    "gs_mse_loss_bwd": [_P, _I64, _P, _P, _P, _P],
    "gs_l1_ssim_workspace_size": [_I, _I, _I],
    "gs_l1_ssim": [_P, _I, _I, _I, _P, _P, _P, _I, _P, _SZ],
    "gs_l1_ssim_bwd": [_P, _I, _I, _I, _P, _P, _P, _P, _SZ, _P],
    "gs_l1_ssim_window_workspace_size": [_I, _I, _I, _I],
    "gs_l1_ssim_window": [_P, _I, _I, _I, _I, _P, _P, _P, _I, _P, _SZ],
    "gs_l1_ssim_window_bwd": [_P, _I, _I, _I, _I, _P, _P, _P, _P, _SZ, _P],
    "gs_densify_workspace_size": [_I64],
    "gs_densify_and_prune": [_P, _I64, _I, _P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _I, ctypes.c_double,
                             ctypes.c_double, ctypes.c_double, ctypes.c_double, _P, _SZ, _P],
    "gs_reset_opacities": [_P, _I64, _P, ctypes.c_double, _P],
    "gs_ply_pack": [_P, _I64, _I, _P, _P, _P, _P, _P, _P],
    "gs_ply_unpack": [_P, _I64, _I, _P, _P, _P, _P, _P, _P],
    "gs_preprocess_bwd_adam": [_P, _I64, _I, _I, _P, _P, _P, _P, _P, _P, _I, _I, _F, _F, _F, _F, _P, _P, _P, _I,
                               ctypes.c_double, ctypes.c_double, ctypes.c_double, _P, _P, _P, _F, _F, _P, _P, _P],
    "gs_l1_ssim_terms": [_P, _P, ctypes.c_double, _P],
    "gs_adam_step": [_P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I, ctypes.c_double, ctypes.c_double,
                     ctypes.c_double],
    "gs_densify_accumulate": [_P, _I64, _P, _P, _P, _F, _F, _P, _P, _P, _P, _P, _P],
}
_RESTYPE = {"gs_last_error": ctypes.c_char_p, "gs_bin_workspace_size": _SZ, "gs_l1_ssim_workspace_size": _SZ,
            "gs_bin_deferred_workspace_size": _SZ,
            "gs_bin_reference_workspace_size": _SZ, "gs_preprocess_bwd_w2c_workspace_size": _SZ,
            "gs_l1_ssim_window_workspace_size": _SZ,
            "gs_densify_workspace_size": _SZ, "gs_composite_l1_out_size": _I64}

_lib = None


ABI_VERSION = 14  # gs_abi_version() of the signatures bound below


class NativeLibraryMissing(RuntimeError):
    pass


def lib():
    """Load libgsraster.so (once).  Raises NativeLibraryMissing if it was not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIBPATH):
            raise NativeLibraryMissing(
                f"{LIBPATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                "(hipcc --offload-arch=gfx950).  There is no CPU fallback.")
        L = ctypes.CDLL(LIBPATH)
        for name, args in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _RESTYPE.get(name, ctypes.c_int)
        if L.gs_abi_version() != ABI_VERSION:
            raise NativeLibraryMissing(f"{LIBPATH} implements ABI {L.gs_abi_version()}, this module binds ABI "
                                       f"{ABI_VERSION}: rebuild it")
        _lib = L
    return _lib


def call(name: str, *args) -> None:
    """Call an int-returning entry point and raise on a non-zero status."""
    rc = getattr(lib(), name)(*args)
    if rc != GS_OK:
        msg = lib().gs_last_error().decode("utf-8", "replace")
        if rc == 1:
            raise ValueError(f"{name}: {msg}")
        raise RuntimeError(f"{name} failed ({rc}): {msg}")


def ptr(t: torch.Tensor | None):
    """Device pointer of a contiguous tensor (None -> NULL)."""
    if t is None:
        return None
    if not t.is_contiguous():
        raise ValueError("tensor must be contiguous")
    return ctypes.c_void_p(t.data_ptr())


def stream_handle(device: torch.device):
    """The current torch stream of `device` as a hipStream_t."""
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
