"""PLY checkpoints of the Gaussians (jax_gs/io/ply.py:6-123), byte-compatible with the
reference's files: binary little-endian, one vertex element of 62 float32 properties
(x y z, zero normals, f_dc_0..2, f_rest_0..44 coefficient-major, opacity, scale_0..2,
rot_0..3).  The records are packed and unpacked on the GPU (``gs_ply_pack`` /
``gs_ply_unpack``), so the arrays cross PCIe as one contiguous block.  Paths go through
fsspec, as in the reference.
"""
from __future__ import annotations

import fsspec
import numpy as np
import torch

from .. import _lib
from ..core.gaussians import Gaussians

PLY_PROPERTIES = (["x", "y", "z", "nx", "ny", "nz", "f_dc_0", "f_dc_1", "f_dc_2"] +
                  [f"f_rest_{i}" for i in range(45)] +
                  ["opacity", "scale_0", "scale_1", "scale_2", "rot_0", "rot_1", "rot_2", "rot_3"])
PLY_FLOATS = len(PLY_PROPERTIES)  # 62


def ply_header(num_points: int) -> bytes:
    """ply.py:58-64."""
    lines = [b"ply\n", b"format binary_little_endian 1.0\n", f"element vertex {num_points}\n".encode()]
    lines += [f"property float {name}\n".encode() for name in PLY_PROPERTIES]
    lines.append(b"end_header\n")
    return b"".join(lines)


def save_ply(path, gaussians: Gaussians) -> None:
    """ply.py:6-66: write the Gaussians (device tensors, 16 SH coefficients) to path."""
    dev = gaussians.means.device
    if dev.type != "cuda":
        raise ValueError("save_ply: the Gaussians must be on the GPU")
    n = gaussians.means.shape[0]
    k = gaussians.sh_coeffs.shape[1]
    records = torch.empty((n, PLY_FLOATS), dtype=torch.float32, device=dev)
    arrs = [getattr(gaussians, f).detach().to(torch.float32).contiguous()
            for f in ("means", "scales", "quaternions", "opacities", "sh_coeffs")]
    _lib.call("gs_ply_pack", _lib.stream_handle(dev), n, k, *[_lib.ptr(a) for a in arrs], _lib.ptr(records))
    data = records.cpu().numpy().astype("<f4", copy=False).tobytes()
    with fsspec.open(path, "wb") as f:
        f.write(ply_header(n))
        f.write(data)


def load_ply(path, device="cuda:0") -> Gaussians:
    """ply.py:68-123: read a file written by save_ply (the vertex count from the header)."""
    with fsspec.open(path, "rb") as f:
        line = f.readline()
        num_points = 0
        while line and line.strip() != b"end_header":
            if b"element vertex" in line:
                num_points = int(line.split()[-1])
            line = f.readline()
        data = f.read(num_points * PLY_FLOATS * 4)
    if len(data) != num_points * PLY_FLOATS * 4:
        raise ValueError(f"load_ply: {path} holds {len(data)} bytes of vertex data, {num_points} vertices need "
                         f"{num_points * PLY_FLOATS * 4}")
    dev = torch.device(device)
    rec = torch.from_numpy(np.frombuffer(data, dtype="<f4").astype(np.float32).reshape(num_points, PLY_FLOATS))
    rec = rec.to(dev)
    g = Gaussians(torch.empty((num_points, 3), device=dev), torch.empty((num_points, 3), device=dev),
                  torch.empty((num_points, 4), device=dev), torch.empty((num_points, 1), device=dev),
                  torch.empty((num_points, 16, 3), device=dev))
    _lib.call("gs_ply_unpack", _lib.stream_handle(dev), num_points, 16, _lib.ptr(rec), _lib.ptr(g.means),
              _lib.ptr(g.scales), _lib.ptr(g.quaternions), _lib.ptr(g.opacities), _lib.ptr(g.sh_coeffs))
    return g
