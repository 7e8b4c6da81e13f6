"""Opaque forward-state buffers of the raw rasterizer ABI.

Counterpart of gswarp/_internal/backends/warp/packing.py:37-121.  The raw
forward (18 arguments -> 11-tuple) hands the state its backward needs to the
caller as three uint8 tensors, geom, binning and img, and the raw backward
(27 arguments -> 8 gradients) reads them back.  Callers treat them as opaque;
their layouts are this build's own:

* geom: N render records of 48 bytes, then N SH clamp bytes (49 B per
  Gaussian).  The preprocess writes the records and clamp bits straight into
  this buffer, so the raw forward does no packing copy.
* binning: point_list (R int32) then ranges (T x 2 int32), the reference's
  layout.  The packed-key binning writes both in place.
* img: n_contrib (H*W int32), a byte view of the render's own output.

The backward recomputes the 3D covariance from scales / rotations (or reads
cov3D_precomp, which it receives as an argument), so geom carries no cov3D.
When a buffer does not have the expected size the backward rebuilds the
state from the inputs, as the reference does when unpacking fails
(backward_ops.py:425-470).
"""

from __future__ import annotations

import torch

from ._lib import GS_RECORD_FLOATS
from ._state import BinningState, PreprocessOutputs

RECORD_BYTES = 4 * GS_RECORD_FLOATS
GEOM_STRIDE_BYTES = RECORD_BYTES + 1
BLOCK = 16


def geom_bytes(num_points: int) -> int:
    return GEOM_STRIDE_BYTES * num_points


def binning_bytes(num_rendered: int, num_tiles: int) -> int:
    return 4 * (num_rendered + 2 * num_tiles)


def allocate_geom(num_points: int, device) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(geom, records (N, 12) fp32 view, clamped (N,) uint8 view)."""
    geom = torch.empty((geom_bytes(num_points),), dtype=torch.uint8, device=device)
    return (geom, *geom_views(geom, num_points))


def geom_views(geom: torch.Tensor, num_points: int) -> tuple[torch.Tensor, torch.Tensor]:
    records = geom[: RECORD_BYTES * num_points].view(torch.float32).view(num_points, GS_RECORD_FLOATS)
    clamped = geom[RECORD_BYTES * num_points: GEOM_STRIDE_BYTES * num_points]
    return records, clamped


def allocate_binning(num_rendered: int, num_tiles: int, device) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(int32 buffer, point_list (R,) view, ranges (T, 2) view)."""
    buf = torch.empty((num_rendered + 2 * num_tiles,), dtype=torch.int32, device=device)
    return buf, buf[:num_rendered], buf[num_rendered:].view(num_tiles, 2)


def empty_buffers(device) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The three zero-length buffers of an N == 0 forward (preprocess_ops.py:45-71)."""
    return tuple(torch.empty((0,), dtype=torch.uint8, device=device) for _ in range(3))


def pack(pre: PreprocessOutputs, bins: BinningState, n_contrib: torch.Tensor):
    """(geom, binning, img) byte tensors of one forward; views, not copies."""
    if pre.geom is None or bins.buffer is None:
        raise RuntimeError("forward state was not allocated in raw-ABI layout")
    return pre.geom, bins.buffer.view(torch.uint8), n_contrib.reshape(-1).view(torch.uint8)


def unpack(geom: torch.Tensor, binning: torch.Tensor, img: torch.Tensor, num_rendered: int, image_height: int,
           image_width: int, radii: torch.Tensor):
    """(PreprocessOutputs, BinningState, n_contrib) viewing the three buffers, or
    None when any has the wrong size (packing.py:63-121).  Only the fields the
    backward reads are populated; the others are empty."""
    if geom.numel() == 0 or binning.numel() == 0 or img.numel() == 0:
        return None
    if geom.dtype != torch.uint8 or binning.dtype != torch.uint8 or img.dtype != torch.uint8:
        return None
    num_points = radii.shape[0]
    grid_x = (image_width + BLOCK - 1) // BLOCK
    grid_y = (image_height + BLOCK - 1) // BLOCK
    num_tiles = grid_x * grid_y
    num_rendered = int(num_rendered)
    if (geom.numel() != geom_bytes(num_points) or binning.numel() != binning_bytes(num_rendered, num_tiles)
            or img.numel() != 4 * image_height * image_width):
        return None
    geom, binning, img = geom.contiguous(), binning.contiguous(), img.contiguous()
    records, clamped = geom_views(geom, num_points)
    device = geom.device
    empty_f = torch.empty((0,), dtype=torch.float32, device=device)
    pre = PreprocessOutputs(radii=radii, depths=empty_f, proj_2d=empty_f, conic_2d=empty_f, conic_2d_inv=empty_f,
                            tiles_touched=torch.empty((0,), dtype=torch.int32, device=device), records=records,
                            clamped=clamped, geom=geom)
    ints = binning.view(torch.int32)
    bins = BinningState(grid_x, grid_y, ints[:num_rendered], ints[num_rendered:].view(num_tiles, 2), num_rendered,
                        buffer=ints)
    n_contrib = img.view(torch.int32).view(image_height * image_width)
    return pre, bins, n_contrib
