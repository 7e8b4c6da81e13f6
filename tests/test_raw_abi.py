"""Host-side checks of the raw ABI's opaque buffers (no GPU needed).

The raw forward returns its state as three byte tensors and the raw backward
reads them back (packing.py:37-121).  These tests pin the layout arithmetic,
that the unpacked tensors are views (no copies) of the buffers, and that
buffers of the wrong size are refused, which sends the backward down its
rebuild path (backward_ops.py:425-470).
"""

from __future__ import annotations

import pytest
import torch

from gswarp_amd import _packing, _rasterizer, _rasterizer_flow
from gswarp_amd._lib import GS_RECORD_FLOATS


def _buffers(P=7, R=11, H=20, W=35):
    T = ((W + 15) // 16) * ((H + 15) // 16)
    geom, records, clamped = _packing.allocate_geom(P, "cpu")
    records.copy_(torch.arange(P * GS_RECORD_FLOATS, dtype=torch.float32).view(P, GS_RECORD_FLOATS))
    clamped.copy_(torch.arange(P, dtype=torch.uint8) * 3)
    buf, point_list, ranges = _packing.allocate_binning(R, T, "cpu")
    point_list.copy_(torch.arange(R, dtype=torch.int32) * 5)
    ranges.copy_(torch.arange(2 * T, dtype=torch.int32).view(T, 2))
    n_contrib = torch.arange(H * W, dtype=torch.int32)
    return P, R, H, W, T, geom, buf, n_contrib


def test_layout_sizes():
    P, R, H, W, T, geom, buf, n_contrib = _buffers()
    assert _packing.RECORD_BYTES == 48 and _packing.GEOM_STRIDE_BYTES == 49
    assert geom.numel() == 49 * P
    assert buf.numel() == R + 2 * T and _packing.binning_bytes(R, T) == 4 * (R + 2 * T)


def test_unpack_round_trip_returns_views():
    P, R, H, W, T, geom, buf, n_contrib = _buffers()
    radii = torch.ones(P, dtype=torch.int32)
    bbytes, img = buf.view(torch.uint8), n_contrib.view(torch.uint8)
    pre, bins, nc = _packing.unpack(geom, bbytes, img, R, H, W, radii)
    assert torch.equal(pre.records.reshape(-1), torch.arange(P * GS_RECORD_FLOATS, dtype=torch.float32))
    assert torch.equal(pre.clamped, torch.arange(P, dtype=torch.uint8) * 3)
    assert torch.equal(bins.point_list, torch.arange(R, dtype=torch.int32) * 5)
    assert torch.equal(bins.ranges.reshape(-1), torch.arange(2 * T, dtype=torch.int32))
    assert bins.num_rendered == R and bins.grid_x * bins.grid_y == T
    assert torch.equal(nc, n_contrib)
    # views, not copies
    assert pre.records.data_ptr() == geom.data_ptr()
    assert pre.clamped.data_ptr() == geom.data_ptr() + 48 * P
    assert bins.point_list.data_ptr() == buf.data_ptr()
    assert bins.ranges.data_ptr() == buf.data_ptr() + 4 * R
    assert nc.data_ptr() == n_contrib.data_ptr()


@pytest.mark.parametrize("which", ["geom", "binning", "img", "count", "empty", "dtype"])
def test_unpack_refuses_wrong_sizes(which):
    P, R, H, W, T, geom, buf, n_contrib = _buffers()
    radii = torch.ones(P, dtype=torch.int32)
    bbytes, img = buf.view(torch.uint8), n_contrib.view(torch.uint8)
    num_rendered = R
    if which == "geom":
        geom = geom[:-1]
    elif which == "binning":
        bbytes = bbytes[:-4]
    elif which == "img":
        img = img[:-4]
    elif which == "count":
        num_rendered = R + 1
    elif which == "empty":
        geom = geom[:0]
    else:
        img = n_contrib
    assert _packing.unpack(geom, bbytes, img, num_rendered, H, W, radii) is None


def test_pack_refuses_state_not_in_raw_layout():
    from gswarp_amd._state import BinningState, PreprocessOutputs
    e = torch.empty(0)
    pre = PreprocessOutputs(e, e, e, e, e, e, e, e)
    bins = BinningState(1, 1, e, e, 0)
    with pytest.raises(RuntimeError):
        _packing.pack(pre, bins, e)


def test_raw_entry_points_check_argument_counts():
    with pytest.raises(TypeError, match="18 arguments"):
        _rasterizer.rasterize_gaussians(*range(17))
    with pytest.raises(TypeError, match="27 arguments"):
        _rasterizer.rasterize_gaussians_backward(*range(26))
    with pytest.raises(TypeError, match="18 arguments"):
        _rasterizer_flow.rasterize_gaussians(*range(19))
    with pytest.raises(TypeError, match="31 arguments"):
        _rasterizer_flow.rasterize_gaussians_backward(*range(27))


def test_alias_modules_export_the_reference_names():
    import gswarp._rasterizer as raw
    import gswarp._rasterizer_flow as raw_flow
    for name in ("rasterize_gaussians", "rasterize_gaussians_backward", "rasterize_gaussians_typed",
                 "rasterize_gaussians_backward_typed", "mark_visible", "is_available", "set_compute_depth"):
        assert callable(getattr(raw, name))
    for name in ("rasterize_gaussians", "rasterize_gaussians_backward", "rasterize_gaussians_flow_backward_typed",
                 "get_flow_topk", "set_compute_flow_aux"):
        assert callable(getattr(raw_flow, name))
