"""Typed state carried from the forward stages to the backward.

Counterparts of gswarp/_internal/backends/warp/state.py:48-110.  The render
stage reads one packed 48-byte record per Gaussian (``records``) instead of
separate points_xy / conic_opacity / features / depths arrays.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch


@dataclass(slots=True)
class PreprocessOutputs:
    radii: torch.Tensor  # (N,) int32
    depths: torch.Tensor  # (N,) view-space z of visible Gaussians, 0 otherwise
    proj_2d: torch.Tensor  # (N, 2) pixel-space centre (= the reference's points_xy_image)
    conic_2d: torch.Tensor  # (N, 3)
    conic_2d_inv: torch.Tensor  # (N, 3) 2D covariance incl. the 0.3 dilation
    tiles_touched: torch.Tensor  # (N,) int32
    records: torch.Tensor  # (N, 12) fp32 render records
    clamped: torch.Tensor  # (N,) uint8 SH clamp bits
    coverage_mode: int = 1
    geom: torch.Tensor | None = None  # raw-ABI byte buffer that records and clamped are views of
    coverage: torch.Tensor | None = None  # (N, 4) int32 cover words for the emission, or None (re-derived)
    band_store: torch.Tensor | None = None  # int32 coverage bands of the banded Gaussians, or None
    # gs_scan_tiles_onepass state that the preprocess prepared (serves one scan), or None
    scan_state: torch.Tensor | None = None


@dataclass(slots=True)
class KeyLayout:
    """Fields of the 64-bit binning key, from high to low:
    tile | float_bits(depth) - depth_min (depth_bits wide) | point index (value_bits wide, 0 = not packed)."""

    depth_min: int = 0
    depth_bits: int = 32
    value_bits: int = 0

    @property
    def tile_shift(self) -> int:
        return self.depth_bits + self.value_bits


@dataclass(slots=True)
class RenderImages:
    """Forward render outputs allocated before the binning, so that the binning
    call can launch the render into them."""

    background: torch.Tensor  # (3,) fp32, contiguous
    color: torch.Tensor  # (3, H, W)
    depth: torch.Tensor  # (1, H, W)
    alpha: torch.Tensor  # (1, H, W)
    n_contrib: torch.Tensor  # (H*W,) int32
    compute_depth: bool = True


@dataclass(slots=True)
class BinningState:
    grid_x: int
    grid_y: int
    point_list: torch.Tensor  # (R,) int32
    ranges: torch.Tensor  # (T, 2) int32
    num_rendered: int
    sorted_keys: torch.Tensor | None = None  # (R,) int64 sorted binning keys (see KeyLayout)
    key_layout: KeyLayout = field(default_factory=KeyLayout)
    buffer: torch.Tensor | None = None  # raw-ABI (R + 2T) int32 buffer that point_list and ranges are views of
    rendered: bool = False  # the standard forward render was launched with the binning (RenderImages)
    tile_order: torch.Tensor | None = None  # (T,) int32 buffer the forward render was given (gs_tile_order)

    def decode_keys(self) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """(tile id, depth float bits, sort field = tile and depth fields as one
        non-negative int64) of every sorted pair, from sorted_keys."""
        k = self.sorted_keys
        lay = self.key_layout
        field_ = (k >> lay.value_bits) & ((1 << (64 - lay.value_bits)) - 1) if lay.value_bits else k
        tile = (k >> lay.tile_shift) & ((1 << (64 - lay.tile_shift)) - 1)
        depth = (field_ & ((1 << lay.depth_bits) - 1)) + lay.depth_min
        return tile, depth, field_


@dataclass(slots=True)
class RenderStageResult:
    color: torch.Tensor
    depth: torch.Tensor
    alpha: torch.Tensor
    n_contrib: torch.Tensor
    aux: tuple[torch.Tensor, ...] = ()


@dataclass(slots=True)
class ForwardState:
    preprocess: PreprocessOutputs
    binning: BinningState
    n_contrib: torch.Tensor
    # (N, 10) float32 gradient accumulator that the forward render zeroed on
    # its way (None when the forward made none); one backward takes it
    grad_gauss: torch.Tensor | None = None


@dataclass(slots=True)
class ForwardResult:
    num_rendered: int
    color: torch.Tensor
    depth: torch.Tensor
    alpha: torch.Tensor
    radii: torch.Tensor
    proj_2d: torch.Tensor
    conic_2d: torch.Tensor
    conic_2d_inv: torch.Tensor
    state: ForwardState | None
    aux: tuple[torch.Tensor, ...] = field(default_factory=tuple)
