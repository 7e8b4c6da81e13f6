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


@dataclass(slots=True)
class BinningState:
    grid_x: int
    grid_y: int
    point_list: torch.Tensor  # (R,) int32
    ranges: torch.Tensor  # (T, 2) int32
    num_rendered: int
    sorted_keys: torch.Tensor | None = None  # (R,) int64: tile << 32 | depth bits


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
