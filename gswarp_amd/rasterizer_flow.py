"""Flow rasterizer API: a drop-in for ``gswarp.rasterizer_flow``.

Mirrors gswarp/rasterizer_flow.py:1-215: the standard settings plus
``enable_flow_grad`` (default True) and ``compute_flow_aux`` (default: the
module flag), a flat 10-tuple return ending (gs_per_pixel (K,H,W) int32,
weight_per_gs_pixel (K,H,W), x_mu (2,K,H,W)), and get/set of the top-K
count and of the aux flag.
"""

from __future__ import annotations

from typing import NamedTuple

import torch
import torch.nn as nn

from . import _pipeline, _runtime
from ._autograd import RasterizeGaussiansFlow
from ._validation import normalize_gaussian_inputs, validate_rasterizer_inputs
from .rasterizer import (  # noqa: F401
    clear_warp_caches,
    get_default_parameter_info,
    get_runtime_auto_tuning_config,
    get_runtime_tuning_report,
    get_warp_cache_report,
    initialize_runtime_tuning,
)


class GaussianRasterizationSettings(NamedTuple):
    image_height: int
    image_width: int
    tanfovx: float
    tanfovy: float
    bg: torch.Tensor
    scale_modifier: float
    viewmatrix: torch.Tensor
    projmatrix: torch.Tensor
    sh_degree: int
    campos: torch.Tensor
    prefiltered: bool
    debug: bool = False
    antialiasing: bool = False
    enable_flow_grad: bool = True
    compute_flow_aux: bool | None = None
    backward_mode: str | None = None
    binning_sort_mode: str | None = None
    auto_tune: bool = True
    auto_tune_verbose: bool = True


def rasterize_gaussians(means3D, means2D, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp,
                        raster_settings):
    """Validated, differentiable forward -> flat 10-tuple."""
    validate_rasterizer_inputs(means3D, means2D, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp,
                               raster_settings)
    return RasterizeGaussiansFlow.apply(means3D, means2D, sh, colors_precomp, opacities, scales, rotations,
                                        cov3Ds_precomp, raster_settings)


class GaussianRasterizer(nn.Module):
    def __init__(self, raster_settings):
        super().__init__()
        self.raster_settings = raster_settings

    def markVisible(self, positions):
        with torch.no_grad():
            return _pipeline.mark_visible(positions, self.raster_settings.viewmatrix)

    def forward(self, means3D, means2D, opacities, dc=None, shs=None, colors_precomp=None, scales=None,
                rotations=None, cov3D_precomp=None):
        inputs = normalize_gaussian_inputs(dc=dc, shs=shs, colors_precomp=colors_precomp, scales=scales,
                                           rotations=rotations, cov3D_precomp=cov3D_precomp)
        return rasterize_gaussians(means3D, means2D, inputs.shs, inputs.colors_precomp, opacities, inputs.scales,
                                   inputs.rotations, inputs.cov3D_precomp, self.raster_settings)


get_backward_mode = _runtime.get_backward_mode
set_backward_mode = _runtime.set_backward_mode
get_binning_sort_mode = _runtime.get_binning_sort_mode
set_binning_sort_mode = _runtime.set_binning_sort_mode
get_tile_coverage_mode = _runtime.get_tile_coverage_mode
set_tile_coverage_mode = _runtime.set_tile_coverage_mode
get_compute_depth = _runtime.get_compute_depth
set_compute_depth = _runtime.set_compute_depth
get_compute_flow_aux = _runtime.get_compute_flow_aux
set_compute_flow_aux = _runtime.set_compute_flow_aux
get_flow_topk = _runtime.get_flow_topk
set_flow_topk = _runtime.set_flow_topk

__all__ = [
    "GaussianRasterizationSettings",
    "GaussianRasterizer",
    "rasterize_gaussians",
    "initialize_runtime_tuning",
    "get_runtime_tuning_report",
    "clear_warp_caches",
    "get_warp_cache_report",
    "get_backward_mode",
    "set_backward_mode",
    "get_compute_depth",
    "set_compute_depth",
    "get_binning_sort_mode",
    "set_binning_sort_mode",
    "get_tile_coverage_mode",
    "set_tile_coverage_mode",
    "get_compute_flow_aux",
    "set_compute_flow_aux",
    "get_flow_topk",
    "set_flow_topk",
]
