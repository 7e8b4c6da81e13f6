"""Mip-Splatting-compatible rasterizer: a drop-in for ``gswarp.methods.mip_3dgs``.

Same names, settings and return values as gswarp/methods/mip_3dgs.py:29-160:
the standard settings plus ``filter_variance`` (default 0.3), validated to be
finite and non-negative, with ``antialiasing`` required to stay False.  The
forward adds the variance to each kept Gaussian's 2D covariance and recomputes
its conic, radius and tile count inside the preprocess kernel
(backend_mip_3dgs.py:63-102); the backward adds the same variance where it
recomputes the 2D covariance (backward_kernels.py:176-178).  A variance of 0
is the standard rasterizer.
"""

from __future__ import annotations

import math
from typing import NamedTuple

import torch
import torch.nn as nn

from .. import _pipeline
from .._autograd import RasterizeGaussians
from .._validation import normalize_gaussian_inputs, validate_rasterizer_inputs
from ..rasterizer import RasterizerMeta


class MethodSpec(NamedTuple):
    name: str
    output_mode: str
    filtering: str


METHOD = MethodSpec(name="mip_3dgs", output_mode="standard_meta", filtering="mip")


class MipGaussianRasterizationSettings(NamedTuple):
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
    backward_mode: str | None = None
    binning_sort_mode: str | None = None
    auto_tune: bool = True
    auto_tune_verbose: bool = True
    filter_variance: float = 0.3


def _check_filter(raster_settings) -> None:
    if raster_settings.antialiasing:
        raise ValueError("mip_3dgs uses filter_variance; antialiasing must remain False")
    filter_variance = float(raster_settings.filter_variance)
    if not math.isfinite(filter_variance) or filter_variance < 0.0:
        raise ValueError("filter_variance must be finite and non-negative")


def rasterize_gaussians(means3D, means2D, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp,
                        raster_settings):
    """Render with the screen-space Mip low-pass variance -> (color, radii, RasterizerMeta)."""
    validate_rasterizer_inputs(means3D, means2D, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp,
                               raster_settings)
    _check_filter(raster_settings)
    color, radii, depth, alpha, proj_2D, conic_2D, conic_2D_inv = RasterizeGaussians.apply(
        means3D, means2D, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp, raster_settings)
    return color, radii, RasterizerMeta(depth=depth, alpha=alpha, proj_2D=proj_2D, conic_2D=conic_2D,
                                        conic_2D_inv=conic_2D_inv)


class MipGaussianRasterizer(nn.Module):
    """Module wrapper with the Mip settings and the standard inputs."""

    def __init__(self, raster_settings: MipGaussianRasterizationSettings):
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


__all__ = [
    "METHOD",
    "MipGaussianRasterizationSettings",
    "MipGaussianRasterizer",
    "rasterize_gaussians",
]
