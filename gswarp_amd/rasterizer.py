"""Public rasterizer API: a drop-in for ``gswarp.rasterizer``.

Same names, fields, defaults and return values as gswarp/rasterizer.py:11-241
(GaussianRasterizationSettings, GaussianRasterizer, RasterizerMeta,
rasterize_gaussians and the runtime getters/setters); the work runs in the
gfx950 HIP library on the current stream.
"""

from __future__ import annotations

from typing import NamedTuple

import torch
import torch.nn as nn

from . import _pipeline, _runtime, _workspace
from ._autograd import RasterizeGaussians
from ._validation import normalize_gaussian_inputs, validate_rasterizer_inputs


class RasterizerMeta(NamedTuple):
    """Auxiliary outputs from the non-flow rasterizer forward pass."""

    depth: torch.Tensor
    alpha: torch.Tensor
    proj_2D: torch.Tensor
    conic_2D: torch.Tensor
    conic_2D_inv: torch.Tensor


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
    backward_mode: str | None = None
    binning_sort_mode: str | None = None
    auto_tune: bool = True
    auto_tune_verbose: bool = True


def rasterize_gaussians(means3D, means2D, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp,
                        raster_settings):
    """Validated, differentiable forward -> (color, radii, RasterizerMeta)."""
    validate_rasterizer_inputs(means3D, means2D, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp,
                               raster_settings)
    color, radii, depth, alpha, proj_2D, conic_2D, conic_2D_inv = RasterizeGaussians.apply(
        means3D, means2D, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp, raster_settings)
    return color, radii, RasterizerMeta(depth=depth, alpha=alpha, proj_2D=proj_2D, conic_2D=conic_2D,
                                        conic_2D_inv=conic_2D_inv)


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
get_default_parameter_info = _runtime.get_default_parameter_info


def initialize_runtime_tuning(device=None, verbose=True):
    """Load the HIP library and report the launch configuration of this build.

    There is nothing to auto-tune: every kernel uses fixed wave64 launch
    shapes.  Returns the same report as get_runtime_tuning_report.
    """
    from . import _lib

    _lib.load()
    report = get_runtime_tuning_report(device)
    if verbose:
        print(f"[gswarp_amd] {report['device_name']} ({report['arch']}): "
              f"{report['compute_units']} CUs, wavefront {report['wavefront_size']}")
    return report


def get_runtime_tuning_report(device=None) -> dict:
    from . import _lib

    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    props = torch.cuda.get_device_properties(dev)
    return {
        "device": str(dev),
        "device_name": props.name,
        "arch": getattr(props, "gcnArchName", "unknown"),
        "compute_units": props.multi_processor_count,
        "wavefront_size": getattr(props, "warp_size", 64),
        "total_memory_bytes": props.total_memory,
        "library": str(_lib.LIB_PATH),
        "workgroup_size": 256,
        "tile": (16, 16),
    }


def get_runtime_auto_tuning_config():
    return False, False


def set_runtime_auto_tuning(enabled: bool | None = None, verbose: bool | None = None) -> None:
    """Accepted for compatibility (runtime.py:162-167); launch shapes are fixed."""


def is_available() -> bool:
    """True when the gfx950 HIP library loads (runtime.py:439-440 asks the same of Warp)."""
    from . import _lib

    try:
        _lib.load()
    except (OSError, RuntimeError):
        return False
    return True


def clear_warp_caches():
    """Release the per-stream host workspaces (the name is kept for compatibility)."""
    _workspace.clear_caches()


def get_warp_cache_report():
    """Workspace occupancy and retained bytes (the name is kept for compatibility)."""
    return _workspace.cache_report()


__all__ = [
    "GaussianRasterizationSettings",
    "GaussianRasterizer",
    "RasterizerMeta",
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
]
