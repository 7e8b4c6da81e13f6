"""gswarp_amd — 3D Gaussian Splatting rasterizer for AMD Instinct MI355X (gfx950).

A drop-in for the rasterizer surface of ``gswarp`` 1.1.0 (gswarp/__init__.py:5-26):
the same settings, module, functions and runtime controls, computed by
hand-written HIP kernels (``libgswarp_hip.so``, C ABI in include/gswarp_hip.h)
on the current PyTorch-ROCm stream.  ``fused_ssim`` and ``distCUDA2`` belong
to other subsystems of the reference and are not provided.
"""

__version__ = "1.1.0+gfx950.0"

from .rasterizer import (  # noqa: F401
    GaussianRasterizationSettings,
    GaussianRasterizer,
    RasterizerMeta,
    clear_warp_caches,
    get_backward_mode,
    get_binning_sort_mode,
    get_compute_depth,
    get_runtime_tuning_report,
    get_tile_coverage_mode,
    get_warp_cache_report,
    initialize_runtime_tuning,
    rasterize_gaussians,
    set_backward_mode,
    set_binning_sort_mode,
    set_compute_depth,
    set_tile_coverage_mode,
)
from . import _lib

_lib.preload()


def fused_ssim(*args, **kwargs):
    raise NotImplementedError("fused_ssim is not part of the gfx950 rasterizer build")


def distCUDA2(*args, **kwargs):
    raise NotImplementedError("distCUDA2 is not part of the gfx950 rasterizer build")
