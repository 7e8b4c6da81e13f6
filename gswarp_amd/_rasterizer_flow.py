"""Raw entry points of the flow rasterizer: a drop-in for ``gswarp._rasterizer_flow``.

* ``rasterize_gaussians(*18 args)`` -> the standard 11-tuple followed by
  (gs_per_pixel, weight_per_gs_pixel, x_mu) (backend_3dgs_flow.py:113-220);
* ``rasterize_gaussians_backward(*31 args)`` -> the eight gradients
  (flow_ops.py:196-512).  The 31 arguments are the standard 27 with the three
  flow outputs' gradients after grad_conic_2D_inv (all three ignored, as the
  reference ignores them) and enable_flow_grad last; with enable_flow_grad the
  render gradients of the projected means and conics enter the preprocess
  backward twice (flow_ops.py:337-360).

The byte buffers are those of :mod:`gswarp_amd._packing`.
"""

from __future__ import annotations

from typing import Any

from . import _runtime
from ._rasterizer import (  # noqa: F401
    clear_warp_caches,
    get_backward_mode,
    get_binning_sort_mode,
    get_compute_depth,
    get_default_parameter_info,
    get_runtime_auto_tuning_config,
    get_runtime_tuning_report,
    get_tile_coverage_mode,
    get_warp_cache_report,
    initialize_runtime_tuning,
    is_available,
    mark_visible,
    raw_backward,
    raw_forward,
    set_backward_mode,
    set_binning_sort_mode,
    set_compute_depth,
    set_runtime_auto_tuning,
    set_tile_coverage_mode,
    typed_forward,
)
from ._pipeline import RasterInputs
from ._state import ForwardResult

BACKWARD_ARG_COUNT = 31


def _backward_args(args):
    if len(args) != BACKWARD_ARG_COUNT:
        raise TypeError(f"rasterize_gaussians_backward expects {BACKWARD_ARG_COUNT} arguments, got {len(args)}")
    (background, means3D, radii, colors, opacities, scales, rotations, scale_modifier, cov3D_precomp, viewmatrix,
     projmatrix, tan_fovx, tan_fovy, grad_color, grad_depth, grad_alpha, grad_proj_2D, grad_conic_2D,
     grad_conic_2D_inv, _grad_gs_per_pixel, _grad_weight_per_gs_pixel, _grad_x_mu, sh, degree, campos, geom_buffer,
     num_rendered, binning_buffer, img_buffer, alphas, enable_flow_grad) = args
    inputs = RasterInputs(background, means3D, colors, opacities, scales, rotations, scale_modifier, cov3D_precomp,
                          viewmatrix, projmatrix, tan_fovx, tan_fovy, grad_color.shape[1], grad_color.shape[2], sh,
                          degree, campos, False)
    grads = (grad_color, grad_depth, grad_alpha, grad_proj_2D, grad_conic_2D, grad_conic_2D_inv)
    return (inputs, radii, grads, geom_buffer, num_rendered, binning_buffer, img_buffer, alphas,
            bool(enable_flow_grad))


def rasterize_gaussians(*args: Any):
    """Raw flow forward with opaque packed state (backend_3dgs_flow.py:223-224)."""
    return raw_forward(args, flow=True)


def rasterize_gaussians_typed(*args: Any) -> ForwardResult:
    """Flow forward with the typed state object (backend_3dgs_flow.py:227-228)."""
    return typed_forward(args, flow=True)


def rasterize_gaussians_backward(*args: Any):
    """Raw flow backward (flow_ops.py:515-517)."""
    inputs, radii, grads, geom, num_rendered, binning, img, alphas, flow_double = _backward_args(args)
    return raw_backward(inputs, radii, grads, geom, num_rendered, binning, img, alphas, flow=True,
                        flow_double=flow_double)


def rasterize_gaussians_flow_backward_typed(*args: Any, forward_state):
    """Raw flow backward arguments with a typed forward state (flow_ops.py:520-522)."""
    inputs, radii, grads, geom, num_rendered, binning, img, alphas, flow_double = _backward_args(args)
    return raw_backward(inputs, radii, grads, geom, num_rendered, binning, img, alphas, flow=True,
                        flow_double=flow_double, forward_state=forward_state, unpack=False)


get_compute_flow_aux = _runtime.get_compute_flow_aux
set_compute_flow_aux = _runtime.set_compute_flow_aux
get_flow_topk = _runtime.get_flow_topk
set_flow_topk = _runtime.set_flow_topk

__all__ = [
    "clear_warp_caches",
    "get_warp_cache_report",
    "get_default_parameter_info",
    "is_available",
    "get_backward_mode",
    "set_backward_mode",
    "get_binning_sort_mode",
    "set_binning_sort_mode",
    "get_tile_coverage_mode",
    "set_tile_coverage_mode",
    "get_runtime_auto_tuning_config",
    "get_runtime_tuning_report",
    "initialize_runtime_tuning",
    "rasterize_gaussians",
    "rasterize_gaussians_typed",
    "mark_visible",
    "rasterize_gaussians_backward",
    "rasterize_gaussians_flow_backward_typed",
    "set_runtime_auto_tuning",
    "get_compute_depth",
    "set_compute_depth",
    "get_compute_flow_aux",
    "set_compute_flow_aux",
    "get_flow_topk",
    "set_flow_topk",
]
