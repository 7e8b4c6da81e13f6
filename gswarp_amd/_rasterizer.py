"""Raw, diff_gaussian_rasterization-style entry points of the standard rasterizer.

A drop-in for ``gswarp._rasterizer`` (gswarp/_rasterizer.py:1-48):

* ``rasterize_gaussians(*18 args) -> (num_rendered, color, depth, alpha, radii,
  geom_buffer, binning_buffer, img_buffer, proj_2D, conic_2D, conic_2D_inv)``
  (backend_3dgs.py:112-248);
* ``rasterize_gaussians_backward(*27 args) -> (grad_means2D, grad_colors,
  grad_opacities, grad_means3D, grad_cov3D, grad_sh, grad_scales,
  grad_rotations)`` (backward_ops.py:376-746);
* the typed pair ``rasterize_gaussians_typed`` / ``rasterize_gaussians_backward_typed``
  that carries the forward state as an object instead of byte buffers;
* ``mark_visible(means3D, viewmatrix, projmatrix)`` and the runtime getters / setters.

The three byte buffers are opaque; their layout is documented in
:mod:`gswarp_amd._packing`.  Neither entry point records an autograd graph.
Runtime options come from the enclosing call's snapshot when there is one,
else from the module flags, as in the reference (runtime.py:60-100).
"""

from __future__ import annotations

from typing import Any

import torch

from . import _packing, _pipeline, _runtime
from ._state import ForwardResult, ForwardState
from .rasterizer import (  # noqa: F401
    clear_warp_caches,
    get_default_parameter_info,
    get_runtime_auto_tuning_config,
    get_runtime_tuning_report,
    get_warp_cache_report,
    initialize_runtime_tuning,
    is_available,
    set_runtime_auto_tuning,
)

FORWARD_ARG_COUNT = 18
BACKWARD_ARG_COUNT = 27


def _options(flow: bool) -> _runtime.ExecutionOptions:
    active = _runtime.active_options()
    return active if active is not None else _runtime.resolve_execution_options(None, flow=flow)


def forward_inputs(args) -> _pipeline.RasterInputs:
    """The 18 raw forward arguments, in the order of backend_3dgs.py:114-133:
    background, means3D, colors, opacities, scales, rotations, scale_modifier,
    cov3D_precomp, viewmatrix, projmatrix, tan_fovx, tan_fovy, image_height,
    image_width, sh, degree, campos, prefiltered."""
    if len(args) != FORWARD_ARG_COUNT:
        raise TypeError(f"rasterize_gaussians expects {FORWARD_ARG_COUNT} arguments, got {len(args)}")
    return _pipeline.RasterInputs(*args)


def raw_forward(args, *, flow: bool):
    inputs = forward_inputs(args)
    options = _options(flow)
    with torch.no_grad(), _runtime.execution_options(options):
        result = _pipeline.forward(inputs, options, flow=flow, pack=True)
    if result.state is None:
        buffers = _packing.empty_buffers(inputs.means3d.device)
    else:
        buffers = _packing.pack(result.state.preprocess, result.state.binning, result.state.n_contrib)
    return (result.num_rendered, result.color, result.depth, result.alpha, result.radii, *buffers,
            result.proj_2d, result.conic_2d, result.conic_2d_inv, *result.aux)


def raw_backward(inputs: _pipeline.RasterInputs, radii, grads, geom, num_rendered, binning, img, alphas, *,
                 flow: bool, flow_double: bool, forward_state: ForwardState | None = None, unpack: bool = True):
    options = _options(flow)
    state = forward_state
    if state is None and unpack:
        unpacked = _packing.unpack(geom, binning, img, num_rendered, inputs.image_height, inputs.image_width,
                                   radii)
        if unpacked is not None:
            state = ForwardState(*unpacked)
    with torch.no_grad(), _runtime.execution_options(options):
        return _pipeline.backward(inputs, radii, alphas, *grads, options, state, flow_double=flow_double)


def _backward_args(args):
    if len(args) != BACKWARD_ARG_COUNT:
        raise TypeError(f"rasterize_gaussians_backward expects {BACKWARD_ARG_COUNT} arguments, got {len(args)}")
    (background, means3D, radii, colors, opacities, scales, rotations, scale_modifier, cov3D_precomp, viewmatrix,
     projmatrix, tan_fovx, tan_fovy, grad_color, grad_depth, grad_alpha, grad_proj_2D, grad_conic_2D,
     grad_conic_2D_inv, sh, degree, campos, geom_buffer, num_rendered, binning_buffer, img_buffer, alphas) = args
    inputs = _pipeline.RasterInputs(background, means3D, colors, opacities, scales, rotations, scale_modifier,
                                    cov3D_precomp, viewmatrix, projmatrix, tan_fovx, tan_fovy, grad_color.shape[1],
                                    grad_color.shape[2], sh, degree, campos, False)
    grads = (grad_color, grad_depth, grad_alpha, grad_proj_2D, grad_conic_2D, grad_conic_2D_inv)
    return inputs, radii, grads, geom_buffer, num_rendered, binning_buffer, img_buffer, alphas


def rasterize_gaussians(*args: Any):
    """Raw forward with opaque packed state (backend_3dgs.py:234-236)."""
    return raw_forward(args, flow=False)


def typed_forward(args, *, flow: bool) -> ForwardResult:
    inputs = forward_inputs(args)
    options = _options(flow)
    with torch.no_grad(), _runtime.execution_options(options):
        return _pipeline.forward(inputs, options, flow=flow)


def rasterize_gaussians_typed(*args: Any) -> ForwardResult:
    """Forward with the typed state object and no packed buffers (backend_3dgs.py:239-241)."""
    return typed_forward(args, flow=False)


def rasterize_gaussians_backward(*args: Any):
    """Raw backward over the 27 arguments of backward_ops.py:377-405; the state
    comes from the byte buffers, or is rebuilt when they do not unpack."""
    inputs, radii, grads, geom, num_rendered, binning, img, alphas = _backward_args(args)
    return raw_backward(inputs, radii, grads, geom, num_rendered, binning, img, alphas, flow=False,
                        flow_double=False)


def rasterize_gaussians_backward_typed(*args: Any, forward_state):
    """Raw backward arguments with a typed forward state (backward_ops.py:753-755)."""
    inputs, radii, grads, geom, num_rendered, binning, img, alphas = _backward_args(args)
    return raw_backward(inputs, radii, grads, geom, num_rendered, binning, img, alphas, flow=False,
                        flow_double=False, forward_state=forward_state, unpack=False)


def mark_visible(means3D, viewmatrix, projmatrix):
    """view-space z > 0.2 as bool (preprocess_ops.py:584-595)."""
    return _pipeline.mark_visible(means3D, viewmatrix)


get_backward_mode = _runtime.get_backward_mode
set_backward_mode = _runtime.set_backward_mode
get_binning_sort_mode = _runtime.get_binning_sort_mode
set_binning_sort_mode = _runtime.set_binning_sort_mode
get_tile_coverage_mode = _runtime.get_tile_coverage_mode
set_tile_coverage_mode = _runtime.set_tile_coverage_mode
get_compute_depth = _runtime.get_compute_depth
set_compute_depth = _runtime.set_compute_depth

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
    "rasterize_gaussians_backward_typed",
    "set_runtime_auto_tuning",
    "get_compute_depth",
    "set_compute_depth",
]
