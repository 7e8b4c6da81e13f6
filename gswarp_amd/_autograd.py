"""torch.autograd Functions of the standard and flow rasterizers.

Same contract as gswarp/_internal/frontend/standard_autograd.py:36-188 and
flow_autograd.py:36-196: the forward snapshots the runtime options, saves
(colors, opacities, means3D, scales, rotations, cov3D, radii, sh, alpha),
keeps the typed forward state on ctx until the first backward releases it
(in ``finally``), and the backward maps the eight gradients onto the ten
inputs.  A second backward through a retained graph recomputes the state.
"""

from __future__ import annotations

import torch

from . import _pipeline
from ._runtime import execution_options, resolve_execution_options


def _forward_args(means3D, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp, raster_settings):
    return _pipeline.RasterInputs(
        raster_settings.bg, means3D, colors_precomp, opacities, scales, rotations, raster_settings.scale_modifier,
        cov3Ds_precomp, raster_settings.viewmatrix, raster_settings.projmatrix, raster_settings.tanfovx,
        raster_settings.tanfovy, raster_settings.image_height, raster_settings.image_width, sh,
        raster_settings.sh_degree, raster_settings.campos, raster_settings.prefiltered,
        float(getattr(raster_settings, "filter_variance", 0.0)))


def _run_forward(ctx, means3D, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp, raster_settings,
                 flow: bool):
    options = resolve_execution_options(raster_settings, flow=flow)
    inputs = _forward_args(means3D, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp, raster_settings)
    with execution_options(options):
        result = _pipeline.forward(inputs, options, flow=flow,
                                   grad_buffer=_pipeline.ACCUMULATOR_IN_FORWARD and any(ctx.needs_input_grad))
    ctx.raster_settings = raster_settings
    ctx.execution_options = options
    ctx.num_rendered = result.num_rendered
    ctx.forward_state = result.state
    ctx.save_for_backward(colors_precomp, opacities, means3D, scales, rotations, cov3Ds_precomp, result.radii, sh,
                          result.alpha)
    ctx.mark_non_differentiable(result.radii)
    # Outputs the loss does not use reach backward as None, which the kernels
    # read as zero gradients, instead of as materialised zero tensors.
    ctx.set_materialize_grads(False)
    return result


def _run_backward(ctx, grad_color, grad_depth, grad_alpha, grad_proj_2D, grad_conic_2D, grad_conic_2D_inv,
                  flow_double: bool):
    colors_precomp, opacities, means3D, scales, rotations, cov3Ds_precomp, radii, sh, alpha = ctx.saved_tensors
    raster_settings = ctx.raster_settings
    inputs = _forward_args(means3D, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp, raster_settings)
    try:
        with execution_options(ctx.execution_options):
            grads = _pipeline.backward(inputs, radii, alpha, grad_color, grad_depth, grad_alpha, grad_proj_2D,
                                       grad_conic_2D, grad_conic_2D_inv, ctx.execution_options, ctx.forward_state,
                                       flow_double=flow_double)
    finally:
        # Arbitrary ctx attributes are not released by PyTorch.
        ctx.forward_state = None
    (grad_means2D, grad_colors_precomp, grad_opacities, grad_means3D, grad_cov3Ds_precomp, grad_sh, grad_scales,
     grad_rotations) = grads
    return (grad_means3D, grad_means2D, grad_sh, grad_colors_precomp, grad_opacities, grad_scales, grad_rotations,
            grad_cov3Ds_precomp, None)


class RasterizeGaussians(torch.autograd.Function):
    """Standard rasterizer: outputs (color, radii, depth, alpha, proj_2D, conic_2D, conic_2D_inv)."""

    @staticmethod
    def forward(ctx, means3D, means2D, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp,
                raster_settings):
        result = _run_forward(ctx, means3D, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp,
                              raster_settings, flow=False)
        return (result.color, result.radii, result.depth, result.alpha, result.proj_2d, result.conic_2d,
                result.conic_2d_inv)

    @staticmethod
    def backward(ctx, grad_color, grad_radii, grad_depth, grad_alpha, grad_proj_2D, grad_conic_2D,
                 grad_conic_2D_inv):
        return _run_backward(ctx, grad_color, grad_depth, grad_alpha, grad_proj_2D, grad_conic_2D,
                             grad_conic_2D_inv, flow_double=False)


class RasterizeGaussiansFlow(torch.autograd.Function):
    """Flow rasterizer: the standard outputs plus (gs_per_pixel, weight_per_gs_pixel, x_mu).

    The gradient arriving on x_mu is ignored and, with enable_flow_grad, the
    render gradients of the projected means and conics enter the
    preprocess backward twice, as in the reference (flow_ops.py:219, 337-360).
    """

    @staticmethod
    def forward(ctx, means3D, means2D, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp,
                raster_settings):
        result = _run_forward(ctx, means3D, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp,
                              raster_settings, flow=True)
        ctx.mark_non_differentiable(result.radii, result.aux[0])
        return (result.color, result.radii, result.depth, result.alpha, result.proj_2d, result.conic_2d,
                result.conic_2d_inv, *result.aux)

    @staticmethod
    def backward(ctx, grad_color, grad_radii, grad_depth, grad_alpha, grad_proj_2D, grad_conic_2D,
                 grad_conic_2D_inv, grad_gs_per_pixel, grad_weight_per_gs_pixel, grad_x_mu):
        flow_double = bool(getattr(ctx.raster_settings, "enable_flow_grad", True))
        return _run_backward(ctx, grad_color, grad_depth, grad_alpha, grad_proj_2D, grad_conic_2D,
                             grad_conic_2D_inv, flow_double=flow_double)
