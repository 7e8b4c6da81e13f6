"""The public input checks report what the reference reports, in its order.

gswarp/_internal/api/validation.py:22-202 raises ValueError with fixed
messages in a fixed order; callers (and the reference's tests) match on
them.  Every check after the first needs means3D on a GPU, so these CPU
tests wrap CPU tensors in a subclass that reports is_cuda: the device
comparisons then run against the CPU device, and each check in turn can be
made to fail on its own, or together with a later one to pin the order.
"""

from __future__ import annotations

import re

import pytest
import torch

from gswarp_amd import _validation
from gswarp_amd.rasterizer import GaussianRasterizationSettings


class _OnGpu(torch.Tensor):
    """A CPU tensor that passes the means3D is_cuda check."""

    @property
    def is_cuda(self):  # noqa: D401
        return True


def _gpu(t: torch.Tensor) -> torch.Tensor:
    return t.as_subclass(_OnGpu)


def _settings(**kw):
    base = dict(image_height=16, image_width=16, tanfovx=1.0, tanfovy=1.0, bg=torch.zeros(3), scale_modifier=1.0,
                viewmatrix=torch.eye(4), projmatrix=torch.eye(4), sh_degree=0, campos=torch.zeros(3),
                prefiltered=False)
    base.update(kw)
    return GaussianRasterizationSettings(**base)


def _args(n=4, **kw):
    args = dict(means3D=_gpu(torch.zeros(n, 3)), means2D=torch.zeros(n, 3), sh=torch.zeros(n, 1, 3),
                colors_precomp=torch.empty(0), opacities=torch.zeros(n, 1), scales=torch.ones(n, 3),
                rotations=torch.ones(n, 4), cov3Ds_precomp=torch.empty(0), raster_settings=_settings())
    args.update(kw)
    return args


def _raises(message: str, **kw):
    with pytest.raises(ValueError, match="^" + re.escape(message) + "$"):
        _validation.validate_rasterizer_inputs(**_args(**kw))


def test_valid_inputs_pass():
    _validation.validate_rasterizer_inputs(**_args())
    _validation.validate_rasterizer_inputs(**_args(raster_settings=_settings(debug=True)))
    # N == 0: the exclusivity checks are skipped
    _validation.validate_rasterizer_inputs(**_args(n=0, sh=torch.empty(0), scales=torch.empty(0),
                                                   rotations=torch.empty(0)))


def test_tensor_type_checks_come_first_in_argument_order():
    _raises("means3D must be a torch.Tensor", means3D=[0.0], means2D="x")
    _raises("means2D must be a torch.Tensor", means2D="x", opacities=None)
    _raises("opacities must be a torch.Tensor", opacities=None, means3D=torch.zeros(4, 3))
    _raises("means3D must be a CUDA tensor", means3D=torch.zeros(4, 3))


def test_per_gaussian_tensors():
    _raises("means3D must have dtype torch.float32, got torch.float64",
            means3D=_gpu(torch.zeros(4, 3, dtype=torch.float64)))
    _raises("means3D must have shape ('N', 3), got (4, 2)", means3D=_gpu(torch.zeros(4, 2)))
    _raises("means3D must have shape ('N', 3), got (12,)", means3D=_gpu(torch.zeros(12)))
    _raises("means2D must have dtype torch.float32, got torch.float16", means2D=torch.zeros(4, 3).half())
    _raises("means2D must have shape (4, 3), got (5, 3)", means2D=torch.zeros(5, 3))
    _raises("opacities must have dtype torch.float32, got torch.int32",
            opacities=torch.zeros(4, 1, dtype=torch.int32))
    _raises("opacities must contain one value per Gaussian (4), got 3", opacities=torch.zeros(3))


def test_settings_scalars_and_tensors():
    _raises("image_height and image_width must be positive integers", raster_settings=_settings(image_height=0))
    _raises("image_height and image_width must be positive integers", raster_settings=_settings(image_width=16.0))
    _raises("image_height * image_width must fit in a signed 32-bit index",
            raster_settings=_settings(image_height=1 << 16, image_width=1 << 16))
    _raises("tanfovx, tanfovy, and scale_modifier must be finite and positive",
            raster_settings=_settings(tanfovy=float("inf")))
    _raises("tanfovx, tanfovy, and scale_modifier must be finite and positive",
            raster_settings=_settings(scale_modifier=0.0))
    _raises("sh_degree must be a non-negative integer", raster_settings=_settings(sh_degree=-1))
    _raises("raster_settings.bg must be a torch.Tensor", raster_settings=_settings(bg=[0, 0, 0]))
    _raises("raster_settings.viewmatrix must have shape (4, 4), got (3, 3)",
            raster_settings=_settings(viewmatrix=torch.eye(3)))
    _raises("raster_settings.projmatrix must have dtype torch.float32, got torch.float64",
            raster_settings=_settings(projmatrix=torch.eye(4, dtype=torch.float64)))
    _raises("raster_settings.campos must have shape (3,), got (4,)", raster_settings=_settings(campos=torch.zeros(4)))


def test_missing_settings_field():
    class Partial:
        image_height = image_width = 16
        tanfovx = tanfovy = scale_modifier = 1.0
        sh_degree = 0
        bg = torch.zeros(3)

    _raises("raster_settings is missing a required field", raster_settings=Partial())


def test_scalars_are_checked_before_settings_tensors():
    # both wrong: the image size is reported
    _raises("image_height and image_width must be positive integers",
            raster_settings=_settings(image_height=-1, campos=torch.zeros(5)))
    # a non-tensor settings field is reported before the scalar checks run
    _raises("raster_settings.campos must be a torch.Tensor", raster_settings=_settings(image_height=-1, campos=None))


def test_optional_inputs():
    _raises("sh must be a torch.Tensor", sh=None)
    _raises("colors_precomp must have dtype torch.float32, got torch.float64",
            colors_precomp=torch.zeros(4, 3, dtype=torch.float64))
    # placement is checked input by input: sh (non-empty, wrong dtype) before colors_precomp's type
    _raises("sh must have dtype torch.float32, got torch.float64", sh=torch.zeros(4, 1, 3, dtype=torch.float64),
            colors_precomp=None)
    _raises("provide exactly one of sh or colors_precomp", colors_precomp=torch.zeros(4, 3))
    _raises("provide exactly one of sh or colors_precomp", sh=torch.empty(0))
    _raises("provide exactly one of scales/rotations or cov3Ds_precomp", rotations=torch.empty(0))
    _raises("provide exactly one of scales/rotations or cov3Ds_precomp", cov3Ds_precomp=torch.zeros(4, 6))
    _raises("provide exactly one of scales/rotations or cov3Ds_precomp", scales=torch.empty(0),
            rotations=torch.empty(0))
    _raises("colors_precomp must have shape (4, 3), got (4, 4)", sh=torch.empty(0), colors_precomp=torch.zeros(4, 4))
    _raises("scales must have shape (4, 3), got (3, 3)", scales=torch.zeros(3, 3))
    _raises("rotations must have shape (4, 4), got (4, 3)", rotations=torch.zeros(4, 3))
    _raises("cov3Ds_precomp must have shape (4, 6), got (4, 9)", scales=torch.empty(0), rotations=torch.empty(0),
            cov3Ds_precomp=torch.zeros(4, 9))
    _raises("sh must contain a whole number of RGB coefficients per Gaussian", sh=torch.zeros(4, 5))
    _raises("sh does not contain enough coefficients for sh_degree", raster_settings=_settings(sh_degree=1))
    # shapes come after exclusivity: both wrong, exclusivity is reported
    _raises("provide exactly one of sh or colors_precomp", colors_precomp=torch.zeros(4, 4))


def test_debug_finite_checks_in_order():
    bad = torch.zeros(4, 3)
    bad[1, 2] = float("nan")
    _raises("means2D contains NaN or Inf values", means2D=bad, raster_settings=_settings(debug=True))
    scales = torch.ones(4, 3)
    scales[0, 0] = float("inf")
    _raises("scales contains NaN or Inf values", scales=scales, raster_settings=_settings(debug=True))
    # without debug the values are not inspected
    _validation.validate_rasterizer_inputs(**_args(means2D=bad, scales=scales))
    # the first non-finite input in the reference's order is reported
    _raises("means2D contains NaN or Inf values", means2D=bad, scales=scales, raster_settings=_settings(debug=True))
