"""Checks on the public rasterizer inputs, run on the host before any launch.

The errors are the reference's interface (gswarp/_internal/api/validation.py:
22-202): ValueError with the same messages, raised in the same order, so
that the first problem a caller has is reported as the reference reports it.
The checks are written here as a table of tensor specifications walked in
stages:

1. the three per-Gaussian tensors exist, means3D is on a GPU; it fixes the
   device and N;
2. means3D / means2D / opacities: placement (device, float32) and shape;
3. the settings: scalar fields, then the four settings tensors;
4. the optional inputs: placement when non-empty;
5. which optional inputs were given (exactly one colour source and one
   covariance source when N > 0), then their shapes;
6. with ``raster_settings.debug``, finiteness of every tensor.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import NamedTuple

import torch

INT32_MAX = 2**31 - 1
N = None  # the Gaussian count in a shape specification


class GaussianInputs(NamedTuple):
    """The optional inputs after normalisation; an absent one is an empty tensor."""

    shs: torch.Tensor
    colors_precomp: torch.Tensor
    scales: torch.Tensor
    rotations: torch.Tensor
    cov3D_precomp: torch.Tensor


def _error(message: str):
    raise ValueError(message)


@dataclass(frozen=True)
class Spec:
    """A tensor input: the name used in messages and its shape (N = Gaussian count)."""

    name: str
    shape: tuple | None = None  # None: no fixed shape

    def as_tensor(self, value) -> torch.Tensor:
        if not isinstance(value, torch.Tensor):
            _error(f"{self.name} must be a torch.Tensor")
        return value

    def check_placement(self, value: torch.Tensor, device: torch.device) -> None:
        if value.device != device:
            _error(f"{self.name} must be on {device}, got {value.device}")
        if value.dtype != torch.float32:
            _error(f"{self.name} must have dtype torch.float32, got {value.dtype}")

    def check_shape(self, value: torch.Tensor, count: int | None = None) -> None:
        """Shape check; N dims must equal count, or are free (shown as "N") without one."""
        want = tuple(count if d is N else d for d in self.shape)
        fits = value.ndim == len(want) and all(w is None or a == w for a, w in zip(value.shape, want))
        if not fits:
            shown = tuple("N" if d is None else d for d in want)
            _error(f"{self.name} must have shape {shown}, got {tuple(value.shape)}")

    def check_finite(self, value: torch.Tensor) -> None:
        if value.numel() and not bool(torch.isfinite(value).all()):
            _error(f"{self.name} contains NaN or Inf values")


MEANS3D = Spec("means3D", (N, 3))
MEANS2D = Spec("means2D", (N, 3))
OPACITIES = Spec("opacities")
SETTINGS_TENSORS = (Spec("raster_settings.bg", (3,)), Spec("raster_settings.viewmatrix", (4, 4)),
                    Spec("raster_settings.projmatrix", (4, 4)), Spec("raster_settings.campos", (3,)))
SH = Spec("sh")
COLORS = Spec("colors_precomp", (N, 3))
SCALES = Spec("scales", (N, 3))
ROTATIONS = Spec("rotations", (N, 4))
COV3D = Spec("cov3Ds_precomp", (N, 6))
OPTIONAL = (SH, COLORS, SCALES, ROTATIONS, COV3D)
_SETTINGS_SCALARS = ("image_height", "image_width", "tanfovx", "tanfovy", "scale_modifier", "sh_degree")


def _settings_values(raster_settings) -> tuple[dict, list[torch.Tensor]]:
    """The scalar fields and the four tensors of the settings (stage 3's reads)."""
    try:
        scalars = {field: getattr(raster_settings, field) for field in _SETTINGS_SCALARS}
        tensors = [spec.as_tensor(getattr(raster_settings, spec.name.split(".", 1)[1]))
                   for spec in SETTINGS_TENSORS]
    except AttributeError as exc:
        raise ValueError("raster_settings is missing a required field") from exc
    return scalars, tensors


def _check_scalars(s: dict) -> None:
    h, w = s["image_height"], s["image_width"]
    if not (isinstance(h, int) and isinstance(w, int) and h > 0 and w > 0):
        _error("image_height and image_width must be positive integers")
    if h * w > INT32_MAX:
        _error("image_height * image_width must fit in a signed 32-bit index")
    if not all(math.isfinite(float(s[k])) and float(s[k]) > 0.0 for k in ("tanfovx", "tanfovy", "scale_modifier")):
        _error("tanfovx, tanfovy, and scale_modifier must be finite and positive")
    if not isinstance(s["sh_degree"], int) or s["sh_degree"] < 0:
        _error("sh_degree must be a non-negative integer")


def _check_sources(count: int, given: dict) -> None:
    """Exactly one colour source and one covariance source (stage 5)."""
    if count == 0:
        return
    if given["sh"] == given["colors_precomp"]:
        _error("provide exactly one of sh or colors_precomp")
    if given["scales"] != given["rotations"] or given["scales"] == given["cov3Ds_precomp"]:
        _error("provide exactly one of scales/rotations or cov3Ds_precomp")


def _check_sh(sh: torch.Tensor, count: int, degree: int) -> None:
    per_gaussian, rest = divmod(sh.numel(), 3 * count) if count else (0, sh.numel())
    if rest:
        _error("sh must contain a whole number of RGB coefficients per Gaussian")
    if per_gaussian < (degree + 1) ** 2:
        _error("sh does not contain enough coefficients for sh_degree")


def validate_rasterizer_inputs(means3D, means2D, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp,
                               raster_settings) -> None:
    """Raise ValueError for the first input the reference would reject."""
    means3D, means2D, opacities = (spec.as_tensor(v) for spec, v in
                                   ((MEANS3D, means3D), (MEANS2D, means2D), (OPACITIES, opacities)))
    if not means3D.is_cuda:
        _error("means3D must be a CUDA tensor")
    device = means3D.device
    MEANS3D.check_placement(means3D, device)
    MEANS3D.check_shape(means3D)
    count = means3D.shape[0]
    if count > INT32_MAX:
        _error("the Gaussian count must fit in a signed 32-bit index")
    MEANS2D.check_placement(means2D, device)
    MEANS2D.check_shape(means2D, count)
    OPACITIES.check_placement(opacities, device)
    if opacities.numel() != count:
        _error(f"opacities must contain one value per Gaussian ({count}), got {opacities.numel()}")

    scalars, settings_tensors = _settings_values(raster_settings)
    _check_scalars(scalars)
    for spec, value in zip(SETTINGS_TENSORS, settings_tensors):
        spec.check_placement(value, device)
        spec.check_shape(value, count)

    optional = []
    for spec, value in zip(OPTIONAL, (sh, colors_precomp, scales, rotations, cov3Ds_precomp)):
        optional.append(spec.as_tensor(value))
        if value.numel():
            spec.check_placement(value, device)
    given = {spec.name: value.numel() != 0 for spec, value in zip(OPTIONAL, optional)}
    _check_sources(count, given)
    for spec, value in zip(OPTIONAL[1:], optional[1:]):
        if given[spec.name]:
            spec.check_shape(value, count)
    if given["sh"]:
        _check_sh(optional[0], count, scalars["sh_degree"])

    if getattr(raster_settings, "debug", False):
        for spec, value in ((MEANS3D, means3D), (MEANS2D, means2D), (OPACITIES, opacities),
                            *zip(SETTINGS_TENSORS, settings_tensors), *zip(OPTIONAL, optional)):
            spec.check_finite(value)


def normalize_gaussian_inputs(*, dc, shs, colors_precomp, scales, rotations, cov3D_precomp) -> GaussianInputs:
    """Join the SH DC band onto the rest (dim 1) and replace absent inputs by empty tensors.

    Exactly one colour source (SH or precomputed colours) and one covariance
    source (scales with rotations, or precomputed covariances) must be given.
    """
    if dc is not None:
        shs = dc if shs is None else torch.cat([dc, shs], dim=1)
    if (shs is None) == (colors_precomp is None):
        _error("provide exactly one of shs or colors_precomp")
    has_scale_rotation = scales is not None and rotations is not None
    has_any_scale_rotation = scales is not None or rotations is not None
    if has_scale_rotation == (cov3D_precomp is not None) or has_any_scale_rotation == (cov3D_precomp is not None):
        _error("provide exactly one of scales/rotations or cov3D_precomp")
    empty = torch.Tensor([])
    return GaussianInputs(*(empty if v is None else v for v in (shs, colors_precomp, scales, rotations,
                                                               cov3D_precomp)))
