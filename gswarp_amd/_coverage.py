"""Tile-coverage modes of the binning stage.

Each public name selects one of the coverage routines compiled into
libgswarp_hip.so (the ``coverage_mode`` argument, ``GS_COVERAGE_*`` in
include/gswarp_hip.h):

  ``snugbox``         0  the Gaussian's alpha-cut-off box, intersected with its
                         3-sigma tile rectangle: every tile of that box;
  ``accutile_sweep``  1  the exact interval of the cut-off ellipse in each tile
                         row (or column) of the box;
  ``conic_rect``      2  an ellipse/tile test per tile of boxes of at most 64
                         tiles, the row/column intervals beyond that.

``auto`` means accutile_sweep for a splat whose footprint is exactly the EWA
screen-space conic sampled at pixel centres with the 3-sigma clamp (every
method this package provides), and snugbox for any other footprint, for which
only the conservative box is safe; the two exact modes are refused there.
The public names, their ids and the auto rule are the reference's interface
(gswarp/_internal/coverage.py:94-110, test_tile_coverage.py:167-230).
"""

from __future__ import annotations

import enum


class CoverageMode(enum.IntEnum):
    """Kernel id of a concrete coverage mode."""

    SNUGBOX = 0
    ACCUTILE_SWEEP = 1
    CONIC_RECT = 2

    @property
    def public_name(self) -> str:
        return self.name.lower()

    @classmethod
    def from_public_name(cls, name: str) -> "CoverageMode":
        return cls[name.upper()]


PUBLIC_NAMES = ("auto",) + tuple(mode.public_name for mode in CoverageMode)


def check_mode_name(name: str) -> str:
    """Validate a public mode name (set_tile_coverage_mode's check)."""
    if name not in PUBLIC_NAMES:
        raise ValueError("mode must be one of " + ", ".join(repr(n) for n in PUBLIC_NAMES))
    return name


def kernel_mode(name: str, *, exact_conic: bool = True) -> CoverageMode:
    """The concrete mode a public name selects for a footprint.

    exact_conic: the splat's footprint is the screen-space conic itself, so the
    culling modes that test tiles against the ellipse are exact for it.
    """
    check_mode_name(name)
    if name == "auto":
        return CoverageMode.ACCUTILE_SWEEP if exact_conic else CoverageMode.SNUGBOX
    mode = CoverageMode.from_public_name(name)
    if mode is not CoverageMode.SNUGBOX and not exact_conic:
        raise ValueError(f"tile coverage mode {name!r} culls tiles against the screen-space conic; "
                         "a footprint other than that conic allows only 'snugbox'")
    return mode
