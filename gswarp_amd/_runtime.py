"""Module-level rasterizer options and their per-call immutable snapshot.

Mirrors gswarp/_internal/backends/warp/runtime.py:32-100 and 443-471 and
gswarp/_internal/api/runtime_context.py:12-36: module defaults (backward
mode "manual", sort mode "warp_depth_stable_tile", coverage "auto", depth
on unless GSWARP_COMPUTE_DEPTH=0), per-call settings override them, and one
frozen ``ExecutionOptions`` is bound to a forward and reused by its backward.
The flow variant adds compute_flow_aux (GSWARP_COMPUTE_FLOW_AUX) and the
top-K count (GSWARP_FLOW_TOPK, default 20) of flow_ops.py:42-59.

The three sort-mode names select how the (tile, depth, index) order of the
pairs is produced (gswarp_amd/_pipeline.py:binning); every one gives the
reference's lists bit for bit.
"""

from __future__ import annotations

import os
from contextlib import contextmanager
from contextvars import ContextVar
from dataclasses import dataclass

from ._coverage import check_mode_name, kernel_mode

BINNING_SORT_MODES = ("warp_radix", "torch", "warp_depth_stable_tile")
DEFAULT_BACKWARD_MODE = "manual"
DEFAULT_BINNING_SORT_MODE = "warp_depth_stable_tile"
DEFAULT_TILE_COVERAGE_MODE = "auto"

_BACKWARD_MODE = DEFAULT_BACKWARD_MODE
_BINNING_SORT_MODE = DEFAULT_BINNING_SORT_MODE
_TILE_COVERAGE_MODE = DEFAULT_TILE_COVERAGE_MODE
_COMPUTE_DEPTH = os.environ.get("GSWARP_COMPUTE_DEPTH", "1") != "0"
_COMPUTE_FLOW_AUX = os.environ.get("GSWARP_COMPUTE_FLOW_AUX", "1") != "0"
_FLOW_TOPK = int(os.environ.get("GSWARP_FLOW_TOPK", "20"))


@dataclass(frozen=True, slots=True)
class ExecutionOptions:
    """Immutable runtime choices owned by one frontend invocation."""

    backward_mode: str
    binning_sort_mode: str
    tile_coverage_mode: str
    compute_depth: bool
    auto_tune: bool
    auto_tune_verbose: bool
    compute_flow_aux: bool | None = None
    flow_topk: int | None = None


_ACTIVE: ContextVar[ExecutionOptions | None] = ContextVar("gswarp_amd_active_execution_options", default=None)


@contextmanager
def execution_options(options: ExecutionOptions):
    token = _ACTIVE.set(options)
    try:
        yield options
    finally:
        _ACTIVE.reset(token)


def active_options() -> ExecutionOptions | None:
    return _ACTIVE.get()


def get_backward_mode() -> str:
    return _BACKWARD_MODE


def set_backward_mode(mode: str) -> None:
    global _BACKWARD_MODE
    if mode != "manual":
        raise ValueError("mode must be 'manual'")
    _BACKWARD_MODE = mode


def get_binning_sort_mode() -> str:
    return _BINNING_SORT_MODE


def set_binning_sort_mode(mode: str) -> None:
    global _BINNING_SORT_MODE
    if mode not in BINNING_SORT_MODES:
        raise ValueError("mode must be one of 'torch', 'warp_radix', or 'warp_depth_stable_tile'")
    _BINNING_SORT_MODE = mode


def get_tile_coverage_mode() -> str:
    return _TILE_COVERAGE_MODE


def set_tile_coverage_mode(mode: str) -> None:
    global _TILE_COVERAGE_MODE
    _TILE_COVERAGE_MODE = check_mode_name(mode)


def get_compute_depth() -> bool:
    return _COMPUTE_DEPTH


def set_compute_depth(enabled: bool) -> None:
    global _COMPUTE_DEPTH
    _COMPUTE_DEPTH = bool(enabled)


def get_compute_flow_aux() -> bool:
    return _COMPUTE_FLOW_AUX


def set_compute_flow_aux(enabled: bool) -> None:
    global _COMPUTE_FLOW_AUX
    _COMPUTE_FLOW_AUX = bool(enabled)


def get_flow_topk() -> int:
    return _FLOW_TOPK


def set_flow_topk(k: int) -> None:
    global _FLOW_TOPK
    if int(k) <= 0:
        raise ValueError("flow_topk must be positive")
    _FLOW_TOPK = int(k)


def resolve_execution_options(raster_settings, *, flow: bool = False, exact_conic: bool = True) -> ExecutionOptions:
    """Merge module defaults and per-call settings into an immutable snapshot.

    exact_conic: the method's footprint is the screen-space conic (true for
    every method of this package), so "auto" coverage means accutile_sweep."""
    backward_mode = getattr(raster_settings, "backward_mode", None)
    binning_sort_mode = getattr(raster_settings, "binning_sort_mode", None)
    compute_flow_aux = getattr(raster_settings, "compute_flow_aux", None) if flow else None
    return ExecutionOptions(
        backward_mode=_BACKWARD_MODE if backward_mode is None else backward_mode,
        binning_sort_mode=_BINNING_SORT_MODE if binning_sort_mode is None else binning_sort_mode,
        tile_coverage_mode=kernel_mode(_TILE_COVERAGE_MODE, exact_conic=exact_conic).public_name,
        compute_depth=_COMPUTE_DEPTH,
        auto_tune=bool(getattr(raster_settings, "auto_tune", True)),
        auto_tune_verbose=bool(getattr(raster_settings, "auto_tune_verbose", True)),
        compute_flow_aux=(_COMPUTE_FLOW_AUX if compute_flow_aux is None else bool(compute_flow_aux)) if flow else None,
        flow_topk=_FLOW_TOPK if flow else None,
    )


def get_default_parameter_info() -> dict:
    """Compile-time and default parameters of this build."""
    return {
        "BLOCK_X": {"value": 16, "category": "kernel_tile", "auto_tunable": False,
                    "description": "Tile width of the render kernels (pixels)."},
        "BLOCK_Y": {"value": 16, "category": "kernel_tile", "auto_tunable": False,
                    "description": "Tile height of the render kernels (pixels)."},
        "DEFAULT_BACKWARD_MODE": {"value": DEFAULT_BACKWARD_MODE, "category": "mode", "auto_tunable": False,
                                  "description": "Only the manual backward is implemented."},
        "DEFAULT_BINNING_SORT_MODE": {"value": DEFAULT_BINNING_SORT_MODE, "category": "mode", "auto_tunable": False,
                                      "description": "Packed 64-bit keys below 4 pairs per Gaussian, depth then tile above."},
        "DEFAULT_TILE_COVERAGE_MODE": {"value": DEFAULT_TILE_COVERAGE_MODE, "category": "mode",
                                       "auto_tunable": False, "description": "auto resolves to accutile_sweep."},
        "WORKGROUP_SIZE": {"value": 256, "category": "launch", "auto_tunable": False,
                           "description": "Threads per workgroup (four wave64) of every kernel."},
    }
