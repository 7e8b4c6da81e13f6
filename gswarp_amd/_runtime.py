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
import threading
from contextlib import contextmanager
from typing import NamedTuple

from ._coverage import check_mode_name, kernel_mode

BINNING_SORT_MODES = ("warp_radix", "torch", "warp_depth_stable_tile")
DEFAULT_BACKWARD_MODE = "manual"
DEFAULT_BINNING_SORT_MODE = "warp_depth_stable_tile"
DEFAULT_TILE_COVERAGE_MODE = "auto"


class _ModuleDefaults:
    """The process-wide values the getters read and the setters change;
    environment variables give the start values of the two flags and K."""

    def __init__(self) -> None:
        self.backward_mode = DEFAULT_BACKWARD_MODE
        self.binning_sort_mode = DEFAULT_BINNING_SORT_MODE
        self.tile_coverage_mode = DEFAULT_TILE_COVERAGE_MODE
        self.compute_depth = os.environ.get("GSWARP_COMPUTE_DEPTH", "1") != "0"
        self.compute_flow_aux = os.environ.get("GSWARP_COMPUTE_FLOW_AUX", "1") != "0"
        self.flow_topk = int(os.environ.get("GSWARP_FLOW_TOPK", "20"))


_defaults = _ModuleDefaults()


class ExecutionOptions(NamedTuple):
    """The option values a rasterizer call runs with: the module values
    merged with the call's settings when the forward starts, then handed
    unchanged to the backward of the same call, so that setters used in
    between change neither.  Flow fields are None for the standard path."""

    backward_mode: str
    binning_sort_mode: str
    tile_coverage_mode: str
    compute_depth: bool
    auto_tune: bool
    auto_tune_verbose: bool
    compute_flow_aux: bool | None = None
    flow_topk: int | None = None


class _ScopeStack(threading.local):
    """Per thread, the options of the calls in progress, innermost last."""

    def __init__(self) -> None:
        self.frames: list[ExecutionOptions] = []


_scopes = _ScopeStack()


@contextmanager
def execution_options(options: ExecutionOptions):
    """Run the body with ``options`` as this thread's innermost call options
    (what a raw-ABI call made inside it resolves to)."""
    _scopes.frames.append(options)
    try:
        yield options
    finally:
        _scopes.frames.pop()


def active_options() -> ExecutionOptions | None:
    """This thread's innermost call options, or None outside any call."""
    frames = _scopes.frames
    return frames[-1] if frames else None


def get_backward_mode() -> str:
    return _defaults.backward_mode


def set_backward_mode(mode: str) -> None:
    if mode != "manual":
        raise ValueError("mode must be 'manual'")
    _defaults.backward_mode = mode


def get_binning_sort_mode() -> str:
    return _defaults.binning_sort_mode


def set_binning_sort_mode(mode: str) -> None:
    if mode not in BINNING_SORT_MODES:
        raise ValueError("mode must be one of 'torch', 'warp_radix', or 'warp_depth_stable_tile'")
    _defaults.binning_sort_mode = mode


def get_tile_coverage_mode() -> str:
    return _defaults.tile_coverage_mode


def set_tile_coverage_mode(mode: str) -> None:
    _defaults.tile_coverage_mode = check_mode_name(mode)


def get_compute_depth() -> bool:
    return _defaults.compute_depth


def set_compute_depth(enabled: bool) -> None:
    _defaults.compute_depth = bool(enabled)


def get_compute_flow_aux() -> bool:
    return _defaults.compute_flow_aux


def set_compute_flow_aux(enabled: bool) -> None:
    _defaults.compute_flow_aux = bool(enabled)


def get_flow_topk() -> int:
    return _defaults.flow_topk


def set_flow_topk(k: int) -> None:
    if int(k) <= 0:
        raise ValueError("flow_topk must be positive")
    _defaults.flow_topk = int(k)


def resolve_execution_options(raster_settings, *, flow: bool = False, exact_conic: bool = True) -> ExecutionOptions:
    """The options of one call: a settings field that is present and not
    None wins over the module value.

    exact_conic: the method's footprint is the screen-space conic (true for
    every method of this package), so "auto" coverage means accutile_sweep."""
    d = _defaults

    def setting(name, default):
        value = getattr(raster_settings, name, None)
        return default if value is None else value

    return ExecutionOptions(
        backward_mode=setting("backward_mode", d.backward_mode),
        binning_sort_mode=setting("binning_sort_mode", d.binning_sort_mode),
        tile_coverage_mode=kernel_mode(d.tile_coverage_mode, exact_conic=exact_conic).public_name,
        compute_depth=d.compute_depth,
        auto_tune=bool(setting("auto_tune", True)),
        auto_tune_verbose=bool(setting("auto_tune_verbose", True)),
        compute_flow_aux=bool(setting("compute_flow_aux", d.compute_flow_aux)) if flow else None,
        flow_topk=d.flow_topk if flow else None,
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
