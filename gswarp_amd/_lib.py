"""ctypes binding of ``libgswarp_hip.so`` (declared in include/gswarp_hip.h).

The library is the only compute path: if it cannot be loaded, every
rasterizer call raises ``RuntimeError`` — there is no CPU or eager fallback.
"""

from __future__ import annotations

import atexit
import ctypes
import os
import threading
from pathlib import Path

# GSWARP_AMD_LIB selects another build of the same library (e.g. one compiled
# with different pixels-per-lane settings).
LIB_PATH = Path(os.environ.get("GSWARP_AMD_LIB", Path(__file__).resolve().parent / "libgswarp_hip.so"))

GS_OK = 0
GS_RECORD_FLOATS = 12
GS_GRAD_FLOATS = 10

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); must match include/gswarp_hip.h
SIGNATURES = {
    "gs_version": (ctypes.c_int, []),
    "gs_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "gs_preprocess_fwd": (
        ctypes.c_int,
        [_i32, _i32, _i32, _vp, _vp, _vp, _vp, _f32, _vp, _vp, _vp, _vp, _vp, _vp, _f32, _f32, _f32, _f32, _i32,
         _i32, _i32, _f32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _sz, _vp],
    ),
    "gs_band_store_words": (_i64, [_i32]),
    "gs_mark_visible": (ctypes.c_int, [_i32, _vp, _vp, _vp, _vp]),
    "gs_count_tiles": (ctypes.c_int, [_i32, _vp, _vp, _vp, _i32, _i32, _i32, _vp, _vp, _vp]),
    "gs_scan_scratch_bytes": (_sz, [_i32]),
    "gs_depth_keys": (ctypes.c_int, [_i32, _vp, _vp, _vp, _vp, _vp]),
    "gs_scan_tiles": (ctypes.c_int, [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "gs_scan_tiles_static_max_points": (_i32, []),
    "gs_scan_tiles_static": (ctypes.c_int, [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "gs_readback_slot_bytes": (_sz, []),
    "gs_num_rendered_readback": (ctypes.c_int, [_vp, _vp, _i64, _vp]),
    "gs_scan_tiles_entries": (ctypes.c_int, [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "gs_info_readback": (ctypes.c_int, [_vp, _vp, _i64, _i32, _vp]),
    "gs_scan_state_bytes": (_sz, [_i32]),
    "gs_scan_state_status_offset": (_i64, [_i32]),
    "gs_scan_state_status_words": (_i64, [_i32]),
    "gs_scan_state_prepare": (ctypes.c_int, [_i32, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "gs_scan_tiles_onepass": (ctypes.c_int, [_i32, _vp, _vp, _vp, _vp, _sz, _i32, _i32, _vp]),
    "gs_bin_buckets_workspace_bytes": (_sz, [_i32, _i32, _i64, _i32, _i32]),
    "gs_bin_buckets": (ctypes.c_int, [_i32, _i32, _i64, _i64, _vp, ctypes.c_uint32, ctypes.c_uint32, _vp, _vp, _vp,
                                      _i32, _i32, _vp, _sz, _vp, _vp, _vp, _vp]),
    "gs_duplicate_keys": (
        ctypes.c_int,
        [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i64, ctypes.c_uint32, _i32, _i32, _vp, _vp, _vp],
    ),
    "gs_duplicate_tiles": (
        ctypes.c_int, [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i64, _vp, _vp, _vp],
    ),
    "gs_sort_num_passes": (ctypes.c_int, [_i32]),
    "gs_sort_scratch_bytes": (_sz, [_i64]),
    "gs_sort_pairs_u64": (ctypes.c_int, [_i64, _i32, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "gs_sort_keys_u64": (ctypes.c_int, [_i64, _i32, _i32, _vp, _vp, _vp, _sz, _vp]),
    "gs_sort_pairs_u32": (ctypes.c_int, [_i64, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "gs_tile_ranges": (ctypes.c_int, [_i64, _vp, _i32, _i32, _i32, _vp, _vp, _vp]),
    "gs_tile_ranges_u32": (ctypes.c_int, [_i64, _vp, _i32, _vp, _vp]),
    "gs_sort_tile_segments": (ctypes.c_int, [_i64, _vp, _vp, _i32, _vp, _i32, _i32, _i32, _vp, _i32, _vp]),
    "gs_bin_packed_workspace_bytes": (ctypes.c_size_t, [_i64]),
    "gs_readback_bin_packed": (ctypes.c_int, [_vp, _vp, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32,
                                              _i64, _vp, _sz, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _i64,
                                              _vp, _vp, _vp, _vp]),
    "gs_bin_packed": (ctypes.c_int, [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i64, ctypes.c_uint32,
                                     _i32, _i32, _vp, _sz, _vp, _vp, _vp, _vp, _vp]),
    "gs_tile_order": (ctypes.c_int, [_i32, _vp, _vp, _vp]),
    "gs_render_fwd": (ctypes.c_int, [_i32, _i32, _i32, _i64, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp]),
    "gs_render_fwd_clear": (
        ctypes.c_int, [_i32, _i32, _i32, _i64, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp]),
    "gs_render_fwd_flow": (
        ctypes.c_int,
        [_i32, _i32, _i32, _i64, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
    ),
    "gs_render_bwd": (
        ctypes.c_int, [_i32, _i32, _i32, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp],
    ),
    "gs_preprocess_bwd": (
        ctypes.c_int,
        [_i32, _i32, _i32, _vp, _vp, _vp, _vp, _f32, _vp, _vp, _vp, _vp, _f32, _f32, _f32, _f32, _vp, _vp, _vp, _vp,
         _i32, _i32, _vp, _vp, _vp, _i32, _f32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
    ),
}

_lock = threading.Lock()
_handle = None


class _Lib:
    """Loaded library whose gs_* calls raise RuntimeError on a non-zero status."""

    def __init__(self, handle: ctypes.CDLL):
        self.handle = handle
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes

    def status_string(self, status: int) -> str:
        return self.handle.gs_status_string(int(status)).decode()

    def call(self, name: str, *args):
        status = getattr(self.handle, name)(*args)
        if status != GS_OK:
            raise RuntimeError(f"{name} failed with status {status}: {self.status_string(status)}")
        return status

    def __getattr__(self, name: str):
        return getattr(self.handle, name)


def _synchronize_at_exit() -> None:
    """Wait for the work of every device the rasterizer ran on before the
    interpreter exits, so that none of the library's kernels is still running
    when the process tears down the HIP runtime and unregisters the library's
    code objects (the reference synchronises before a workspace is evicted or
    cleared, gswarp/_internal/backends/warp/memory.py:209-230, 381-385)."""
    from . import _workspace

    try:
        import torch

        if torch.cuda.is_initialized():
            for index in sorted(_workspace.used_devices()):
                torch.cuda.synchronize(index)
    except Exception:  # a device already in an error state has nothing left to wait for
        pass


def load() -> _Lib:
    """Load the HIP library; raises RuntimeError when it is not built."""
    global _handle
    if _handle is None:
        with _lock:
            if _handle is None:
                if not LIB_PATH.exists():
                    raise RuntimeError(
                        f"{LIB_PATH.name} is not built; run `python -m gswarp_amd._build` "
                        "(hipcc, gfx950) before using the rasterizer"
                    )
                _handle = _Lib(ctypes.CDLL(str(LIB_PATH)))
                atexit.register(_synchronize_at_exit)
    return _handle


def preload() -> None:
    """Load the library at package import when it is built (a missing or
    stale library raises at the first call instead).  Loaded then, before any GPU work, its
    code objects are registered with the HIP runtime in the same order as
    torch's own kernels, and unregistered after the runtime's exit handlers as
    theirs are, rather than by a library that a first call loaded after the
    GPU was initialised."""
    import torch  # noqa: F401  (its HIP runtime must be the one the library binds to)

    if LIB_PATH.exists():
        try:
            load()
        except (AttributeError, OSError):
            # A library built from other sources (a symbol missing) or not
            # loadable: the package still imports, so that it can be rebuilt,
            # and the first call raises the same error again.
            pass


def ptr(tensor) -> int | None:
    """Raw device address of a tensor (None for an absent optional input)."""
    if tensor is None:
        return None
    return tensor.data_ptr()
