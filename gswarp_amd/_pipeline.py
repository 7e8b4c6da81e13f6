"""Host orchestration of the rasterizer stages on the current HIP stream.

Stage order and semantics follow the reference pipeline
(gswarp/_internal/methods/pipeline.py:11-45): empty scene -> preprocess ->
binning -> features -> render -> state, and the manual backward of
gswarp/_internal/backends/warp/backward_ops.py:376-746 (flow variant:
flow_ops.py:196-512).  Every stage allocates its tensors with torch on the
input's device and enqueues the gfx950 kernels through the C ABI on
``torch.cuda.current_stream(device)``; the only host synchronisation is the
pair-count readback of the binning stage.
"""

from __future__ import annotations

import contextlib
import ctypes
from dataclasses import dataclass

import torch

from . import _lib, _packing, _workspace
from ._coverage import kernel_mode
from ._runtime import BINNING_SORT_MODES, ExecutionOptions
from ._state import (BinningState, ForwardResult, ForwardState, KeyLayout, PreprocessOutputs, RenderImages,
                     RenderStageResult)

BLOCK_X = 16
BLOCK_Y = 16
NUM_CHANNELS = 3
MAX_BINNING_PAIRS = (1 << 31) - 1

# Optional per-stage timer: a callable(stage_name) returning a context
# manager that brackets the stage's launches (used by bench.py to record
# HIP events on the launch stream).  None disables it.
STAGE_TIMER = None

# The autograd forward allocates the backward's (N, 10) gradient accumulator
# and has its render zero it (gs_render_fwd_clear), which spares the backward
# a fill launch; the buffer (40 B per Gaussian) is then held from the forward
# until its backward.  A loop that runs several forwards before one backward
# holds one per pending forward: with False the backward allocates and fills
# its own, one at a time.
ACCUMULATOR_IN_FORWARD = True


def _stage(name: str):
    timer = STAGE_TIMER
    return timer(name) if timer is not None else contextlib.nullcontext()


def _stage_chain(names):
    """Raw event handles (a ctypes array) bracketing consecutive stages inside
    one C call, when the stage timer offers them; None otherwise."""
    timer = STAGE_TIMER
    if timer is None or not hasattr(timer, "chain"):
        return None
    return timer.chain(names)


@dataclass(slots=True)
class RasterInputs:
    """The 18-argument forward tuple of the reference raw ABI, typed."""

    background: torch.Tensor
    means3d: torch.Tensor
    colors: torch.Tensor
    opacities: torch.Tensor
    scales: torch.Tensor
    rotations: torch.Tensor
    scale_modifier: float
    cov3d_precomp: torch.Tensor
    viewmatrix: torch.Tensor
    projmatrix: torch.Tensor
    tan_fovx: float
    tan_fovy: float
    image_height: int
    image_width: int
    sh: torch.Tensor
    degree: int
    campos: torch.Tensor
    prefiltered: bool
    # Mip-Splatting screen-space variance, the Mip method's 19th forward
    # argument (mip_autograd.py:51-71); 0 for the standard rasterizer.
    filter_variance: float = 0.0

    @classmethod
    def from_args(cls, args) -> "RasterInputs":
        return cls(*args)


def validate_pair_count(value: int) -> int:
    """binning_ops.py:75-81."""
    if value < 0 or value > MAX_BINNING_PAIRS:
        raise OverflowError(
            "binning tile-reference count exceeds signed int32; reduce Gaussian footprint or image size"
        )
    return value


def grid_dims(width: int, height: int) -> tuple[int, int]:
    return (width + BLOCK_X - 1) // BLOCK_X, (height + BLOCK_Y - 1) // BLOCK_Y


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _f32c(t: torch.Tensor, align16: bool = False) -> torch.Tensor:
    t = t.detach()
    if t.dtype != torch.float32:
        t = t.to(torch.float32)
    t = t.contiguous()
    if align16 and t.numel() and t.data_ptr() % 16:
        t = t.clone()
    return t


def _focal(size: int, tanfov: float) -> float:
    return size / (2.0 * tanfov)


def empty_forward(inputs: RasterInputs, flow_aux_k: int | None = None) -> ForwardResult:
    """N == 0: background image and zeros (preprocess_ops.py:45-71, flow_ops.py:62-106)."""
    device = inputs.means3d.device
    H, W, n = inputs.image_height, inputs.image_width, inputs.means3d.shape[0]
    bg = inputs.background.to(device=device, dtype=torch.float32).reshape(NUM_CHANNELS, 1, 1)
    aux: tuple[torch.Tensor, ...] = ()
    if flow_aux_k is not None:
        aux = _empty_flow_aux(flow_aux_k, H, W, device)
    return ForwardResult(
        num_rendered=0,
        color=bg.expand(NUM_CHANNELS, H, W).clone(),
        depth=torch.zeros((1, H, W), dtype=torch.float32, device=device),
        alpha=torch.zeros((1, H, W), dtype=torch.float32, device=device),
        radii=torch.zeros((n,), dtype=torch.int32, device=device),
        proj_2d=torch.zeros((n, 2), dtype=torch.float32, device=device),
        conic_2d=torch.zeros((n, 3), dtype=torch.float32, device=device),
        conic_2d_inv=torch.zeros((n, 3), dtype=torch.float32, device=device),
        state=None,
        aux=aux,
    )


def _empty_flow_aux(k: int, H: int, W: int, device) -> tuple[torch.Tensor, ...]:
    if k <= 0:
        return (
            torch.empty((0,), dtype=torch.int32, device=device),
            torch.empty((0,), dtype=torch.float32, device=device),
            torch.empty((0,), dtype=torch.float32, device=device),
        )
    return (
        torch.full((k, H, W), -1, dtype=torch.int32, device=device),
        torch.zeros((k, H, W), dtype=torch.float32, device=device),
        torch.zeros((2, k, H, W), dtype=torch.float32, device=device),
    )


def _covariance_inputs(inputs: RasterInputs, P: int):
    """(scales, rotations, None) or (None, None, cov3D (P, 6)) as contiguous fp32, the
    two covariance sources of preprocess_ops.py:289-581."""
    if inputs.cov3d_precomp.numel() != 0:
        cov = _f32c(inputs.cov3d_precomp).reshape(-1)
        if cov.numel() != 6 * P:
            raise ValueError("cov3D_precomp must hold 6 values per Gaussian")
        return None, None, cov
    return _f32c(inputs.scales), _f32c(inputs.rotations, align16=True), None


def preprocess(inputs: RasterInputs, options: ExecutionOptions, *, pack: bool = False) -> PreprocessOutputs:
    """Fused projection / covariance / coverage / SH colour (preprocess_ops.py:289-581).
    With ``pack`` the records and clamp bits live in one raw-ABI geom buffer."""
    if inputs.prefiltered:
        raise NotImplementedError("prefiltered=True is not supported by the gfx950 preprocess path.")
    has_cov = inputs.cov3d_precomp.numel() != 0
    has_sr = inputs.scales.numel() != 0 and inputs.rotations.numel() != 0
    if has_cov == has_sr:
        raise ValueError("Provide exactly one of cov3D_precomp or scales/rotations")
    lib = _lib.load()
    means = inputs.means3d
    if means.ndim != 2 or means.shape[1] != 3:
        raise ValueError("means3D must have dimensions (num_points, 3)")
    device = means.device
    P = means.shape[0]
    W, H = inputs.image_width, inputs.image_height
    f = dict(dtype=torch.float32, device=device)
    if pack:
        geom, records, clamped = _packing.allocate_geom(P, device)
    else:
        geom = None
        records = torch.empty((P, _lib.GS_RECORD_FLOATS), **f)
        clamped = torch.empty((P,), dtype=torch.uint8, device=device)
    out = PreprocessOutputs(
        radii=torch.empty((P,), dtype=torch.int32, device=device),
        depths=torch.empty((P,), **f),
        proj_2d=torch.empty((P, 2), **f),
        conic_2d=torch.empty((P, 3), **f),
        conic_2d_inv=torch.empty((P, 3), **f),
        tiles_touched=torch.empty((P,), dtype=torch.int32, device=device),
        records=records,
        clamped=clamped,
        coverage_mode=int(kernel_mode(options.tile_coverage_mode)),
        geom=geom,
        coverage=torch.empty((P, 4), dtype=torch.int32, device=device),
    )
    if buckets_expected(options, W, H, P, device):
        # the bucketed binning reads the banded Gaussians' coverage bands instead of recomputing them
        out.band_store = torch.empty((max(int(lib.gs_band_store_words(P)), 1),), dtype=torch.int32, device=device)
    if SCAN_ONEPASS and P > 0:
        # the binning's one-pass scan state, which the preprocess prepares
        out.scan_state = torch.empty((int(lib.gs_scan_state_bytes(P)) // 8,), dtype=torch.int64, device=device)
    colors = _f32c(inputs.colors) if inputs.colors.numel() != 0 else None
    shs = None
    K = 0
    if colors is None:
        if inputs.sh.numel() == 0:
            raise ValueError("provide exactly one of sh or colors_precomp")
        shs = _f32c(inputs.sh).reshape(P, -1, NUM_CHANNELS)
        K = shs.shape[1]
    tanfovx, tanfovy = float(inputs.tan_fovx), float(inputs.tan_fovy)
    # Locals keep every converted input alive until the launch is enqueued.
    means_c = _f32c(means)
    scales_c, rot_c, cov_c = _covariance_inputs(inputs, P)
    opac_c = _f32c(inputs.opacities)
    view_c = _f32c(inputs.viewmatrix)
    proj_c = _f32c(inputs.projmatrix)
    campos_c = _f32c(inputs.campos)
    with _stage("preprocess"):
        lib.call(
            "gs_preprocess_fwd", P, K, int(inputs.degree), means_c.data_ptr(), _lib.ptr(scales_c),
            _lib.ptr(rot_c), _lib.ptr(cov_c), float(inputs.scale_modifier), opac_c.data_ptr(), _lib.ptr(shs),
            _lib.ptr(colors),
            view_c.data_ptr(), proj_c.data_ptr(), campos_c.data_ptr(), tanfovx, tanfovy, _focal(W, tanfovx),
            _focal(H, tanfovy), W, H, out.coverage_mode, float(inputs.filter_variance), out.radii.data_ptr(),
            out.depths.data_ptr(),
            out.proj_2d.data_ptr(), out.conic_2d.data_ptr(), out.conic_2d_inv.data_ptr(),
            out.tiles_touched.data_ptr(), out.coverage.data_ptr(), out.records.data_ptr(), out.clamped.data_ptr(),
            _lib.ptr(out.band_store), 0 if out.band_store is None else out.band_store.numel(),
            _lib.ptr(out.scan_state), 0 if out.scan_state is None else out.scan_state.numel() * 8, _stream(device))
    return out


def buckets_possible(options: ExecutionOptions, image_width: int, image_height: int) -> bool:
    """Whether the binning may take the bucketed dataflow: the default sort mode
    with it selected, on images of at most BUCKET_MAX_GRID tiles per side."""
    grid_x, grid_y = grid_dims(image_width, image_height)
    return (options.binning_sort_mode == "warp_depth_stable_tile" and HEAVY_DATAFLOW == "buckets"
            and grid_x <= BUCKET_MAX_GRID and grid_y <= BUCKET_MAX_GRID)


def buckets_expected(options: ExecutionOptions, image_width: int, image_height: int, num_points: int,
                     device: torch.device) -> bool:
    """Whether this forward prepares the bucketed binning (BUCKET_SIZING): the
    preprocess and the binning of one forward agree, since the device's pair
    count history only changes at the binning's read-back."""
    if not buckets_possible(options, image_width, image_height):
        return False
    return (BUCKET_SIZING == "always"
            or _workspace.last_pairs(device) > DEPTH_TILE_MIN_PAIRS_PER_GAUSSIAN * num_points)


def key_layout(P: int, T: int, depth_min: int, depth_max: int) -> KeyLayout:
    """Binning key fields: tile id above the visible depth range's bits above the
    packed point index; the index is carried separately when the three do not fit."""
    tile_bits = (T - 1).bit_length()
    depth_bits = (depth_max - depth_min).bit_length() if depth_max >= depth_min else 0
    value_bits = max(1, (P - 1).bit_length())
    if tile_bits + depth_bits + value_bits > 64:
        value_bits = 0
    return KeyLayout(depth_min=depth_min, depth_bits=depth_bits, value_bits=value_bits)


# How the packed-key dataflow orders its pairs: "segmented" sorts the keys
# stably by the tile field only and then each tile's segment by depth on chip
# (gs_sort_tile_segments); "full" runs the radix sort over tile and depth bits.
PACKED_SORT = "segmented"

# Above this many pairs per Gaussian the default mode sorts the Gaussians by
# depth and builds the tile lists from that order instead of sorting one
# 64-bit key per pair.
DEPTH_TILE_MIN_PAIRS_PER_GAUSSIAN = 4

# How the default mode builds the lists above that ratio: "buckets" writes
# each pair once through 8 x 8-tile squares (gs_bin_buckets); "depth_tile"
# emits (tile, point) pairs in depth order and sorts them by tile, the
# reference's dataflow (also the fallback when the image or a Gaussian's
# tile rectangle is too large for the bucketed binning's cover words).
HEAVY_DATAFLOW = "buckets"
BUCKET_MAX_GRID = 255  # tiles per image side the bucketed binning takes
# When the forward prepares the bucketed binning (the preprocess stores the
# coverage bands, the scan sizes the entries): "auto" when the last forward on
# the device had more than DEPTH_TILE_MIN_PAIRS_PER_GAUSSIAN pairs per
# Gaussian (a forward without that history bins by the depth-then-tile sort),
# "always" on every forward that may take it.
BUCKET_SIZING = "auto"

# The binning's point-order scan: one kernel (gs_scan_tiles_onepass, a
# decoupled look-back over a state that the preprocess prepares) when True,
# else the two-pass gs_scan_tiles.  SCAN_SPIN_LIMIT bounds the rounds of each
# of its waits; a round is an agent-scope load of 256 status words across the
# XCDs, two ballots, two workgroup barriers and a short sleep (on the order of
# a microsecond), so the bound is about a second, where a real wait (blocks
# start in index order) takes a few microseconds.  A timed-out wait falls back
# to summing the counts directly (exact, slower).
SCAN_ONEPASS = True
SCAN_SPIN_LIMIT = 1 << 20


def binning(pre: PreprocessOutputs, image_height: int, image_width: int, options: ExecutionOptions,
            keep_keys: bool = False, pack: bool = False, images: RenderImages | None = None,
            grad_clear: torch.Tensor | None = None) -> BinningState:
    """Per-tile Gaussian lists (binning_ops.py:84-431) in the requested sort mode.

    Every mode yields the same lists: per tile, the Gaussians in (depth, index)
    order.  A point-order scan of the tile counts always runs first; it gives
    the pair count (the forward's one host sync) and the visible depth range.
    ``warp_radix`` then sorts one packed 64-bit (tile, depth, point) key per
    pair with the HIP radix sort.  ``torch`` sorts the Gaussians by depth and
    the (tile, point) pairs by tile with ``torch.sort`` (stable), as the
    reference's torch mode does.  ``warp_depth_stable_tile`` (the default)
    runs the reference's depth-then-tile dataflow with the HIP radix sort when
    there are more than DEPTH_TILE_MIN_PAIRS_PER_GAUSSIAN pairs per Gaussian,
    and the single packed-key sort otherwise, where one sort of the pairs is
    cheaper than two sorts and the extra gathers.  With ``pack`` point_list and
    ranges are views of one raw-ABI binning buffer.  With ``images`` the
    packed path may launch the standard forward render into them right after
    the binning (then the returned state has ``rendered`` set).
    """
    mode = options.binning_sort_mode
    if mode not in BINNING_SORT_MODES:
        raise ValueError("sort_mode must be one of 'torch', 'warp_radix', or 'warp_depth_stable_tile'")
    lib = _lib.load()
    device = pre.radii.device
    P = pre.radii.shape[0]
    grid_x, grid_y = grid_dims(image_width, image_height)
    T = grid_x * grid_y
    stream = _stream(device)
    offsets = torch.empty((P,), dtype=torch.int32, device=device)
    info = torch.empty((4,), dtype=torch.int64, device=device)
    # the default mode's scan also sizes the bucketed binning (entries and
    # valid Gaussians in info[2] and info[3]) for the case of many pairs per Gaussian
    sized = buckets_expected(options, image_width, image_height, P, device) and pre.coverage is not None
    scan_state, pre.scan_state = pre.scan_state, None  # a prepared state serves one scan
    with _stage("scan"):
        if scan_state is not None:
            lib.call("gs_scan_tiles_onepass", P, pre.tiles_touched.data_ptr(), offsets.data_ptr(), info.data_ptr(),
                     scan_state.data_ptr(), scan_state.numel() * 8, int(sized), SCAN_SPIN_LIMIT, stream)
        elif sized:
            scan_scratch = torch.empty((max(int(lib.gs_scan_scratch_bytes(P)), 1),), dtype=torch.uint8,
                                       device=device)
            lib.call("gs_scan_tiles_entries", P, pre.tiles_touched.data_ptr(), pre.radii.data_ptr(),
                     pre.depths.data_ptr(), pre.coverage.data_ptr(), offsets.data_ptr(), info.data_ptr(),
                     scan_scratch.data_ptr(), scan_scratch.numel(), stream)
        else:
            scan_scratch = torch.empty((max(int(lib.gs_scan_scratch_bytes(P)), 1),), dtype=torch.uint8,
                                       device=device)
            lib.call("gs_scan_tiles", P, pre.tiles_touched.data_ptr(), None, pre.radii.data_ptr(),
                     pre.depths.data_ptr(), offsets.data_ptr(), info.data_ptr(), scan_scratch.data_ptr(),
                     scan_scratch.numel(), stream)
    slot = _workspace.readback_slot(device, torch.cuda.current_stream(device))
    capacity = _workspace.pair_capacity(device) if (not pack and not keep_keys and mode != "torch"
                                                    and PACKED_SORT == "segmented" and P > 0) else 0
    if mode == "warp_depth_stable_tile" and _workspace.last_pairs(device) > DEPTH_TILE_MIN_PAIRS_PER_GAUSSIAN * P:
        # the last forward on this device took the depth-then-tile dataflow, which this one will most
        # likely take too: provisioning the packed path's buffers would only raise the peak memory
        capacity = 0
    if capacity > 0:
        # Buffers for the expected pair count are allocated before the count
        # is read back, so that one C call reads it and launches the whole
        # packed binning; it declines (result[4] == 0) when the count does not
        # fit or the default mode picks the depth-then-tile dataflow.
        point_list = torch.empty((capacity,), dtype=torch.int32, device=device)
        ranges = torch.empty((T, 2), dtype=torch.int32, device=device)
        ws = torch.empty((int(lib.gs_bin_packed_workspace_bytes(capacity)),), dtype=torch.uint8, device=device)
        result = (ctypes.c_int64 * 6)()
        events = _stage_chain(("duplicate", "sort", "ranges", "sort") + (("render",) if images is not None else ()))
        img = images
        order = None if img is None else tile_order_buffer(image_width, image_height, device)
        lib.call("gs_readback_bin_packed", info.data_ptr(), slot.address, slot.next_seq(), P, pre.radii.data_ptr(),
                 pre.records.data_ptr(), pre.conic_2d_inv.data_ptr(), _lib.ptr(pre.coverage), _depths_or_none(pre),
                 offsets.data_ptr(), image_width, image_height, pre.coverage_mode, DEPTH_TILE_MIN_PAIRS_PER_GAUSSIAN if mode == "warp_depth_stable_tile" else 0,
                 capacity, ws.data_ptr(), ws.numel(), ranges.data_ptr(), point_list.data_ptr(),
                 None if img is None else img.background.data_ptr(), int(img is not None and img.compute_depth),
                 None if img is None else img.color.data_ptr(), None if img is None else img.depth.data_ptr(),
                 None if img is None else img.alpha.data_ptr(), None if img is None else img.n_contrib.data_ptr(),
                 _lib.ptr(grad_clear), 0 if grad_clear is None else grad_clear.numel(), events, result,
                 _lib.ptr(order), stream)
        R = validate_pair_count(int(result[0]))
        _workspace.note_pairs(device, R)
        _note("num_rendered", R)
        if result[4]:
            _note("binning_dataflow", "packed_key")
            _note("sort_passes", int(lib.gs_sort_num_passes((T - 1).bit_length())))
            layout = KeyLayout(depth_min=int(result[1]), depth_bits=int(result[2]), value_bits=int(result[3]))
            return BinningState(grid_x, grid_y, point_list[:R], ranges, R, None, layout, rendered=bool(result[5]),
                                tile_order=order if result[5] else None)
        depth_range = slot[1] & 0xFFFFFFFFFFFFFFFF
        # declined: release the provisioned buffers before the exact-size binning allocates its own
        del ws, result, events
        point_list = ranges = None
        if sized:  # the fast path read back two values only
            lib.call("gs_info_readback", info.data_ptr(), slot.address, slot.next_seq(), 4, stream)
    else:
        point_list = ranges = None
        lib.call("gs_info_readback", info.data_ptr(), slot.address, slot.next_seq(), 4 if sized else 2, stream)
        R = validate_pair_count(slot[0])
        depth_range = slot[1] & 0xFFFFFFFFFFFFFFFF
        _workspace.note_pairs(device, R)
        _note("num_rendered", R)
    entries, valid_points = (slot[2], slot[3]) if sized else (-1, 0)
    buffer = None
    if pack:
        buffer, point_list, ranges = _packing.allocate_binning(R, T, device)
    if R == 0:
        if ranges is None:
            ranges = torch.empty((T, 2), dtype=torch.int32, device=device)
        ranges.zero_()
        return BinningState(grid_x, grid_y, torch.empty((0,), dtype=torch.int32, device=device), ranges, 0,
                            buffer=buffer)
    layout = key_layout(P, T, depth_range & 0xFFFFFFFF, depth_range >> 32)
    if mode == "warp_radix" or (mode == "warp_depth_stable_tile" and layout.value_bits > 0
                                and R <= DEPTH_TILE_MIN_PAIRS_PER_GAUSSIAN * P):
        _note("binning_dataflow", "packed_key")
        bins = _binning_packed(pre, image_width, image_height, offsets, R, layout, keep_keys, point_list, ranges)
    elif sized and 0 <= entries <= MAX_BINNING_PAIRS:
        _note("binning_dataflow", "buckets")
        _note("bucket_entries", entries)
        _note("bucket_valid", valid_points)
        bins = _binning_buckets(pre, image_width, image_height, R, entries, valid_points,
                                depth_range & 0xFFFFFFFF, depth_range >> 32, keep_keys, ranges)
    else:
        _note("binning_dataflow", "depth_then_tile")
        bins = _binning_depth_tile(pre, image_width, image_height, R, keep_keys, mode == "torch", ranges)
    if buffer is not None:
        if bins.point_list.data_ptr() != point_list.data_ptr():
            point_list.copy_(bins.point_list)
            bins.point_list = point_list
        bins.buffer = buffer
    return bins


def tile_order_buffer(image_width: int, image_height: int, device) -> torch.Tensor:
    """Buffer for the blend kernels' tile order (gs_tile_order, one int32 per
    16 x 16 tile): the forward render orders the tiles into it, longest list
    first, when that pays (R <= 4 N, R >= 192 T), and the backward, given the
    same buffer (BinningState.tile_order), takes the tiles in that order."""
    num_tiles = ((image_width + 15) // 16) * ((image_height + 15) // 16)
    return torch.empty((max(num_tiles, 1),), dtype=torch.int32, device=device)


def _note(key: str, value) -> None:
    if STAGE_TIMER is not None and hasattr(STAGE_TIMER, "note"):
        STAGE_TIMER.note(key, value)


def _binning_depth_tile(pre: PreprocessOutputs, image_width: int, image_height: int, R: int, keep_keys: bool,
                        use_torch: bool, ranges: torch.Tensor | None = None) -> BinningState:
    """Depth sort of the Gaussians, tile counts scanned in depth order, (tile, point)
    pairs emitted in that order and sorted stably by tile (binning_ops.py:152-343)."""
    lib = _lib.load()
    device = pre.radii.device
    P = pre.radii.shape[0]
    grid_x, grid_y = grid_dims(image_width, image_height)
    T = grid_x * grid_y
    stream = _stream(device)
    dkeys = torch.empty((P,), dtype=torch.int32, device=device)
    order = torch.empty((P,), dtype=torch.int32, device=device)
    with _stage("depth_sort"):
        lib.call("gs_depth_keys", P, pre.radii.data_ptr(), pre.depths.data_ptr(), dkeys.data_ptr(),
                 order.data_ptr(), stream)
        if use_torch:
            dkeys, perm = torch.sort(dkeys, stable=True)
            order = order[perm]
        else:
            dkeys_alt = torch.empty_like(dkeys)
            order_alt = torch.empty_like(order)
            scratch = torch.empty((max(int(lib.gs_sort_scratch_bytes(P)), 1),), dtype=torch.uint8, device=device)
            lib.call("gs_sort_pairs_u32", P, 0, 32, dkeys.data_ptr(), order.data_ptr(), dkeys_alt.data_ptr(),
                     order_alt.data_ptr(), scratch.data_ptr(), scratch.numel(), stream)
            if lib.gs_sort_num_passes(32) % 2:
                dkeys, order = dkeys_alt, order_alt
    # depth-order offsets; the total is the R already read back
    offsets = torch.empty((P,), dtype=torch.int32, device=device)
    info = torch.empty((2,), dtype=torch.int64, device=device)
    scan_scratch = torch.empty((max(int(lib.gs_scan_scratch_bytes(P)), 1),), dtype=torch.uint8, device=device)
    with _stage("scan"):
        lib.call("gs_scan_tiles", P, pre.tiles_touched.data_ptr(), order.data_ptr(), None, None, offsets.data_ptr(),
                 info.data_ptr(), scan_scratch.data_ptr(), scan_scratch.numel(), stream)
    tiles = torch.empty((R,), dtype=torch.int32, device=device)
    vals = torch.empty((R,), dtype=torch.int32, device=device)
    with _stage("duplicate"):
        lib.call("gs_duplicate_tiles", P, order.data_ptr(), pre.radii.data_ptr(), pre.records.data_ptr(),
                 pre.conic_2d_inv.data_ptr(), _lib.ptr(pre.coverage), offsets.data_ptr(), image_width, image_height,
                 pre.coverage_mode, R,
                 tiles.data_ptr(), vals.data_ptr(), stream)
    tile_bits = (T - 1).bit_length()
    _note("sort_passes", int(lib.gs_sort_num_passes(tile_bits)))
    with _stage("sort"):
        if use_torch:
            tiles, perm = torch.sort(tiles, stable=True)
            vals = vals[perm]
        elif tile_bits > 0:
            tiles_alt = torch.empty_like(tiles)
            vals_alt = torch.empty_like(vals)
            scratch = torch.empty((max(int(lib.gs_sort_scratch_bytes(R)), 1),), dtype=torch.uint8, device=device)
            lib.call("gs_sort_pairs_u32", R, 0, tile_bits, tiles.data_ptr(), vals.data_ptr(), tiles_alt.data_ptr(),
                     vals_alt.data_ptr(), scratch.data_ptr(), scratch.numel(), stream)
            if lib.gs_sort_num_passes(tile_bits) % 2:
                tiles, vals = tiles_alt, vals_alt
    if ranges is None:
        ranges = torch.empty((T, 2), dtype=torch.int32, device=device)
    with _stage("ranges"):
        lib.call("gs_tile_ranges_u32", R, tiles.data_ptr(), T, ranges.data_ptr(), stream)
    keys = None
    if keep_keys:  # tile << 32 | depth bits, for tests
        keys = (tiles.to(torch.int64) << 32) | (pre.depths.view(torch.int32)[vals.long()].to(torch.int64)
                                                & 0xFFFFFFFF)
    return BinningState(grid_x, grid_y, vals, ranges, R, keys, KeyLayout(depth_min=0, depth_bits=32, value_bits=0))


def _binning_buckets(pre: PreprocessOutputs, image_width: int, image_height: int, R: int, entries: int,
                     valid_points: int, depth_min: int, depth_max: int, keep_keys: bool,
                     ranges: torch.Tensor | None = None) -> BinningState:
    """Depth order of the Gaussians, then per 8 x 8-tile square entries with
    tile masks, then the tile lists, each pair written once (gs_bin_buckets):
    the lists and ranges of binning_ops.py:152-431."""
    lib = _lib.load()
    device = pre.radii.device
    P = pre.radii.shape[0]
    grid_x, grid_y = grid_dims(image_width, image_height)
    T = grid_x * grid_y
    stream = _stream(device)
    point_list = torch.empty((R,), dtype=torch.int32, device=device)
    if ranges is None:
        ranges = torch.empty((T, 2), dtype=torch.int32, device=device)
    nbytes = int(lib.gs_bin_buckets_workspace_bytes(P, valid_points, entries, image_width, image_height))
    ws = torch.empty((max(nbytes, 1),), dtype=torch.uint8, device=device)
    events = _stage_chain(("depth_sort", "bucket", "bucket_tiles"))
    lib.call("gs_bin_buckets", P, valid_points, entries, R, pre.depths.data_ptr(), depth_min, depth_max,
             pre.coverage.data_ptr(), _lib.ptr(pre.band_store), pre.records.data_ptr(), image_width, image_height,
             ws.data_ptr(), ws.numel(), ranges.data_ptr(), point_list.data_ptr(), events, stream)
    keys = None
    if keep_keys:  # tile << 32 | depth bits, for tests
        lengths = (ranges[:, 1] - ranges[:, 0]).long()
        tiles = torch.repeat_interleave(torch.arange(T, device=device, dtype=torch.int64), lengths)
        keys = (tiles << 32) | (pre.depths.view(torch.int32)[point_list.long()].to(torch.int64) & 0xFFFFFFFF)
    return BinningState(grid_x, grid_y, point_list, ranges, R, keys, KeyLayout(depth_min=0, depth_bits=32, value_bits=0))


def _binning_packed(pre: PreprocessOutputs, image_width: int, image_height: int, offsets: torch.Tensor, R: int,
                    layout: KeyLayout, keep_keys: bool, point_list: torch.Tensor | None = None,
                    ranges: torch.Tensor | None = None) -> BinningState:
    """One packed 64-bit key per pair, emitted in point order and sorted."""
    lib = _lib.load()
    device = pre.radii.device
    P = pre.radii.shape[0]
    grid_x, grid_y = grid_dims(image_width, image_height)
    T = grid_x * grid_y
    stream = _stream(device)
    packed = layout.value_bits > 0
    tile_bits = (T - 1).bit_length()
    if ranges is None:
        ranges = torch.empty((T, 2), dtype=torch.int32, device=device)
    if packed and PACKED_SORT == "segmented":
        # One host call launches emission, the stable sort on the tile field,
        # the tile ranges and each tile's on-chip depth sort back to back.
        _note("sort_passes", int(lib.gs_sort_num_passes(tile_bits)))
        if point_list is None:
            point_list = torch.empty((R,), dtype=torch.int32, device=device)
        ws = torch.empty((max(int(lib.gs_bin_packed_workspace_bytes(R)), 1),), dtype=torch.uint8, device=device)
        keys_out = torch.empty((R,), dtype=torch.int64, device=device) if keep_keys else None
        events = _stage_chain(("duplicate", "sort", "ranges", "sort"))
        lib.call("gs_bin_packed", P, pre.radii.data_ptr(), pre.records.data_ptr(), pre.conic_2d_inv.data_ptr(),
                 _lib.ptr(pre.coverage), _depths_or_none(pre), offsets.data_ptr(), image_width, image_height, pre.coverage_mode, R, layout.depth_min,
                 layout.depth_bits, layout.value_bits, ws.data_ptr(), ws.numel(), ranges.data_ptr(),
                 point_list.data_ptr(), _lib.ptr(keys_out), events, stream)
        return BinningState(grid_x, grid_y, point_list, ranges, R, keys_out, layout)
    keys = torch.empty((R,), dtype=torch.int64, device=device)
    keys_alt = torch.empty((R,), dtype=torch.int64, device=device)
    vals = vals_alt = None
    if not packed:
        vals = torch.empty((R,), dtype=torch.int32, device=device)
        vals_alt = torch.empty((R,), dtype=torch.int32, device=device)
    with _stage("duplicate"):
        lib.call("gs_duplicate_keys", P, pre.radii.data_ptr(), pre.records.data_ptr(),
                 pre.conic_2d_inv.data_ptr(), _lib.ptr(pre.coverage), _depths_or_none(pre), offsets.data_ptr(),
                 image_width, image_height, pre.coverage_mode, R,
                 layout.depth_min, layout.depth_bits, layout.value_bits, keys.data_ptr(), _lib.ptr(vals), stream)
    sort_bits = tile_bits + layout.depth_bits
    sort_scratch = torch.empty((max(int(lib.gs_sort_scratch_bytes(R)), 1),), dtype=torch.uint8, device=device)
    _note("sort_passes", int(lib.gs_sort_num_passes(sort_bits)))
    with _stage("sort"):
        if packed:
            lib.call("gs_sort_keys_u64", R, layout.value_bits, sort_bits, keys.data_ptr(), keys_alt.data_ptr(),
                     sort_scratch.data_ptr(), sort_scratch.numel(), stream)
        else:
            lib.call("gs_sort_pairs_u64", R, sort_bits, keys.data_ptr(), vals.data_ptr(), keys_alt.data_ptr(),
                     vals_alt.data_ptr(), sort_scratch.data_ptr(), sort_scratch.numel(), stream)
    if lib.gs_sort_num_passes(sort_bits) % 2:
        keys, vals = keys_alt, vals_alt
    if not packed:
        point_list = vals
    elif point_list is None:
        point_list = torch.empty((R,), dtype=torch.int32, device=device)
    with _stage("ranges"):
        lib.call("gs_tile_ranges", R, keys.data_ptr(), layout.tile_shift, layout.value_bits, T, ranges.data_ptr(),
                 point_list.data_ptr() if packed else None, stream)
    return BinningState(grid_x, grid_y, point_list, ranges, R, keys if keep_keys else None, layout)


def render_images(background: torch.Tensor, image_height: int, image_width: int, options: ExecutionOptions,
                  device: torch.device) -> RenderImages:
    """The forward render's outputs, allocated ahead of the binning."""
    f = dict(dtype=torch.float32, device=device)
    H, W = image_height, image_width
    return RenderImages(_f32c(background.to(device)), torch.empty((NUM_CHANNELS, H, W), **f),
                        torch.empty((1, H, W), **f), torch.empty((1, H, W), **f),
                        torch.empty((H * W,), dtype=torch.int32, device=device), bool(options.compute_depth))


def render(pre: PreprocessOutputs, bins: BinningState, background: torch.Tensor, image_height: int,
           image_width: int, options: ExecutionOptions, *, flow: bool = False,
           images: RenderImages | None = None, grad_clear: torch.Tensor | None = None) -> RenderStageResult:
    """Tile blend (render_ops.py:16-93; flow: flow_ops.py:109-193).  ``images``
    are preallocated outputs; when the binning already launched the render into
    them (``bins.rendered``) nothing more is launched.  ``grad_clear`` (the
    backward's gradient accumulator, if any) is zeroed by the render kernel,
    or by the binning's render when that ran."""
    lib = _lib.load()
    device = pre.radii.device
    P = pre.radii.shape[0]
    H, W = image_height, image_width
    f = dict(dtype=torch.float32, device=device)
    if images is None:
        images = render_images(background, H, W, options, device)
    bg, color, depth, alpha, n_contrib = images.background, images.color, images.depth, images.alpha, images.n_contrib
    aux: tuple[torch.Tensor, ...] = ()
    if bins.rendered and not flow:
        return RenderStageResult(color, depth, alpha, n_contrib, aux)
    write_aux = bool(flow and options.compute_flow_aux)
    k = int(options.flow_topk or 0) if write_aux else 0
    if grad_clear is not None and (flow or bins.num_rendered == 0):
        grad_clear.zero_()
        grad_clear = None
    if bins.num_rendered == 0:
        color.copy_(bg.reshape(NUM_CHANNELS, 1, 1).expand_as(color))
        depth.zero_()
        alpha.zero_()
        n_contrib.zero_()
        if flow:
            aux = _empty_flow_aux(k, H, W, device)
        return RenderStageResult(color, depth, alpha, n_contrib, aux)
    compute_depth = int(bool(options.compute_depth))
    stream = _stream(device)
    if bins.tile_order is None:
        bins.tile_order = tile_order_buffer(W, H, device)
    if flow:
        if write_aux:
            aux = (torch.empty((k, H, W), dtype=torch.int32, device=device), torch.empty((k, H, W), **f),
                   torch.empty((2, k, H, W), **f))
        else:
            aux = _empty_flow_aux(0, H, W, device)
        with _stage("render"):
            lib.call("gs_render_fwd_flow", W, H, P, bins.num_rendered, bins.ranges.data_ptr(),
                     bins.point_list.data_ptr(), pre.records.data_ptr(), bg.data_ptr(), compute_depth,
                     int(write_aux), k, color.data_ptr(), depth.data_ptr(), alpha.data_ptr(), n_contrib.data_ptr(),
                     aux[0].data_ptr() if write_aux else None, aux[1].data_ptr() if write_aux else None,
                     aux[2].data_ptr() if write_aux else None, bins.tile_order.data_ptr(), stream)
    else:
        with _stage("render"):
            lib.call("gs_render_fwd_clear", W, H, P, bins.num_rendered, bins.ranges.data_ptr(),
                     bins.point_list.data_ptr(), pre.records.data_ptr(), bg.data_ptr(), compute_depth,
                     color.data_ptr(), depth.data_ptr(), alpha.data_ptr(), n_contrib.data_ptr(),
                     _lib.ptr(grad_clear), 0 if grad_clear is None else grad_clear.numel(),
                     bins.tile_order.data_ptr(), stream)
    return RenderStageResult(color, depth, alpha, n_contrib, aux)


def forward(inputs: RasterInputs, options: ExecutionOptions, *, flow: bool = False,
            pack: bool = False, grad_buffer: bool = False) -> ForwardResult:
    """One typed forward: the reference's execute_typed_forward (pipeline.py:11-45).
    ``pack`` lays the state out in the raw ABI's geom / binning buffers.
    ``grad_buffer`` has the render zero the backward's (N, 10) gradient
    accumulator on its way, kept in the state for one backward."""
    means = inputs.means3d
    if means.ndim != 2 or means.shape[1] != 3:
        raise ValueError("means3D must have dimensions (num_points, 3)")
    device = means.device
    with torch.cuda.device(device), _workspace.device_lock(device):
        if means.shape[0] == 0:
            k = (options.flow_topk if options.compute_flow_aux else 0) if flow else None
            return empty_forward(inputs, k)
        pre = preprocess(inputs, options, pack=pack)
        images = render_images(inputs.background, inputs.image_height, inputs.image_width, options, device)
        grad_gauss = torch.empty((means.shape[0], _lib.GS_GRAD_FLOATS), dtype=torch.float32,
                                 device=device) if grad_buffer else None
        bins = binning(pre, inputs.image_height, inputs.image_width, options, pack=pack,
                       images=None if flow else images, grad_clear=grad_gauss)
        res = render(pre, bins, inputs.background, inputs.image_height, inputs.image_width, options, flow=flow,
                     images=images, grad_clear=grad_gauss)
        _note("n_contrib", res.n_contrib)
        _note("alpha", res.alpha)
    return ForwardResult(
        num_rendered=bins.num_rendered,
        color=res.color,
        depth=res.depth,
        alpha=res.alpha,
        radii=pre.radii,
        proj_2d=pre.proj_2d,
        conic_2d=pre.conic_2d,
        conic_2d_inv=pre.conic_2d_inv,
        state=ForwardState(pre, bins, res.n_contrib, grad_gauss),
        aux=res.aux,
    )


def _depths_or_none(pre: PreprocessOutputs) -> int | None:
    """Address of the preprocess depths for the emission's key field, or None
    (a state restored from raw buffers has none; the records hold a copy)."""
    return pre.depths.data_ptr() if pre.depths.numel() == pre.radii.numel() and pre.radii.numel() > 0 else None


def _f32c_or_none(t: torch.Tensor | None) -> torch.Tensor | None:
    """Contiguous fp32 upstream gradient, or None (the kernels read an absent
    gradient as zero)."""
    return None if t is None else _f32c(t)


def backward(inputs: RasterInputs, radii: torch.Tensor, alpha: torch.Tensor, grad_color, grad_depth, grad_alpha,
             grad_proj_2d, grad_conic_2d, grad_conic_2d_inv, options: ExecutionOptions,
             forward_state: ForwardState | None, *, flow_double: bool = False):
    """Manual backward -> (grad_means2D, grad_colors, grad_opacities, grad_means3D, grad_cov3D,
    grad_sh, grad_scales, grad_rotations), the order of backward_ops.py:746."""
    lib = _lib.load()
    means = inputs.means3d
    device = means.device
    P = means.shape[0]
    H, W = inputs.image_height, inputs.image_width
    grad_colors = torch.empty_like(inputs.colors)
    grad_cov3d = torch.empty_like(inputs.cov3d_precomp)
    if P == 0:
        return (torch.zeros((0, 3), dtype=torch.float32, device=device), grad_colors,
                torch.empty_like(inputs.opacities), torch.zeros_like(means), grad_cov3d,
                torch.empty_like(inputs.sh), torch.zeros_like(inputs.scales), torch.zeros_like(inputs.rotations))
    with torch.cuda.device(device), _workspace.device_lock(device):
        if forward_state is None:
            # Second backward of a retained graph: rebuild the forward state.
            pre = preprocess(inputs, options)
            bins = binning(pre, H, W, options)
            n_contrib = render(pre, bins, inputs.background, H, W, options).n_contrib
        else:
            pre, bins, n_contrib = forward_state.preprocess, forward_state.binning, forward_state.n_contrib
        stream = _stream(device)
        # the accumulator the forward render zeroed serves one backward
        grad_gauss = None if forward_state is None else forward_state.grad_gauss
        if grad_gauss is not None:
            forward_state.grad_gauss = None
        if grad_gauss is None or grad_gauss.shape[0] != P:
            grad_gauss = torch.zeros((P, _lib.GS_GRAD_FLOATS), dtype=torch.float32, device=device)
        if bins.num_rendered != 0:
            bg = _f32c(inputs.background.to(device))
            gc = _f32c_or_none(grad_color)
            gd = _f32c_or_none(grad_depth)
            ga = _f32c_or_none(grad_alpha)
            alpha_c = _f32c(alpha)
            with _stage("render_bwd"):
                lib.call("gs_render_bwd", W, H, P, bins.num_rendered, bins.ranges.data_ptr(),
                         bins.point_list.data_ptr(), pre.records.data_ptr(), bg.data_ptr(), alpha_c.data_ptr(),
                         n_contrib.data_ptr(), _lib.ptr(gc), _lib.ptr(gd), _lib.ptr(ga),
                         int(bool(options.compute_depth)), grad_gauss.data_ptr(), _lib.ptr(bins.tile_order),
                         stream)
        has_sh = inputs.sh.numel() != 0
        shs = _f32c(inputs.sh).reshape(P, -1, NUM_CHANNELS) if has_sh else None
        K = shs.shape[1] if has_sh else 0
        grad_sh = torch.empty((P, K, NUM_CHANNELS), dtype=torch.float32, device=device) if has_sh else \
            torch.empty_like(inputs.sh)
        f = dict(dtype=torch.float32, device=device)
        grad_means3d = torch.empty((P, 3), **f)
        grad_means2d = torch.empty((P, 3), **f)
        scales_c, rot_c, cov_c = _covariance_inputs(inputs, P)
        if cov_c is None:
            grad_scales = torch.empty((P, 3), **f)
            grad_rotations = torch.empty((P, 4), **f)
        else:
            # The precomputed-covariance branch of backward_ops.py:733-737.
            grad_scales = torch.zeros_like(inputs.scales)
            grad_rotations = torch.zeros_like(inputs.rotations)
            grad_cov3d = torch.empty((P, 6), **f)
        tanfovx, tanfovy = float(inputs.tan_fovx), float(inputs.tan_fovy)
        means_c = _f32c(means)
        campos_c = _f32c(inputs.campos)
        view_c = _f32c(inputs.viewmatrix)
        proj_c = _f32c(inputs.projmatrix)
        radii_c = radii.contiguous()
        # The opacity and colour gradients are columns 5 and 6-8 of grad_gauss
        # (the reference returns views of its render gradients,
        # backward_ops.py:538-541); they are written out contiguously here so
        # that autograd does not copy a strided view into each leaf.
        grad_opacities = torch.empty((P,), **f)
        grad_colors_out = torch.empty((P, NUM_CHANNELS), **f) if inputs.colors.numel() != 0 else None
        gp2 = _f32c_or_none(grad_proj_2d)
        gcon = _f32c_or_none(grad_conic_2d)
        gcov = _f32c_or_none(grad_conic_2d_inv)
        with _stage("preprocess_bwd"):
            lib.call(
                "gs_preprocess_bwd", P, K, int(inputs.degree), means_c.data_ptr(), _lib.ptr(scales_c),
                _lib.ptr(rot_c), _lib.ptr(cov_c), float(inputs.scale_modifier), _lib.ptr(shs), campos_c.data_ptr(),
                view_c.data_ptr(), proj_c.data_ptr(), tanfovx, tanfovy, _focal(W, tanfovx), _focal(H, tanfovy),
                radii_c.data_ptr(), pre.clamped.data_ptr(), grad_gauss.data_ptr(), pre.records.data_ptr(), W, H,
                _lib.ptr(gp2), _lib.ptr(gcon),
                _lib.ptr(gcov), int(bool(flow_double)), float(inputs.filter_variance), grad_means3d.data_ptr(),
                grad_means2d.data_ptr(),
                _lib.ptr(grad_scales) if cov_c is None else None,
                _lib.ptr(grad_rotations) if cov_c is None else None,
                _lib.ptr(grad_cov3d) if cov_c is not None else None,
                grad_sh.data_ptr() if has_sh else None, grad_opacities.data_ptr(),
                _lib.ptr(grad_colors_out), stream)
    grad_opacities = grad_opacities.reshape(inputs.opacities.shape)
    if grad_colors_out is not None:
        grad_colors = grad_colors_out.reshape(inputs.colors.shape)
    if has_sh:
        grad_sh = grad_sh.reshape(inputs.sh.shape)
    if grad_cov3d.numel() != 0:
        grad_cov3d = grad_cov3d.reshape(inputs.cov3d_precomp.shape)
    return (grad_means2d, grad_colors, grad_opacities, grad_means3d, grad_cov3d, grad_sh,
            grad_scales.reshape(inputs.scales.shape), grad_rotations.reshape(inputs.rotations.shape))


def mark_visible(positions: torch.Tensor, viewmatrix: torch.Tensor) -> torch.Tensor:
    """view-space z > 0.2 as bool (preprocess_ops.py:584-595)."""
    points = positions.contiguous()
    if points.ndim != 2 or points.shape[1] != 3:
        raise ValueError("means3D must have dimensions (num_points, 3)")
    device = points.device
    if points.shape[0] == 0:
        return torch.empty((0,), dtype=torch.bool, device=device)
    lib = _lib.load()
    out = torch.empty((points.shape[0],), dtype=torch.uint8, device=device)
    points_c = _f32c(points)
    view_c = _f32c(viewmatrix)
    with torch.cuda.device(device), _workspace.device_lock(device):
        lib.call("gs_mark_visible", points.shape[0], points_c.data_ptr(), view_c.data_ptr(), out.data_ptr(),
                 _stream(device))
    return out.view(torch.bool)
