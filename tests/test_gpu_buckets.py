"""The bucketed binning (gs_bin_buckets) and its sizing scan against the CPU oracle.

The default sort mode bins scenes with more than four pairs per Gaussian by
8 x 8-tile squares: the Gaussians in depth order give one entry per square
their tile rectangle meets, with the mask of the tiles they cover there, and
each square's entries are written into its tiles' lists.  The lists and
ranges must equal the oracle's (binning_ops.py:152-431 semantics) bit for
bit.  The cases force the dataflow at any pair ratio and cover the three
coverage modes (full rectangles, cover masks, coverage bands by rows and by
columns), partial squares at the image edge, and groups of Gaussians whose
entries exceed one assembly window.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gswarp_amd import _lib, _pipeline, configs
from helpers import gpu_forward, options, oracle_forward, raster_inputs, to_np

pytestmark = pytest.mark.gpu


def _spy_calls(monkeypatch):
    lib = _lib.load()
    names = []
    real = lib.call

    def call(name, *args):
        names.append(name)
        return real(name, *args)

    monkeypatch.setattr(lib, "call", call)
    return names


def _force_buckets(monkeypatch):
    monkeypatch.setattr(_pipeline, "DEPTH_TILE_MIN_PAIRS_PER_GAUSSIAN", 0)
    monkeypatch.setattr(_pipeline, "HEAVY_DATAFLOW", "buckets")
    monkeypatch.setattr(_pipeline, "BUCKET_SIZING", "always")


def _large_splats(device, count=3000, width=960, height=540, seed=3):
    """The config-3 distributions with every scale at least 0.4: tile rectangles
    of tens of tiles by tens, about ten 8 x 8-tile squares per Gaussian, so a
    wave's 64 Gaussians have more entries than one 512-entry window."""
    scene = configs.make_scene(3, count=count, width=width, height=height, seed=seed, device=device)
    scene["scales"] = torch.clamp(scene["scales"] * 4.0, min=0.4)
    return scene


SCENES = {
    "c3_small": lambda dev: configs.make_scene(3, count=60_000, width=480, height=270, device=dev),
    "c2_small": lambda dev: configs.make_scene(2, count=60_000, width=480, height=270, device=dev),
    "c1_ragged": lambda dev: configs.make_scene(1, count=5_000, width=203, height=117, device=dev),
    "large": lambda dev: _large_splats(dev),
}


def _check_lists(scene, coverage_mode, monkeypatch):
    names = _spy_calls(monkeypatch)
    opts = options(coverage_mode=coverage_mode)
    print(f"[buckets] N={scene['means3D'].shape[0]} {scene['width']}x{scene['height']} cov={coverage_mode}",
          flush=True)
    out = gpu_forward(scene, opts)
    host, ref = oracle_forward(scene, coverage_mode=coverage_mode)
    bins, res, rb, rf = out["bins"], out["res"], ref["bins"], ref["fwd"]
    assert bins.num_rendered == rb["num_rendered"]
    if bins.num_rendered:
        assert "gs_bin_buckets" in names
        assert np.array_equal(to_np(bins.point_list), rb["point_list"])
    assert np.array_equal(to_np(bins.ranges), rb["ranges"])
    assert np.array_equal(to_np(res.n_contrib).reshape(rf["n_contrib"].shape), rf["n_contrib"])
    assert np.array_equal(to_np(res.color), rf["color"])
    return out, ref


@pytest.mark.parametrize("coverage_mode", [0, 1, 2])
@pytest.mark.parametrize("name", list(SCENES))
def test_bucketed_lists_match_oracle(name, coverage_mode, device, monkeypatch):
    _force_buckets(monkeypatch)
    _check_lists(SCENES[name](device), coverage_mode, monkeypatch)


def _decode_words(words: np.ndarray):
    x, y = words[:, 0].astype(np.int64) & 0xFFFFFFFF, words[:, 1].astype(np.int64) & 0xFFFFFFFF
    rx, ry = x & 0xFFFF, x >> 16
    sw, sh = y & 0xFF, (y >> 8) & 0xFF
    valid = ((y >> 18) & 1).astype(bool)
    return rx, ry, sw, sh, valid


@pytest.mark.parametrize("name", ["c3_small", "large", "c1_ragged"])
def test_scan_sizes_the_buckets(name, device):
    """gs_scan_tiles_entries: info[0] is the pair count, info[2] the number of
    (Gaussian, 8 x 8-tile square) entries of the valid cover words and info[3]
    the number of valid words; every tile the oracle bins a Gaussian to lies in
    its word's rectangle, and every Gaussian with tiles has a valid word."""
    scene = SCENES[name](device)
    opts = options()
    inputs = raster_inputs(scene)
    lib = _lib.load()
    with torch.cuda.device(device):
        pre = _pipeline.preprocess(inputs, opts)
        P = pre.radii.shape[0]
        offsets = torch.empty((P,), dtype=torch.int32, device=device)
        info = torch.full((4,), -7, dtype=torch.int64, device=device)
        scratch = torch.empty((int(lib.gs_scan_scratch_bytes(P)),), dtype=torch.uint8, device=device)
        stream = torch.cuda.current_stream(device).cuda_stream
        lib.call("gs_scan_tiles_entries", P, pre.tiles_touched.data_ptr(), pre.radii.data_ptr(),
                 pre.depths.data_ptr(), pre.coverage.data_ptr(), offsets.data_ptr(), info.data_ptr(),
                 scratch.data_ptr(), scratch.numel(), stream)
    torch.cuda.synchronize()
    host, ref = oracle_forward(scene)
    words = to_np(pre.coverage)
    rx, ry, sw, sh, valid = _decode_words(words)
    units = (((rx + sw - 1) // 8 - rx // 8 + 1) * ((ry + sh - 1) // 8 - ry // 8 + 1))[valid]
    got = to_np(info)
    assert got[0] == ref["bins"]["num_rendered"]
    assert got[2] == int(units.sum())
    assert got[3] == int(valid.sum())
    touched = to_np(pre.tiles_touched)
    assert np.all(valid[touched > 0])
    # the oracle's tiles of each Gaussian lie inside its word's rectangle
    rb = ref["bins"]
    tiles = rb["tile_ids"].astype(np.int64)
    pts = rb["point_list"].astype(np.int64)
    gx = (scene["width"] + 15) // 16
    tx, ty = tiles % gx, tiles // gx
    assert np.all((tx >= rx[pts]) & (tx < rx[pts] + sw[pts]) & (ty >= ry[pts]) & (ty < ry[pts] + sh[pts]))
    # offsets are the point-order scan of gs_scan_tiles
    assert np.array_equal(to_np(offsets), np.cumsum(touched, dtype=np.int64).astype(np.int32))


def test_default_mode_takes_buckets_for_many_pairs(device, monkeypatch):
    """Unforced: a forward of the heavy-tailed scene (more than four pairs per
    Gaussian) after one with that ratio on the device takes the bucketed
    binning in the default sort mode and matches the oracle; without the
    history the forward bins by the depth-then-tile sort, with the same lists."""
    from gswarp_amd import _workspace

    scene = configs.make_scene(3, count=20_000, width=960, height=540, device=device)
    host, ref = oracle_forward(scene)
    R = ref["bins"]["num_rendered"]
    assert R > 4 * scene["means3D"].shape[0]
    monkeypatch.setattr(_workspace, "last_pairs", lambda dev: 0)
    names = _spy_calls(monkeypatch)
    out = gpu_forward(scene, options())
    assert "gs_bin_buckets" not in names and "gs_duplicate_tiles" in names
    assert np.array_equal(to_np(out["bins"].point_list), ref["bins"]["point_list"])
    monkeypatch.setattr(_workspace, "last_pairs", lambda dev: R)
    _check_lists(scene, 1, monkeypatch)


def test_oversized_image_falls_back_to_depth_tile(device, monkeypatch):
    """Images wider than 255 tiles exceed the cover words' spans: the default
    mode then bins by the depth-then-tile sort, with the same lists."""
    monkeypatch.setattr(_pipeline, "DEPTH_TILE_MIN_PAIRS_PER_GAUSSIAN", 0)
    scene = configs.make_scene(1, count=3_000, width=4112, height=64, device=device)
    names = _spy_calls(monkeypatch)
    out = gpu_forward(scene, options())
    host, ref = oracle_forward(scene)
    assert "gs_bin_buckets" not in names and "gs_duplicate_tiles" in names
    assert np.array_equal(to_np(out["bins"].point_list), ref["bins"]["point_list"])
    assert np.array_equal(to_np(out["bins"].ranges), ref["bins"]["ranges"])
