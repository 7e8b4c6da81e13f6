"""Tile count == emission at numeric boundaries, through the HIP count and emission.

Restates test_rasterizer_cuda_contracts.py:176-336 of the reference for the
gfx950 path: Gaussians centred one ulp either side of tile edges and with
opacities one ulp either side of 1/255 are counted by gs_count_tiles (the
preprocess's flattened band walk and cover masks, on given 2D inputs) and
emitted by gs_duplicate_keys, once from the cover words and once by the band
walk, in all three coverage modes.  Counts, the emitted tile set of every
Gaussian and the packed key fields must equal the C oracle's exactly, and the
count must equal what is emitted.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from gswarp_amd import _lib

pytestmark = pytest.mark.gpu

MODES = {"snugbox": 0, "accutile_sweep": 1, "conic_rect": 2}


def _f32_next(x: float, toward: float) -> float:
    return float(np.nextafter(np.float32(x), np.float32(toward)))


def _reference_case():
    """The six Gaussians of test_rasterizer_cuda_contracts.py:177-233 on an 8x8 tile grid."""
    b16, a16 = _f32_next(16.0, -np.inf), _f32_next(16.0, np.inf)
    cut = np.float32(1.0 / 255.0)
    pts = np.array([[b16, b16], [16.0, 16.0], [a16, a16], [31.999, 48.001], [64.0, 63.999], [1.0, 126.0]],
                   np.float32)
    cov = np.array([[20.0, 8.0, 12.0], [20.0, -8.0, 12.0], [0.5, 0.49, 0.5], [80.0, 0.0, 0.4],
                    [0.4, -0.15, 30.0], [4.0, 1.5, 4.0]], np.float32)
    opac = np.array([0.8, 0.8, 0.3, 0.5, _f32_next(cut, np.inf), _f32_next(cut, -np.inf)], np.float32)
    return pts, cov, opac, 8, 8


def _random_boundary_case(seed: int, n: int = 4096, grid: int = 24):
    """Centres on tile edges (multiples of 16), one ulp either side, and tile
    centres; covariances from tiny to a few tiles wide, isotropic to
    needle-thin, with either sign of correlation; opacities at 1/255 and one or
    two ulp either side, or uniform."""
    rng = np.random.default_rng(seed)
    edges = np.arange(0, grid + 1, dtype=np.float32) * 16.0
    base = rng.choice(edges, size=(n, 2)).astype(np.float32)
    which = rng.integers(0, 4, size=(n, 2))
    ups = np.nextafter(base, np.float32(np.inf))
    downs = np.nextafter(base, np.float32(-np.inf))
    pts = np.where(which == 0, base, np.where(which == 1, ups, np.where(which == 2, downs, base + 8.0)))
    pts = pts.astype(np.float32)
    s1 = np.exp(rng.uniform(np.log(0.3), np.log(900.0), n))
    s2 = s1 * np.exp(rng.uniform(np.log(0.01), 0.0, n))
    th = rng.uniform(0, np.pi, n)
    c, s = np.cos(th), np.sin(th)
    a = c * c * s1 + s * s * s2
    b = c * s * (s1 - s2)
    d = s * s * s1 + c * c * s2
    cov = np.stack([a, b, d], 1).astype(np.float32)
    cut = np.float32(1.0 / 255.0)
    near = np.array([np.nextafter(np.nextafter(cut, np.float32(-1)), np.float32(-1)), np.nextafter(cut, np.float32(-1)),
                     cut, np.nextafter(cut, np.float32(1)),
                     np.nextafter(np.nextafter(cut, np.float32(1)), np.float32(1))], np.float32)
    opac = np.where(rng.random(n) < 0.5, rng.choice(near, n), rng.uniform(0.01, 0.99, n)).astype(np.float32)
    return pts, cov, opac, grid, grid


def _conic_and_radius(cov: np.ndarray):
    """Conic and 3-sigma radius in float32, as the reference test forms them."""
    det = cov[:, 0] * cov[:, 2] - cov[:, 1] * cov[:, 1]
    conic = np.stack([cov[:, 2] / det, -cov[:, 1] / det, cov[:, 0] / det], 1).astype(np.float32)
    tr = cov[:, 0] + cov[:, 2]
    disc = np.maximum(np.float32(0.25) * tr * tr - det, np.float32(0.0))
    lam = np.float32(0.5) * tr + np.sqrt(disc)
    radii = np.ceil(np.float32(3.0) * np.sqrt(lam)).astype(np.int32)
    return conic, radii


def _gpu_count_and_emit(pts, cov, conic, opac, radii, grid_x, grid_y, mode, device, use_cover: bool):
    lib = _lib.load()
    n = pts.shape[0]
    W, H = 16 * grid_x, 16 * grid_y
    rec = np.zeros((n, 12), np.float32)
    rec[:, 0:2] = pts
    rec[:, 2:4] = conic[:, 0:2]
    rec[:, 4] = conic[:, 2]
    rec[:, 5] = opac
    rec[:, 6] = np.arange(1, n + 1, dtype=np.float32)  # depths, as the reference test
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    t_rec, t_cov, t_rad = d(rec), d(cov), d(radii)
    touched = torch.full((n,), -1, dtype=torch.int32, device=device)
    cover = torch.zeros((n, 4), dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    lib.call("gs_count_tiles", n, t_rad.data_ptr(), t_rec.data_ptr(), t_cov.data_ptr(), W, H, mode,
             touched.data_ptr(), cover.data_ptr(), stream)
    counts = touched.cpu().numpy()
    offsets = np.cumsum(counts, dtype=np.int64).astype(np.int32)
    total = int(offsets[-1])
    depth_bits_arr = rec[:, 6].view(np.uint32)
    dmin, dmax = int(depth_bits_arr.min()), int(depth_bits_arr.max())
    depth_bits = (dmax - dmin).bit_length()
    value_bits = max(1, (n - 1).bit_length())
    keys = torch.full((max(total, 1),), -1, dtype=torch.int64, device=device)
    if total:
        lib.call("gs_duplicate_keys", n, t_rad.data_ptr(), t_rec.data_ptr(), t_cov.data_ptr(),
                 cover.data_ptr() if use_cover else None, None, d(offsets).data_ptr(), W, H, mode, total, dmin,
                 depth_bits, value_bits, keys.data_ptr(), None, stream)
    torch.cuda.synchronize(device)
    k = keys.cpu().numpy()[:total].view(np.uint64)
    point = (k & np.uint64((1 << value_bits) - 1)).astype(np.int64)
    depth_field = ((k >> np.uint64(value_bits)) & np.uint64((1 << depth_bits) - 1)).astype(np.int64)
    tile = (k >> np.uint64(value_bits + depth_bits)).astype(np.int64)
    return counts, offsets, tile, point, depth_field, depth_bits_arr.astype(np.int64) - dmin


def _check(pts, cov, opac, grid_x, grid_y, device):
    conic, radii = _conic_and_radius(cov)
    co = np.concatenate([conic, opac[:, None]], 1).astype(np.float32)
    n = pts.shape[0]
    for name, mode in MODES.items():
        ref_counts = oracle.count_covered_tiles(pts, cov, co, radii, grid_x, grid_y, mode)
        ref_tiles, ref_points, ref_offsets = oracle.emit_covered_tiles(pts, cov, co, radii, grid_x, grid_y, mode)
        for use_cover in (True, False):
            print(f"[boundary] n={n} grid={grid_x}x{grid_y} mode={name} cover_words={use_cover}", flush=True)
            counts, offsets, tile, point, depth_field, depth_of = _gpu_count_and_emit(
                pts, cov, conic, opac, radii, grid_x, grid_y, mode, device, use_cover)
            assert np.array_equal(counts, ref_counts), (name, np.flatnonzero(counts != ref_counts)[:10])
            assert tile.size == int(counts.sum()) == ref_tiles.size
            assert np.all((tile >= 0) & (tile < grid_x * grid_y))
            starts = np.concatenate([[0], offsets[:-1]])
            for i in range(n):
                s, e = int(starts[i]), int(offsets[i])
                assert np.all(point[s:e] == i), (name, i)
                assert np.all(depth_field[s:e] == depth_of[i]), (name, i)
                rs, re = (int(ref_offsets[i - 1]) if i else 0), int(ref_offsets[i])
                assert np.array_equal(np.sort(tile[s:e]), np.sort(ref_tiles[rs:re].astype(np.int64))), (name, i)
    return radii


def test_reference_boundary_points_count_equals_emit(device):
    pts, cov, opac, gx, gy = _reference_case()
    _check(pts, cov, opac, gx, gy, device)
    # the Gaussian just below the 1/255 cut-off covers no tile; every other one covers some
    conic, radii = _conic_and_radius(cov)
    co = np.concatenate([conic, opac[:, None]], 1).astype(np.float32)
    for mode in MODES.values():
        counts = oracle.count_covered_tiles(pts, cov, co, radii, gx, gy, mode)
        assert counts[-1] == 0 and np.all(counts[:-1] > 0)


@pytest.mark.parametrize("seed", [0, 1])
def test_random_boundary_points_count_equals_emit(seed, device):
    pts, cov, opac, gx, gy = _random_boundary_case(seed)
    _check(pts, cov, opac, gx, gy, device)
