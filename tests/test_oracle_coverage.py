"""Pins the oracle's tile coverage (count and emit) without the reference.

The reference's own CPU test of coverage (tests/test_tile_coverage.py:245-279)
checks, on 253 seeded footprints in a 96x64 image, that every tile holding a
pixel whose Gaussian exponent reaches the alpha cut-off (inside the CUDA
3-sigma rectangle) is covered by the exact modes, and that the exact modes
never cover more than SnugBox.  Those properties are restated here against
the C oracle (oracle/gs_oracle.c), with the same seeded case generator, plus:

* float64 restatements of the SnugBox rectangle, the AccuTile band sweep
  and the conic-rectangle test (math_kernels.py:151-390) that the float32
  oracle must reproduce tile for tile on every seeded case;
* the count/emit boundary cases of test_rasterizer_cuda_contracts.py:176-336
  (points on tile edges, cut-off opacities) with count == emitted pairs.
"""

from __future__ import annotations

import math
import random

import numpy as np
import pytest

import oracle

BLOCK = 16
Q_EPS = 1.0e-4
W, H = 96, 64
GX, GY = (W + BLOCK - 1) // BLOCK, (H + BLOCK - 1) // BLOCK
MODES = {"snugbox": 0, "accutile_sweep": 1, "conic_rect": 2}


def f32(x):
    return float(np.float32(x))


def seeded_cases():
    """The three fixed footprints and 250 random ones (conic eigenvalues
    10^U(-1.3, 0.7), uniform angle, centres slightly outside the image), in the
    reference test's draw order (test_tile_coverage.py:246-271)."""
    rng = random.Random(20260713)
    cases = [
        ((31.4, 16.9), (2.220537, -2.480092, 3.196566), 0.12),
        ((0.25, 0.75), (0.08, 0.075, 0.09), 0.95),
        ((79.2, 47.8), (1.5, -0.02, 0.04), 0.5),
    ]
    for _ in range(250):
        angle = rng.uniform(-math.pi, math.pi)
        ca, sa = math.cos(angle), math.sin(angle)
        e1 = 10.0 ** rng.uniform(-1.3, 0.7)
        e2 = 10.0 ** rng.uniform(-1.3, 0.7)
        conic = (e1 * ca * ca + e2 * sa * sa, (e1 - e2) * ca * sa, e1 * sa * sa + e2 * ca * ca)
        centre = (rng.uniform(-4.0, 100.0), rng.uniform(-4.0, 68.0))
        cases.append((centre, conic, rng.uniform(0.01, 0.99)))
    # every value as the float32 the kernels see
    return [((f32(p[0]), f32(p[1])), tuple(f32(v) for v in c), f32(o)) for p, c, o in cases]


def cov_of(conic):
    a, b, c = conic
    det = a * c - b * b
    return c / det, -b / det, a / det


def cuda_radius(cov):
    xx, xy, yy = cov
    mid = 0.5 * (xx + yy)
    lam = mid + math.sqrt(max(0.0, mid * mid - (xx * yy - xy * xy)))
    return int(math.ceil(3.0 * math.sqrt(lam)))


def rect(px, py, rx, ry):
    """Tile rectangle [x0, x1) x [y0, y1) of a centre and radii (truncating casts, clamp to grid)."""
    def clamp(v, hi):
        return min(hi, max(0, v))
    return (clamp(int((px - rx) / BLOCK), GX), clamp(int((py - ry) / BLOCK), GY),
            clamp(int((px + rx + BLOCK - 1) / BLOCK), GX), clamp(int((py + ry + BLOCK - 1) / BLOCK), GY))


def threshold_of(opacity):
    return 2.0 * math.log(max(255.0 * opacity, 1.0))


def snug_rect(point, conic, opacity):
    cov = cov_of(conic)
    r = cuda_radius(cov)
    outer = rect(point[0], point[1], r, r)
    t = threshold_of(opacity)
    if t <= 0.0:
        return (0, 0, 0, 0)
    rx = math.ceil(math.sqrt(max(t * cov[0], 0.0)) + 1.0)
    ry = math.ceil(math.sqrt(max(t * cov[2], 0.0)) + 1.0)
    inner = rect(point[0], point[1], rx, ry)
    return (max(outer[0], inner[0]), max(outer[1], inner[1]), min(outer[2], inner[2]), min(outer[3], inner[3]))


def band_tiles(pu, pv, cuu, cuv, cvv, t, band, lo, hi):
    """Tiles along u of the band `band` (pixels band*16 .. band*16+15 along v):
    the conic's u-interval at both band edges and at the ellipse's u-extremes
    when they fall inside the band, padded by Q_EPS, floor-divided into tiles."""
    det = cuu * cvv - cuv * cuv
    t = t + Q_EPS
    v0 = band * BLOCK - pv
    v1 = band * BLOCK + BLOCK - 1 - pv
    us = []
    for v in (v0, v1):
        disc = cuu * t - det * v * v
        if disc >= -Q_EPS:
            half = math.sqrt(max(disc, 0.0)) / cuu
            centre = -cuv * v / cuu
            us += [centre - half, centre + half]
    ext = math.sqrt(max(t * cvv / det, 0.0))
    for u in (-ext, ext):
        if v0 - Q_EPS <= -cuv * u / cvv <= v1 + Q_EPS:
            us.append(u)
    if not us:
        return lo, lo
    first = math.floor((pu + min(us)) / BLOCK)
    last = math.floor((pu + max(us)) / BLOCK) + 1
    return max(lo, min(hi, first)), max(lo, min(hi, last))


def accutile_tiles(point, conic, opacity):
    r = snug_rect(point, conic, opacity)
    sx, sy = r[2] - r[0], r[3] - r[1]
    if sx * sy <= 1:
        return {(x, y) for y in range(r[1], r[3]) for x in range(r[0], r[2])}
    t = threshold_of(opacity)
    a, b, c = conic
    out = set()
    if sy <= sx:
        for y in range(r[1], r[3]):
            lo, hi = band_tiles(point[0], point[1], a, b, c, t, y, r[0], r[2])
            out.update((x, y) for x in range(lo, hi))
    else:
        for x in range(r[0], r[2]):
            lo, hi = band_tiles(point[1], point[0], c, b, a, t, x, r[1], r[3])
            out.update((x, y) for y in range(lo, hi))
    return out


def accepted_tiles(point, conic, opacity):
    """Tiles of every pixel centre whose exponent reaches the cut-off, inside the 3-sigma rect."""
    a, b, c = conic
    r = cuda_radius(cov_of(conic))
    outer = rect(point[0], point[1], r, r)
    ys, xs = np.mgrid[0:H, 0:W].astype(np.float64)
    dx, dy = xs - point[0], ys - point[1]
    q = a * dx * dx + 2.0 * b * dx * dy + c * dy * dy
    ok = q <= threshold_of(opacity)
    tx, ty = xs.astype(int) // BLOCK, ys.astype(int) // BLOCK
    ok &= (tx >= outer[0]) & (tx < outer[2]) & (ty >= outer[1]) & (ty < outer[3])
    return set(zip(tx[ok].tolist(), ty[ok].tolist()))


def oracle_tiles(cases, mode):
    """Tile sets emitted by the C oracle, one set per case, and its per-case counts."""
    pts = np.array([p for p, _, _ in cases], dtype=np.float32)
    cov = np.array([cov_of(c) for _, c, _ in cases], dtype=np.float32)
    co = np.array([(*c, o) for _, c, o in cases], dtype=np.float32)
    radii = np.array([cuda_radius(cov_of(c)) for _, c, _ in cases], dtype=np.int32)
    counts = oracle.count_covered_tiles(pts, cov, co, radii, GX, GY, mode)
    tiles, points, offsets = oracle.emit_covered_tiles(pts, cov, co, radii, GX, GY, mode)
    sets = [set() for _ in cases]
    for t, p in zip(tiles.tolist(), points.tolist()):
        sets[p].add((t % GX, t // GX))
    return sets, counts, tiles, points, offsets


@pytest.fixture(scope="module")
def cases():
    return seeded_cases()


@pytest.fixture(scope="module")
def emitted(cases):
    return {name: oracle_tiles(cases, mode) for name, mode in MODES.items()}


def test_case_generator_gives_positive_definite_conics(cases):
    assert len(cases) == 253
    for _point, (a, b, c), opacity in cases:
        assert a > 0.0 and c > 0.0 and a * c - b * b > 0.0 and 0.0 < opacity < 1.0


def test_exact_modes_cover_every_accepted_pixel_tile(cases, emitted):
    snug_sets = emitted["snugbox"][0]
    for mode in ("accutile_sweep", "conic_rect"):
        sets = emitted[mode][0]
        for i, (point, conic, opacity) in enumerate(cases):
            expected = accepted_tiles(point, conic, opacity)
            assert expected <= snug_sets[i], (i, expected - snug_sets[i])
            assert expected <= sets[i], (mode, i, expected - sets[i])
            assert sets[i] <= snug_sets[i], (mode, i, sets[i] - snug_sets[i])


def test_snugbox_is_the_float64_rectangle(cases, emitted):
    sets = emitted["snugbox"][0]
    for i, (point, conic, opacity) in enumerate(cases):
        r = snug_rect(point, conic, opacity)
        assert sets[i] == {(x, y) for y in range(r[1], r[3]) for x in range(r[0], r[2])}, i


def test_accutile_matches_float64_sweep(cases, emitted):
    """The float32 sweep reproduces the float64 restatement tile for tile on
    every seeded case (an interval end within rounding of a tile edge would
    show up here as a one-tile difference)."""
    sets = emitted["accutile_sweep"][0]
    for i, (point, conic, opacity) in enumerate(cases):
        ref = accutile_tiles(point, conic, opacity)
        assert sets[i] == ref, (i, sets[i] ^ ref)


def conic_rect_hits(point, conic, t, tx, ty):
    """Minimum of the conic form over the tile's pixel-centre rectangle, from
    the clamped stationary points on its four edges, against t + Q_EPS."""
    a, b, c = conic
    x0, x1 = tx * BLOCK - point[0], tx * BLOCK + BLOCK - 1 - point[0]
    y0, y1 = ty * BLOCK - point[1], ty * BLOCK + BLOCK - 1 - point[1]
    if x0 <= 0.0 <= x1 and y0 <= 0.0 <= y1:
        return True
    q = []
    for x in (x0, x1):
        y = min(y1, max(y0, -b * x / c))
        q.append(a * x * x + 2.0 * b * x * y + c * y * y)
    for y in (y0, y1):
        x = min(x1, max(x0, -b * y / a))
        q.append(a * x * x + 2.0 * b * x * y + c * y * y)
    return min(q) <= t + Q_EPS


def test_conic_rect_matches_float64_test(cases, emitted):
    sets = emitted["conic_rect"][0]
    for i, (point, conic, opacity) in enumerate(cases):
        r = snug_rect(point, conic, opacity)
        if (r[2] - r[0]) * (r[3] - r[1]) <= 1:
            ref = {(x, y) for y in range(r[1], r[3]) for x in range(r[0], r[2])}
        else:
            t = threshold_of(opacity)
            ref = {(x, y) for y in range(r[1], r[3]) for x in range(r[0], r[2])
                   if conic_rect_hits(point, conic, t, x, y)}
        assert sets[i] == ref, (i, sets[i] ^ ref)


def test_accutile_is_strictly_tighter_somewhere(cases, emitted):
    """A coverage that silently fell back to the rectangle would pass the
    subset checks; the sweep must drop tiles on elongated rotated footprints."""
    acc = sum(len(s) for s in emitted["accutile_sweep"][0])
    snug = sum(len(s) for s in emitted["snugbox"][0])
    rect = sum(len(s) for s in emitted["conic_rect"][0])
    assert acc < snug and rect < snug


def test_count_equals_emitted_pairs(cases, emitted):
    for name in MODES:
        _sets, counts, tiles, points, offsets = emitted[name]
        assert int(counts.sum()) == tiles.size == points.size
        assert np.all((tiles >= 0) & (tiles < GX * GY))
        starts = np.concatenate([[0], offsets[:-1]])
        for i, (s, e) in enumerate(zip(starts, offsets)):
            assert np.all(points[s:e] == i)


def test_boundary_points_and_cutoff_opacities():
    """Count/emit agreement at tile-edge centres and at opacities one ulp
    either side of 1/255 (test_rasterizer_cuda_contracts.py:176-336): the
    sub-cut-off Gaussian covers no tile, every other one covers some."""
    below16 = float(np.nextafter(np.float32(16.0), np.float32(-np.inf)))
    above16 = float(np.nextafter(np.float32(16.0), np.float32(np.inf)))
    cut = np.float32(1.0 / 255.0)
    below_cut = float(np.nextafter(cut, np.float32(-np.inf)))
    above_cut = float(np.nextafter(cut, np.float32(np.inf)))
    pts = np.array([[below16, below16], [16.0, 16.0], [above16, above16], [31.999, 48.001], [64.0, 63.999],
                    [1.0, 126.0]], dtype=np.float32)
    cov = np.array([[20.0, 8.0, 12.0], [20.0, -8.0, 12.0], [0.5, 0.49, 0.5], [80.0, 0.0, 0.4], [0.4, -0.15, 30.0],
                    [4.0, 1.5, 4.0]], dtype=np.float32)
    det = cov[:, 0] * cov[:, 2] - cov[:, 1] ** 2
    conic = np.stack([cov[:, 2] / det, -cov[:, 1] / det, cov[:, 0] / det], axis=1)
    opac = np.array([0.8, 0.8, 0.3, 0.5, above_cut, below_cut], dtype=np.float32)
    co = np.concatenate([conic, opac[:, None]], axis=1).astype(np.float32)
    tr = cov[:, 0] + cov[:, 2]
    lam = 0.5 * tr + np.sqrt(np.maximum(0.25 * tr * tr - det, 0.0))
    radii = np.ceil(3.0 * np.sqrt(lam)).astype(np.int32)
    for mode in MODES.values():
        counts = oracle.count_covered_tiles(pts, cov, co, radii, 8, 8, mode)
        tiles, points, offsets = oracle.emit_covered_tiles(pts, cov, co, radii, 8, 8, mode)
        assert counts[-1] == 0
        assert np.all(counts[:-1] > 0)
        assert tiles.size == int(counts.sum())
        assert np.all((tiles >= 0) & (tiles < 64))


def test_zero_radius_emits_nothing():
    pts = np.array([[8.0, 8.0]], dtype=np.float32)
    cov = np.array([[4.0, 0.0, 4.0]], dtype=np.float32)
    co = np.array([[0.25, 0.0, 0.25, 0.9]], dtype=np.float32)
    for mode in MODES.values():
        tiles, _points, _offsets = oracle.emit_covered_tiles(pts, cov, co, np.array([0], np.int32), 4, 4, mode)
        assert tiles.size == 0
