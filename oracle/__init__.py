"""CPU oracle for the rasterizer path — TEST INFRASTRUCTURE ONLY.

This package restates the fancifulland2718/gswarp 1.1.0 rasterizer (Warp
backend) in plain C (``gs_oracle.c``) and exposes it through ctypes/numpy.
Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker or the timed CPU
baseline.  The product package ``gswarp_amd`` never imports it.

Every wrapper takes and returns numpy arrays (float32 / int32, C-contiguous).
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
SOURCE = ORACLE_DIR / "gs_oracle.c"
# GS_ORACLE_LIB selects another build of the same source (the sanitizer
# build of oracle/sanitize.sh).
LIB_PATH = Path(os.environ.get("GS_ORACLE_LIB", ORACLE_DIR / "libgs_oracle.so"))

CFLAGS = (
    "-O2",
    "-std=c11",
    "-fPIC",
    "-shared",
    "-fopenmp",
    "-ffp-contract=off",
    "-mfma",
    "-fno-fast-math",
    "-fno-finite-math-only",
)

BLOCK = 16

_lib = None


def build(verbose: bool = False) -> Path:
    """Compile gs_oracle.c with gcc into libgs_oracle.so next to it."""
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = ["gcc", *CFLAGS, str(SOURCE), "-o", str(tmp), "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


_F = ctypes.POINTER(ctypes.c_float)
_D = ctypes.POINTER(ctypes.c_double)
_I = ctypes.POINTER(ctypes.c_int)
_c_int = ctypes.c_int
_c_float = ctypes.c_float
_c_ll = ctypes.c_longlong

_SIGNATURES = {
    "or_exp": (_c_float, [_c_float]),
    "or_log": (_c_float, [_c_float]),
    "or_count_covered_tiles": (None, [_c_int, _F, _F, _F, _I, _c_int, _c_int, _c_int, _I]),
    "or_emit_covered_tiles": (None, [_c_int, _F, _F, _F, _I, _c_int, _c_int, _c_int, _I, _I, _I]),
    "or_preprocess": (
        None,
        [_c_int, _c_int, _c_int, _F, _F, _F, _F, _c_float, _F, _F, _F, _F, _F, _F, _c_float, _c_float, _c_float,
         _c_float, _c_int, _c_int, _c_int, _c_float, _I, _F, _F, _F, _F, _I, _F, _F, _I, _I],
    ),
    "or_mark_visible": (None, [_c_int, _F, _F, _I]),
    "or_num_rendered": (_c_ll, [_c_int, _I]),
    "or_binning": (None, [_c_int, _I, _F, _I, _F, _F, _F, _c_int, _c_int, _c_int, _c_ll, _I, _I, _I]),
    "or_render_fwd": (
        None,
        [_c_int, _c_int, _I, _I, _F, _F, _F, _F, _F, _c_int, _c_int, _F, _F, _F, _I, _I, _F, _F],
    ),
    "or_render_bwd": (
        None,
        [_c_int, _c_int, _c_int, _I, _I, _F, _F, _F, _F, _F, _F, _I, _F, _F, _F, _c_int, _c_int, _F, _D, _D, _D],
    ),
    "or_preprocess_bwd": (
        None,
        [_c_int, _c_int, _c_int, _F, _F, _F, _c_float, _F, _F, _F, _I, _F, _F, _c_float, _c_float, _c_float,
         _c_float, _I, _F, _F, _F, _F, _c_int, _c_int, _c_float, _F, _F, _F, _F, _F, _F],
    ),
    "or_num_threads": (_c_int, []),
    "or_set_num_threads": (None, [_c_int]),
}


def lib():
    """Load (building first if absent) the oracle shared library."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int32)


def _fp(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(_F)


def _ip(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(_I)


def _dp(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(_D)


def exp(x: float) -> float:
    return float(lib().or_exp(float(x)))


def log(x: float) -> float:
    return float(lib().or_log(float(x)))


def grid_dims(width: int, height: int) -> tuple[int, int]:
    return (width + BLOCK - 1) // BLOCK, (height + BLOCK - 1) // BLOCK


def set_num_threads(n: int) -> None:
    lib().or_set_num_threads(int(n))


def num_threads() -> int:
    return int(lib().or_num_threads())


def count_covered_tiles(points_xy, cov2d, conic_opacity, radii, grid_x, grid_y, mode=1) -> np.ndarray:
    points_xy, cov2d, conic_opacity, radii = _f32(points_xy), _f32(cov2d), _f32(conic_opacity), _i32(radii)
    n = radii.shape[0]
    out = np.zeros(n, dtype=np.int32)
    lib().or_count_covered_tiles(n, _fp(points_xy), _fp(cov2d), _fp(conic_opacity), _ip(radii), grid_x, grid_y,
                                 mode, _ip(out))
    return out


def emit_covered_tiles(points_xy, cov2d, conic_opacity, radii, grid_x, grid_y, mode=1):
    """(tile_ids, point_list, inclusive offsets) in point order."""
    points_xy, cov2d, conic_opacity, radii = _f32(points_xy), _f32(cov2d), _f32(conic_opacity), _i32(radii)
    counts = count_covered_tiles(points_xy, cov2d, conic_opacity, radii, grid_x, grid_y, mode)
    counts = np.where(radii > 0, counts, 0).astype(np.int32)
    offsets = np.cumsum(counts, dtype=np.int64).astype(np.int32)
    total = int(offsets[-1]) if offsets.size else 0
    tiles = np.full(total, -1, dtype=np.int32)
    points = np.full(total, -1, dtype=np.int32)
    n = radii.shape[0]
    lib().or_emit_covered_tiles(n, _fp(points_xy), _fp(cov2d), _fp(conic_opacity), _ip(radii), grid_x, grid_y,
                                mode, _ip(offsets), _ip(tiles), _ip(points))
    return tiles, points, offsets


def preprocess(means3d, scales, rotations, opacities, view, proj, campos, *, tanfovx, tanfovy, width, height,
               scale_modifier=1.0, shs=None, degree=0, colors=None, coverage_mode=1, cov3d_precomp=None,
               filter_variance=0.0) -> dict:
    """Reference preprocess + SH colour: the fused scales/rotations path, or the
    masked path for precomputed 3D covariances (cov3d_precomp (N, 6)); a
    non-zero filter_variance applies the Mip-Splatting screen-space filter."""
    means3d = _f32(means3d)
    if cov3d_precomp is not None:
        cov3d_precomp = _f32(cov3d_precomp).reshape(-1, 6)
        scales = rotations = None
    else:
        scales, rotations = _f32(scales), _f32(rotations)
    opacities = _f32(opacities).reshape(-1)
    view, proj, campos = _f32(view).reshape(16), _f32(proj).reshape(16), _f32(campos).reshape(3)
    P = means3d.shape[0]
    K = 0
    if shs is not None:
        shs = _f32(shs).reshape(P, -1, 3)
        K = shs.shape[1]
    if colors is not None:
        colors = _f32(colors).reshape(P, 3)
    focal_x = np.float32(width / (2.0 * tanfovx))
    focal_y = np.float32(height / (2.0 * tanfovy))
    out = {
        "radii": np.zeros(P, np.int32),
        "depths": np.zeros(P, np.float32),
        "proj_2d": np.zeros((P, 2), np.float32),
        "conic_2d": np.zeros((P, 3), np.float32),
        "conic_2d_inv": np.zeros((P, 3), np.float32),
        "tiles_touched": np.zeros(P, np.int32),
        "cov3d": np.zeros((P, 6), np.float32),
        "rgb": np.zeros((P, 3), np.float32),
        "clamped": np.zeros((P, 3), np.int32),
        "visible": np.zeros(P, np.int32),
    }
    lib().or_preprocess(
        P, K, degree, _fp(means3d), _fp(scales), _fp(rotations), _fp(cov3d_precomp), float(scale_modifier),
        _fp(opacities),
        _fp(shs), _fp(colors), _fp(view), _fp(proj), _fp(campos), float(np.float32(tanfovx)),
        float(np.float32(tanfovy)), float(focal_x), float(focal_y), width, height, coverage_mode,
        float(np.float32(filter_variance)), _ip(out["radii"]), _fp(out["depths"]), _fp(out["proj_2d"]), _fp(out["conic_2d"]), _fp(out["conic_2d_inv"]),
        _ip(out["tiles_touched"]), _fp(out["cov3d"]), _fp(out["rgb"]), _ip(out["clamped"]), _ip(out["visible"]))
    out["conic_opacity"] = np.concatenate([out["conic_2d"], opacities.reshape(P, 1)], axis=1)
    out["conic_opacity"][out["radii"] <= 0] = 0.0
    return out


def mark_visible(means3d, view) -> np.ndarray:
    means3d, view = _f32(means3d), _f32(view).reshape(16)
    out = np.zeros(means3d.shape[0], np.int32)
    lib().or_mark_visible(means3d.shape[0], _fp(means3d), _fp(view), _ip(out))
    return out.astype(bool)


def binning(pre: dict, width: int, height: int, coverage_mode=1) -> dict:
    """Reference binning (depth sort, scan, duplicate, tile sort, ranges)."""
    radii = _i32(pre["radii"])
    P = radii.shape[0]
    tiles_touched = _i32(pre["tiles_touched"])
    R = int(lib().or_num_rendered(P, _ip(tiles_touched)))
    grid_x, grid_y = grid_dims(width, height)
    point_list = np.zeros(max(R, 1), np.int32)
    tile_ids = np.zeros(max(R, 1), np.int32)
    ranges = np.zeros((grid_x * grid_y, 2), np.int32)
    lib().or_binning(P, _ip(radii), _fp(_f32(pre["depths"])), _ip(tiles_touched), _fp(_f32(pre["proj_2d"])),
                     _fp(_f32(pre["conic_2d_inv"])), _fp(_f32(pre["conic_opacity"])), width, height, coverage_mode,
                     R, _ip(point_list), _ip(tile_ids), _ip(ranges))
    return {"num_rendered": R, "point_list": point_list[:R], "tile_ids": tile_ids[:R], "ranges": ranges}


def render_fwd(pre: dict, bins: dict, features, background, width, height, *, compute_depth=True, top_k=0) -> dict:
    features = _f32(features).reshape(-1, 3)
    bg = _f32(background).reshape(3)
    P = width * height
    out = {
        "color": np.zeros((3, height, width), np.float32),
        "depth": np.zeros((1, height, width), np.float32),
        "alpha": np.zeros((1, height, width), np.float32),
        "n_contrib": np.zeros((height, width), np.int32),
    }
    ids = weights = x_mu = None
    if top_k > 0:
        ids = np.zeros((top_k, height, width), np.int32)
        weights = np.zeros((top_k, height, width), np.float32)
        x_mu = np.zeros((2, top_k, height, width), np.float32)
    point_list = _i32(bins["point_list"]) if bins["num_rendered"] > 0 else np.zeros(1, np.int32)
    lib().or_render_fwd(width, height, _ip(_i32(bins["ranges"])), _ip(point_list), _fp(_f32(pre["proj_2d"])),
                        _fp(features), _fp(_f32(pre["depths"])), _fp(_f32(pre["conic_opacity"])), _fp(bg),
                        int(bool(compute_depth)), int(top_k), _fp(out["color"]), _fp(out["depth"]),
                        _fp(out["alpha"]), _ip(out["n_contrib"]), _ip(ids), _fp(weights), _fp(x_mu))
    del P
    if top_k > 0:
        out.update(gs_per_pixel=ids, weight_per_gs_pixel=weights, x_mu=x_mu)
    return out


def render_bwd(pre: dict, bins: dict, features, background, width, height, fwd: dict, grad_color, grad_depth,
               grad_alpha, *, compute_depth=True, bound=False, value_mode=0):
    """Per-Gaussian (N, 10) render gradients: dx, dy, conic a, b, c, opacity, rgb, depth.

    With bound=True also returns (err, mag), two (N, 10) float64 arrays: the
    summed first-order bound on the fp32 rounding of each column's per-pixel
    terms under any evaluation order, and the summed term magnitudes (every
    sum in absolute values), which scale the rounding of summing the terms.
    value_mode 1 (double values from the fp32 inputs) and 2 (a second fp32
    evaluation order) return the float64 sums instead of float32; they exist
    to check that bound.
    """
    features = _f32(features).reshape(-1, 3)
    N = features.shape[0]
    out = np.zeros((N, 10), np.float32)
    out64 = np.zeros((N, 10), np.float64) if value_mode else None
    err = np.zeros((N, 10), np.float64) if bound else None
    mag = np.zeros((N, 10), np.float64) if bound else None
    point_list = _i32(bins["point_list"]) if bins["num_rendered"] > 0 else np.zeros(1, np.int32)
    lib().or_render_bwd(width, height, N, _ip(_i32(bins["ranges"])), _ip(point_list), _fp(_f32(pre["proj_2d"])),
                        _fp(features), _fp(_f32(pre["depths"])), _fp(_f32(pre["conic_opacity"])),
                        _fp(_f32(background).reshape(3)), _fp(_f32(fwd["alpha"])), _ip(_i32(fwd["n_contrib"])),
                        _fp(_f32(grad_color)), _fp(_f32(grad_depth)), _fp(_f32(grad_alpha)),
                        int(bool(compute_depth)), int(value_mode), _fp(out), _dp(out64), _dp(err), _dp(mag))
    res = out64 if value_mode else out
    if bound:
        return res, err, mag
    return res


def preprocess_bwd(pre: dict, grad_gauss, means3d, scales, rotations, view, proj, campos, *, tanfovx, tanfovy,
                   width, height, scale_modifier=1.0, shs=None, degree=0, grad_proj_2d=None, grad_conic_2d=None,
                   grad_conic_2d_inv=None, flow_double=False, cov3d_precomp=None, filter_variance=0.0) -> dict:
    means3d = _f32(means3d)
    precomp = cov3d_precomp is not None
    if not precomp:
        scales, rotations = _f32(scales), _f32(rotations)
    else:
        scales = rotations = None
    P = means3d.shape[0]
    K = 0
    if shs is not None:
        shs = _f32(shs).reshape(P, -1, 3)
        K = shs.shape[1]
    zeros = lambda *s: np.zeros(s, np.float32)  # noqa: E731
    grad_proj_2d = zeros(P, 2) if grad_proj_2d is None else _f32(grad_proj_2d)
    grad_conic_2d = zeros(P, 3) if grad_conic_2d is None else _f32(grad_conic_2d)
    grad_conic_2d_inv = zeros(P, 3) if grad_conic_2d_inv is None else _f32(grad_conic_2d_inv)
    focal_x = np.float32(width / (2.0 * tanfovx))
    focal_y = np.float32(height / (2.0 * tanfovy))
    out = {
        "means3D": zeros(P, 3),
        "means2D": zeros(P, 3),
        "scales": zeros(P, 3),
        "rotations": zeros(P, 4),
        "cov3D": zeros(P, 6),
        "sh": zeros(P, max(K, 1), 3)[:, :K],
    }
    out["sh"] = np.ascontiguousarray(out["sh"])
    lib().or_preprocess_bwd(
        P, K, degree, _fp(means3d), _fp(scales), _fp(rotations), float(scale_modifier), _fp(_f32(pre["cov3d"])),
        _fp(shs), _fp(_f32(campos).reshape(3)), _ip(_i32(pre["clamped"])), _fp(_f32(view).reshape(16)),
        _fp(_f32(proj).reshape(16)), float(np.float32(tanfovx)), float(np.float32(tanfovy)), float(focal_x),
        float(focal_y), _ip(_i32(pre["radii"])), _fp(_f32(grad_gauss)), _fp(grad_proj_2d), _fp(grad_conic_2d),
        _fp(grad_conic_2d_inv), int(bool(flow_double)), int(precomp), float(np.float32(filter_variance)),
        _fp(out["means3D"]), _fp(out["means2D"]),
        _fp(out["scales"]), _fp(out["rotations"]), _fp(out["cov3D"]), _fp(out["sh"]) if K > 0 else None)
    gg = _f32(grad_gauss)
    out["opacities"] = gg[:, 5:6].copy()
    out["colors"] = gg[:, 6:9].copy()
    return out


def rasterize(scene: dict, *, coverage_mode=1, compute_depth=True, top_k=0) -> dict:
    """Full forward on a scene dict (numpy arrays) as produced by gswarp_amd.configs."""
    s = scene
    pre = preprocess(s["means3D"], s.get("scales"), s.get("rotations"), s["opacities"], s["viewmatrix"],
                     s["projmatrix"], s["campos"], tanfovx=s["tanfovx"], tanfovy=s["tanfovy"], width=s["width"],
                     height=s["height"], scale_modifier=s.get("scale_modifier", 1.0), shs=s.get("shs"),
                     degree=s.get("sh_degree", 0), colors=s.get("colors_precomp"), coverage_mode=coverage_mode,
                     cov3d_precomp=s.get("cov3D_precomp"), filter_variance=s.get("filter_variance", 0.0))
    bins = binning(pre, s["width"], s["height"], coverage_mode)
    fwd = render_fwd(pre, bins, pre["rgb"], s["bg"], s["width"], s["height"], compute_depth=compute_depth,
                     top_k=top_k)
    return {"pre": pre, "bins": bins, "fwd": fwd}


# Unit roundoff of binary32.
U32 = 2.0 ** -24
# Partial sums per (tile, Gaussian) and gradient component that an fp32
# implementation may add up in an arbitrary order (one per pixel slice of a
# tile that visits the Gaussian; four 16x4 slices at most).
PARTIALS_PER_TILE = 4
# Depth of the summation tree inside one partial sum (pixels of a lane, lane
# folds, a quad of slots and its shuffles).
TREE_DEPTH = 8
# Rounding of the per-Gaussian chain itself (SH, projection, cov2D -> cov3D ->
# scale / rotation), in units of u times the magnitude of its linear output.
CHAIN_DEPTH = 64

_OUTPUT_KEYS = ("means3D", "means2D", "scales", "rotations", "cov3D", "sh")


def _backward_chain(scene, pre, gg, grad_proj_2d=None, grad_conic_2d=None, grad_conic_2d_inv=None,
                    flow_double=False) -> dict:
    s = scene
    return preprocess_bwd(pre, gg, s["means3D"], s.get("scales"), s.get("rotations"), s["viewmatrix"],
                          s["projmatrix"], s["campos"], tanfovx=s["tanfovx"], tanfovy=s["tanfovy"],
                          width=s["width"], height=s["height"], scale_modifier=s.get("scale_modifier", 1.0),
                          shs=s.get("shs"), degree=s.get("sh_degree", 0), grad_proj_2d=grad_proj_2d,
                          grad_conic_2d=grad_conic_2d, grad_conic_2d_inv=grad_conic_2d_inv,
                          flow_double=flow_double, cov3d_precomp=s.get("cov3D_precomp"),
                          filter_variance=s.get("filter_variance", 0.0))


def gradient_bound(scene: dict, result: dict, gg, err, mag, *, grad_proj_2d=None, grad_conic_2d=None,
                   grad_conic_2d_inv=None, flow_double=False) -> dict:
    """Per-element bound on |fp32 implementation - oracle| for every output gradient.

    The render stage's bound per Gaussian and column is
        B = 2 err + (TREE_DEPTH + PARTIALS_PER_TILE tiles_touched) u mag
    (each side errs by at most err in its terms; the summation of the terms,
    in any order over that many partial sums, by the second part).  The
    per-Gaussian backward is linear in the render gradients, so B reaches
    each output through the absolute value of its Jacobian: column k's
    Jacobian J_k is the backward of a unit render gradient in column k alone
    (Gaussians are independent, so one run gives it for all of them), and
    the bound is  sum_k |J_k| B_k + CHAIN_DEPTH u (M + max M over the Gaussian's
    components of the same output), M = sum_k |J_k| |g_k| + |J_meta g_meta|: the
    rounding of the chain itself, whose intermediate values are on the scale
    of the Gaussian's largest output component.  Returns a dict of float64
    arrays keyed like the gradients (plus "grad_gauss").
    """
    pre = result["pre"]
    tt = np.asarray(pre["tiles_touched"], np.float64)[:, None]
    B = 2.0 * err + (TREE_DEPTH + PARTIALS_PER_TILE * tt) * U32 * mag
    N = gg.shape[0]
    out = {"grad_gauss": B, "opacities": B[:, 5:6].copy(), "colors": B[:, 6:9].copy()}
    acc_b = {}
    acc_m = {}
    zeros_meta = dict(grad_proj_2d=np.zeros((N, 2), np.float32), grad_conic_2d=np.zeros((N, 3), np.float32),
                      grad_conic_2d_inv=np.zeros((N, 3), np.float32))
    absg = np.abs(gg)
    B32 = B.astype(np.float32)  # bound arithmetic needs a few significant digits, not 16

    def add(acc, key, value, index=None):
        if key not in acc:
            acc[key] = np.zeros(value.shape if index is None else jac_shapes[key], np.float32)
        if index is None:
            acc[key] += value
        else:
            acc[key][index] += value

    jac_shapes = {}
    for k in range(10):
        # column 5 (opacity) leaves the chain untouched; only the colour columns reach the SH gradients
        if k == 5 or (not np.any(B[:, k]) and not np.any(gg[:, k])):
            continue
        unit = np.zeros((N, 10), np.float32)
        unit[:, k] = 1.0
        jac = _backward_chain(scene, pre, unit, flow_double=flow_double, **zeros_meta)
        for key in _OUTPUT_KEYS:
            if key == "sh":
                if k not in (6, 7, 8) or not jac[key].size:
                    continue
                # colour channel c reaches only the channel-c SH coefficients
                jac_shapes[key] = jac[key].shape
                index = (slice(None), slice(None), k - 6)
                a = np.abs(jac[key][index])
                add(acc_b, key, a * B32[:, k:k + 1], index)
                add(acc_m, key, a * absg[:, k:k + 1], index)
                continue
            a = np.abs(jac[key])
            if not a.size or not a.any():
                continue
            shape = (-1,) + (1,) * (a.ndim - 1)
            add(acc_b, key, a * B32[:, k].reshape(shape))
            add(acc_m, key, a * absg[:, k].reshape(shape))
    meta = {"grad_proj_2d": grad_proj_2d, "grad_conic_2d": grad_conic_2d, "grad_conic_2d_inv": grad_conic_2d_inv}
    for name, value in meta.items():
        if value is None or not np.any(value):
            continue
        args = dict(zeros_meta)
        args[name] = np.ascontiguousarray(value, np.float32)
        part = _backward_chain(scene, pre, np.zeros((N, 10), np.float32), flow_double=flow_double, **args)
        for key in _OUTPUT_KEYS:
            if part[key].size:
                add(acc_m, key, np.abs(part[key]))
    for key in _OUTPUT_KEYS:
        m = acc_m.get(key, 0.0)
        if np.ndim(m):
            # intermediate values of one Gaussian's chain (dL/dcov3D, dL/dM, ...) are on the scale of its
            # largest output component, so a component that cancels to near zero still errs by that much
            m = m + m.reshape(m.shape[0], -1).max(axis=1, initial=0.0).reshape((-1,) + (1,) * (m.ndim - 1))
        b = acc_b.get(key, 0.0) + CHAIN_DEPTH * U32 * m
        out[key] = np.asarray(b, np.float64)  # a scalar 0 where no column reaches this output
    return out


def rasterize_backward(scene: dict, result: dict, grad_color, grad_depth, grad_alpha, *, compute_depth=True,
                       grad_proj_2d=None, grad_conic_2d=None, grad_conic_2d_inv=None, flow_double=False,
                       with_bound=False) -> dict:
    """Full backward matching the reference's gradient tuple (as a dict).

    with_bound=True adds grads["bound"]: gradient_bound() of every output.
    """
    s = scene
    pre, bins, fwd = result["pre"], result["bins"], result["fwd"]
    rb = render_bwd(pre, bins, pre["rgb"], s["bg"], s["width"], s["height"], fwd, grad_color,
                    grad_depth if grad_depth is not None else np.zeros_like(fwd["depth"]), grad_alpha,
                    compute_depth=compute_depth, bound=with_bound)
    gg = rb[0] if with_bound else rb
    grads = _backward_chain(s, pre, gg, grad_proj_2d=grad_proj_2d, grad_conic_2d=grad_conic_2d,
                            grad_conic_2d_inv=grad_conic_2d_inv, flow_double=flow_double)
    grads["grad_gauss"] = gg
    if with_bound:
        bound = gradient_bound(s, result, gg, rb[1], rb[2], grad_proj_2d=grad_proj_2d,
                               grad_conic_2d=grad_conic_2d, grad_conic_2d_inv=grad_conic_2d_inv,
                               flow_double=flow_double)
        grads["bound"] = {k: np.broadcast_to(v, grads[k].shape).copy() if k in grads else v
                          for k, v in bound.items()}
    return grads
