"""Pins the C oracle's preprocess, SH, binning, render and backward.

The reference cannot run here (its kernels need NVIDIA Warp, which is not
installed), so each oracle function is checked against what fixes it
independently:

* exp / log against libm;
* preprocess against closed forms (identity rotation and view: cov2D =
  (f/z)^2 s^2 + 0.3, conic its inverse, radius from the larger eigenvalue) and
  against the float64 matrix-form restatement in dense_ref.py;
* SH against the float64 basis and the degree-0 special case;
* binning against a brute-force numpy lexsort of the emitted pairs;
* render against single-Gaussian closed-form compositing
  (test_rasterizer_cuda_contracts.py:482-505), an empty scene, the depth-off
  invariance (test_rasterizer_cuda_contracts.py:129-174) and the dense
  float64 blend, flow top-K included;
* backward against torch.autograd through the float64 restatement, and the
  flow doubling (flow_ops.py:337-360 with backward_kernels.py:95-98).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import dense_ref
import oracle
from gswarp_amd import configs
from helpers import grad_mismatch

BLOCK = 16


def tiny_scene(seed: int, n: int = 40, width: int = 64, height: int = 48, degree: int = 3, spread: float = 0.6,
               log_scale: float = -2.3) -> dict:
    """Small world-space scene seen by a rotated camera (numpy float32 arrays)."""
    g = torch.Generator().manual_seed(seed)
    means = torch.randn(n, 3, generator=g) * spread
    scales = torch.exp(torch.randn(n, 3, generator=g) * 0.4 + log_scale)
    quats = torch.randn(n, 4, generator=g)
    quats = quats / quats.norm(dim=1, keepdim=True) * (0.8 + 0.4 * torch.rand(n, 1, generator=g))
    opac = torch.clamp(torch.sigmoid(torch.randn(n, 1, generator=g)), 0.05, 0.95)
    shs = torch.randn(n, (degree + 1) ** 2, 3, generator=g) * 0.2
    shs[:, 0] = torch.randn(n, 3, generator=g) * 0.5
    fov = math.radians(55.0)
    fovy = 2.0 * math.atan(math.tan(fov / 2) * height / width)
    cam = configs.camera(width, height, fov, fovy, configs.look_at((0.5, -0.4, -3.5)))
    bg = torch.tensor([0.1, 0.25, 0.4])
    scene = {"means3D": means, "scales": scales, "rotations": quats, "opacities": opac, "shs": shs,
             "sh_degree": degree, "bg": bg, "scale_modifier": 1.0, **cam}
    return {k: (v.numpy().astype(np.float32) if isinstance(v, torch.Tensor) else v) for k, v in scene.items()}


def t64(a):
    return torch.tensor(np.asarray(a, dtype=np.float64))


def dense_pre(s: dict, *, grad: bool = False):
    leaves = {k: t64(s[k]).requires_grad_(grad) for k in ("means3D", "scales", "rotations", "opacities", "shs")}
    pre = dense_ref.preprocess(leaves["means3D"], leaves["scales"], leaves["rotations"], t64(s["viewmatrix"]),
                               t64(s["projmatrix"]), t64(s["campos"]), s["tanfovx"], s["tanfovy"], s["width"],
                               s["height"], shs=leaves["shs"], degree=s["sh_degree"])
    return pre, leaves


def tile_sets_of(res: dict, n: int, width: int) -> list:
    """Tile ids each Gaussian is binned to, from the oracle's sorted lists."""
    sets = [set() for _ in range(n)]
    bins = res["bins"]
    for tile, pid in zip(bins["tile_ids"].tolist(), bins["point_list"].tolist()):
        sets[pid].add(tile)
    return sets


# ---------------------------------------------------------------- math

def test_exp_matches_libm():
    # within 0.9 ulp (every float of [-87, 0] was checked against a long double
    # exp); 0.9 ulp is at most 1.08e-7 relative
    xs = np.concatenate([np.linspace(-87.0, 88.0, 20001), -np.logspace(-8, 1.9, 2000), [0.0, -1e-30]])
    for x in xs.astype(np.float32):
        got = oracle.exp(float(x))
        want = math.exp(float(x))
        assert abs(got - want) <= 1.1e-7 * want, (x, got, want)
    assert oracle.exp(-87.5) == 0.0


def test_log_matches_libm():
    ys = np.concatenate([np.logspace(-37, 38, 20001), np.linspace(0.5, 2.0, 4001)]).astype(np.float32)
    for y in ys:
        got = oracle.log(float(y))
        want = math.log(float(y))
        assert abs(got - want) <= 2e-7 * max(1.0, abs(want)), (y, got, want)


# ---------------------------------------------------------------- preprocess

def identity_camera(width=64, height=64, tan=1.0):
    view = np.eye(4, dtype=np.float32)
    return dict(view=view, proj=view.copy(), campos=np.zeros(3, np.float32), tanfovx=tan, tanfovy=tan,
                width=width, height=height)


def test_preprocess_closed_form_on_axis():
    """Identity view and projection (the reference tests' camera), identity
    rotation: cov2D = (f/z)^2 s^2 + 0.3, conic = its inverse, radius =
    ceil(3 sqrt(lambda_max)), pixel = ((ndc + 1) S - 1) / 2 with ndc = x / (w + 1e-7)."""
    cam = identity_camera()
    z, s = 2.0, 0.05
    means = np.array([[0.0, 0.0, z], [0.1, -0.2, z]], np.float32)
    scales = np.full((2, 3), s, np.float32)
    rots = np.tile(np.array([1, 0, 0, 0], np.float32), (2, 1))
    op = np.full((2, 1), 0.8, np.float32)
    pre = oracle.preprocess(means, scales, rots, op, cam["view"], cam["proj"], cam["campos"],
                            tanfovx=cam["tanfovx"], tanfovy=cam["tanfovy"], width=64, height=64,
                            colors=np.full((2, 3), 0.2, np.float32))
    f = 64 / 2.0
    var = (f / z) ** 2 * s * s + 0.3
    np.testing.assert_allclose(pre["conic_2d_inv"][0], [var, 0.0, var], rtol=1e-5)
    np.testing.assert_allclose(pre["conic_2d"][0], [1 / var, 0.0, 1 / var], rtol=1e-5)
    mid = var
    assert pre["radii"][0] == math.ceil(3.0 * math.sqrt(mid + math.sqrt(max(0.1, mid * mid - var * var))))
    assert pre["depths"][0] == np.float32(z)
    # identity projection: w = 1, ndc = (x, y) / (1 + 1e-7)
    ndc = np.array([0.1, -0.2]) / (1 + 1e-7)
    np.testing.assert_allclose(pre["proj_2d"][1], ((ndc + 1) * 64 - 1) * 0.5, rtol=1e-6)
    # the off-axis point's Jacobian adds the -f x / z^2 column
    J = np.array([[f / z, 0, -f * 0.1 / z**2], [0, f / z, f * 0.2 / z**2]])
    cov = J @ (np.eye(3) * s * s) @ J.T + 0.3 * np.eye(2)
    np.testing.assert_allclose(pre["conic_2d_inv"][1], [cov[0, 0], cov[0, 1], cov[1, 1]], rtol=1e-5)


def test_preprocess_culls_behind_near_plane_and_keeps_subthreshold_geometry():
    """z <= 0.2 culls with every output zero (test_rasterizer_cuda_contracts.py:355-366);
    a sub-threshold opacity keeps its radius but touches no tile
    (test_rasterizer_cuda_contracts.py:432-449)."""
    cam = identity_camera(16, 16)
    means = np.array([[0.0, 0.0, -2.0], [0.0, 0.0, 0.2], [0.0, 0.0, 2.0]], np.float32)
    scales = np.full((3, 3), 0.5, np.float32)
    rots = np.tile(np.array([1, 0, 0, 0], np.float32), (3, 1))
    op = np.array([[0.8], [0.8], [1e-4]], np.float32)
    for mode in (0, 1, 2):
        pre = oracle.preprocess(means, scales, rots, op, cam["view"], cam["proj"], cam["campos"], tanfovx=1.0,
                                tanfovy=1.0, width=16, height=16, colors=np.full((3, 3), 0.2, np.float32),
                                coverage_mode=mode)
        assert list(pre["radii"][:2]) == [0, 0]
        for key in ("depths", "proj_2d", "conic_2d", "conic_2d_inv", "tiles_touched"):
            assert not np.any(pre[key][:2]), key
        assert pre["radii"][2] > 0 and pre["tiles_touched"][2] == 0


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_preprocess_matches_float64_restatement(seed):
    s = tiny_scene(seed, n=200, spread=1.0)
    res = oracle.rasterize(s)
    pre, _ = dense_pre(s)
    op = res["pre"]
    vis = pre["radii"] > 0
    assert vis.sum() > 50
    # radii: equal unless 3 sqrt(lambda) sits within rounding of an integer
    a, b, c = (pre["cov2d"][:, i].detach().numpy() for i in range(3))
    mid = 0.5 * (a + c)
    lam = mid + np.sqrt(np.maximum(0.1, mid * mid - (a * c - b * b)))
    r3 = 3.0 * np.sqrt(lam)
    near_int = np.abs(r3 - np.round(r3)) < 1e-4
    assert np.array_equal(op["radii"][~near_int], pre["radii"][~near_int])
    v = vis & (op["radii"] > 0)
    np.testing.assert_allclose(op["depths"][v], pre["depth"].detach().numpy()[v], rtol=1e-6)
    np.testing.assert_allclose(op["proj_2d"][v], pre["pix"].detach().numpy()[v], atol=2e-4 * max(s["width"], 1))
    np.testing.assert_allclose(op["conic_2d_inv"][v], pre["cov2d"].detach().numpy()[v], rtol=2e-5, atol=1e-6)
    np.testing.assert_allclose(op["conic_2d"][v], pre["conic"].detach().numpy()[v], rtol=1e-4, atol=1e-7)
    # colour for every Gaussian (the reference evaluates SH for all N)
    np.testing.assert_allclose(op["rgb"], pre["rgb"].detach().numpy(), atol=2e-6)
    assert np.array_equal(op["clamped"].astype(bool), pre["clamped"].numpy())


@pytest.mark.parametrize("degree", [0, 1, 2, 3])
def test_sh_colour_against_float64_basis(degree):
    s = tiny_scene(7, n=64, degree=degree)
    res = oracle.rasterize(s)
    pre, _ = dense_pre(s)
    np.testing.assert_allclose(res["pre"]["rgb"], pre["rgb"].detach().numpy(), atol=2e-6)
    if degree == 0:
        dc = s["shs"][:, 0, :].astype(np.float64)
        np.testing.assert_allclose(res["pre"]["rgb"], np.maximum(0.28209479177387814 * dc + 0.5, 0.0), atol=1e-6)


# ---------------------------------------------------------------- binning

@pytest.mark.parametrize("mode", [0, 1, 2])
def test_binning_against_brute_force_sort(mode):
    s = tiny_scene(3, n=300, width=96, height=80, spread=1.2)
    res = oracle.rasterize(s, coverage_mode=mode)
    pre, bins = res["pre"], res["bins"]
    gx, gy = oracle.grid_dims(96, 80)
    tiles, points, _ = oracle.emit_covered_tiles(pre["proj_2d"], pre["conic_2d_inv"], pre["conic_opacity"],
                                                 pre["radii"], gx, gy, mode)
    depth_bits = pre["depths"].view(np.uint32)[points]
    order = np.lexsort((points, depth_bits, tiles))
    assert bins["num_rendered"] == tiles.size == int(pre["tiles_touched"][pre["radii"] > 0].sum())
    assert np.array_equal(bins["point_list"], points[order])
    assert np.array_equal(bins["tile_ids"], tiles[order])
    ranges = bins["ranges"]
    # ranges partition [0, R) in tile order; empty tiles are [0, 0)
    covered = 0
    for t in range(gx * gy):
        lo, hi = ranges[t]
        if hi > lo:
            assert lo == covered
            assert np.all(bins["tile_ids"][lo:hi] == t)
            d = pre["depths"][bins["point_list"][lo:hi]]
            assert np.all(np.diff(d) >= 0)
            covered = hi
        else:
            assert lo == hi == 0
    assert covered == bins["num_rendered"]


# ---------------------------------------------------------------- render

def test_render_single_rotated_gaussian_closed_form():
    """One Gaussian, per-pixel alpha = min(0.99, o e^power) cut at 1/255 and
    blended over the background (test_rasterizer_cuda_contracts.py:482-505)."""
    s = tiny_scene(11, n=1, width=64, height=64, spread=0.0, log_scale=-1.6)
    res = oracle.rasterize(s)
    pre = res["pre"]
    assert pre["radii"][0] > 0
    ys, xs = np.mgrid[0:64, 0:64].astype(np.float64)
    (px, py), (a, b, c), o = pre["proj_2d"][0], pre["conic_2d"][0], float(s["opacities"][0, 0])
    dx, dy = px - xs, py - ys
    power = -0.5 * (a * dx * dx + c * dy * dy) - b * dx * dy
    alpha = np.minimum(0.99, o * np.exp(power))
    alpha = np.where((alpha >= 1 / 255) & (power <= 0), alpha, 0.0)
    # pixels outside the binned tiles are not blended
    gx = 4
    tiles = set(res["bins"]["tile_ids"].tolist())
    in_tile = np.vectorize(lambda x, y: (y // 16) * gx + x // 16 in tiles)(xs.astype(int), ys.astype(int))
    alpha = np.where(in_tile, alpha, 0.0)
    rgb = pre["rgb"][0].astype(np.float64)
    expected = rgb[:, None, None] * alpha[None] + s["bg"].astype(np.float64)[:, None, None] * (1 - alpha[None])
    np.testing.assert_allclose(res["fwd"]["color"], expected, atol=2e-5, rtol=2e-4)
    np.testing.assert_allclose(res["fwd"]["alpha"][0], alpha, atol=2e-6)
    assert alpha.max() > 0.3


def test_render_alpha_cap_and_stop_rule_closed_form():
    """Opaque Gaussians centred on one pixel: alpha is capped at 0.99, so T
    falls to 1 - 0.99f = 0.0099999905 after the first; the second would leave
    T (1 - alpha) = 9.99998e-5 < 1e-4, so the pixel stops without it (and
    without the third), keeping n_contrib = 1 and T_final = 1 - 0.99f."""
    cam = identity_camera(32, 32)
    z = np.array([2.0, 2.5, 3.0], np.float32)
    x = np.full(3, (2 * 15 + 1) / 32 - 1, np.float32)  # identity projection: ndc = x, pixel 15
    means = np.stack([x, x, z], axis=1).astype(np.float32)
    scales = np.full((3, 3), 0.3, np.float32)
    rots = np.tile(np.array([1, 0, 0, 0], np.float32), (3, 1))
    rgb = np.array([[0.9, 0.1, 0.2], [0.3, 0.8, 0.1], [0.5, 0.5, 0.9]], np.float32)
    scene = {"means3D": means, "scales": scales, "rotations": rots, "opacities": np.ones((3, 1), np.float32),
             "colors_precomp": rgb, "shs": None, "sh_degree": 0, "bg": np.array([0.2, 0.4, 0.6], np.float32),
             "viewmatrix": cam["view"], "projmatrix": cam["proj"], "campos": cam["campos"], "tanfovx": 1.0,
             "tanfovy": 1.0, "width": 32, "height": 32}
    res = oracle.rasterize(scene, top_k=3)
    f = res["fwd"]
    assert abs(res["pre"]["proj_2d"][0, 0] - 15.0) < 1e-3
    a1 = np.float32(0.99)
    t1 = np.float32(1) - a1
    assert t1 * (np.float32(1) - a1) < np.float32(1e-4)
    np.testing.assert_allclose(f["color"][:, 15, 15], rgb[0] * a1 + t1 * scene["bg"], rtol=1e-6)
    assert f["alpha"][0, 15, 15] == a1
    assert f["n_contrib"][15, 15] == 1
    assert list(f["gs_per_pixel"][:, 15, 15]) == [0, -1, -1]
    # one pixel away the first alpha is below the cap and the second Gaussian blends
    assert f["n_contrib"][15, 18] >= 2 and f["alpha"][0, 15, 18] < a1


def test_render_empty_and_all_culled_scenes_return_background():
    s = tiny_scene(0, n=5)
    s["means3D"] = s["means3D"] * 0 + np.array([0.5, -0.4, -10.0], np.float32)  # behind the camera
    res = oracle.rasterize(s)
    assert res["bins"]["num_rendered"] == 0
    np.testing.assert_array_equal(res["fwd"]["color"], np.broadcast_to(s["bg"][:, None, None], (3, 48, 64)))
    assert not res["fwd"]["alpha"].any() and not res["fwd"]["n_contrib"].any()


def test_render_depth_off_keeps_colour_and_zeroes_depth():
    s = tiny_scene(5)
    on = oracle.rasterize(s, compute_depth=True)["fwd"]
    off = oracle.rasterize(s, compute_depth=False)["fwd"]
    np.testing.assert_array_equal(on["color"], off["color"])
    np.testing.assert_array_equal(on["alpha"], off["alpha"])
    np.testing.assert_array_equal(on["n_contrib"], off["n_contrib"])
    assert not off["depth"].any() and on["depth"].any()


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_render_matches_dense_float64_blend(seed):
    s = tiny_scene(seed, n=60)
    top_k = 4
    res = oracle.rasterize(s, top_k=top_k)
    pre, _ = dense_pre(s)
    n = s["means3D"].shape[0]
    op = res["pre"]
    out = dense_ref.render(t64(op["proj_2d"]), t64(op["conic_2d"]), t64(s["opacities"][:, 0]), t64(op["rgb"]),
                           t64(op["depths"]), op["radii"], tile_sets_of(res, n, s["width"]), s["width"],
                           s["height"], t64(s["bg"]), top_k=top_k)
    f = res["fwd"]
    assert f["alpha"].max() > 0.5
    np.testing.assert_allclose(f["color"], out["color"].numpy(), atol=1e-5)
    np.testing.assert_allclose(f["alpha"], out["alpha"].numpy(), atol=1e-5)
    np.testing.assert_allclose(f["depth"], out["depth"].numpy(), atol=1e-4, rtol=1e-5)
    assert np.array_equal(f["n_contrib"], out["n_contrib"].numpy())
    assert np.array_equal(f["gs_per_pixel"], out["ids"].numpy())
    np.testing.assert_allclose(f["weight_per_gs_pixel"], out["weights"].numpy(), atol=1e-6)
    np.testing.assert_allclose(f["x_mu"], out["x_mu"].numpy(), atol=2e-5)
    # slots with no contributor keep -1 / 0 / 0
    empty = f["gs_per_pixel"] < 0
    assert empty.any() and not f["weight_per_gs_pixel"][empty].any()
    assert not f["x_mu"][:, empty].any()


@pytest.mark.parametrize("seed", [0, 1])
def test_render_saturating_scene_matches_dense_blend(seed):
    """Opaque, heavily overlapping Gaussians: alpha hits its 0.99 cap and
    pixels reach the T (1 - alpha) < 1e-4 stop, which the sparse scenes never do."""
    s = tiny_scene(seed, n=150, spread=0.25, log_scale=-1.4)
    s["opacities"] = np.random.default_rng(seed).uniform(0.9, 1.0, (150, 1)).astype(np.float32)
    s["opacities"][::3] = 1.0
    res = oracle.rasterize(s, top_k=3)
    op = res["pre"]
    out = dense_ref.render(t64(op["proj_2d"]), t64(op["conic_2d"]), t64(s["opacities"][:, 0]), t64(op["rgb"]),
                           t64(op["depths"]), op["radii"], tile_sets_of(res, 150, s["width"]), s["width"],
                           s["height"], t64(s["bg"]), top_k=3)
    f = res["fwd"]
    assert (1.0 - f["alpha"]).min() < 1e-3
    np.testing.assert_allclose(f["color"], out["color"].numpy(), atol=1e-5)
    np.testing.assert_allclose(f["alpha"], out["alpha"].numpy(), atol=1e-5)
    assert np.array_equal(f["n_contrib"], out["n_contrib"].numpy())
    assert np.array_equal(f["gs_per_pixel"], out["ids"].numpy())


def test_render_with_float64_preprocess_inputs():
    """Same comparison with the blend fed by the float64 preprocess: the whole
    forward chain, not just the blend, agrees."""
    s = tiny_scene(9, n=60)
    res = oracle.rasterize(s)
    pre, _ = dense_pre(s)
    n = s["means3D"].shape[0]
    out = dense_ref.render(pre["pix"], pre["conic"], t64(s["opacities"][:, 0]), pre["rgb"], pre["depth"],
                           res["pre"]["radii"], tile_sets_of(res, n, s["width"]), s["width"], s["height"],
                           t64(s["bg"]))
    np.testing.assert_allclose(res["fwd"]["color"], out["color"].detach().numpy(), atol=2e-4)
    np.testing.assert_allclose(res["fwd"]["alpha"], out["alpha"].detach().numpy(), atol=2e-4)


# ---------------------------------------------------------------- backward

@pytest.mark.parametrize("seed,compute_depth", [(0, True), (1, True), (2, False), (4, True)])
def test_backward_matches_float64_autograd(seed, compute_depth):
    s = tiny_scene(seed, n=50)
    res = oracle.rasterize(s, compute_depth=compute_depth)
    g = torch.Generator().manual_seed(100 + seed)
    H, W = s["height"], s["width"]
    gc = torch.randn(3, H, W, generator=g, dtype=torch.float64)
    gd = torch.randn(1, H, W, generator=g, dtype=torch.float64) if compute_depth else torch.zeros(1, H, W,
                                                                                                  dtype=torch.float64)
    ga = torch.randn(1, H, W, generator=g, dtype=torch.float64)
    grads = oracle.rasterize_backward(s, res, gc.numpy().astype(np.float32), gd.numpy().astype(np.float32),
                                      ga.numpy().astype(np.float32), compute_depth=compute_depth, with_bound=True)

    pre, leaves = dense_pre(s, grad=True)
    pre["ndc"].retain_grad()
    n = s["means3D"].shape[0]
    out = dense_ref.render(pre["pix"], pre["conic"], leaves["opacities"][:, 0], pre["rgb"], pre["depth"],
                           res["pre"]["radii"], tile_sets_of(res, n, W), W, H, t64(s["bg"]),
                           compute_depth=compute_depth)
    np.testing.assert_allclose(res["fwd"]["color"], out["color"].detach().numpy(), atol=2e-4)
    loss = (out["color"] * gc).sum() + (out["alpha"] * ga).sum()
    if compute_depth:
        loss = loss + (out["depth"] * gd).sum()
    loss.backward()
    checks = {
        "means3D": leaves["means3D"].grad,
        "scales": leaves["scales"].grad,
        "rotations": leaves["rotations"].grad,
        "opacities": leaves["opacities"].grad,
        "sh": leaves["shs"].grad,
    }
    for name, expected in checks.items():
        bad, worst, _, _ = grad_mismatch(grads[name], expected.numpy(), grads["bound"][name])
        assert bad == 0, (name, worst)
        assert np.abs(expected.numpy()).max() > 0
    # means2D carries dL/d(ndc) with z = 0
    bad, worst, _, _ = grad_mismatch(grads["means2D"][:, :2], pre["ndc"].grad.numpy(),
                                     grads["bound"]["means2D"][:, :2])
    assert bad == 0, ("means2D", worst)
    assert not grads["means2D"][:, 2].any()


def test_backward_culled_gaussians_get_zero_gradients():
    s = tiny_scene(2, n=30)
    s["means3D"][:10] = np.array([0.5, -0.4, -10.0], np.float32)  # behind the camera
    res = oracle.rasterize(s)
    H, W = s["height"], s["width"]
    grads = oracle.rasterize_backward(s, res, np.ones((3, H, W), np.float32), np.ones((1, H, W), np.float32),
                                      np.ones((1, H, W), np.float32))
    assert np.all(res["pre"]["radii"][:10] == 0)
    for name in ("means3D", "scales", "rotations", "opacities", "means2D"):
        assert not grads[name][:10].any(), name
    assert np.abs(grads["means3D"][10:]).max() > 0


def test_flow_doubling_adds_render_grads_once_more():
    """With enable_flow_grad the reference adds the render's xy and conic
    gradients to the upstream proj_2D / conic_2D gradients and the fused
    backward adds them again (flow_ops.py:337-360, backward_kernels.py:95-98,
    182-184): the result equals a standard backward whose upstream proj_2D and
    conic_2D gradients are the render gradients themselves."""
    s = tiny_scene(6, n=50)
    res = oracle.rasterize(s)
    H, W = s["height"], s["width"]
    g = np.random.default_rng(0)
    gc = g.standard_normal((3, H, W)).astype(np.float32)
    zeros = np.zeros((1, H, W), np.float32)
    doubled = oracle.rasterize_backward(s, res, gc, zeros, zeros, flow_double=True)
    gg = doubled["grad_gauss"]
    explicit = oracle.rasterize_backward(s, res, gc, zeros, zeros, grad_proj_2d=gg[:, 0:2],
                                         grad_conic_2d=gg[:, 2:5])
    single = oracle.rasterize_backward(s, res, gc, zeros, zeros)
    for name in ("means3D", "scales", "rotations"):
        np.testing.assert_allclose(doubled[name], explicit[name], rtol=1e-5, atol=1e-7)
        assert not np.allclose(doubled[name], single[name])
    np.testing.assert_array_equal(doubled["opacities"], single["opacities"])
    np.testing.assert_array_equal(doubled["sh"], single["sh"])


# ---------------------------------------------------------------- precomputed 3D covariances

def cov3d_of(s: dict) -> np.ndarray:
    """Upper triangle (xx, xy, xz, yy, yz, zz) of R diag(s^2) R^T in float64."""
    return dense_ref.covariance_upper(s["scales"], s["rotations"])


def precomp_scene(seed: int, n: int = 50) -> dict:
    s = tiny_scene(seed, n=n)
    s["cov3D_precomp"] = cov3d_of(s).astype(np.float32)
    return s


def test_precomputed_covariance_matches_scale_rotation_path():
    """The masked path fed R diag(s^2) R^T reproduces the fused path's outputs
    (same mathematics, different float evaluation order)."""
    s = precomp_scene(4, n=200)
    ref = oracle.rasterize({k: v for k, v in s.items() if k != "cov3D_precomp"})
    got = oracle.rasterize({k: v for k, v in s.items() if k not in ("scales", "rotations")})
    assert np.mean(got["pre"]["radii"] == ref["pre"]["radii"]) > 0.98
    vis = (got["pre"]["radii"] > 0) & (ref["pre"]["radii"] > 0)
    np.testing.assert_allclose(got["pre"]["conic_2d_inv"][vis], ref["pre"]["conic_2d_inv"][vis], rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(got["fwd"]["color"], ref["fwd"]["color"], atol=2e-3)


def test_precomputed_covariance_masked_path_details():
    """The masked kernel culls |det| < 1e-7 (strict) and stores the given
    covariance for the backward (preprocess_kernels.py:420-422)."""
    s = precomp_scene(5, n=20)
    s.pop("scales")
    s.pop("rotations")
    res = oracle.rasterize(s)
    np.testing.assert_array_equal(res["pre"]["cov3d"], s["cov3D_precomp"])
    assert (res["pre"]["radii"] > 0).sum() > 5


@pytest.mark.parametrize("seed", [0, 3])
def test_precomputed_covariance_backward_matches_float64_autograd(seed):
    s = precomp_scene(seed)
    s.pop("scales")
    s.pop("rotations")
    res = oracle.rasterize(s)
    g = torch.Generator().manual_seed(200 + seed)
    H, W = s["height"], s["width"]
    gc = torch.randn(3, H, W, generator=g, dtype=torch.float64)
    gd = torch.randn(1, H, W, generator=g, dtype=torch.float64)
    ga = torch.randn(1, H, W, generator=g, dtype=torch.float64)
    grads = oracle.rasterize_backward(s, res, gc.numpy().astype(np.float32), gd.numpy().astype(np.float32),
                                      ga.numpy().astype(np.float32), with_bound=True)
    leaves = {k: t64(s[k]).requires_grad_(True) for k in ("means3D", "opacities", "shs", "cov3D_precomp")}
    pre = dense_ref.preprocess(leaves["means3D"], None, None, t64(s["viewmatrix"]), t64(s["projmatrix"]),
                               t64(s["campos"]), s["tanfovx"], s["tanfovy"], W, H, shs=leaves["shs"],
                               degree=s["sh_degree"], cov3d=leaves["cov3D_precomp"])
    n = s["means3D"].shape[0]
    out = dense_ref.render(pre["pix"], pre["conic"], leaves["opacities"][:, 0], pre["rgb"], pre["depth"],
                           res["pre"]["radii"], tile_sets_of(res, n, W), W, H, t64(s["bg"]))
    ((out["color"] * gc).sum() + (out["alpha"] * ga).sum() + (out["depth"] * gd).sum()).backward()
    for name, key in (("means3D", "means3D"), ("cov3D", "cov3D_precomp"), ("opacities", "opacities"),
                      ("sh", "shs")):
        expected = leaves[key].grad.numpy()
        bad, worst, _, _ = grad_mismatch(grads[name], expected, grads["bound"][name])
        assert bad == 0, (name, worst)
        assert np.abs(expected).max() > 0


# ---------------------------------------------------------------- Mip-Splatting filter variance

def mip_scene(seed: int, f: float, n: int = 120, precomp: bool = False) -> dict:
    s = tiny_scene(seed, n=n, spread=0.8)
    s["filter_variance"] = f
    if precomp:
        s["cov3D_precomp"] = cov3d_of(s).astype(np.float32)
        s.pop("scales")
        s.pop("rotations")
    return s


def test_mip_filter_closed_form_on_axis():
    """Identity camera and rotation, on-axis point: filtered cov2D =
    (f/z)^2 s^2 + 0.3 + v on the diagonal, conic its inverse, and with the
    discriminant zero the radius is ceil(3 sqrt(cov2D))."""
    cam = identity_camera()
    z, s, v = 2.0, 0.05, 1.0
    means = np.array([[0.0, 0.0, z]], np.float32)
    kw = dict(tanfovx=cam["tanfovx"], tanfovy=cam["tanfovy"], width=64, height=64,
              colors=np.full((1, 3), 0.2, np.float32))
    args = (means, np.full((1, 3), s, np.float32), np.array([[1, 0, 0, 0]], np.float32),
            np.full((1, 1), 0.8, np.float32), cam["view"], cam["proj"], cam["campos"])
    base = oracle.preprocess(*args, **kw)
    pre = oracle.preprocess(*args, filter_variance=v, **kw)
    var = (64 / 2.0 / z) ** 2 * s * s + 0.3 + v
    np.testing.assert_allclose(pre["conic_2d_inv"][0], [var, 0.0, var], rtol=1e-5)
    np.testing.assert_allclose(pre["conic_2d"][0], [1 / var, 0.0, 1 / var], rtol=1e-5)
    assert pre["radii"][0] == math.ceil(3.0 * math.sqrt(var))
    assert pre["radii"][0] > base["radii"][0]
    assert pre["depths"][0] == base["depths"][0] and np.array_equal(pre["proj_2d"], base["proj_2d"])
    # a point-like Gaussian: cov2D ~ 0.3 + v, radius ceil(3 sqrt(0.4)) = 2
    tiny = oracle.preprocess(means, np.full((1, 3), 1e-4, np.float32), *args[2:], filter_variance=0.1, **kw)
    assert tiny["radii"][0] == 2
    # the 0.1 eigenvalue floor: precomputed cov3D with cov2D = -0.15 I before
    # and -0.1 I after the filter (determinant 0.01, kept) gives radius
    # ceil(3 sqrt(0.1)) = 1
    v = -0.45 / (64 / 2.0 / z) ** 2
    cov = np.array([[v, 0.0, 0.0, v, 0.0, v]], np.float32)
    neg = oracle.preprocess(means, None, None, *args[3:], cov3d_precomp=cov, filter_variance=0.05, **kw)
    np.testing.assert_allclose(neg["conic_2d_inv"][0], [-0.1, 0.0, -0.1], atol=1e-6)
    assert neg["radii"][0] == 1


def test_mip_zero_filter_is_the_base_path():
    s = tiny_scene(3, n=80)
    base = oracle.rasterize(s)
    zero = oracle.rasterize({**s, "filter_variance": 0.0})
    for key in ("radii", "conic_2d", "conic_2d_inv", "tiles_touched"):
        assert np.array_equal(base["pre"][key], zero["pre"][key])
    assert np.array_equal(base["fwd"]["color"], zero["fwd"]["color"])


@pytest.mark.parametrize("seed,f", [(0, 0.3), (1, 0.1), (2, 2.0)])
def test_mip_filter_matches_float64_restatement(seed, f):
    s = mip_scene(seed, f, n=200)
    res = oracle.rasterize(s)
    op = res["pre"]
    leaves = {k: t64(s[k]) for k in ("means3D", "scales", "rotations", "shs")}
    pre = dense_ref.preprocess(leaves["means3D"], leaves["scales"], leaves["rotations"], t64(s["viewmatrix"]),
                               t64(s["projmatrix"]), t64(s["campos"]), s["tanfovx"], s["tanfovy"], s["width"],
                               s["height"], shs=leaves["shs"], degree=s["sh_degree"], filter_variance=f)
    a, b, c = (pre["cov2d"][:, i].numpy() for i in range(3))
    lam = 0.5 * (a + c) + np.sqrt(np.maximum(0.25 * (a - c) ** 2 + b * b, 0.0))
    r3 = 3.0 * np.sqrt(np.maximum(lam, 0.1))
    near_int = np.abs(r3 - np.round(r3)) < 1e-4
    assert np.array_equal(op["radii"][~near_int], pre["radii"][~near_int])
    v = (op["radii"] > 0) & (pre["radii"] > 0)
    assert v.sum() > 50
    np.testing.assert_allclose(op["conic_2d_inv"][v], pre["cov2d"].numpy()[v], rtol=2e-5, atol=1e-6)
    np.testing.assert_allclose(op["conic_2d"][v], pre["conic"].numpy()[v], rtol=1e-4, atol=1e-7)
    # tile counts are recounted from the filtered values
    gx, gy = oracle.grid_dims(s["width"], s["height"])
    recount = oracle.count_covered_tiles(op["proj_2d"], op["conic_2d_inv"], op["conic_opacity"], op["radii"],
                                         gx, gy, 1)
    assert np.array_equal(recount, op["tiles_touched"])
    base = oracle.rasterize({k: val for k, val in s.items() if k != "filter_variance"})
    assert (op["tiles_touched"] > base["pre"]["tiles_touched"]).sum() > 5


@pytest.mark.parametrize("seed,precomp", [(0, False), (5, False), (1, True)])
def test_mip_filter_backward_matches_float64_autograd(seed, precomp):
    f = 0.3
    s = mip_scene(seed, f, n=50, precomp=precomp)
    res = oracle.rasterize(s)
    g = torch.Generator().manual_seed(300 + seed)
    H, W = s["height"], s["width"]
    gc = torch.randn(3, H, W, generator=g, dtype=torch.float64)
    gd = torch.randn(1, H, W, generator=g, dtype=torch.float64)
    ga = torch.randn(1, H, W, generator=g, dtype=torch.float64)
    grads = oracle.rasterize_backward(s, res, gc.numpy().astype(np.float32), gd.numpy().astype(np.float32),
                                      ga.numpy().astype(np.float32), with_bound=True)
    names = ("means3D", "opacities", "shs") + (("cov3D_precomp",) if precomp else ("scales", "rotations"))
    leaves = {k: t64(s[k]).requires_grad_(True) for k in names}
    pre = dense_ref.preprocess(leaves["means3D"], leaves.get("scales"), leaves.get("rotations"),
                               t64(s["viewmatrix"]), t64(s["projmatrix"]), t64(s["campos"]), s["tanfovx"],
                               s["tanfovy"], W, H, shs=leaves["shs"], degree=s["sh_degree"],
                               cov3d=leaves.get("cov3D_precomp"), filter_variance=f)
    n = s["means3D"].shape[0]
    out = dense_ref.render(pre["pix"], pre["conic"], leaves["opacities"][:, 0], pre["rgb"], pre["depth"],
                           res["pre"]["radii"], tile_sets_of(res, n, W), W, H, t64(s["bg"]))
    np.testing.assert_allclose(res["fwd"]["color"], out["color"].detach().numpy(), atol=2e-4)
    ((out["color"] * gc).sum() + (out["alpha"] * ga).sum() + (out["depth"] * gd).sum()).backward()
    key_of = {"cov3D_precomp": "cov3D", "shs": "sh"}
    for name in names:
        expected = leaves[name].grad.numpy()
        key = key_of.get(name, name)
        bad, worst, _, _ = grad_mismatch(grads[key], expected, grads["bound"][key])
        assert bad == 0, (name, worst)
        assert np.abs(expected).max() > 0
