"""Parity of every gfx950 stage with the CPU oracle on seeded scenes.

Bar (from the build's north star): radii, tile counts, sorted keys, point
lists and tile ranges bit-exact; colour / depth / alpha within 1e-4
absolute; flow top-K ids exact; gradients within 1e-3 relative + 1e-5
absolute plus, per element, twice the oracle's bound on the fp32 rounding of
that element's sum of per-pixel terms (helpers.grad_mismatch).

The forward kernels evaluate every fp32 expression in the oracle's order
with the same exp/log, so the forward is asserted stricter than the bar:
colour, depth, alpha and the flow weights / x_mu equal the oracle's bit for
bit (EXACT_FORWARD).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gswarp_amd import _pipeline, configs
from helpers import gpu_forward, options, oracle_forward, report_grad, to_np, with_precomputed_covariance

pytestmark = pytest.mark.gpu

CASES = {
    "c0_full": dict(config=0),
    "c1_full": dict(config=1),
    "c2_small": dict(config=2, count=60_000, width=480, height=270),
    "c3_small": dict(config=3, count=60_000, width=480, height=270),
    "c4_small": dict(config=4, count=40_000, width=320, height=180),
    "c1_ragged": dict(config=1, count=5_000, width=203, height=117),
}

COLOR_ATOL = 1e-4
EXACT_FORWARD = True


def _scene(name, device, seed=0):
    kw = dict(CASES[name])
    cfg = kw.pop("config")
    return configs.make_scene(cfg, seed=seed, device=device, **kw)


def _check_forward(scene, opts, *, coverage_mode=1, flow=False, top_k=0, colors=False):
    print(f"[parity] N={scene['means3D'].shape[0]} {scene['width']}x{scene['height']} cov={coverage_mode} "
          f"flow={flow} colors={colors}", flush=True)
    out = gpu_forward(scene, opts, flow=flow, colors=colors)
    host, ref = oracle_forward(scene, coverage_mode=coverage_mode, compute_depth=opts.compute_depth,
                               top_k=top_k, colors=colors)
    pre, bins, res = out["pre"], out["bins"], out["res"]
    rp, rb, rf = ref["pre"], ref["bins"], ref["fwd"]
    # preprocess: integer outputs bit-exact, float outputs bit-exact too
    assert np.array_equal(to_np(pre.radii), rp["radii"])
    assert np.array_equal(to_np(pre.tiles_touched), rp["tiles_touched"])
    for key in ("proj_2d", "conic_2d", "conic_2d_inv", "depths"):
        assert np.array_equal(to_np(getattr(pre, key)), rp[key]), key
    vis = rp["radii"] > 0
    rgb = to_np(pre.records)[:, 8:11]
    assert np.array_equal(rgb[vis], rp["rgb"][vis])
    # binning
    assert bins.num_rendered == rb["num_rendered"]
    if bins.num_rendered:
        assert np.array_equal(to_np(bins.point_list), rb["point_list"])
        tile, depth, _ = bins.decode_keys()
        assert np.array_equal(to_np(tile), rb["tile_ids"].astype(np.int64))
        assert np.array_equal(to_np(depth).astype(np.uint32), rp["depths"].view(np.uint32)[rb["point_list"]])
        lay = bins.key_layout
        if lay.value_bits:  # the packed low bits are the point list itself
            low = to_np(bins.sorted_keys) & ((1 << lay.value_bits) - 1)
            assert np.array_equal(low, rb["point_list"].astype(np.int64))
    assert np.array_equal(to_np(bins.ranges), rb["ranges"])
    # render
    assert np.array_equal(to_np(res.n_contrib).reshape(rf["n_contrib"].shape), rf["n_contrib"])
    floats = [("color", res.color, rf["color"]), ("depth", res.depth, rf["depth"]), ("alpha", res.alpha, rf["alpha"])]
    if flow and top_k:
        assert np.array_equal(to_np(res.aux[0]), rf["gs_per_pixel"])
        floats += [("weights", res.aux[1], rf["weight_per_gs_pixel"]), ("x_mu", res.aux[2], rf["x_mu"])]
    for key, t, expected in floats:
        got = to_np(t)
        err = float(np.abs(got - expected).max()) if got.size else 0.0
        assert err <= COLOR_ATOL, (key, err)
        if EXACT_FORWARD:
            assert np.array_equal(got, expected), (key, err)
    return out, host, ref


@pytest.mark.parametrize("case", list(CASES))
def test_forward_stages_match_oracle(case, device):
    scene = _scene(case, device)
    flow = CASES[case]["config"] == 4
    _check_forward(scene, options(flow=flow), flow=flow, top_k=20 if flow else 0)


@pytest.mark.parametrize("sort_mode", ["warp_radix", "torch", "depth_then_tile", "buckets"])
@pytest.mark.parametrize("case", ["c0_full", "c2_small", "c3_small", "c1_ragged"])
def test_other_sort_modes_match_oracle(case, sort_mode, device, monkeypatch):
    """Every binning dataflow gives the oracle's bit-exact lists: the packed
    64-bit key sort, the torch.sort dataflow, and the default mode's two
    dataflows for many pairs per Gaussian, the HIP depth-then-tile sort and the
    bucketed binning (both forced here at any pair-count ratio)."""
    scene = _scene(case, device)
    if sort_mode in ("depth_then_tile", "buckets"):
        monkeypatch.setattr(_pipeline, "DEPTH_TILE_MIN_PAIRS_PER_GAUSSIAN", 0)
        monkeypatch.setattr(_pipeline, "HEAVY_DATAFLOW", "depth_tile" if sort_mode == "depth_then_tile" else "buckets")
        monkeypatch.setattr(_pipeline, "BUCKET_SIZING", "always")
        sort_mode = "warp_depth_stable_tile"
    _check_forward(scene, options(sort_mode=sort_mode))


COVERAGE_SCENES = {
    "c1": dict(config=1, count=20_000, width=320, height=256),
    # large splats: tile rectangles beyond 64 cells take the band walk, the rest the cover masks
    "c3": dict(config=3, count=20_000, width=480, height=270),
}


@pytest.mark.parametrize("coverage_mode", [0, 1, 2])
@pytest.mark.parametrize("scene_name", list(COVERAGE_SCENES))
def test_alternative_coverage_modes_match_oracle(scene_name, coverage_mode, device):
    kw = dict(COVERAGE_SCENES[scene_name])
    scene = configs.make_scene(kw.pop("config"), device=device, **kw)
    _check_forward(scene, options(coverage_mode=coverage_mode), coverage_mode=coverage_mode)


def test_depth_off_matches_oracle(device):
    scene = configs.make_scene(2, count=20_000, width=320, height=200, device=device)
    _check_forward(scene, options(compute_depth=False))


def test_colors_precomp_matches_oracle(device):
    scene = configs.make_scene(1, count=20_000, width=256, height=256, device=device)
    _check_forward(scene, options(), colors=True)


def _upstream(scene, seed, with_meta=True):
    H, W, N = scene["height"], scene["width"], scene["means3D"].shape[0]
    g = torch.Generator().manual_seed(seed)
    dev = scene["means3D"].device
    grads = {
        "color": torch.randn(3, H, W, generator=g),
        "depth": torch.randn(1, H, W, generator=g),
        "alpha": torch.randn(1, H, W, generator=g),
        "proj_2d": torch.randn(N, 2, generator=g) * (1e-2 if with_meta else 0.0),
        "conic_2d": torch.randn(N, 3, generator=g) * (1e-2 if with_meta else 0.0),
        "conic_2d_inv": torch.randn(N, 3, generator=g) * (1e-2 if with_meta else 0.0),
    }
    return {k: v.to(dev) for k, v in grads.items()}


def _check_backward(scene, *, flow_double=False, compute_depth=True, colors=False, seed=3):
    opts = options(compute_depth=compute_depth)
    # the forward render zeroes the backward's NaN-filled accumulator
    out = gpu_forward(scene, opts, colors=colors, grad_buffer=True)
    host, ref = oracle_forward(scene, compute_depth=compute_depth, colors=colors)
    up = _upstream(scene, seed)
    with torch.cuda.device(scene["means3D"].device):
        grads = _pipeline.backward(out["inputs"], out["pre"].radii, out["res"].alpha, up["color"], up["depth"],
                                   up["alpha"], up["proj_2d"], up["conic_2d"], up["conic_2d_inv"], opts,
                                   _pipeline.ForwardState(out["pre"], out["bins"], out["res"].n_contrib,
                                                          out["grad_gauss"]),
                                   flow_double=flow_double)
    torch.cuda.synchronize()
    g_means2d, g_colors, g_opac, g_means3d, g_cov, g_sh, g_scales, g_rot = grads
    ref_g = __import__("oracle").rasterize_backward(
        host, ref, to_np(up["color"]), to_np(up["depth"]), to_np(up["alpha"]), compute_depth=compute_depth,
        grad_proj_2d=to_np(up["proj_2d"]), grad_conic_2d=to_np(up["conic_2d"]),
        grad_conic_2d_inv=to_np(up["conic_2d_inv"]), flow_double=flow_double, with_bound=True)
    checks = [("means2D", g_means2d, ref_g["means2D"]), ("opacities", g_opac, ref_g["opacities"]),
              ("means3D", g_means3d, ref_g["means3D"])]
    if "cov3D_precomp" in scene:
        checks.append(("cov3D", g_cov, ref_g["cov3D"]))
        assert g_scales.numel() == 0 and g_rot.numel() == 0
    else:
        checks += [("scales", g_scales, ref_g["scales"]), ("rotations", g_rot, ref_g["rotations"])]
    if colors:
        checks.append(("colors", g_colors, ref_g["colors"]))
    else:
        checks.append(("sh", g_sh, ref_g["sh"]))
    failures = []
    for name, actual, expected in checks:
        a = to_np(actual).reshape(expected.shape)
        bad, worst = report_grad(name, a, expected, ref_g["bound"][name])
        if bad:
            failures.append((name, bad, worst))
    assert not failures, failures


@pytest.mark.parametrize("case", ["c1_full", "c2_small", "c3_small", "c1_ragged"])
def test_backward_matches_oracle(case, device):
    _check_backward(_scene(case, device))


def test_flow_backward_doubling_matches_oracle(device):
    _check_backward(_scene("c4_small", device), flow_double=True)


def test_backward_depth_off_and_colors_precomp(device):
    scene = configs.make_scene(2, count=20_000, width=320, height=200, device=device)
    _check_backward(scene, compute_depth=False, colors=True)


@pytest.mark.parametrize("case", ["c1_full", "c2_small", "c1_ragged"])
def test_precomputed_covariance_forward_matches_oracle(case, device):
    """cov3D_precomp input (preprocess_kernels.py:345-477): every stage bit-exact."""
    scene = with_precomputed_covariance(_scene(case, device))
    _check_forward(scene, options())


@pytest.mark.parametrize("coverage_mode", [0, 2])
def test_precomputed_covariance_coverage_modes_match_oracle(coverage_mode, device):
    scene = with_precomputed_covariance(configs.make_scene(1, count=20_000, width=320, height=256, device=device))
    _check_forward(scene, options(coverage_mode=coverage_mode), coverage_mode=coverage_mode)


@pytest.mark.parametrize("case,flow_double", [("c1_full", False), ("c2_small", False), ("c4_small", True)])
def test_precomputed_covariance_backward_matches_oracle(case, flow_double, device):
    """dL/dcov3D from the chain of backward_ops.py:679-744 instead of scale / rotation."""
    _check_backward(with_precomputed_covariance(_scene(case, device)), flow_double=flow_double)


@pytest.mark.parametrize("case,f,coverage_mode", [("c1_full", 0.3, 1), ("c2_small", 0.1, 1), ("c1_ragged", 2.0, 1),
                                                   ("c1_full", 0.3, 0), ("c1_full", 0.3, 2)])
def test_mip_filter_forward_matches_oracle(case, f, coverage_mode, device):
    """Mip-Splatting filter variance (backend_mip_3dgs.py:63-102): filtered
    conics, radii and recounted tiles, then every later stage, bit-exact."""
    scene = dict(_scene(case, device), filter_variance=f)
    _check_forward(scene, options(coverage_mode=coverage_mode), coverage_mode=coverage_mode)


def test_mip_filter_with_precomputed_covariance_matches_oracle(device):
    scene = dict(with_precomputed_covariance(_scene("c1_full", device)), filter_variance=0.3)
    _check_forward(scene, options())
    _check_backward(scene)


@pytest.mark.parametrize("case", ["c1_full", "c2_small"])
def test_mip_filter_backward_matches_oracle(case, device):
    _check_backward(dict(_scene(case, device), filter_variance=0.3))


def test_stacked_opaque_gaussians_terminate_like_oracle(device):
    """Eight wide, opaque Gaussians stacked on the view axis: alpha is capped
    at 0.99, so a pixel where two or more reach the cap has T <= 1e-4 and
    stops at the next one it would blend (the oracle stops about 300 of the
    7680 pixels before the eighth).  The stop decisions, n_contrib and the
    colours match the oracle bit for bit."""
    k = 8
    scene = configs.make_scene(1, count=k, width=96, height=80, device=device)
    z = torch.arange(k, dtype=torch.float32, device=device) * 0.05
    scene["means3D"] = torch.stack([torch.zeros_like(z), torch.zeros_like(z), z], dim=1).contiguous()
    scene["scales"] = torch.full((k, 3), 0.8, device=device)
    scene["opacities"] = torch.full((k, 1), 0.999, device=device)
    out, _host, ref = _check_forward(scene, options())
    n_contrib = ref["fwd"]["n_contrib"].reshape(-1)
    alpha = ref["fwd"]["alpha"].reshape(-1)
    stopped = (n_contrib > 0) & (n_contrib < k) & (alpha > 0.9998)
    assert stopped.sum() > 100, int(stopped.sum())
