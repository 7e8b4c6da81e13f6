"""The production forward's fast path against the CPU oracle.

The typed forward provisions its pair buffers before the pair count is known
(from the previous forward's count on the device) and makes one C call,
gs_readback_bin_packed, that reads the count back and launches the packed
binning and the standard render.  It declines, and the Python path bins into
exact buffers, when the count exceeds the provision or the default sort mode
picks the depth-then-tile dataflow.  The stage-by-stage parity tests bin
through the explicit path (they keep the sorted keys), so these tests pin the
fast path itself: taken or declined as expected, and every output of a
forward + backward through it equal to the oracle's to the parity bar.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from gswarp_amd import _pipeline, _workspace, configs
from helpers import options, oracle_forward, raster_inputs, report_grad, to_np

pytestmark = pytest.mark.gpu

CASES = {
    "c1_full": dict(config=1),
    "c2_small": dict(config=2, count=60_000, width=480, height=270),
    # the heavy tail at half resolution: about 8 pairs per Gaussian
    "c3_half": dict(config=3, count=20_000, width=960, height=540),
    "c1_ragged": dict(config=1, count=5_000, width=203, height=117),
}


def _scene(name, device, seed=0):
    kw = dict(CASES[name])
    cfg = kw.pop("config")
    return configs.make_scene(cfg, seed=seed, device=device, **kw)


def _forward(scene, opts):
    inputs = raster_inputs(scene)
    with torch.cuda.device(scene["means3D"].device):
        result = _pipeline.forward(inputs, opts)
    torch.cuda.synchronize()
    return inputs, result


def _check_against_oracle(scene, result, ref):
    rp, rb, rf = ref["pre"], ref["bins"], ref["fwd"]
    pre, bins = result.state.preprocess, result.state.binning
    assert np.array_equal(to_np(result.radii), rp["radii"])
    assert bins.num_rendered == rb["num_rendered"]
    assert np.array_equal(to_np(bins.point_list), rb["point_list"])
    assert np.array_equal(to_np(bins.ranges), rb["ranges"])
    assert np.array_equal(to_np(result.state.n_contrib).reshape(rf["n_contrib"].shape), rf["n_contrib"])
    for key, t in (("color", result.color), ("depth", result.depth), ("alpha", result.alpha)):
        err = float(np.abs(to_np(t) - rf[key]).max())
        assert err <= 1e-4, (key, err)
    del pre


@pytest.mark.parametrize("case", ["c1_full", "c2_small", "c1_ragged"])
def test_fast_path_forward_matches_oracle(case, device):
    """With a provision that fits, one call bins and renders: the state says
    the render was launched with the binning, and every forward output equals
    the oracle's."""
    scene = _scene(case, device)
    host, ref = oracle_forward(scene)
    _workspace.note_pairs(device, ref["bins"]["num_rendered"])
    print(f"[fast] {case} R={ref['bins']['num_rendered']}", flush=True)
    _, result = _forward(scene, options())
    assert result.state.binning.rendered
    _check_against_oracle(scene, result, ref)


def test_fast_path_declines_over_capacity(device):
    """A provision far below the pair count: the call only reads the count
    back, the exact-buffer path bins and renders, and the outputs still equal
    the oracle's; the next forward is provisioned from this count and takes
    the fast path."""
    scene = _scene("c2_small", device)
    host, ref = oracle_forward(scene)
    _workspace.note_pairs(device, 1)
    _, result = _forward(scene, options())
    assert not result.state.binning.rendered
    _check_against_oracle(scene, result, ref)
    _, again = _forward(scene, options())
    assert again.state.binning.rendered
    _check_against_oracle(scene, again, ref)


def _spy_calls(monkeypatch):
    """Names of the C entry points the pipeline calls."""
    from gswarp_amd import _lib

    lib = _lib.load()
    names = []
    real = lib.call

    def call(name, *args):
        names.append(name)
        return real(name, *args)

    monkeypatch.setattr(lib, "call", call)
    return names


def test_fast_path_declines_for_depth_then_tile(device, monkeypatch):
    """The heavy-tailed config-3 scene at half resolution has more than four
    pairs per Gaussian.  Provisioned for its count regardless of the last
    forward, the one-call path declines (the default mode's dataflow for many
    pairs per Gaussian applies) and the outputs still equal the oracle's."""
    scene = _scene("c3_half", device)
    host, ref = oracle_forward(scene)
    R = ref["bins"]["num_rendered"]
    assert R > 4 * scene["means3D"].shape[0]
    monkeypatch.setattr(_workspace, "pair_capacity", lambda dev: 2 * R)
    monkeypatch.setattr(_workspace, "last_pairs", lambda dev: 1)
    names = _spy_calls(monkeypatch)
    _, result = _forward(scene, options())
    assert "gs_readback_bin_packed" in names
    assert "gs_bin_buckets" in names or "gs_duplicate_tiles" in names
    assert not result.state.binning.rendered
    _check_against_oracle(scene, result, ref)


def test_no_provision_after_a_depth_then_tile_forward(device, monkeypatch):
    """After a forward with many pairs per Gaussian the next one does not
    provision the packed path's buffers: it reads the counts back alone (the
    pair count and the bucketed binning's sizes) and bins by buckets."""
    scene = _scene("c3_half", device)
    host, ref = oracle_forward(scene)
    _workspace.note_pairs(device, ref["bins"]["num_rendered"])
    names = _spy_calls(monkeypatch)
    _, result = _forward(scene, options())
    assert "gs_readback_bin_packed" not in names and "gs_info_readback" in names
    # the sizing scan: one pass by default (its state cleared by the preprocess), else two
    scan = "gs_scan_tiles_onepass" if _pipeline.SCAN_ONEPASS else "gs_scan_tiles_entries"
    assert scan in names and "gs_bin_buckets" in names
    assert not result.state.binning.rendered
    _check_against_oracle(scene, result, ref)


def test_fast_path_explicit_warp_radix_takes_it_at_any_ratio(device):
    """In warp_radix mode the packed dataflow applies at any pairs-per-Gaussian
    ratio, so the heavy-tailed scene also bins and renders in one call."""
    scene = _scene("c3_half", device)
    host, ref = oracle_forward(scene)
    _workspace.note_pairs(device, ref["bins"]["num_rendered"])
    _, result = _forward(scene, options(sort_mode="warp_radix"))
    assert result.state.binning.rendered
    _check_against_oracle(scene, result, ref)


@pytest.mark.parametrize("case", ["c1_full", "c2_small"])
def test_fast_path_backward_matches_oracle(case, device):
    """Gradients through a fast-path forward (its point list is a view of the
    provisioned buffer) match the oracle's to the gradient bar."""
    scene = _scene(case, device)
    host, ref = oracle_forward(scene)
    _workspace.note_pairs(device, ref["bins"]["num_rendered"])
    opts = options()
    inputs, result = _forward(scene, opts)
    assert result.state.binning.rendered
    H, W = scene["height"], scene["width"]
    g = torch.Generator().manual_seed(9)
    up = {k: torch.randn(*shape, generator=g).to(device)
          for k, shape in (("color", (3, H, W)), ("depth", (1, H, W)), ("alpha", (1, H, W)))}
    with torch.cuda.device(device):
        grads = _pipeline.backward(inputs, result.radii, result.alpha, up["color"], up["depth"], up["alpha"],
                                   None, None, None, opts, result.state)
    torch.cuda.synchronize()
    g_means2d, _g_colors, g_opac, g_means3d, _g_cov, g_sh, g_scales, g_rot = grads
    zeros2 = np.zeros((scene["means3D"].shape[0], 2), np.float32)
    zeros3 = np.zeros((scene["means3D"].shape[0], 3), np.float32)
    ref_g = oracle.rasterize_backward(host, ref, to_np(up["color"]), to_np(up["depth"]), to_np(up["alpha"]),
                                      grad_proj_2d=zeros2, grad_conic_2d=zeros3, grad_conic_2d_inv=zeros3,
                                      with_bound=True)
    failures = []
    for name, actual, key in (("means2D", g_means2d, "means2D"), ("opacities", g_opac, "opacities"),
                              ("means3D", g_means3d, "means3D"), ("scales", g_scales, "scales"),
                              ("rotations", g_rot, "rotations"), ("sh", g_sh, "sh")):
        expected = ref_g[key]
        bad, worst = report_grad(name, to_np(actual).reshape(expected.shape), expected, ref_g["bound"][key])
        if bad:
            failures.append((name, bad, worst))
    assert not failures, failures
