"""The raw ABI on the GPU: 18 -> 11 (flow: 14) forward and 27 -> 8 (flow: 31 -> 8)
backward with opaque geom / binning / img buffers (backend_3dgs.py:112-248,
backward_ops.py:376-746, flow_ops.py:196-512).

The raw forward must equal the typed forward bit for bit (it is the same
pipeline with its state laid out in the byte buffers), the raw backward must
meet the gradient bar against the oracle, and a backward whose buffers do not
unpack must rebuild the state and give the same gradients.
"""

from __future__ import annotations

from dataclasses import fields

import numpy as np
import pytest
import torch

import oracle
from gswarp_amd import _pipeline, _rasterizer, _rasterizer_flow, configs
from helpers import oracle_forward, raster_inputs, report_grad, to_np, with_precomputed_covariance

pytestmark = pytest.mark.gpu

GRAD_NAMES = ("means2D", "colors", "opacities", "means3D", "cov3D", "sh", "scales", "rotations")


def _raw_args(scene, colors=False):
    inputs = raster_inputs(scene, colors=colors)
    return [getattr(inputs, f.name) for f in fields(_pipeline.RasterInputs)][:18]


def _upstream(scene, seed=3):
    H, W, N = scene["height"], scene["width"], scene["means3D"].shape[0]
    g = torch.Generator().manual_seed(seed)
    dev = scene["means3D"].device
    out = {"color": torch.randn(3, H, W, generator=g), "depth": torch.randn(1, H, W, generator=g),
           "alpha": torch.randn(1, H, W, generator=g), "proj_2d": torch.randn(N, 2, generator=g) * 1e-2,
           "conic_2d": torch.randn(N, 3, generator=g) * 1e-2, "conic_2d_inv": torch.randn(N, 3, generator=g) * 1e-2}
    return {k: v.to(dev) for k, v in out.items()}


def _backward_args(fargs, fwd, up, geom=None, binning=None, img=None):
    (bg, means, colors, opac, scales, rots, smod, cov, view, proj, tx, ty, _H, _W, sh, deg, campos, _pf) = fargs
    num_rendered, _color, _depth, alpha, radii, g, b, i = fwd[:8]
    return [bg, means, radii, colors, opac, scales, rots, smod, cov, view, proj, tx, ty, up["color"], up["depth"],
            up["alpha"], up["proj_2d"], up["conic_2d"], up["conic_2d_inv"], sh, deg, campos,
            g if geom is None else geom, num_rendered, b if binning is None else binning, i if img is None else img,
            alpha]


def _oracle_grads(scene, up, *, colors=False, flow_double=False):
    host, ref = oracle_forward(scene, colors=colors)
    return oracle.rasterize_backward(
        host, ref, to_np(up["color"]), to_np(up["depth"]), to_np(up["alpha"]), grad_proj_2d=to_np(up["proj_2d"]),
        grad_conic_2d=to_np(up["conic_2d"]), grad_conic_2d_inv=to_np(up["conic_2d_inv"]), flow_double=flow_double,
        with_bound=True)


def _check_grads(scene, grads, ref_g, *, colors=False):
    grads = dict(zip(GRAD_NAMES, grads))
    names = ["means2D", "opacities", "means3D"]
    names += ["colors"] if colors else ["sh"]
    names += ["cov3D"] if "cov3D_precomp" in scene else ["scales", "rotations"]
    failures = []
    for name in names:
        expected = ref_g[name]
        bad, worst = report_grad(name, to_np(grads[name]).reshape(expected.shape), expected, ref_g["bound"][name])
        if bad:
            failures.append((name, bad, worst))
    assert not failures, failures


def test_raw_forward_backward_compatibility_round_trip(device):
    """test_rasterizer_cuda_contracts.py:806-878: one Gaussian through the raw
    forward and backward; 8 finite gradients, a non-zero scale gradient."""
    n = 1
    bg = torch.zeros(3, device=device)
    means = torch.tensor([[0.0, 0.0, 2.0]], device=device)
    colors = torch.full((n, 3), 0.2, device=device)
    opac = torch.full((n, 1), 0.8, device=device)
    scales = torch.full((n, 3), 0.5, device=device)
    rots = torch.tensor([[1.0, 0.0, 0.0, 0.0]], device=device)
    empty = torch.empty((0,), device=device)
    eye = torch.eye(4, device=device)
    fwd = _rasterizer.rasterize_gaussians(bg, means, colors, opac, scales, rots, 1.0, empty, eye, eye, 1.0, 1.0, 16,
                                          16, empty, 0, torch.zeros(3, device=device), False)
    assert len(fwd) == 11
    num_rendered, color, depth, alpha, radii, geom, binning, img, proj_2d, conic_2d, conic_2d_inv = fwd
    assert isinstance(num_rendered, int) and num_rendered > 0
    assert geom.dtype == binning.dtype == img.dtype == torch.uint8
    grads = _rasterizer.rasterize_gaussians_backward(
        bg, means, radii, colors, opac, scales, rots, 1.0, empty, eye, eye, 1.0, 1.0, torch.ones_like(color),
        torch.zeros_like(depth), torch.zeros_like(alpha), torch.zeros_like(proj_2d), torch.zeros_like(conic_2d),
        torch.zeros_like(conic_2d_inv), empty, 0, torch.zeros(3, device=device), geom, num_rendered, binning, img,
        alpha)
    torch.cuda.synchronize()
    assert len(grads) == 8
    assert all(torch.isfinite(g).all() for g in grads)
    assert grads[6].abs().sum().item() > 0.0


@pytest.mark.parametrize("sort_mode", ["warp_depth_stable_tile", "warp_radix", "torch"])
def test_raw_forward_matches_typed_forward(sort_mode, device):
    scene = configs.make_scene(1, count=30_000, width=320, height=240, device=device)
    args = _raw_args(scene)
    original = _rasterizer.get_binning_sort_mode()
    try:
        _rasterizer.set_binning_sort_mode(sort_mode)
        raw = _rasterizer.rasterize_gaussians(*args)
        typed = _rasterizer.rasterize_gaussians_typed(*args)
    finally:
        _rasterizer.set_binning_sort_mode(original)
    torch.cuda.synchronize()
    num_rendered, color, depth, alpha, radii, geom, binning, img, proj_2d, conic_2d, conic_2d_inv = raw
    assert num_rendered == typed.num_rendered > 0
    for a, b in ((color, typed.color), (depth, typed.depth), (alpha, typed.alpha), (radii, typed.radii),
                 (proj_2d, typed.proj_2d), (conic_2d, typed.conic_2d), (conic_2d_inv, typed.conic_2d_inv)):
        assert torch.equal(a, b)
    st = typed.state
    P = radii.shape[0]
    assert torch.equal(geom[: 48 * P].view(torch.float32).view(P, 12), st.preprocess.records)
    assert torch.equal(geom[48 * P:], st.preprocess.clamped)
    ints = binning.view(torch.int32)
    assert torch.equal(ints[:num_rendered], st.binning.point_list)
    assert torch.equal(ints[num_rendered:].view(-1, 2), st.binning.ranges)
    assert torch.equal(img.view(torch.int32), st.n_contrib.reshape(-1))


@pytest.mark.parametrize("variant", ["sh", "colors", "precomputed_covariance"])
def test_raw_backward_matches_oracle(variant, device):
    scene = configs.make_scene(2, count=20_000, width=320, height=200, device=device)
    if variant == "precomputed_covariance":
        scene = with_precomputed_covariance(scene)
    colors = variant == "colors"
    args = _raw_args(scene, colors=colors)
    fwd = _rasterizer.rasterize_gaussians(*args)
    up = _upstream(scene)
    grads = _rasterizer.rasterize_gaussians_backward(*_backward_args(args, fwd, up))
    torch.cuda.synchronize()
    assert len(grads) == 8
    _check_grads(scene, grads, _oracle_grads(scene, up, colors=colors), colors=colors)


def test_raw_backward_rebuilds_state_when_buffers_do_not_unpack(device):
    """A wrong-sized buffer sends the backward down the rebuild path
    (backward_ops.py:425-470); the gradients still meet the bar."""
    scene = configs.make_scene(1, count=20_000, width=256, height=256, device=device)
    args = _raw_args(scene)
    fwd = _rasterizer.rasterize_gaussians(*args)
    up = _upstream(scene)
    broken = torch.empty((0,), dtype=torch.uint8, device=device)
    grads = _rasterizer.rasterize_gaussians_backward(*_backward_args(args, fwd, up, geom=broken))
    torch.cuda.synchronize()
    _check_grads(scene, grads, _oracle_grads(scene, up))


def test_raw_typed_backward_uses_the_given_state(device):
    scene = configs.make_scene(1, count=20_000, width=256, height=256, device=device)
    args = _raw_args(scene)
    typed = _rasterizer.rasterize_gaussians_typed(*args)
    fwd = (typed.num_rendered, typed.color, typed.depth, typed.alpha, typed.radii, None, None, None)
    up = _upstream(scene)
    empty = torch.empty((0,), dtype=torch.uint8, device=device)
    grads = _rasterizer.rasterize_gaussians_backward_typed(
        *_backward_args(args, fwd, up, geom=empty, binning=empty, img=empty), forward_state=typed.state)
    torch.cuda.synchronize()
    _check_grads(scene, grads, _oracle_grads(scene, up))


def test_raw_empty_scene(device):
    bg = torch.tensor([0.1, 0.4, 0.8], device=device)
    empty = torch.empty((0,), device=device)
    eye = torch.eye(4, device=device)
    args = [bg, torch.empty((0, 3), device=device), empty, torch.empty((0, 1), device=device), empty, empty, 1.0,
            empty, eye, eye, 1.0, 1.0, 16, 16, empty, 0, torch.zeros(3, device=device), False]
    fwd = _rasterizer.rasterize_gaussians(*args)
    assert fwd[0] == 0 and all(t.numel() == 0 for t in fwd[5:8])
    torch.testing.assert_close(fwd[1], bg[:, None, None].expand(3, 16, 16))
    up = {"color": torch.ones(3, 16, 16, device=device), "depth": torch.zeros(1, 16, 16, device=device),
          "alpha": torch.zeros(1, 16, 16, device=device), "proj_2d": torch.zeros(0, 2, device=device),
          "conic_2d": torch.zeros(0, 3, device=device), "conic_2d_inv": torch.zeros(0, 3, device=device)}
    grads = _rasterizer.rasterize_gaussians_backward(*_backward_args(args, fwd, up))
    assert len(grads) == 8 and grads[3].shape == (0, 3)
    flow = _rasterizer_flow.rasterize_gaussians(*args)
    assert len(flow) == 14


@pytest.mark.parametrize("enable_flow_grad", [True, False])
def test_raw_flow_forward_and_backward(enable_flow_grad, device):
    scene = configs.make_scene(4, count=20_000, width=320, height=180, device=device)
    args = _raw_args(scene)
    original = _rasterizer_flow.get_compute_flow_aux()
    try:
        _rasterizer_flow.set_compute_flow_aux(True)
        fwd = _rasterizer_flow.rasterize_gaussians(*args)
        typed = _rasterizer_flow.rasterize_gaussians_typed(*args)
    finally:
        _rasterizer_flow.set_compute_flow_aux(original)
    assert len(fwd) == 14
    for a, b in zip(fwd[11:], typed.aux):
        assert torch.equal(a, b)
    assert torch.equal(fwd[1], typed.color)
    k = _rasterizer_flow.get_flow_topk()
    assert fwd[11].shape == (k, scene["height"], scene["width"])
    up = _upstream(scene)
    bargs = _backward_args(args, fwd, up)
    # the flow outputs' gradients sit after grad_conic_2D_inv and are ignored
    flow_grads = [None, None, torch.randn_like(fwd[13])]
    bargs = bargs[:19] + flow_grads + bargs[19:] + [enable_flow_grad]
    grads = _rasterizer_flow.rasterize_gaussians_backward(*bargs)
    torch.cuda.synchronize()
    _check_grads(scene, grads, _oracle_grads(scene, up, flow_double=enable_flow_grad))
