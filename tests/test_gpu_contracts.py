"""Public-API contracts on the GPU, restating the reference's CUDA contract
tests (tests/test_rasterizer_cuda_contracts.py) for the scales/rotations path,
plus full-size (config 2) structural properties of the binning.

Every test runs the HIP library through the public API; none can fall back to
the CPU (the library raises if it is missing).
"""

from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor
from threading import Barrier

import pytest
import torch

from gswarp_amd import _runtime, _workspace, configs
from gswarp_amd.rasterizer import GaussianRasterizationSettings as Settings
from gswarp_amd.rasterizer import GaussianRasterizer, clear_warp_caches, get_warp_cache_report, rasterize_gaussians
from gswarp_amd.rasterizer_flow import GaussianRasterizationSettings as FlowSettings
from gswarp_amd.rasterizer_flow import rasterize_gaussians as rasterize_flow
from helpers import gpu_forward, options

pytestmark = pytest.mark.gpu


def _empty(device):
    return torch.empty((0,), dtype=torch.float32, device=device)


def _settings(device, bg, *, flow=False, size=16, **extra):
    common = dict(image_height=size, image_width=size, tanfovx=1.0, tanfovy=1.0, bg=bg, scale_modifier=1.0,
                  viewmatrix=torch.eye(4, device=device), projmatrix=torch.eye(4, device=device), sh_degree=0,
                  campos=torch.zeros(3, device=device), prefiltered=False, auto_tune=False, auto_tune_verbose=False)
    common.update(extra)
    if flow:
        return FlowSettings(**common, enable_flow_grad=False, compute_flow_aux=False)
    return Settings(**common)


def _inputs(device, means, *, scales=None, sh=None, covariances=None):
    n = means.shape[0]
    if scales is None and covariances is None:
        scales = torch.full((n, 3), 0.5, device=device)
    return dict(
        means3D=means,
        means2D=torch.zeros((n, 3), device=device, requires_grad=True),
        sh=_empty(device) if sh is None else sh,
        colors_precomp=torch.full((n, 3), 0.2, device=device) if sh is None else _empty(device),
        opacities=torch.full((n, 1), 0.8, device=device),
        scales=_empty(device) if covariances is not None else scales,
        rotations=_empty(device) if covariances is not None else
        torch.tensor([[1.0, 0.0, 0.0, 0.0]], device=device).expand(n, -1).clone(),
        cov3Ds_precomp=_empty(device) if covariances is None else covariances,
    )


def _std(device, inputs, settings):
    return rasterize_gaussians(inputs["means3D"], inputs["means2D"], inputs["sh"], inputs["colors_precomp"],
                               inputs["opacities"], inputs["scales"], inputs["rotations"], inputs["cov3Ds_precomp"],
                               settings)


def _flow(device, inputs, settings):
    return rasterize_flow(inputs["means3D"], inputs["means2D"], inputs["sh"], inputs["colors_precomp"],
                          inputs["opacities"], inputs["scales"], inputs["rotations"], inputs["cov3Ds_precomp"],
                          settings)


@pytest.fixture(autouse=True)
def _fresh_caches():
    clear_warp_caches()
    yield


def test_depth_disable_preserves_colour_and_returns_zero_depth(device):
    bg = torch.tensor([0.1, 0.2, 0.3], device=device)
    inputs = _inputs(device, torch.tensor([[-0.2, 0.1, 2.0], [0.25, -0.15, 2.5]], device=device))
    settings = _settings(device, bg, size=64)
    fsettings = _settings(device, bg, size=64, flow=True)
    original = _runtime.get_compute_depth()
    try:
        _runtime.set_compute_depth(True)
        on = _std(device, inputs, settings)
        fon = _flow(device, inputs, fsettings)
        _runtime.set_compute_depth(False)
        off = _std(device, inputs, settings)
        foff = _flow(device, inputs, fsettings)
        torch.cuda.synchronize()
    finally:
        _runtime.set_compute_depth(original)
    torch.testing.assert_close(off[0], on[0])
    torch.testing.assert_close(off[1], on[1])
    torch.testing.assert_close(off[2].alpha, on[2].alpha)
    assert torch.count_nonzero(off[2].depth) == 0 and torch.count_nonzero(on[2].depth) > 0
    torch.testing.assert_close(foff[0], fon[0])
    torch.testing.assert_close(foff[3], fon[3])
    assert torch.count_nonzero(foff[2]) == 0


def test_empty_inputs_return_background_for_both_backends(device):
    bg = torch.tensor([0.1, 0.4, 0.8], device=device)
    inputs = _inputs(device, torch.empty((0, 3), device=device))
    expected = bg[:, None, None].expand(3, 16, 16)
    color, radii, _ = _std(device, inputs, _settings(device, bg))
    fout = _flow(device, inputs, _settings(device, bg, flow=True))
    torch.testing.assert_close(color, expected)
    torch.testing.assert_close(fout[0], expected)
    assert radii.numel() == 0 and fout[1].numel() == 0


def test_all_culled_inputs_return_background_and_zero_gradients(device):
    bg = torch.tensor([0.2, 0.6, 0.3], device=device)
    means = torch.tensor([[0.0, 0.0, -2.0]], device=device, requires_grad=True)
    inputs = _inputs(device, means)
    inputs["colors_precomp"] = torch.full((1, 3), 0.2, device=device, requires_grad=True)
    inputs["opacities"] = torch.full((1, 1), 0.8, device=device, requires_grad=True)
    inputs["scales"] = torch.full((1, 3), 0.5, device=device, requires_grad=True)
    color, radii, meta = _std(device, inputs, _settings(device, bg))
    color.sum().backward()
    torch.testing.assert_close(color, bg[:, None, None].expand(3, 16, 16))
    assert torch.count_nonzero(radii) == 0
    assert torch.count_nonzero(meta.proj_2D) == 0 and torch.count_nonzero(meta.conic_2D) == 0
    for t in (means, inputs["colors_precomp"], inputs["opacities"], inputs["scales"]):
        assert torch.count_nonzero(t.grad) == 0


def test_subthreshold_opacity_preserves_geometric_visibility(device):
    bg = torch.tensor([0.2, 0.6, 0.3], device=device)
    inputs = _inputs(device, torch.tensor([[0.0, 0.0, 2.0]], device=device))
    inputs["opacities"] = torch.full((1, 1), 1e-4, device=device)
    color, radii, _ = _std(device, inputs, _settings(device, bg))
    torch.testing.assert_close(color, bg[:, None, None].expand(3, 16, 16))
    assert radii.item() > 0


def test_rotated_gaussian_matches_per_pixel_compositing(device):
    """test_rasterizer_cuda_contracts.py:482-505 with a scales/rotations Gaussian."""
    size = 64
    bg = torch.tensor([0.1, 0.2, 0.3], device=device)
    opacity = 0.2
    rgb = torch.tensor([[0.7, 0.4, 0.2]], device=device)
    inputs = _inputs(device, torch.tensor([[-0.5, -0.5, 2.0]], device=device),
                     scales=torch.tensor([[0.25, 0.03, 0.1]], device=device))
    inputs["rotations"] = torch.tensor([[0.92, 0.0, 0.0, 0.39]], device=device)
    inputs["colors_precomp"] = rgb
    inputs["opacities"] = torch.full((1, 1), opacity, device=device)
    rendered, _, meta = _std(device, inputs, _settings(device, bg, size=size))
    point, conic = meta.proj_2D[0], meta.conic_2D[0]
    pix = torch.arange(size, dtype=torch.float32, device=device)
    py, px = torch.meshgrid(pix, pix, indexing="ij")
    dx, dy = point[0] - px, point[1] - py
    power = -0.5 * (conic[0] * dx * dx + conic[2] * dy * dy) - conic[1] * dx * dy
    alpha = torch.clamp(opacity * torch.exp(power), max=0.99)
    alpha = torch.where(alpha >= 1.0 / 255.0, alpha, 0.0)
    expected = rgb[0, :, None, None] * alpha[None] + bg[:, None, None] * (1.0 - alpha[None])
    torch.testing.assert_close(rendered, expected, atol=2e-5, rtol=2e-4)
    assert alpha.max() > 0.15


def test_coverage_modes_agree_on_a_large_rotated_gaussian(device):
    size = 128
    bg = torch.tensor([0.1, 0.2, 0.3], device=device)
    inputs = _inputs(device, torch.tensor([[-0.15, 0.1, 2.0]], device=device),
                     scales=torch.tensor([[0.6, 0.04, 0.1]], device=device))
    inputs["rotations"] = torch.tensor([[0.92, 0.0, 0.0, 0.39]], device=device)
    inputs["opacities"] = torch.full((1, 1), 0.35, device=device)
    original = _runtime.get_tile_coverage_mode()
    outs = {}
    try:
        for mode in ("snugbox", "accutile_sweep", "conic_rect", "auto"):
            _runtime.set_tile_coverage_mode(mode)
            outs[mode] = _std(device, inputs, _settings(device, bg, size=size))
            torch.cuda.synchronize()
    finally:
        _runtime.set_tile_coverage_mode(original)
    ref = outs["snugbox"]
    for mode in ("accutile_sweep", "conic_rect", "auto"):
        torch.testing.assert_close(outs[mode][0], ref[0], atol=2e-5, rtol=2e-4)
        torch.testing.assert_close(outs[mode][1], ref[1])
        for a, e in zip(outs[mode][2], ref[2]):
            torch.testing.assert_close(a, e, atol=2e-5, rtol=2e-4)


def test_mark_visible_returns_owned_bool_tensor(device):
    rast = GaussianRasterizer(_settings(device, torch.zeros(3, device=device)))
    first = rast.markVisible(torch.tensor([[0.0, 0.0, 2.0], [0.2, 0.0, 2.0]], device=device))
    torch.cuda.synchronize()
    expected = first.clone()
    second = rast.markVisible(torch.tensor([[0.0, 0.0, -2.0], [0.2, 0.0, 0.1]], device=device))
    torch.cuda.synchronize()
    assert first.dtype == torch.bool and first.data_ptr() != second.data_ptr()
    torch.testing.assert_close(first, expected)
    assert bool(first.all()) and not bool(second.any())


def test_conic_inverse_gradient_matches_finite_difference(device):
    bg = torch.zeros(3, device=device)
    means = torch.tensor([[0.0, 0.0, 2.0]], device=device)

    def loss_for(value, grad):
        scales = torch.full((1, 3), value, device=device, requires_grad=grad)
        _, _, meta = _std(device, _inputs(device, means, scales=scales), _settings(device, bg))
        return meta.conic_2D_inv.sum(), scales

    loss, scales = loss_for(0.5, True)
    loss.backward()
    analytic = scales.grad.sum().item()
    eps = 1e-3
    numeric = (loss_for(0.5 + eps, False)[0].item() - loss_for(0.5 - eps, False)[0].item()) / (2 * eps)
    assert analytic != 0.0
    assert abs(analytic - numeric) <= max(1e-2, abs(numeric) * 5e-2)


def _iso_cov(device, var=0.25, grad=False):
    return torch.tensor([[var, 0.0, 0.0, var, 0.0, var]], device=device, requires_grad=grad)


def test_precomputed_covariance_preprocess_avoids_host_scalar_readback(device):
    """test_rasterizer_cuda_contracts.py:368-395: a culled cov3D_precomp point
    preprocesses with no Tensor.item() and leaves zero radii and conics."""
    from unittest.mock import patch

    from gswarp_amd import _pipeline
    from helpers import raster_inputs
    scene = dict(means3D=torch.tensor([[0.0, 0.0, -2.0]], device=device), cov3D_precomp=_iso_cov(device),
                 opacities=torch.full((1, 1), 0.8, device=device), bg=torch.zeros(3, device=device),
                 viewmatrix=torch.eye(4, device=device), projmatrix=torch.eye(4, device=device),
                 tanfovx=1.0, tanfovy=1.0, height=16, width=16, campos=torch.zeros(3, device=device),
                 sh_degree=0, colors_precomp=torch.full((1, 3), 0.2, device=device))
    inputs = raster_inputs(scene, colors=True)
    with patch.object(torch.Tensor, "item", side_effect=AssertionError):
        pre = _pipeline.preprocess(inputs, options())
    torch.cuda.synchronize()
    assert torch.count_nonzero(pre.radii) == 0
    assert torch.count_nonzero(pre.conic_2d) == 0 and torch.count_nonzero(pre.tiles_touched) == 0


def test_all_culled_precomputed_covariance_has_zero_gradients(device):
    """test_rasterizer_cuda_contracts.py:397-433."""
    bg = torch.tensor([0.2, 0.6, 0.3], device=device)
    means = torch.tensor([[0.0, 0.0, -2.0]], device=device, requires_grad=True)
    cov = _iso_cov(device, grad=True)
    inputs = _inputs(device, means, covariances=cov)
    inputs["colors_precomp"] = torch.full((1, 3), 0.2, device=device, requires_grad=True)
    inputs["opacities"] = torch.full((1, 1), 0.8, device=device, requires_grad=True)
    color, radii, meta = _std(device, inputs, _settings(device, bg))
    color.sum().backward()
    torch.testing.assert_close(color, bg[:, None, None].expand(3, 16, 16))
    assert torch.count_nonzero(radii) == 0
    assert torch.count_nonzero(meta.proj_2D) == 0 and torch.count_nonzero(meta.conic_2D) == 0
    for t in (means, cov, inputs["colors_precomp"], inputs["opacities"]):
        assert t.grad is not None and t.grad.shape == t.shape
        assert torch.count_nonzero(t.grad) == 0


def test_conic_inverse_gradient_reaches_precomputed_covariance_path(device):
    """test_rasterizer_cuda_contracts.py:609-623, with a central-difference check
    of each of the six covariance entries added."""
    bg = torch.zeros(3, device=device)
    means = torch.tensor([[0.0, 0.0, 2.0]], device=device)
    base = torch.tensor([[0.25, 0.03, -0.02, 0.2, 0.04, 0.3]], device=device)

    def loss_for(cov, grad):
        cov = cov.clone().requires_grad_(grad)
        _, _, meta = _std(device, _inputs(device, means, covariances=cov), _settings(device, bg))
        return meta.conic_2D_inv.sum(), cov

    loss, cov = loss_for(base, True)
    loss.backward()
    assert torch.isfinite(cov.grad).all() and cov.grad.abs().sum().item() > 0
    eps = 1e-3
    for j in range(6):
        step = torch.zeros_like(base)
        step[0, j] = eps
        numeric = (loss_for(base + step, False)[0].item() - loss_for(base - step, False)[0].item()) / (2 * eps)
        assert abs(cov.grad[0, j].item() - numeric) <= max(1e-2, abs(numeric) * 5e-2), (j, cov.grad, numeric)


def test_rotated_precomputed_covariance_matches_per_pixel_compositing(device):
    """The rotated-Gaussian compositing contract (test_rasterizer_cuda_contracts.py:482-505)
    fed the same Gaussian as a precomputed covariance."""
    import numpy as np

    import dense_ref
    size = 64
    bg = torch.tensor([0.1, 0.2, 0.3], device=device)
    opacity = 0.2
    rgb = torch.tensor([[0.7, 0.4, 0.2]], device=device)
    cov = dense_ref.covariance_upper(np.array([[0.25, 0.03, 0.1]]), np.array([[0.92, 0.0, 0.0, 0.39]]))
    inputs = _inputs(device, torch.tensor([[-0.5, -0.5, 2.0]], device=device),
                     covariances=torch.tensor(cov, dtype=torch.float32, device=device))
    inputs["colors_precomp"] = rgb
    inputs["opacities"] = torch.full((1, 1), opacity, device=device)
    rendered, _, meta = _std(device, inputs, _settings(device, bg, size=size))
    point, conic = meta.proj_2D[0], meta.conic_2D[0]
    pix = torch.arange(size, dtype=torch.float32, device=device)
    py, px = torch.meshgrid(pix, pix, indexing="ij")
    dx, dy = point[0] - px, point[1] - py
    power = -0.5 * (conic[0] * dx * dx + conic[2] * dy * dy) - conic[1] * dx * dy
    alpha = torch.clamp(opacity * torch.exp(power), max=0.99)
    alpha = torch.where(alpha >= 1.0 / 255.0, alpha, 0.0)
    expected = rgb[0, :, None, None] * alpha[None] + bg[:, None, None] * (1.0 - alpha[None])
    torch.testing.assert_close(rendered, expected, atol=2e-5, rtol=2e-4)
    assert alpha.max() > 0.15


def _mip_settings(device, bg, f, **extra):
    from gswarp_amd.methods.mip_3dgs import MipGaussianRasterizationSettings
    common = _settings(device, bg)._asdict()
    common.update(extra)
    return MipGaussianRasterizationSettings(**common, filter_variance=f)


def _two_gaussian_inputs(device):
    means = torch.tensor([[-0.15, 0.05, 2.0], [0.2, -0.1, 2.4]], device=device, requires_grad=True)
    inputs = _inputs(device, means, scales=torch.tensor([[0.25, 0.1, 0.05], [0.12, 0.3, 0.2]], device=device))
    inputs["rotations"] = torch.tensor([[0.9, 0.1, 0.0, 0.4], [1.0, 0.0, 0.2, 0.0]], device=device)
    for key in ("colors_precomp", "opacities", "scales", "rotations"):
        inputs[key] = inputs[key].clone().requires_grad_(True)
    return inputs


def test_mip_zero_filter_matches_baseline_and_filtered_gradients_are_finite(device):
    """test_classic_variant_methods_cuda.py:144-162."""
    from gswarp_amd.methods.mip_3dgs import rasterize_gaussians as rasterize_mip
    bg = torch.tensor([0.05, 0.15, 0.25], device=device)

    def loss(out):
        return out[0].square().mean() + out[2].alpha.mean() + out[2].depth.mean()

    base_in = _two_gaussian_inputs(device)
    base = _std(device, base_in, _settings(device, bg))
    loss(base).backward()
    zero_in = _two_gaussian_inputs(device)
    zero = rasterize_mip(*(zero_in[k] for k in ("means3D", "means2D", "sh", "colors_precomp", "opacities", "scales",
                                                "rotations", "cov3Ds_precomp")), _mip_settings(device, bg, 0.0))
    torch.testing.assert_close(zero[0], base[0], rtol=2e-5, atol=2e-5)
    torch.testing.assert_close(zero[2].alpha, base[2].alpha, rtol=2e-5, atol=2e-5)
    loss(zero).backward()
    torch.testing.assert_close(zero_in["means3D"].grad, base_in["means3D"].grad, rtol=3e-4, atol=3e-5)
    filt_in = _two_gaussian_inputs(device)
    filt = rasterize_mip(*(filt_in[k] for k in ("means3D", "means2D", "sh", "colors_precomp", "opacities", "scales",
                                                "rotations", "cov3Ds_precomp")), _mip_settings(device, bg, 0.25))
    loss(filt).backward()
    for name in ("means3D", "means2D", "colors_precomp", "opacities", "scales", "rotations"):
        assert torch.isfinite(filt_in[name].grad).all(), name
    # the filter only widens each footprint (every conic shrinks), so the
    # accumulated alpha grows
    assert float(filt[2].alpha.detach().sum()) > float(base[2].alpha.detach().sum())


def test_mip_settings_are_validated(device):
    from gswarp_amd.methods.mip_3dgs import MipGaussianRasterizer
    bg = torch.zeros(3, device=device)
    inputs = _inputs(device, torch.tensor([[0.0, 0.0, 2.0]], device=device))
    for bad in (dict(f=-0.1), dict(f=float("inf")), dict(f=0.3, antialiasing=True)):
        f = bad.pop("f")
        rast = MipGaussianRasterizer(_mip_settings(device, bg, f, **bad))
        with pytest.raises(ValueError):
            rast(inputs["means3D"], inputs["means2D"], inputs["opacities"], colors_precomp=inputs["colors_precomp"],
                 scales=inputs["scales"], rotations=inputs["rotations"])


def test_mip_filter_conic_inverse_gradient_matches_finite_difference(device):
    """The filter variance enters the backward's recomputed cov2D: the analytic
    dL/dscale of sum(conic_2D_inv) under the filter matches central differences."""
    from gswarp_amd.methods.mip_3dgs import rasterize_gaussians as rasterize_mip
    bg = torch.zeros(3, device=device)
    means = torch.tensor([[0.1, 0.0, 2.0]], device=device)

    def loss_for(value, grad):
        scales = torch.tensor([[value, 0.3, 0.2]], device=device, requires_grad=grad)
        inp = _inputs(device, means, scales=scales)
        out = rasterize_mip(*(inp[k] for k in ("means3D", "means2D", "sh", "colors_precomp", "opacities", "scales",
                                               "rotations", "cov3Ds_precomp")), _mip_settings(device, bg, 0.5))
        return out[2].conic_2D.sum(), scales

    loss, scales = loss_for(0.5, True)
    loss.backward()
    analytic = scales.grad[0, 0].item()
    eps = 1e-3
    numeric = (loss_for(0.5 + eps, False)[0].item() - loss_for(0.5 - eps, False)[0].item()) / (2 * eps)
    assert analytic != 0.0
    assert abs(analytic - numeric) <= max(1e-4, abs(numeric) * 2e-2), (analytic, numeric)


def test_colour_gradient_matches_finite_difference(device):
    """Central differences of sum(colour * W) through the GPU forward against
    the GPU backward, for the mean, scales and rotation of one Gaussian.  W is
    a ramp times a bump that vanishes two sigma from the centre, so the loss
    is smooth: the alpha cut-off contour (3.3 sigma), where the colour jumps
    by 1/255 of a contrast and the analytic gradient has no term, lies outside
    the weight's support."""
    size = 32
    bg = torch.tensor([0.1, 0.2, 0.3], device=device)
    settings = _settings(device, bg, size=size)
    base = {"means3D": torch.tensor([[0.05, -0.03, 2.0]], device=device),
            "scales": torch.tensor([[0.4, 0.35, 0.3]], device=device),
            "rotations": torch.tensor([[0.95, 0.1, -0.2, 0.2]], device=device)}

    def run(params, grad):
        p = {k: v.clone().requires_grad_(grad) for k, v in params.items()}
        inputs = _inputs(device, p["means3D"], scales=p["scales"])
        inputs["rotations"] = p["rotations"]
        inputs["opacities"] = torch.full((1, 1), 0.6, device=device)
        inputs["colors_precomp"] = torch.tensor([[0.9, 0.5, 0.1]], device=device)
        color, _, meta = _std(device, inputs, settings)
        return color, meta, p

    color, meta, p = run(base, True)
    px, py = meta.proj_2D[0].tolist()
    ys, xs = torch.meshgrid(torch.arange(size, dtype=torch.float64), torch.arange(size, dtype=torch.float64),
                            indexing="ij")
    bump = torch.clamp(1 - ((xs - px) ** 2 + (ys - py) ** 2) / 6.4 ** 2, min=0) ** 2
    weight = ((xs / size + 0.5 * ys / size) * bump)[None].expand(3, size, size)
    (color * weight.to(device=device, dtype=torch.float32)).sum().backward()

    def loss(params):
        with torch.no_grad():
            c, _, _ = run(params, False)
        return float((c.double().cpu() * weight).sum())

    eps = 2e-3
    checked = 0
    for name, idx in (("means3D", (0, 0)), ("means3D", (0, 1)), ("means3D", (0, 2)), ("scales", (0, 0)),
                      ("scales", (0, 2)), ("rotations", (0, 1)), ("rotations", (0, 3))):
        plus = {k: v.clone() for k, v in base.items()}
        minus = {k: v.clone() for k, v in base.items()}
        plus[name][idx] += eps
        minus[name][idx] -= eps
        numeric = (loss(plus) - loss(minus)) / (2 * eps)
        analytic = p[name].grad[idx].item()
        assert abs(analytic - numeric) <= 2e-3 * abs(numeric) + 2e-3, (name, idx, analytic, numeric)
        checked += abs(numeric) > 0.1
    assert checked >= 4


def test_flow_conic_inverse_gradient_reaches_scales(device):
    bg = torch.zeros(3, device=device)
    scales = torch.full((1, 3), 0.5, device=device, requires_grad=True)
    out = _flow(device, _inputs(device, torch.tensor([[0.0, 0.0, 2.0]], device=device), scales=scales),
                _settings(device, bg, flow=True))
    out[6].sum().backward()
    assert torch.isfinite(scales.grad).all() and scales.grad.abs().sum().item() > 0


def test_repeated_flow_calls_use_fresh_parameters(device):
    bg = torch.tensor([0.1, 0.2, 0.3], device=device)
    pts = torch.tensor([[-0.15, 0.05, 2.0], [0.2, -0.1, 2.4]], device=device)
    warm_scales = torch.full((2, 3), 0.45, device=device, requires_grad=True)
    warm = _flow(device, _inputs(device, pts, scales=warm_scales), _settings(device, bg, flow=True))
    warm[6].sum().backward()
    cached_scales = torch.full((2, 3), 0.65, device=device, requires_grad=True)
    cached = _flow(device, _inputs(device, pts, scales=cached_scales), _settings(device, bg, flow=True))
    cached[6].sum().backward()
    clear_warp_caches()
    ref_scales = torch.full((2, 3), 0.65, device=device, requires_grad=True)
    ref = _flow(device, _inputs(device, pts, scales=ref_scales), _settings(device, bg, flow=True))
    ref[6].sum().backward()
    torch.testing.assert_close(cached[0], ref[0])
    torch.testing.assert_close(cached[6], ref[6])
    torch.testing.assert_close(cached_scales.grad, ref_scales.grad)


def test_pending_forward_owns_its_binning_state(device):
    bg = torch.zeros(3, device=device)
    pts = torch.tensor([[-0.25, 0.0, 2.0], [0.25, 0.0, 2.0]], device=device)
    ref_scales = torch.full((2, 3), 0.5, device=device, requires_grad=True)
    ref_color, _, _ = _std(device, _inputs(device, pts, scales=ref_scales), _settings(device, bg))
    ref_color.sum().backward()
    clear_warp_caches()
    scales = torch.full((2, 3), 0.5, device=device, requires_grad=True)
    pending, _, _ = _std(device, _inputs(device, pts, scales=scales), _settings(device, bg))
    _std(device, _inputs(device, torch.tensor([[0.0, 0.0, 2.0]], device=device)), _settings(device, bg))
    pending.sum().backward()
    torch.testing.assert_close(scales.grad, ref_scales.grad)


def test_retain_graph_repeats_backward(device):
    bg = torch.zeros(3, device=device)
    scales = torch.full((8, 3), 0.5, device=device, requires_grad=True)
    g = torch.Generator(device="cpu").manual_seed(3)
    sh = torch.randn((8, 16, 3), generator=g).to(device).requires_grad_(True)
    inputs = _inputs(device, torch.tensor([[-0.2, 0.0, 2.0], [0.2, 0.0, 2.0]] * 4, device=device), scales=scales,
                     sh=sh)
    color, _, _ = _std(device, inputs, _settings(device, bg, sh_degree=3))
    loss = color.square().mean()
    loss.backward(retain_graph=True)
    first_scales, first_sh = scales.grad.clone(), sh.grad.clone()
    scales.grad = None
    sh.grad = None
    loss.backward()
    torch.testing.assert_close(scales.grad, first_scales)
    torch.testing.assert_close(sh.grad, first_sh)


def test_two_streams_match_isolated_references(device):
    bg = torch.zeros(3, device=device)
    settings = _settings(device, bg)
    pa = torch.tensor([[-0.25, 0.0, 2.0], [0.25, 0.0, 2.0]], device=device)
    pb = torch.tensor([[0.0, 0.0, 2.0]], device=device)

    def isolated(points):
        scales = torch.full((points.shape[0], 3), 0.5, device=device, requires_grad=True)
        color, _, _ = _std(device, _inputs(device, points, scales=scales), settings)
        color.square().mean().backward()
        torch.cuda.synchronize()
        return color.detach().clone(), scales.grad.detach().clone()

    ea, eb = isolated(pa), isolated(pb)
    clear_warp_caches()
    sa = torch.full((2, 3), 0.5, device=device, requires_grad=True)
    sb = torch.full((1, 3), 0.5, device=device, requires_grad=True)
    stream_a, stream_b = torch.cuda.Stream(device=device), torch.cuda.Stream(device=device)
    with torch.cuda.stream(stream_a):
        ca, _, _ = _std(device, _inputs(device, pa, scales=sa), settings)
        la = ca.square().mean()
    with torch.cuda.stream(stream_b):
        cb, _, _ = _std(device, _inputs(device, pb, scales=sb), settings)
        lb = cb.square().mean()
    with torch.cuda.stream(stream_a):
        la.backward()
    with torch.cuda.stream(stream_b):
        lb.backward()
    stream_a.synchronize()
    stream_b.synchronize()
    torch.testing.assert_close(ca, ea[0])
    torch.testing.assert_close(sa.grad, ea[1])
    torch.testing.assert_close(cb, eb[0])
    torch.testing.assert_close(sb.grad, eb[1])
    assert get_warp_cache_report()["workspace_entries"] == 2


def test_two_threads_submit_on_independent_streams(device):
    bg = torch.zeros(3, device=device)
    settings = _settings(device, bg)
    inputs = (_inputs(device, torch.tensor([[-0.2, 0.0, 2.0], [0.2, 0.0, 2.0]], device=device)),
              _inputs(device, torch.tensor([[0.0, 0.0, 2.0]], device=device)))
    with torch.no_grad():
        expected = tuple(_std(device, v, settings)[0].clone() for v in inputs)
    torch.cuda.synchronize()
    clear_warp_caches()
    streams = (torch.cuda.Stream(device=device), torch.cuda.Stream(device=device))
    barrier = Barrier(2)

    def submit(i):
        with torch.cuda.stream(streams[i]), torch.no_grad():
            barrier.wait()
            color, _, _ = _std(device, inputs[i], settings)
        streams[i].synchronize()
        return color

    with ThreadPoolExecutor(max_workers=2) as pool:
        actual = [f.result() for f in [pool.submit(submit, i) for i in range(2)]]
    torch.testing.assert_close(actual[0], expected[0])
    torch.testing.assert_close(actual[1], expected[1])


def test_workspace_stream_slots_are_bounded_and_evict_safely(device):
    bg = torch.zeros(3, device=device)
    settings = _settings(device, bg)
    inputs = _inputs(device, torch.tensor([[0.0, 0.0, 2.0]], device=device))
    with torch.no_grad():
        expected = _std(device, inputs, settings)[0].clone()
    streams = [torch.cuda.Stream(device=device) for _ in range(_workspace.MAX_WORKSPACE_STREAMS + 1)]
    before = get_warp_cache_report()["workspace_evictions"]
    outs = []
    for s in streams:
        with torch.cuda.stream(s), torch.no_grad():
            outs.append(_std(device, inputs, settings)[0])
    for s in streams:
        s.synchronize()
    report = get_warp_cache_report()
    assert report["workspace_entries"] == _workspace.MAX_WORKSPACE_STREAMS
    assert report["workspace_evictions"] > before
    for o in outs:
        torch.testing.assert_close(o, expected)


def test_invalid_settings_raise_before_launch(device):
    bg = torch.zeros(3, device=device)
    inputs = _inputs(device, torch.tensor([[0.0, 0.0, 2.0]], device=device))
    with pytest.raises(NotImplementedError):
        _std(device, inputs, _settings(device, bg, prefiltered=True))
    bad = dict(inputs)
    bad["opacities"] = torch.full((2, 1), 0.8, device=device)
    with pytest.raises(ValueError):
        _std(device, bad, _settings(device, bg))


@pytest.mark.parametrize("sort_mode", ["warp_depth_stable_tile", "warp_radix"])
def test_full_size_config2_binning_structure(sort_mode, device):
    """Config 2 at full size (1M Gaussians, 1920x1080): the sorted keys are
    non-decreasing, every key's tile matches its range, the ranges partition
    [0, R), R equals the sum of visible tile counts, and each tile's depths are
    non-decreasing with index order among equal depths."""
    scene = configs.make_scene(2, seed=0, device=device)
    out = gpu_forward(scene, options(sort_mode=sort_mode))
    pre, bins = out["pre"], out["bins"]
    R = bins.num_rendered
    assert R > 1_000_000
    vis = pre.radii > 0
    assert int(pre.tiles_touched[vis].sum().item()) == R
    tiles, depth, field_ = bins.decode_keys()
    assert bool((field_[1:] >= field_[:-1]).all())
    T = bins.ranges.shape[0]
    assert int(tiles.min()) >= 0 and int(tiles.max()) < T
    counts = torch.bincount(tiles, minlength=T)
    starts = torch.cumsum(counts, 0) - counts
    nonempty = counts > 0
    assert torch.equal(bins.ranges[nonempty, 0].long(), starts[nonempty])
    assert torch.equal(bins.ranges[nonempty, 1].long(), (starts + counts)[nonempty])
    assert int(bins.ranges[~nonempty].abs().sum()) == 0
    # the depth field is the depth of the listed Gaussian, and equal-field runs keep index order
    pts = bins.point_list.long()
    assert torch.equal(depth, pre.depths.view(torch.int32)[pts].to(torch.int64) & 0xFFFFFFFF)
    same = field_[1:] == field_[:-1]
    assert bool((pts[1:][same] > pts[:-1][same]).all())
    if sort_mode == "warp_radix":
        # this workload packs the point index into the key and sorts fewer than 6 passes of bits
        lay = bins.key_layout
        assert lay.value_bits == 20 and (T - 1).bit_length() + lay.depth_bits <= 40
    torch.cuda.synchronize()
