"""gs_render_fwd_clear: the forward blend that also zeroes the backward's
(N, 10) gradient accumulator (backward_ops.py:203 allocates it with
torch.zeros), so the backward needs no fill of its own.

The images must be bit-identical to gs_render_fwd's, exactly clear_floats
floats must be zeroed (float4 body plus a 1-3 float tail, for counts far
above and below the grid's share), nothing past them may be written, and the
autograd path, where the forward hands the zeroed buffer to one backward, must
give the same gradients as a backward that zero-fills its own.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from gswarp_amd import _lib, configs
from gswarp_amd.rasterizer import GaussianRasterizationSettings, GaussianRasterizer
from helpers import gpu_forward, options

pytestmark = pytest.mark.gpu

GUARD = 64


def _images(H, W, device):
    f = dict(dtype=torch.float32, device=device)
    return (torch.empty((3, H, W), **f), torch.empty((1, H, W), **f), torch.empty((1, H, W), **f),
            torch.empty((H * W,), dtype=torch.int32, device=device))


def _render(lib, scene, out, images, clear=None, count=0):
    pre, bins = out["pre"], out["bins"]
    H, W = scene["height"], scene["width"]
    stream = torch.cuda.current_stream(scene["means3D"].device).cuda_stream
    args = (W, H, pre.radii.shape[0], bins.num_rendered, bins.ranges.data_ptr(), bins.point_list.data_ptr(),
            pre.records.data_ptr(), scene["bg"].data_ptr(), 1) + tuple(t.data_ptr() for t in images)
    if clear is None and count == 0:
        return lib.gs_render_fwd(*args, None, stream)
    return lib.gs_render_fwd_clear(*args, clear, count, None, stream)


@pytest.mark.parametrize("count_of", ["p10", "p10_minus_1", "three", "large_plus_5"])
def test_clear_zeroes_exactly_and_keeps_images(count_of, device):
    lib = _lib.load()
    scene = configs.make_scene(2, count=20_000, width=320, height=200, device=device)
    out = gpu_forward(scene, options())
    P = scene["means3D"].shape[0]
    count = {"p10": 10 * P, "p10_minus_1": 10 * P - 1, "three": 3, "large_plus_5": (1 << 22) + 5}[count_of]
    print(f"render clear: count={count} P={P} R={out['bins'].num_rendered}", flush=True)
    buf = torch.full((count + GUARD,), float("nan"), device=device)
    ref = _images(200, 320, device)
    got = _images(200, 320, device)
    assert _render(lib, scene, out, ref) == 0
    assert _render(lib, scene, out, got, buf.data_ptr(), count) == 0
    torch.cuda.synchronize()
    for a, b in zip(ref, got):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    assert bool((buf[:count] == 0).all())
    assert bool(buf[count:].isnan().all()), "written past clear_floats"


def test_clear_argument_checks(device):
    lib = _lib.load()
    scene = configs.make_scene(1, count=2_000, width=64, height=64, device=device)
    out = gpu_forward(scene, options())
    images = _images(64, 64, device)
    buf = torch.zeros((64,), device=device)
    assert _render(lib, scene, out, images, buf.data_ptr() + 4, 8) != 0  # not 16-byte aligned
    assert _render(lib, scene, out, images, buf.data_ptr(), -1) != 0
    assert lib.gs_render_fwd_clear(64, 64, 1, 1, None, None, None, None, 1, None, None, None, None, None, 8,
                                   None, None) != 0
    torch.cuda.synchronize()


def _autograd_step(scene, device, *, twice=False):
    settings = GaussianRasterizationSettings(
        image_height=scene["height"], image_width=scene["width"], tanfovx=scene["tanfovx"],
        tanfovy=scene["tanfovy"], bg=scene["bg"], scale_modifier=1.0, viewmatrix=scene["viewmatrix"],
        projmatrix=scene["projmatrix"], sh_degree=scene["sh_degree"], campos=scene["campos"], prefiltered=False,
        debug=False, auto_tune=False, auto_tune_verbose=False)
    leaves = {k: scene[k].clone().requires_grad_(True) for k in ("means3D", "shs", "opacities", "scales",
                                                                 "rotations")}
    means2d = torch.zeros_like(leaves["means3D"], requires_grad=True)
    color, _radii, _meta = GaussianRasterizer(settings)(
        means3D=leaves["means3D"], means2D=means2d, shs=leaves["shs"], opacities=leaves["opacities"],
        scales=leaves["scales"], rotations=leaves["rotations"])
    g = torch.Generator(device="cpu").manual_seed(7)
    up = torch.randn(color.shape, generator=g).to(device)
    grads = torch.autograd.grad(color, list(leaves.values()) + [means2d], up, retain_graph=twice)
    if twice:
        again = torch.autograd.grad(color, list(leaves.values()) + [means2d], up)
        return grads, again
    return grads


def test_autograd_uses_the_cleared_buffer_once(device):
    """The first backward takes the buffer the forward zeroed; a second one
    over the retained graph zero-fills its own: both give the same result,
    and so does a fresh step."""
    scene = configs.make_scene(2, count=20_000, width=320, height=200, device=device)
    first, second = _autograd_step(scene, device, twice=True)
    fresh = _autograd_step(scene, device)
    torch.cuda.synchronize()
    # The render backward accumulates with float atomics in no fixed order, so
    # runs differ by rounding; a stale or unzeroed accumulator would differ by
    # whole contributions (or be NaN), far beyond this bound.
    for i, (a, b, c) in enumerate(zip(first, second, fresh)):
        assert bool(torch.isfinite(a).all()), i
        scale = float(a.abs().max()) + 1e-30
        for other in (b, c):
            err = float((a - other).abs().max())
            assert err <= 1e-4 * scale, (i, err, scale)


def test_accumulator_allocated_in_backward(device):
    """With ACCUMULATOR_IN_FORWARD off the forward allocates no accumulator
    and the backward allocates and fills its own: the gradients equal those of
    the default path (to the rounding of the atomics' order)."""
    from gswarp_amd import _pipeline

    scene = configs.make_scene(2, count=20_000, width=320, height=200, device=device)
    default = _autograd_step(scene, device)
    _pipeline.ACCUMULATOR_IN_FORWARD = False
    try:
        own = _autograd_step(scene, device)
    finally:
        _pipeline.ACCUMULATOR_IN_FORWARD = True
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(default, own)):
        assert bool(torch.isfinite(b).all()), i
        scale = float(a.abs().max()) + 1e-30
        err = float((a - b).abs().max())
        assert err <= 1e-4 * scale, (i, err, scale)


def _check_order(o, ranges):
    T = ranges.shape[0]
    assert np.array_equal(np.sort(o), np.arange(T))
    r = ranges.cpu().numpy()
    length = np.maximum(r[:, 1] - r[:, 0], 0)[o]
    cls = np.where(length < 512, length >> 2, 128 + np.minimum(127, (length - 512) >> 6))
    assert np.all(np.diff(cls) <= 0)


def test_tile_order_is_longest_first_permutation(device):
    """gs_tile_order: a permutation of the tiles whose list lengths never
    rise by more than the width of its length classes (4 pairs below 512,
    64 above) along the order; the forward render is bit-identical with and
    without it (the order changes only the schedule)."""
    lib = _lib.load()
    scene = configs.make_scene(2, count=150_000, width=480, height=270, device=device)
    out = gpu_forward(scene, options())
    bins = out["bins"]
    T = bins.ranges.shape[0]
    order = torch.full((T + GUARD,), -7, dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    assert lib.gs_tile_order(T, bins.ranges.data_ptr(), order.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    o = order.cpu().numpy()
    assert np.all(o[T:] == -7), "written past num_tiles"
    _check_order(o[:T], bins.ranges)
    a, b = _images(scene["height"], scene["width"], device), _images(scene["height"], scene["width"], device)
    assert _render(lib, scene, out, a) == 0
    args = (scene["width"], scene["height"], out["pre"].radii.shape[0], bins.num_rendered, bins.ranges.data_ptr(),
            bins.point_list.data_ptr(), out["pre"].records.data_ptr(), scene["bg"].data_ptr(), 1)
    P = out["pre"].radii.shape[0]
    assert 192 * T <= bins.num_rendered <= 4 * P, "the order is used at this R"
    order.fill_(-7)
    assert lib.gs_render_fwd(*args, *(t.data_ptr() for t in b), order.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    _check_order(order.cpu().numpy()[:T], bins.ranges)  # the forward wrote an order (ties in any order)
    for x, y in zip(a, b):
        assert torch.equal(x.view(torch.int32), y.view(torch.int32))
    # The backward over the forward's order: the same gradients up to the
    # rounding of its float atomics, whose order the schedule changes.
    g = torch.Generator(device="cpu").manual_seed(3)
    ups = [torch.randn(shape, generator=g).to(device) for shape in ((3,) + a[0].shape[1:], a[1].shape, a[2].shape)]
    grads = []
    for buf in (None, order.data_ptr()):
        gg = torch.zeros((P, _lib.GS_GRAD_FLOATS), dtype=torch.float32, device=device)
        assert lib.gs_render_bwd(scene["width"], scene["height"], P, bins.num_rendered, bins.ranges.data_ptr(),
                                 bins.point_list.data_ptr(), out["pre"].records.data_ptr(), scene["bg"].data_ptr(),
                                 a[2].data_ptr(), a[3].data_ptr(), *(u.data_ptr() for u in ups), 1, gg.data_ptr(),
                                 buf, stream) == 0
        grads.append(gg)
    torch.cuda.synchronize()
    scale = float(grads[0].abs().max()) + 1e-30
    assert float((grads[0] - grads[1]).abs().max()) <= 1e-4 * scale


def test_forward_writes_no_order_when_it_does_not_pay(device):
    """Below 192 pairs a tile the forward leaves the buffer untouched and the
    backward, given it, takes the tiles in tile order (it never reads it)."""
    lib = _lib.load()
    scene = configs.make_scene(1, count=2_000, width=256, height=256, device=device)
    out = gpu_forward(scene, options())
    bins = out["bins"]
    T = bins.ranges.shape[0]
    assert 0 < bins.num_rendered < 192 * T
    order = torch.full((T,), -7, dtype=torch.int32, device=device)
    images = _images(scene["height"], scene["width"], device)
    stream = torch.cuda.current_stream(device).cuda_stream
    args = (scene["width"], scene["height"], out["pre"].radii.shape[0], bins.num_rendered, bins.ranges.data_ptr(),
            bins.point_list.data_ptr(), out["pre"].records.data_ptr(), scene["bg"].data_ptr(), 1)
    assert lib.gs_render_fwd(*args, *(t.data_ptr() for t in images), order.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    assert bool((order == -7).all())
