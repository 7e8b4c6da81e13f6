"""The early-stop rule at its tie: a pixel stops before a Gaussian whose
blend would leave T * (1 - alpha) < 1e-4 (strict, render_kernels.py:126);
when the product is exactly 1e-4f the Gaussian still blends.

Four Gaussians centred exactly on pixel (5, 7) (q = 0 there, so alpha is
the opacity itself) with opacities found by exhaustive search over float32
values: T after the first two is 0.0050018085 and the third takes it to
exactly 1e-4f.  The third therefore blends (n_contrib 3) and the fourth,
which would take T to 5e-5, stops the pixel; a '<=' rule would give 2.  The
oracle is checked on the CPU; the GPU forward (gs_render_fwd on hand-built
records) is checked against it bit for bit.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle

W = H = 16
PX, PY = 5, 7
OPACITY_BITS = (0x3F733299, 0x3F66653C, 0x3F7AE1C1, 0x3F000000)  # 0.9499908, 0.8999822, 0.98000723, 0.5


def _scene():
    o = np.array(OPACITY_BITS, dtype=np.uint32).view(np.float32)
    n = o.shape[0]
    xy = np.tile(np.array([PX, PY], np.float32), (n, 1))
    conic = np.tile(np.array([10.0, 0.0, 10.0], np.float32), (n, 1))
    depths = np.arange(1, n + 1, dtype=np.float32)
    colors = np.array([[0.9, 0.1, 0.2], [0.3, 0.8, 0.1], [0.2, 0.3, 0.7], [0.5, 0.5, 0.5]], np.float32)
    bg = np.array([0.1, 0.2, 0.3], np.float32)
    return o, xy, conic, depths, colors, bg


def _oracle():
    o, xy, conic, depths, colors, bg = _scene()
    pre = {"proj_2d": xy, "depths": depths, "conic_opacity": np.concatenate([conic, o[:, None]], axis=1)}
    bins = {"num_rendered": o.shape[0], "point_list": np.arange(o.shape[0], dtype=np.int32),
            "ranges": np.array([[0, o.shape[0]]], np.int32)}
    return oracle.render_fwd(pre, bins, colors, bg, W, H, compute_depth=True)


def test_search_result_is_an_exact_tie():
    o = np.array(OPACITY_BITS, dtype=np.uint32).view(np.float32)
    one = np.float32(1.0)
    T = one * (one - o[0])
    T = np.float32(T * (one - o[1]))
    assert np.float32(T * (one - o[2])) == np.float32(1e-4)


def test_oracle_blends_at_the_tie():
    out = _oracle()
    assert int(out["n_contrib"][PY, PX]) == 3


@pytest.mark.gpu
def test_gpu_blends_at_the_tie(device):
    import torch

    from gswarp_amd import _lib

    o, xy, conic, depths, colors, bg = _scene()
    n = o.shape[0]
    rec = np.zeros((n, 12), np.float32)
    rec[:, 0:2] = xy
    rec[:, 2] = conic[:, 0]
    rec[:, 3] = conic[:, 1]
    rec[:, 4] = conic[:, 2]
    rec[:, 5] = o
    rec[:, 6] = depths
    # candidate bound on q (the preprocess stores -2 power_cutoff(o)): 174 keeps
    # every pixel with a representable exponential (power >= -87) a candidate,
    # so each decision is taken exactly, as in the oracle
    rec[:, 7] = np.float32(174.0)
    rec[:, 8:11] = colors
    rec[:, 11] = np.array([0x7C007C00], np.uint32).view(np.float32)[0]  # culling half-widths +inf: never culled
    f = dict(dtype=torch.float32, device=device)
    records = torch.from_numpy(rec).to(device)
    ranges = torch.tensor([[0, n]], dtype=torch.int32, device=device)
    point_list = torch.arange(n, dtype=torch.int32, device=device)
    bgt = torch.from_numpy(bg).to(device)
    color, depth, alpha = torch.empty((3, H, W), **f), torch.empty((1, H, W), **f), torch.empty((1, H, W), **f)
    n_contrib = torch.empty((H * W,), dtype=torch.int32, device=device)
    lib = _lib.load()
    stream = torch.cuda.current_stream(device).cuda_stream
    assert lib.gs_render_fwd(W, H, n, n, ranges.data_ptr(), point_list.data_ptr(), records.data_ptr(),
                             bgt.data_ptr(), 1, color.data_ptr(), depth.data_ptr(), alpha.data_ptr(),
                             n_contrib.data_ptr(), None, stream) == 0
    torch.cuda.synchronize()
    ref = _oracle()
    nc = n_contrib.cpu().numpy().reshape(H, W)
    assert int(nc[PY, PX]) == 3
    assert np.array_equal(nc, ref["n_contrib"])
    for name, got in (("color", color), ("depth", depth), ("alpha", alpha)):
        assert np.array_equal(got.cpu().numpy().view(np.int32), ref[name].view(np.int32)), name
