"""Test helpers: run the gfx950 stages and the CPU oracle on the same scene."""

from __future__ import annotations

import numpy as np
import torch

import dense_ref
import oracle
from gswarp_amd import _pipeline, configs
from gswarp_amd._runtime import ExecutionOptions

COVERAGE_NAMES = {0: "snugbox", 1: "accutile_sweep", 2: "conic_rect"}


def options(coverage_mode: int = 1, compute_depth: bool = True, flow: bool = False, top_k: int = 20,
            compute_flow_aux: bool = True, sort_mode: str = "warp_depth_stable_tile") -> ExecutionOptions:
    return ExecutionOptions(
        backward_mode="manual",
        binning_sort_mode=sort_mode,
        tile_coverage_mode=COVERAGE_NAMES[coverage_mode],
        compute_depth=compute_depth,
        auto_tune=False,
        auto_tune_verbose=False,
        compute_flow_aux=compute_flow_aux if flow else None,
        flow_topk=top_k if flow else None,
    )


def raster_inputs(scene: dict, *, colors: bool = False) -> _pipeline.RasterInputs:
    dev = scene["means3D"].device
    empty = torch.empty((0,), dtype=torch.float32, device=dev)
    if colors:
        rgb = scene.get("colors_precomp")
        if rgb is None:
            g = torch.Generator().manual_seed(11)
            rgb = torch.rand(scene["means3D"].shape[0], 3, generator=g).to(dev)
            scene["colors_precomp"] = rgb
    cov = scene.get("cov3D_precomp")
    return _pipeline.RasterInputs(
        scene["bg"], scene["means3D"], scene["colors_precomp"] if colors else empty, scene["opacities"],
        scene["scales"] if cov is None else empty, scene["rotations"] if cov is None else empty,
        float(scene.get("scale_modifier", 1.0)), empty if cov is None else cov, scene["viewmatrix"],
        scene["projmatrix"], scene["tanfovx"], scene["tanfovy"], scene["height"], scene["width"],
        empty if colors else scene["shs"], scene["sh_degree"], scene["campos"], False,
        float(scene.get("filter_variance", 0.0)))


def with_precomputed_covariance(scene: dict, seed: int = 5) -> dict:
    """The scene with cov3D_precomp = R diag(s^2) R^T (float64, rounded to
    float32) whose off-diagonals are shrunk toward zero by a random factor per
    Gaussian, a convex mix of two PSD matrices, so covariances are not all of
    the scale/rotation form.  scales / rotations are dropped."""
    host = {k: scene[k].detach().cpu().numpy() for k in ("scales", "rotations")}
    cov = dense_ref.covariance_upper(host["scales"], host["rotations"], float(scene.get("scale_modifier", 1.0)))
    t = np.random.default_rng(seed).uniform(0.0, 0.6, size=(cov.shape[0], 1))
    cov[:, [1, 2, 4]] *= 1.0 - t
    out = {k: v for k, v in scene.items() if k not in ("scales", "rotations")}
    out["cov3D_precomp"] = torch.from_numpy(cov.astype(np.float32)).to(scene["means3D"].device)
    return out


def gpu_forward(scene: dict, opts: ExecutionOptions, *, flow: bool = False, colors: bool = False) -> dict:
    inputs = raster_inputs(scene, colors=colors)
    with torch.cuda.device(scene["means3D"].device):
        pre = _pipeline.preprocess(inputs, opts)
        bins = _pipeline.binning(pre, scene["height"], scene["width"], opts, keep_keys=True)
        res = _pipeline.render(pre, bins, scene["bg"], scene["height"], scene["width"], opts, flow=flow)
    torch.cuda.synchronize()
    out = {"pre": pre, "bins": bins, "res": res, "inputs": inputs}
    return out


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def oracle_forward(scene: dict, *, coverage_mode: int = 1, compute_depth: bool = True, top_k: int = 0,
                   colors: bool = False) -> tuple[dict, dict]:
    host = configs.scene_to_numpy(scene)
    if not colors:
        host.pop("colors_precomp", None)
    else:
        host["shs"] = None
    return host, oracle.rasterize(host, coverage_mode=coverage_mode, compute_depth=compute_depth, top_k=top_k)


def grad_mismatch(actual: np.ndarray, expected: np.ndarray, rtol: float = 1e-3, atol: float = 1e-5,
                  scale_atol: float = 1e-4) -> tuple[int, float]:
    """Count of elements outside |a-e| <= rtol*|e| + max(atol, scale_atol*max|e|), and the worst ratio.

    Gradients are sums of per-pixel terms accumulated with float atomics in
    unspecified order on the GPU and in double on the CPU; where terms cancel
    the absolute error scales with the tensor's magnitude, hence the
    scale-relative floor.
    """
    actual = np.asarray(actual, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    floor = max(atol, scale_atol * float(np.abs(expected).max(initial=0.0)))
    tol = rtol * np.abs(expected) + floor
    diff = np.abs(actual - expected)
    bad = diff > tol
    worst = float((diff / tol).max(initial=0.0))
    return int(bad.sum()), worst
