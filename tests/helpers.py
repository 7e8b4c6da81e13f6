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


def gpu_forward(scene: dict, opts: ExecutionOptions, *, flow: bool = False, colors: bool = False,
                grad_buffer: bool = False) -> dict:
    """The forward stages; with ``grad_buffer`` the render also zeroes a
    NaN-filled (N, 10) gradient accumulator, returned as ``grad_gauss``."""
    inputs = raster_inputs(scene, colors=colors)
    dev = scene["means3D"].device
    grad_gauss = torch.full((scene["means3D"].shape[0], 10), float("nan"), device=dev) if grad_buffer else None
    with torch.cuda.device(dev):
        pre = _pipeline.preprocess(inputs, opts)
        bins = _pipeline.binning(pre, scene["height"], scene["width"], opts, keep_keys=True)
        res = _pipeline.render(pre, bins, scene["bg"], scene["height"], scene["width"], opts, flow=flow,
                               grad_clear=grad_gauss)
    torch.cuda.synchronize()
    out = {"pre": pre, "bins": bins, "res": res, "inputs": inputs, "grad_gauss": grad_gauss}
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


# Safety factor on the oracle's per-element rounding bound (oracle.gradient_bound):
# it covers the second-order terms the first-order analysis drops.  On the
# CPU the oracle and a second fp32 evaluation order stay within 0.4 of the
# one-sided bound (tests/test_oracle_bound.py).
BOUND_FACTOR = 2.0


def grad_mismatch(actual: np.ndarray, expected: np.ndarray, bound=0.0, rtol: float = 1e-3, atol: float = 1e-5,
                  factor: float = BOUND_FACTOR) -> tuple[int, float, int, float]:
    """Per-element gradient check.

    An element passes when |a - e| <= rtol |e| + atol + factor * bound, where
    bound (broadcast to e's shape) is the oracle's bound on the fp32 rounding
    of that element's sum of per-pixel terms, carried through the
    per-Gaussian backward (oracle.gradient_bound): where those terms cancel,
    the rounding of any fp32 evaluation exceeds the 1e-3 / 1e-5 bar, and the
    bound says by how much for this element alone.

    Returns (failures, worst ratio |a-e| / tolerance, elements outside the
    plain rtol/atol bar, worst ratio against that bar).
    """
    actual = np.asarray(actual, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    bound = np.broadcast_to(np.asarray(bound, dtype=np.float64), expected.shape)
    diff = np.abs(actual - expected)
    strict = rtol * np.abs(expected) + atol
    tol = strict + factor * bound
    bad = int((diff > tol).sum())
    n_strict = int((diff > strict).sum())
    with np.errstate(divide="ignore", invalid="ignore"):  # 0/0 where both are exactly zero
        worst = float(np.nan_to_num(diff / tol, posinf=np.inf).max(initial=0.0))
        worst_strict = float(np.nan_to_num(diff / strict, posinf=np.inf).max(initial=0.0))
    return bad, worst, n_strict, worst_strict


def report_grad(name: str, actual, expected, bound) -> tuple[int, float]:
    """grad_mismatch with one printed line per tensor; returns (failures, worst ratio)."""
    bad, worst, n_strict, worst_strict = grad_mismatch(actual, expected, bound)
    print(f"[grad] {name}: failures={bad} worst={worst:.3f} | outside 1e-3/1e-5 bar: {n_strict} "
          f"(worst {worst_strict:.2f}) of {np.size(expected)}; max|e|={np.abs(expected).max(initial=0):.3e}",
          flush=True)
    return bad, worst
