"""CPU tests of the host side: input normalisation and validation, coverage
policy, runtime options, pair-count checks, the workspace report, the C ABI
library's exports, and the fail-loudly rule when the library is absent.

Restates the reference's CPU contract tests (tests/test_public_contracts.py:16-37,
tests/test_runtime_options.py:47-137, tests/test_tile_coverage.py:167-230).
"""

from __future__ import annotations

import ctypes
import os
import re
import subprocess
import sys
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch

import gswarp_amd
from gswarp_amd import _coverage, _lib, _pipeline, _runtime, _validation, _workspace
from gswarp_amd.rasterizer import GaussianRasterizationSettings

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "gswarp_hip.h"


# ---------------------------------------------------------------- normalisation

def test_requires_exactly_one_color_representation():
    with pytest.raises(ValueError, match="exactly one"):
        _validation.normalize_gaussian_inputs(dc=None, shs=None, colors_precomp=None, scales=torch.empty(0),
                                              rotations=torch.empty(0), cov3D_precomp=torch.empty((1, 6)))
    with pytest.raises(ValueError, match="exactly one"):
        _validation.normalize_gaussian_inputs(dc=None, shs=torch.empty((1, 1, 3)), colors_precomp=torch.empty((1, 3)),
                                              scales=torch.empty((1, 3)), rotations=torch.empty((1, 4)),
                                              cov3D_precomp=None)


def test_requires_complete_scale_rotation_pair():
    with pytest.raises(ValueError, match="scales/rotations"):
        _validation.normalize_gaussian_inputs(dc=None, shs=torch.empty((1, 1, 3)), colors_precomp=None,
                                              scales=torch.empty((1, 3)), rotations=None, cov3D_precomp=None)
    with pytest.raises(ValueError, match="scales/rotations"):
        _validation.normalize_gaussian_inputs(dc=None, shs=torch.empty((1, 1, 3)), colors_precomp=None,
                                              scales=torch.empty((1, 3)), rotations=torch.empty((1, 4)),
                                              cov3D_precomp=torch.empty((1, 6)))


def test_dc_is_concatenated_in_front_of_shs():
    dc = torch.full((2, 1, 3), 1.0)
    rest = torch.full((2, 15, 3), 2.0)
    out = _validation.normalize_gaussian_inputs(dc=dc, shs=rest, colors_precomp=None, scales=torch.ones(2, 3),
                                                rotations=torch.ones(2, 4), cov3D_precomp=None)
    assert out.shs.shape == (2, 16, 3)
    assert torch.equal(out.shs[:, 0], dc[:, 0]) and torch.equal(out.shs[:, 1:], rest)
    assert out.colors_precomp.numel() == 0 and out.cov3D_precomp.numel() == 0
    only_dc = _validation.normalize_gaussian_inputs(dc=dc, shs=None, colors_precomp=None, scales=torch.ones(2, 3),
                                                    rotations=torch.ones(2, 4), cov3D_precomp=None)
    assert only_dc.shs is dc


def _settings(**kw):
    base = dict(image_height=16, image_width=16, tanfovx=1.0, tanfovy=1.0, bg=torch.zeros(3), scale_modifier=1.0,
                viewmatrix=torch.eye(4), projmatrix=torch.eye(4), sh_degree=0, campos=torch.zeros(3),
                prefiltered=False)
    base.update(kw)
    return GaussianRasterizationSettings(**base)


def test_validation_rejects_host_tensors_before_any_launch():
    means = torch.zeros(2, 3)
    with pytest.raises(ValueError, match="CUDA tensor"):
        _validation.validate_rasterizer_inputs(means, torch.zeros(2, 3), torch.zeros(2, 1, 3), torch.empty(0),
                                               torch.ones(2, 1), torch.ones(2, 3), torch.ones(2, 4), torch.empty(0),
                                               _settings())
    with pytest.raises(ValueError, match="means3D"):
        _validation.validate_rasterizer_inputs("not a tensor", None, None, None, None, None, None, None, _settings())


def test_settings_defaults_match_reference_fields():
    s = _settings()
    assert s.debug is False and s.antialiasing is False
    assert s.backward_mode is None and s.binning_sort_mode is None
    assert s.auto_tune is True and s.auto_tune_verbose is True


# ---------------------------------------------------------------- pair count

def test_pair_count_rejects_negative_and_int32_wrap():
    assert _pipeline.validate_pair_count((1 << 31) - 1) == (1 << 31) - 1
    assert _pipeline.validate_pair_count(0) == 0
    for bad in (-1, 1 << 31, (1 << 32) + 17):
        with pytest.raises(OverflowError):
            _pipeline.validate_pair_count(bad)


# ---------------------------------------------------------------- coverage policy

def test_coverage_policy_rejects_exact_culling_for_non_exact_footprints():
    """test_tile_coverage.py:167-230: auto is AccuTile for the exact screen conic
    and the conservative box otherwise; the culling modes need the exact conic."""
    CM = _coverage.CoverageMode
    assert _coverage.kernel_mode("auto") is CM.ACCUTILE_SWEEP
    assert _coverage.kernel_mode("auto", exact_conic=False) is CM.SNUGBOX
    assert _coverage.kernel_mode("snugbox", exact_conic=False) is CM.SNUGBOX
    for name in ("accutile_sweep", "conic_rect"):
        with pytest.raises(ValueError, match="allows only 'snugbox'"):
            _coverage.kernel_mode(name, exact_conic=False)
    # kernel ids are the library's GS_COVERAGE_* values
    header = HEADER.read_text()
    for mode in CM:
        assert f"#define GS_COVERAGE_{mode.name} {int(mode)}" in header
    assert [_coverage.kernel_mode(n) for n in ("snugbox", "accutile_sweep", "conic_rect")] == [0, 1, 2]


def test_coverage_mode_names_are_checked():
    with pytest.raises(ValueError, match="mode must be one of 'auto', 'snugbox', 'accutile_sweep', 'conic_rect'"):
        _coverage.check_mode_name("typo")
    assert _coverage.PUBLIC_NAMES == ("auto", "snugbox", "accutile_sweep", "conic_rect")


# ---------------------------------------------------------------- runtime options

def test_settings_override_defaults_without_mutating_them():
    s = SimpleNamespace(bg=torch.zeros(3), backward_mode=None, binning_sort_mode="torch", auto_tune=False,
                        auto_tune_verbose=False, compute_flow_aux=None)
    opts = _runtime.resolve_execution_options(s)
    assert opts.backward_mode == "manual"
    assert opts.binning_sort_mode == "torch"
    assert opts.tile_coverage_mode == "accutile_sweep"
    assert opts.compute_depth is _runtime.get_compute_depth()
    assert not opts.auto_tune and not opts.auto_tune_verbose
    assert opts.compute_flow_aux is None and opts.flow_topk is None
    assert _runtime.get_binning_sort_mode() == "warp_depth_stable_tile"


def test_flow_options_are_snapshotted_per_call():
    s = SimpleNamespace(bg=torch.zeros(3), backward_mode=None, binning_sort_mode=None, auto_tune=True,
                        auto_tune_verbose=True, compute_flow_aux=False)
    opts = _runtime.resolve_execution_options(s, flow=True)
    assert opts.compute_flow_aux is False and opts.flow_topk == _runtime.get_flow_topk()
    original = _runtime.get_flow_topk()
    try:
        _runtime.set_flow_topk(7)
        assert opts.flow_topk == original
        assert _runtime.resolve_execution_options(s, flow=True).flow_topk == 7
        with pytest.raises(ValueError):
            _runtime.set_flow_topk(0)
    finally:
        _runtime.set_flow_topk(original)


def test_mode_setters_validate_and_restore():
    original = _runtime.get_tile_coverage_mode()
    try:
        _runtime.set_tile_coverage_mode("conic_rect")
        assert _runtime.get_tile_coverage_mode() == "conic_rect"
        with pytest.raises(ValueError, match="accutile_sweep"):
            _runtime.set_tile_coverage_mode("not-a-mode")
    finally:
        _runtime.set_tile_coverage_mode(original)
    with pytest.raises(ValueError):
        _runtime.set_backward_mode("autograd")
    with pytest.raises(ValueError):
        _runtime.set_binning_sort_mode("bogus")
    original_depth = _runtime.get_compute_depth()
    try:
        _runtime.set_compute_depth(False)
        assert gswarp_amd.get_compute_depth() is False
    finally:
        _runtime.set_compute_depth(original_depth)


def test_execution_options_context_nests_and_restores():
    a = _runtime.ExecutionOptions("manual", "torch", "snugbox", True, False, False)
    b = _runtime.ExecutionOptions("manual", "warp_radix", "conic_rect", False, True, True)
    assert _runtime.active_options() is None
    with _runtime.execution_options(a):
        assert _runtime.active_options() is a
        with _runtime.execution_options(b):
            assert _runtime.active_options() is b
        assert _runtime.active_options() is a
    assert _runtime.active_options() is None


def test_cache_report_is_cpu_safe():
    _workspace.clear_caches()
    report = gswarp_amd.get_warp_cache_report()
    assert report["workspace_entries"] == 0
    assert "workspace_evictions" in report


def test_public_surface_matches_reference_exports():
    names = ["GaussianRasterizationSettings", "GaussianRasterizer", "RasterizerMeta", "rasterize_gaussians",
             "initialize_runtime_tuning", "get_runtime_tuning_report", "clear_warp_caches", "get_warp_cache_report",
             "get_backward_mode", "set_backward_mode", "get_compute_depth", "set_compute_depth",
             "get_binning_sort_mode", "set_binning_sort_mode", "get_tile_coverage_mode", "set_tile_coverage_mode"]
    import gswarp
    import gswarp.rasterizer_flow as flow
    for name in names:
        assert hasattr(gswarp, name), name
    for name in ("GaussianRasterizationSettings", "GaussianRasterizer", "rasterize_gaussians", "get_flow_topk",
                 "set_flow_topk", "get_compute_flow_aux", "set_compute_flow_aux"):
        assert hasattr(flow, name), name
    with pytest.raises(NotImplementedError):
        gswarp.fused_ssim(None, None)
    with pytest.raises(NotImplementedError):
        gswarp.distCUDA2(None)


# ---------------------------------------------------------------- C ABI library

def _declared_functions() -> dict:
    """gs_* function name -> parameter count, parsed from the public header."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    decls = {}
    for m in re.finditer(r"\b(gs_\w+)\s*\(([^;{]*?)\)\s*;", text):
        params = m.group(2).strip()
        decls[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return decls


def test_header_declares_the_bound_signatures():
    decls = _declared_functions()
    assert set(decls) == set(_lib.SIGNATURES)
    for name, (_restype, argtypes) in _lib.SIGNATURES.items():
        assert decls[name] == len(argtypes), name


def test_library_loads_and_exports_every_declared_symbol():
    if not _lib.LIB_PATH.exists():
        pytest.skip("libgswarp_hip.so not built (run __graft_entry__.build())")
    handle = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in _declared_functions():
        assert hasattr(handle, name), name
    lib = _lib.load()
    assert lib.gs_version() == 10200
    assert lib.gs_readback_slot_bytes() == 256
    assert lib.status_string(0) == "ok"
    for code in (-1, -2, -3, -4):
        assert lib.status_string(code) and lib.status_string(code) != "ok"
    assert lib.gs_sort_num_passes(45) == 6 and lib.gs_sort_num_passes(40) == 5
    assert lib.gs_sort_scratch_bytes(0) % 256 == 0
    assert lib.gs_scan_scratch_bytes(1_000_000) > 0


def test_sort_pass_count_matches_key_width_rule():
    """passes = ceil((32 + ceil(log2 T)) / 8): 5 at 256 tiles, 6 at 2,500-8,160 tiles."""
    if not _lib.LIB_PATH.exists():
        pytest.skip("libgswarp_hip.so not built")
    lib = _lib.load()
    for tiles, passes in ((256, 5), (2500, 6), (3600, 6), (8160, 6)):
        key_bits = 32 + (tiles - 1).bit_length()
        assert lib.gs_sort_num_passes(key_bits) == passes


def test_missing_library_fails_loudly():
    """No CPU fallback: with the library path pointing nowhere, loading raises."""
    code = ("import gswarp_amd._lib as L\n"
            "try:\n    L.load()\nexcept RuntimeError as e:\n    print('raised', 'not built' in str(e))\n")
    env = dict(os.environ, GSWARP_AMD_LIB=str(ROOT / "no_such_lib.so"), PYTHONPATH=str(ROOT))
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=120)
    assert out.stdout.strip() == "raised True", out.stderr


def test_bench_refuses_more_than_one_gpu():
    out = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 2 and "one GPU" in out.stderr


def test_mip_settings_defaults_and_filter_checks():
    """gswarp/methods/mip_3dgs.py:29-48 defaults; the filter checks of
    mip_3dgs.py:83-87 (antialiasing off, finite non-negative variance)."""
    import math

    from gswarp_amd.methods import mip_3dgs
    import gswarp.methods.mip_3dgs as alias
    assert alias.MipGaussianRasterizationSettings is mip_3dgs.MipGaussianRasterizationSettings
    fields = mip_3dgs.MipGaussianRasterizationSettings._fields
    assert fields[-1] == "filter_variance"
    assert mip_3dgs.MipGaussianRasterizationSettings._field_defaults["filter_variance"] == 0.3
    ok = mip_3dgs.MipGaussianRasterizationSettings(16, 16, 1.0, 1.0, None, 1.0, None, None, 0, None, False)
    mip_3dgs._check_filter(ok)
    for bad in (ok._replace(filter_variance=-1e-3), ok._replace(filter_variance=math.inf),
                ok._replace(filter_variance=math.nan), ok._replace(antialiasing=True)):
        with pytest.raises(ValueError):
            mip_3dgs._check_filter(bad)
