"""gs_scan_tiles_onepass (one kernel, decoupled look-back) against the two-pass scans.

The one-pass scan must give the offsets and info of gs_scan_tiles (and, with
sizes, of gs_scan_tiles_entries) bit for bit: the inclusive prefix sum of
the tile counts in point order (memory.py:539-551), the exact pair total and
the visible depth range (binning_ops.py:62-81), and the bucketed binning's
sizes.  Its state is prepared by gs_scan_state_prepare (on a buffer of
garbage) or by gs_preprocess_fwd.  Cases cover one partial block, exact
multiples of the 4096-Gaussian block, a million counts, and the bounded
waits forced to time out from the host (spin limit 0): blocks then add up
the counts before them directly and every output stays exact.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gswarp_amd import _lib, _pipeline, configs
from helpers import options, raster_inputs, to_np

pytestmark = pytest.mark.gpu


def _inputs(P: int, seed: int, device, big: bool = False):
    g = torch.Generator().manual_seed(seed)
    hi = 5000 if big else 60
    touched = torch.randint(0, hi, (P,), generator=g, dtype=torch.int32)
    radii = torch.randint(0, 4, (P,), generator=g, dtype=torch.int32)
    touched = torch.where(radii > 0, touched, torch.zeros_like(touched))
    depths = torch.rand(P, generator=g) * 50.0 + 0.25
    return {k: v.to(device) for k, v in (("touched", touched), ("radii", radii), ("depths", depths))}


def _state(lib, inp, P, device, *, coverage=None, with_depths=True):
    """A state prepared by gs_scan_state_prepare on a buffer of garbage."""
    nbytes = int(lib.gs_scan_state_bytes(P))
    state = torch.full((max(nbytes // 8, 1),), -123456789, dtype=torch.int64, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    lib.call("gs_scan_state_prepare", P, inp["touched"].data_ptr(),
             inp["radii"].data_ptr() if with_depths else None, inp["depths"].data_ptr() if with_depths else None,
             None if coverage is None else coverage.data_ptr(), state.data_ptr(), nbytes, stream)
    return state


def _onepass(lib, inp, P, device, *, coverage=None, spin_limit=1 << 20, state=None, with_depths=True,
             sized=None):
    offsets = torch.full((P,), -7, dtype=torch.int32, device=device)
    info = torch.full((4,), -7, dtype=torch.int64, device=device)
    if state is None:
        state = _state(lib, inp, P, device, coverage=coverage, with_depths=with_depths)
    sized = coverage is not None if sized is None else sized
    stream = torch.cuda.current_stream(device).cuda_stream
    lib.call("gs_scan_tiles_onepass", P, inp["touched"].data_ptr(), offsets.data_ptr(), info.data_ptr(),
             state.data_ptr(), state.numel() * 8, int(sized), spin_limit, stream)
    torch.cuda.synchronize(device)
    return offsets.cpu().numpy(), info.cpu().numpy()


def _twopass(lib, inp, P, device, *, coverage=None, with_depths=True):
    offsets = torch.full((P,), -7, dtype=torch.int32, device=device)
    info = torch.full((4,), -7, dtype=torch.int64, device=device)
    nbytes = int(lib.gs_scan_scratch_bytes(P))
    scratch = torch.empty((max(nbytes, 1),), dtype=torch.uint8, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    radii = inp["radii"].data_ptr() if with_depths else None
    depths = inp["depths"].data_ptr() if with_depths else None
    if coverage is None:
        lib.call("gs_scan_tiles", P, inp["touched"].data_ptr(), None, radii, depths, offsets.data_ptr(),
                 info.data_ptr(), scratch.data_ptr(), nbytes, stream)
    else:
        lib.call("gs_scan_tiles_entries", P, inp["touched"].data_ptr(), radii, depths, coverage.data_ptr(),
                 offsets.data_ptr(), info.data_ptr(), scratch.data_ptr(), nbytes, stream)
    torch.cuda.synchronize(device)
    return offsets.cpu().numpy(), info.cpu().numpy()


def _expected_range(inp) -> int:
    r = inp["radii"].cpu().numpy()
    bits = inp["depths"].cpu().numpy().view(np.uint32)[r > 0]
    return 0 if bits.size == 0 else (int(bits.max()) << 32) | int(bits.min())


@pytest.mark.parametrize("P", [1, 5, 4095, 4096, 4097, 3 * 4096, 70_001, 1_000_003])
def test_onepass_matches_two_pass_and_numpy(P, device):
    lib = _lib.load()
    print(f"[onepass] P={P}", flush=True)
    inp = _inputs(P, 7 + P % 97, device, big=P == 70_001)
    a_off, a_info = _onepass(lib, inp, P, device)
    e_off, e_info = _twopass(lib, inp, P, device)
    assert np.array_equal(a_off, e_off)
    assert np.array_equal(a_info[:2], e_info[:2])
    t = inp["touched"].cpu().numpy().astype(np.int64)
    assert np.array_equal(a_off, np.cumsum(t).astype(np.int32))
    assert a_info[0] == t.sum()
    assert a_info[1] == _expected_range(inp)


def test_onepass_without_depths(device):
    lib = _lib.load()
    P = 20_000
    inp = _inputs(P, 3, device)
    a_off, a_info = _onepass(lib, inp, P, device, with_depths=False)
    t = inp["touched"].cpu().numpy().astype(np.int64)
    assert np.array_equal(a_off, np.cumsum(t).astype(np.int32))
    assert a_info[0] == t.sum() and a_info[1] == 0


def _scene_pre(device, config=3, count=60_000):
    scene = configs.make_scene(config, count=count, width=480, height=270, device=device)
    with torch.cuda.device(device):
        return _pipeline.preprocess(raster_inputs(scene), options())


def test_onepass_sizes_the_buckets_like_the_entries_scan(device):
    """With cover words: info[2] and info[3] equal gs_scan_tiles_entries'."""
    lib = _lib.load()
    pre = _scene_pre(device)
    P = pre.radii.shape[0]
    inp = {"touched": pre.tiles_touched, "radii": pre.radii, "depths": pre.depths}
    a_off, a_info = _onepass(lib, inp, P, device, coverage=pre.coverage)
    e_off, e_info = _twopass(lib, inp, P, device, coverage=pre.coverage)
    assert np.array_equal(a_off, e_off)
    assert np.array_equal(a_info, e_info)


@pytest.mark.parametrize("config", [2, 3])
def test_preprocess_prepares_the_state(config, device, monkeypatch):
    """The pipeline's preprocess prepares the state it allocates as
    gs_scan_state_prepare does from its outputs (aggregates and zero status
    words); the scan on it equals the two-pass scans, with the sizes.  The
    binning takes the state once (a second binning of the same preprocess
    outputs runs the two-pass scan)."""
    monkeypatch.setattr(_pipeline, "SCAN_ONEPASS", True)
    lib = _lib.load()
    pre = _scene_pre(device, config=config)
    P = pre.radii.shape[0]
    assert pre.scan_state is not None
    inp = {"touched": pre.tiles_touched, "radii": pre.radii, "depths": pre.depths}
    expected = _state(lib, inp, P, device, coverage=pre.coverage)
    torch.cuda.synchronize(device)
    off0 = int(lib.gs_scan_state_status_offset(P))
    used = off0 + int(lib.gs_scan_state_status_words(P))
    assert torch.equal(pre.scan_state[:used], expected[:used])
    assert np.all(to_np(pre.scan_state[off0:used]) == 0)
    e_off, e_info = _twopass(lib, inp, P, device, coverage=pre.coverage)
    a_off, a_info = _onepass(lib, inp, P, device, state=pre.scan_state, sized=True)
    assert np.array_equal(a_off, e_off) and np.array_equal(a_info, e_info)
    if config == 3:
        return
    pre2 = _scene_pre(device, config=2)
    with torch.cuda.device(device):
        b1 = _pipeline.binning(pre2, 270, 480, options())
        assert pre2.scan_state is None
        b2 = _pipeline.binning(pre2, 270, 480, options())
    torch.cuda.synchronize(device)
    assert b1.num_rendered == b2.num_rendered == e_info[0]
    assert np.array_equal(to_np(b1.point_list), to_np(b2.point_list))


@pytest.mark.parametrize("P", [4097, 70_001, 1_000_003])
def test_onepass_forced_timeouts_stay_exact(P, device):
    """spin_limit 0: every wait that finds its predecessor unpublished gives up
    at once.  Blocks then add up the counts before them directly, so offsets
    and the total stay exact; the depth range is exact or the widest one and
    the sizes exact or declined (-1)."""
    lib = _lib.load()
    print(f"[onepass timeout] P={P}", flush=True)
    inp = _inputs(P, 11, device)
    pre = _scene_pre(device) if P == 70_001 else None
    if pre is not None:
        inp = {"touched": pre.tiles_touched, "radii": pre.radii, "depths": pre.depths}
        P = pre.radii.shape[0]
    cov = None if pre is None else pre.coverage
    a_off, a_info = _onepass(lib, inp, P, device, coverage=cov, spin_limit=0)
    e_off, e_info = _twopass(lib, inp, P, device, coverage=cov)
    assert np.array_equal(a_off, e_off)
    assert a_info[0] == e_info[0]
    # the final wait may time out too: then the widest range and no sizes
    assert a_info[1] in (e_info[1], 0x7F7FFFFF << 32)
    if cov is not None:
        assert (a_info[2], a_info[3]) in ((e_info[2], e_info[3]), (-1, 0))


def test_onepass_argument_checks(device):
    lib = _lib.load()
    stream = torch.cuda.current_stream(device).cuda_stream
    info = torch.full((4,), -7, dtype=torch.int64, device=device)
    x = torch.zeros((64,), dtype=torch.int32, device=device)
    state = torch.zeros((64,), dtype=torch.int64, device=device)
    # too small a state, a negative spin limit, an unaligned state
    assert lib.gs_scan_tiles_onepass(100_000, x.data_ptr(), x.data_ptr(), info.data_ptr(), state.data_ptr(), 8, 0,
                                     10, stream) != 0
    assert lib.gs_scan_tiles_onepass(10, x.data_ptr(), x.data_ptr(), info.data_ptr(), state.data_ptr(), 512, 0,
                                     -1, stream) != 0
    assert lib.gs_scan_tiles_onepass(10, x.data_ptr(), x.data_ptr(), info.data_ptr(), state.data_ptr() + 4, 500, 0,
                                     10, stream) != 0
    assert lib.gs_scan_state_prepare(100_000, x.data_ptr(), None, None, None, state.data_ptr(), 8, stream) != 0
    assert lib.gs_scan_state_prepare(10, x.data_ptr(), x.data_ptr(), None, None, state.data_ptr(), 512,
                                     stream) != 0
    # P == 0 zeroes info (all four words with the sizes)
    lib.call("gs_scan_tiles_onepass", 0, None, None, info.data_ptr(), None, 0, 1, 10, stream)
    torch.cuda.synchronize(device)
    assert np.array_equal(info.cpu().numpy(), np.zeros(4, np.int64))
