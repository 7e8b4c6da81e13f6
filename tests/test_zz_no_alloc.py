"""gs_scan_tiles_static (no allocation, fixed device scratch) against gs_scan_tiles.

The allocation-free scan shares its kernels with gs_scan_tiles but keeps its
per-block partial sums in a device array inside the library.  Called through
the C ABI, its offsets and its (total, depth range) info must equal the
caller-scratch scan's bit for bit, on consecutive calls whose second input is
smaller (the array keeps the first call's contents), with and without a
gather order and a depth range.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gswarp_amd import _lib

pytestmark = pytest.mark.gpu


def _inputs(P: int, seed: int, device):
    g = torch.Generator().manual_seed(seed)
    touched = torch.randint(0, 60, (P,), generator=g, dtype=torch.int32)
    radii = torch.randint(0, 4, (P,), generator=g, dtype=torch.int32)
    touched = torch.where(radii > 0, touched, torch.zeros_like(touched))
    depths = torch.rand(P, generator=g) * 50.0 + 0.25
    order = torch.randperm(P, generator=g).to(torch.int32)
    return {k: v.to(device) for k, v in (("touched", touched), ("radii", radii), ("depths", depths),
                                        ("order", order))}


def _scan(lib, inp, P, device, *, static: bool, use_order: bool, use_depths: bool):
    offsets = torch.full((P,), -7, dtype=torch.int32, device=device)
    info = torch.full((2,), -7, dtype=torch.int64, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    order = inp["order"].data_ptr() if use_order else None
    radii = inp["radii"].data_ptr() if use_depths else None
    depths = inp["depths"].data_ptr() if use_depths else None
    if static:
        lib.call("gs_scan_tiles_static", P, inp["touched"].data_ptr(), order, radii, depths, offsets.data_ptr(),
                 info.data_ptr(), stream)
    else:
        nbytes = int(lib.gs_scan_scratch_bytes(P))
        scratch = torch.empty((max(nbytes, 1),), dtype=torch.uint8, device=device)
        lib.call("gs_scan_tiles", P, inp["touched"].data_ptr(), order, radii, depths, offsets.data_ptr(),
                 info.data_ptr(), scratch.data_ptr(), nbytes, stream)
    torch.cuda.synchronize(device)
    return offsets.cpu().numpy(), info.cpu().numpy()


@pytest.mark.parametrize("use_order,use_depths", [(False, True), (True, True), (False, False), (True, False)])
def test_static_scan_matches_scratch_scan_on_consecutive_calls(use_order, use_depths, device):
    lib = _lib.load()
    for P, seed in ((1_000_003, 1), (70_001, 2)):  # the second call is smaller
        print(f"[no-alloc] P={P} order={use_order} depths={use_depths}", flush=True)
        inp = _inputs(P, seed, device)
        a_off, a_info = _scan(lib, inp, P, device, static=True, use_order=use_order, use_depths=use_depths)
        e_off, e_info = _scan(lib, inp, P, device, static=False, use_order=use_order, use_depths=use_depths)
        assert np.array_equal(a_off, e_off)
        assert np.array_equal(a_info, e_info)
        # and against numpy: the inclusive scan of the (gathered) counts and their total
        t = inp["touched"].cpu().numpy().astype(np.int64)
        if use_order:
            t = t[inp["order"].cpu().numpy()]
        assert np.array_equal(a_off, np.cumsum(t).astype(np.int32))
        assert a_info[0] == t.sum()


def test_static_scan_limits(device):
    lib = _lib.load()
    assert lib.gs_scan_tiles_static_max_points() == 1 << 26
    stream = torch.cuda.current_stream(device).cuda_stream
    info = torch.full((2,), -7, dtype=torch.int64, device=device)
    # beyond the fixed scratch: refused before any launch, with its own status
    status = lib.gs_scan_tiles_static((1 << 26) + 1, 1, None, None, None, 1, info.data_ptr(), stream)
    assert status == -5
    assert "fixed scratch" in lib.status_string(status)
    # P == 0: info is zeroed
    lib.call("gs_scan_tiles_static", 0, None, None, None, None, None, info.data_ptr(), stream)
    torch.cuda.synchronize(device)
    assert info.cpu().tolist() == [0, 0]
