"""gs_info_readback / gs_num_rendered_readback: the forward's one device-to-host
read (binning_ops.py:243-252, the num_rendered .item()).

The library publishes the words into a slot of its own pinned host memory
with a small kernel and spins on the slot's flag.  These tests check that a
read sees exactly the values the stream wrote before it (for every count, over
more calls than there are slots, so slots are reused), and that reads from two
threads on two streams never see each other's values.
"""

from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

from gswarp_amd import _lib

pytestmark = pytest.mark.gpu


def _read(lib, info, count, stream):
    out = torch.full((16,), -1, dtype=torch.int64).pin_memory()
    lib.call("gs_info_readback", info.data_ptr(), out.data_ptr(), count, stream.cuda_stream)
    return out.numpy()[:count].copy()


def test_readback_sees_the_stream_order(device):
    """Each read follows a device write of new values on the same stream (no
    host synchronisation in between): 200 reads over counts 1-16."""
    lib = _lib.load()
    stream = torch.cuda.current_stream(device)
    g = torch.Generator().manual_seed(5)
    info = torch.zeros((16,), dtype=torch.int64, device=device)
    for it in range(200):
        values = torch.randint(-2**62, 2**62, (16,), generator=g, dtype=torch.int64)
        info.copy_(values.to(device, non_blocking=False))
        info.add_(it)  # a kernel on the stream right before the read
        count = 1 + it % 16
        got = _read(lib, info, count, stream)
        assert np.array_equal(got, (values + it).numpy()[:count]), (it, count)


def test_num_rendered_readback_two_words(device):
    lib = _lib.load()
    stream = torch.cuda.current_stream(device)
    info = torch.tensor([123456789012, -5, 7, 8], dtype=torch.int64, device=device)
    out = torch.full((2,), -1, dtype=torch.int64).pin_memory()
    lib.call("gs_num_rendered_readback", info.data_ptr(), out.data_ptr(), stream.cuda_stream)
    assert out.tolist() == [123456789012, -5]


def test_readback_two_threads(device):
    """Two threads, each with its own stream, read distinct values 150 times."""
    lib = _lib.load()

    def worker(k):
        torch.cuda.set_device(device)
        stream = torch.cuda.Stream(device)
        with torch.cuda.stream(stream):
            info = torch.zeros((4,), dtype=torch.int64, device=device)
            for it in range(150):
                info.fill_(1000 * k + it)
                got = _read(lib, info, 4, stream)
                if not np.all(got == 1000 * k + it):
                    return (k, it, got.tolist())
        return None

    with ThreadPoolExecutor(2) as pool:
        results = list(pool.map(worker, (1, 2)))
    assert results == [None, None]


def test_readback_argument_checks(device):
    lib = _lib.load()
    stream = torch.cuda.current_stream(device)
    info = torch.zeros((16,), dtype=torch.int64, device=device)
    out = torch.zeros((16,), dtype=torch.int64).pin_memory()
    for count in (0, 17, -1):
        assert lib.gs_info_readback(info.data_ptr(), out.data_ptr(), count, stream.cuda_stream) != 0
    assert lib.gs_info_readback(None, out.data_ptr(), 2, stream.cuda_stream) != 0
    assert lib.gs_num_rendered_readback(info.data_ptr(), None, stream.cuda_stream) != 0
