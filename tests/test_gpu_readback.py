"""gs_info_readback / gs_num_rendered_readback: the forward's one device-to-host
read (binning_ops.py:243-252, the num_rendered .item()).

The caller owns the read-back slot (coherent pinned host memory of
gs_readback_slot_bytes() bytes) and passes a sequence number; the library
publishes the words into the slot with a small kernel, raises the slot's flag
to that number and spins on it, keeping no state of its own.  These tests
check that a read sees exactly the values the stream wrote before it (for
every count, 200 reads through one slot), that slots are independent (two
slots each counting from 1, which a library-wide sequence would confuse),
that reads from two threads on two streams with their own slots never see
each other's values, that a slot in pageable memory is served by the copy,
and the argument checks (including a sequence number the flag already holds).
"""

from __future__ import annotations

import ctypes
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

from gswarp_amd import _lib, _workspace

pytestmark = pytest.mark.gpu


@pytest.fixture
def slots(device):
    """Slots taken from the device's block, returned to it afterwards."""
    index = device.index or 0
    taken = []

    def take():
        s = _workspace._take_slot(index)
        taken.append(s)
        return s

    yield take
    _workspace._free_slots[index].extend(taken)


def _read(lib, info, count, stream, slot):
    seq = slot.next_seq()
    lib.call("gs_info_readback", info.data_ptr(), slot.address, seq, count, stream.cuda_stream)
    assert slot[31] == seq  # the flag word holds this call's number
    return np.array([slot[i] for i in range(count)], dtype=np.int64)


def test_slot_size():
    assert int(_lib.load().gs_readback_slot_bytes()) == 256


def test_readback_sees_the_stream_order(device, slots):
    """Each read follows a device write of new values on the same stream (no
    host synchronisation in between): 200 reads over counts 1-16."""
    lib = _lib.load()
    stream = torch.cuda.current_stream(device)
    slot = slots()
    g = torch.Generator().manual_seed(5)
    info = torch.zeros((16,), dtype=torch.int64, device=device)
    for it in range(200):
        values = torch.randint(-2**62, 2**62, (16,), generator=g, dtype=torch.int64)
        info.copy_(values.to(device, non_blocking=False))
        info.add_(it)  # a kernel on the stream right before the read
        count = 1 + it % 16
        got = _read(lib, info, count, stream, slot)
        assert np.array_equal(got, (values + it).numpy()[:count]), (it, count)


def test_slots_are_independent(device, slots):
    """Two fresh slots, each counting its own uses from 1, used alternately."""
    lib = _lib.load()
    stream = torch.cuda.current_stream(device)
    a, b = slots(), slots()
    for s in (a, b):  # restart both counts at 0, as a fresh block has them
        s.words[31] = 0
        s.uses = 0
    info = torch.zeros((4,), dtype=torch.int64, device=device)
    for it in range(20):
        for k, s in enumerate((a, b)):
            info.fill_(100 * k + it)
            got = _read(lib, info, 4, stream, s)
            assert np.all(got == 100 * k + it), (it, k, got.tolist())
            assert s.uses == it + 1


def test_num_rendered_readback_two_words(device, slots):
    lib = _lib.load()
    stream = torch.cuda.current_stream(device)
    slot = slots()
    info = torch.tensor([123456789012, -5, 7, 8], dtype=torch.int64, device=device)
    lib.call("gs_num_rendered_readback", info.data_ptr(), slot.address, slot.next_seq(), stream.cuda_stream)
    assert [slot[0], slot[1]] == [123456789012, -5]


def test_readback_pageable_slot_copies(device):
    """A slot the device cannot address (pageable memory) is filled by the copy."""
    lib = _lib.load()
    stream = torch.cuda.current_stream(device)
    buf = (ctypes.c_int64 * 32)()
    info = torch.arange(3, 19, dtype=torch.int64, device=device)
    for seq in (1, 2, 3):
        info.add_(1)
        lib.call("gs_info_readback", info.data_ptr(), ctypes.addressof(buf), seq, 16, stream.cuda_stream)
        assert list(buf[:16]) == list(range(3 + seq, 19 + seq))


def test_readback_two_threads(device, slots):
    """Two threads, each with its own stream and slot, read distinct values 150 times."""
    lib = _lib.load()
    own = [slots(), slots()]

    def worker(k):
        torch.cuda.set_device(device)
        stream = torch.cuda.Stream(device)
        with torch.cuda.stream(stream):
            info = torch.zeros((4,), dtype=torch.int64, device=device)
            for it in range(150):
                info.fill_(1000 * k + it)
                got = _read(lib, info, 4, stream, own[k - 1])
                if not np.all(got == 1000 * k + it):
                    return (k, it, got.tolist())
        return None

    with ThreadPoolExecutor(2) as pool:
        results = list(pool.map(worker, (1, 2)))
    assert results == [None, None]


def test_readback_argument_checks(device, slots):
    lib = _lib.load()
    stream = torch.cuda.current_stream(device)
    info = torch.zeros((16,), dtype=torch.int64, device=device)
    slot = slots()
    seq = slot.next_seq()
    for count in (0, 17, -1):
        assert lib.gs_info_readback(info.data_ptr(), slot.address, seq, count, stream.cuda_stream) != 0
    assert lib.gs_info_readback(None, slot.address, seq, 2, stream.cuda_stream) != 0
    assert lib.gs_info_readback(info.data_ptr(), None, seq, 2, stream.cuda_stream) != 0
    assert lib.gs_num_rendered_readback(info.data_ptr(), None, seq, stream.cuda_stream) != 0
    for bad in (0, -3):
        assert lib.gs_info_readback(info.data_ptr(), slot.address, bad, 2, stream.cuda_stream) != 0
    # a sequence number the flag already holds would end the wait before the words arrive
    assert lib.gs_info_readback(info.data_ptr(), slot.address, seq, 2, stream.cuda_stream) == 0
    assert lib.gs_info_readback(info.data_ptr(), slot.address, seq, 2, stream.cuda_stream) != 0
    torch.cuda.synchronize(device)
