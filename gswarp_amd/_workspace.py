"""Per-(device, stream) host workspaces and submission locks.

The forward pass performs one device-to-host read (the pair count).  The
library publishes it into a caller-owned slot of coherent pinned host memory
and spins on the slot's flag (gs_info_readback), so this module owns that
memory: per device one block of slots, allocated once with the HIP runtime's
hipHostMalloc (portable, mapped, coherent) and kept until the process ends,
from which each (device, stream) takes its own slot and counts its uses (the
sequence number the flag is raised to).  At most ``MAX_WORKSPACE_STREAMS``
streams per device hold a slot, with least-recently used eviction; an
evicted or cleared entry's stream is synchronised first, so no publication
into its slot can still be in flight (the contract of the reference's
workspace cache, gswarp/_internal/backends/warp/memory.py:20-22 and 340-393).
Device scratch (scan and sort tables) comes from torch's stream-ordered
caching allocator per call.

Submission from several host threads is serialised per device with an
RLock, as gswarp/_stream.py:128-151 does; calls on different streams still
overlap on the GPU.
"""

from __future__ import annotations

import ctypes
import os
import threading
from collections import OrderedDict

import torch

MAX_WORKSPACE_STREAMS = 4

_lock = threading.Lock()
_device_locks: dict[int, threading.RLock] = {}
_entries: "OrderedDict[tuple[int, int], dict]" = OrderedDict()
_evictions = 0


def device_lock(device: torch.device) -> threading.RLock:
    index = device.index if device.index is not None else torch.cuda.current_device()
    with _lock:
        lock = _device_locks.get(index)
        if lock is None:
            lock = _device_locks[index] = threading.RLock()
        return lock


def used_devices() -> set[int]:
    """Indices of the devices the rasterizer has submitted work to."""
    with _lock:
        return set(_device_locks)


class ReadbackSlot:
    """One read-back slot: gs_readback_slot_bytes() bytes of host memory (the
    info words first, the flag word last) and the count of its uses."""

    def __init__(self, address: int, nbytes: int):
        self.address = address
        self.words = (ctypes.c_int64 * (nbytes // 8)).from_address(address)
        self.uses = int(self.words[-1])

    def next_seq(self) -> int:
        """Sequence number for the next read-back: one above the flag's value."""
        self.uses += 1
        return self.uses

    def __getitem__(self, i: int) -> int:
        return int(self.words[i])


_HIP_HOST_MALLOC_FLAGS = 0x1 | 0x2 | 0x40000000  # portable | mapped | coherent
SLOTS_PER_BLOCK = 2 * MAX_WORKSPACE_STREAMS
_free_slots: dict[int, list] = {}
_slot_blocks: list = []  # (device, address, bytes): kept until the process ends


def _hip_runtime() -> ctypes.CDLL:
    """The HIP runtime the rasterizer library is linked against (already loaded)."""
    from . import _lib

    _lib.load()
    for name in ("libamdhip64.so.7", "libamdhip64.so"):
        try:
            hip = ctypes.CDLL(name, mode=os.RTLD_NOLOAD | os.RTLD_GLOBAL)
        except OSError:
            continue
        hip.hipHostMalloc.restype = ctypes.c_int
        hip.hipHostMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t, ctypes.c_uint]
        return hip
    raise RuntimeError("the HIP runtime (libamdhip64) is not loaded")


def _take_slot(index: int) -> ReadbackSlot:
    """A free slot of the device's blocks (a new block when none is free)."""
    free = _free_slots.setdefault(index, [])
    if not free:
        from . import _lib

        nbytes = int(_lib.load().gs_readback_slot_bytes())
        p = ctypes.c_void_p()
        with torch.cuda.device(index):
            status = _hip_runtime().hipHostMalloc(ctypes.byref(p), nbytes * SLOTS_PER_BLOCK, _HIP_HOST_MALLOC_FLAGS)
        if status != 0 or not p.value:
            raise RuntimeError(f"hipHostMalloc of the read-back slots failed with status {status}")
        ctypes.memset(p.value, 0, nbytes * SLOTS_PER_BLOCK)
        _slot_blocks.append((index, p.value, nbytes * SLOTS_PER_BLOCK))
        free.extend(ReadbackSlot(p.value + k * nbytes, nbytes) for k in reversed(range(SLOTS_PER_BLOCK)))
    return free.pop()


def readback_slot(device: torch.device, stream: torch.cuda.Stream) -> ReadbackSlot:
    """The read-back slot owned by (device, stream): words 0-3 receive the
    pair count, the visible depth-bit range and the bucketed binning's entry
    and valid Gaussian counts."""
    global _evictions
    index = device.index if device.index is not None else torch.cuda.current_device()
    key = (index, stream.cuda_stream)
    with _lock:
        entry = _entries.get(key)
        if entry is not None:
            _entries.move_to_end(key)
            return entry["slot"]
        per_device = [k for k in _entries if k[0] == index]
        while len(per_device) >= MAX_WORKSPACE_STREAMS:
            victim = per_device.pop(0)
            old = _entries.pop(victim)
            old["stream"].synchronize()
            _free_slots[victim[0]].append(old["slot"])
            _evictions += 1
        entry = {"slot": _take_slot(index), "stream": stream}
        _entries[key] = entry
        return entry["slot"]


# Pair count of the last forward per device: the next forward allocates its
# binning buffers for 1.25x that many pairs before its own count is known.
_pair_hint: dict[int, int] = {}
PAIR_HEADROOM = 1.25


def pair_capacity(device: torch.device) -> int:
    """Pairs to provision before the count is read back (0: no estimate yet)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    last = _pair_hint.get(index, 0)
    return int(last * PAIR_HEADROOM) + 1024 if last > 0 else 0


def last_pairs(device: torch.device) -> int:
    """Pair count of the last forward on the device (0 before the first)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    return _pair_hint.get(index, 0)


def note_pairs(device: torch.device, count: int) -> None:
    index = device.index if device.index is not None else torch.cuda.current_device()
    _pair_hint[index] = int(count)


def clear_caches() -> None:
    """Drop every workspace after synchronising the streams that use them
    (their slots return to the free lists; the slot blocks stay allocated)."""
    with _lock:
        for (index, _), entry in _entries.items():
            entry["stream"].synchronize()
            _free_slots[index].append(entry["slot"])
        _entries.clear()
        _pair_hint.clear()


def cache_report() -> dict:
    with _lock:
        return {
            "workspace_entries": len(_entries),
            "workspace_evictions": _evictions,
            "workspace_limit_per_device": MAX_WORKSPACE_STREAMS,
            "retained_host_bytes": sum(b[2] for b in _slot_blocks),
            "retained_device_bytes": 0,
        }
