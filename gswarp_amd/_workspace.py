"""Per-(device, stream) host workspaces and submission locks.

The forward pass performs one device-to-host read (the pair count), which
needs page-locked host memory to be asynchronous on the stream.  Allocating
pinned memory is slow, so one small pinned buffer is kept per (device,
stream), at most ``MAX_WORKSPACE_STREAMS`` per device with least-recently
used eviction; an evicted or cleared entry's stream is synchronised first so
no copy into it can still be in flight (the contract of the reference's
workspace cache, gswarp/_internal/backends/warp/memory.py:20-22 and
340-393).  Device scratch (scan and sort tables) comes from torch's
stream-ordered caching allocator per call.

Submission from several host threads is serialised per device with an
RLock, as gswarp/_stream.py:128-151 does; calls on different streams still
overlap on the GPU.
"""

from __future__ import annotations

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


def readback_buffer(device: torch.device, stream: torch.cuda.Stream) -> torch.Tensor:
    """Pinned int64[4] host buffer owned by (device, stream): the pair count,
    the visible depth-bit range and the bucketed binning's entry and valid
    Gaussian counts."""
    global _evictions
    index = device.index if device.index is not None else torch.cuda.current_device()
    key = (index, stream.cuda_stream)
    with _lock:
        entry = _entries.get(key)
        if entry is not None:
            _entries.move_to_end(key)
            return entry["pinned"]
        per_device = [k for k in _entries if k[0] == index]
        while len(per_device) >= MAX_WORKSPACE_STREAMS:
            victim = per_device.pop(0)
            old = _entries.pop(victim)
            old["stream"].synchronize()
            _evictions += 1
        entry = {"pinned": torch.zeros(4, dtype=torch.int64, pin_memory=True), "stream": stream}
        _entries[key] = entry
        return entry["pinned"]


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
    """Drop every workspace after synchronising the streams that use them."""
    with _lock:
        for entry in _entries.values():
            entry["stream"].synchronize()
        _entries.clear()
        _pair_hint.clear()


def cache_report() -> dict:
    with _lock:
        return {
            "workspace_entries": len(_entries),
            "workspace_evictions": _evictions,
            "workspace_limit_per_device": MAX_WORKSPACE_STREAMS,
            "retained_host_bytes": sum(e["pinned"].numel() * e["pinned"].element_size() for e in _entries.values()),
            "retained_device_bytes": 0,
        }
