"""The radix sort entry points through the C ABI against a stable numpy sort.

gs_sort_keys_u64 / gs_sort_pairs_u64 / gs_sort_pairs_u32 replace the
reference's stable radix sorts (binning_ops.py:152-222 and 337-343,
memory.py:586-600).  Each case draws keys with heavy duplication (few distinct
values per digit, the shape of tile ids and depth exponents) and checks the
sorted keys and the carried values against numpy's stable argsort of the
selected bit field, so stability is checked too; bits above the field must
not take part.  Sizes straddle the 4096-element block.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gswarp_amd import _lib

pytestmark = pytest.mark.gpu


def _keys(n, kind, rng, dtype):
    bits = 64 if dtype == np.uint64 else 32
    if kind == "uniform":
        k = rng.integers(0, 2**62 if bits == 64 else 2**31, size=n, dtype=np.int64).astype(dtype)
        k = k * dtype(3) + rng.integers(0, 3, size=n).astype(dtype)
    elif kind == "few":
        k = rng.integers(0, 37, size=n).astype(dtype) * dtype(0x0101010101 if bits == 64 else 0x01010101)
    elif kind == "equal":
        k = np.full(n, 0xABCDEF if bits == 64 else 0xABCD, dtype=dtype)
    else:  # tile | depth-like: low entropy high bits, dense low bits
        tile = rng.integers(0, 8160, size=n).astype(np.uint64)
        depth = rng.integers(0x3E4CCCCD, 0x41400000, size=n).astype(np.uint64)
        k = ((tile << np.uint64(32)) | depth).astype(np.uint64)
        if bits == 32:
            k = (k & np.uint64(0xFFFFFFFF)).astype(np.uint32)
    return k


def _field(keys, lo_bit, key_bits):
    k = keys.astype(np.uint64) >> np.uint64(lo_bit)
    if key_bits < 64:
        k = k & np.uint64((1 << key_bits) - 1)
    return k


def _sort(name, n, lo_bit, key_bits, keys_np, vals_np, device):
    lib = _lib.load()
    kt = torch.from_numpy(keys_np.view(np.int64 if keys_np.dtype == np.uint64 else np.int32)).to(device)
    k_alt = torch.empty_like(kt)
    vt = v_alt = None
    if vals_np is not None:
        vt = torch.from_numpy(vals_np).to(device)
        v_alt = torch.empty_like(vt)
    scratch = torch.empty((max(int(lib.gs_sort_scratch_bytes(n)), 1),), dtype=torch.uint8, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    print(f"[sort] {name} n={n} lo={lo_bit} bits={key_bits}", flush=True)
    if name == "gs_sort_keys_u64":
        lib.call(name, n, lo_bit, key_bits, kt.data_ptr(), k_alt.data_ptr(), scratch.data_ptr(), scratch.numel(),
                 stream)
    elif name == "gs_sort_pairs_u64":
        assert lo_bit == 0
        lib.call(name, n, key_bits, kt.data_ptr(), vt.data_ptr(), k_alt.data_ptr(), v_alt.data_ptr(),
                 scratch.data_ptr(), scratch.numel(), stream)
    else:
        lib.call(name, n, lo_bit, key_bits, kt.data_ptr(), vt.data_ptr(), k_alt.data_ptr(), v_alt.data_ptr(),
                 scratch.data_ptr(), scratch.numel(), stream)
    torch.cuda.synchronize()
    if lib.gs_sort_num_passes(key_bits) % 2:
        kt, vt = k_alt, v_alt
    out_k = kt.cpu().numpy().view(keys_np.dtype)
    out_v = vt.cpu().numpy() if vt is not None else None
    return out_k, out_v


CASES = [
    ("gs_sort_keys_u64", 1, 20, 39, "uniform"),
    ("gs_sort_keys_u64", 4095, 20, 39, "tile_depth"),
    ("gs_sort_keys_u64", 4097, 0, 64, "uniform"),
    ("gs_sort_keys_u64", 300_001, 20, 44, "tile_depth"),
    ("gs_sort_keys_u64", 2_870_000, 20, 39, "tile_depth"),
    ("gs_sort_keys_u64", 1_000_003, 3, 13, "few"),
    ("gs_sort_keys_u64", 123_457, 0, 64, "equal"),
    ("gs_sort_pairs_u64", 200_003, 0, 45, "tile_depth"),
    ("gs_sort_pairs_u64", 4096, 0, 1, "uniform"),
    ("gs_sort_pairs_u64", 1_500_000, 0, 64, "few"),
    ("gs_sort_pairs_u32", 1_000_000, 0, 32, "uniform"),
    ("gs_sort_pairs_u32", 777_777, 0, 13, "tile_depth"),
    # more than 2048 blocks of 4096 keys: the digit-row scan runs in several chunks
    ("gs_sort_pairs_u32", 9_000_001, 0, 13, "tile_depth"),
    # at least 2^24 keys: 8192-key workgroup tiles
    ("gs_sort_pairs_u32", 17_000_003, 0, 13, "tile_depth"),
    ("gs_sort_keys_u64", 16_777_217, 20, 39, "tile_depth"),
    ("gs_sort_pairs_u32", 65_536, 4, 9, "few"),
    ("gs_sort_pairs_u32", 8191, 0, 32, "equal"),
]


@pytest.mark.parametrize("name,n,lo_bit,key_bits,kind", CASES)
def test_sort_matches_stable_numpy_sort(name, n, lo_bit, key_bits, kind, device):
    rng = np.random.default_rng(n * 31 + key_bits)
    dtype = np.uint32 if name.endswith("u32") else np.uint64
    keys = _keys(n, kind, rng, dtype)
    vals = None if name == "gs_sort_keys_u64" else rng.permutation(n).astype(np.int32)
    out_k, out_v = _sort(name, n, lo_bit, key_bits, keys, vals, device)
    order = np.argsort(_field(keys, lo_bit, key_bits), kind="stable")
    assert np.array_equal(out_k, keys[order])
    if vals is not None:
        assert np.array_equal(out_v, vals[order])


def test_sort_repeated_calls_reuse_scratch(device):
    """Back-to-back sorts of different sizes with one scratch buffer."""
    lib = _lib.load()
    rng = np.random.default_rng(5)
    n = 600_000
    scratch = torch.empty((int(lib.gs_sort_scratch_bytes(n)),), dtype=torch.uint8, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    for rep, m in enumerate((n, n // 3, n)):
        keys = _keys(m, "tile_depth", rng, np.uint64)
        kt = torch.from_numpy(keys.view(np.int64)).to(device)
        alt = torch.empty_like(kt)
        print(f"[sort] repeat {rep} n={m}", flush=True)
        lib.call("gs_sort_keys_u64", m, 0, 45, kt.data_ptr(), alt.data_ptr(), scratch.data_ptr(), scratch.numel(),
                 stream)
        torch.cuda.synchronize()
        res = (alt if lib.gs_sort_num_passes(45) % 2 else kt).cpu().numpy().view(np.uint64)
        assert np.array_equal(res, keys[np.argsort(_field(keys, 0, 45), kind="stable")])


def _tile_sorted_keys(rng, sizes, depth_bits, value_bits, dup):
    """Packed (tile, depth field, point) keys grouped by tile, in point order
    within each tile (the state after the stable tile-field sort)."""
    chunks = []
    for t, c in enumerate(sizes):
        if c == 0:
            continue
        idx = np.sort(rng.choice(1 << value_bits, size=c, replace=False)).astype(np.uint64)
        hi = max(1, (1 << depth_bits) if not dup else min(1 << depth_bits, 7))
        depth = rng.integers(0, hi, size=c, dtype=np.uint64) if depth_bits > 0 else np.zeros(c, np.uint64)
        chunks.append((np.uint64(t) << np.uint64(depth_bits + value_bits)) | (depth << np.uint64(value_bits)) | idx)
    keys = np.concatenate(chunks) if chunks else np.zeros(0, np.uint64)
    ends = np.cumsum(sizes)
    ranges = np.stack([ends - np.asarray(sizes), ends], axis=1).astype(np.int32)
    ranges[np.asarray(sizes) == 0] = 0
    return keys, ranges


SEGMENT_CASES = [
    # tile sizes, depth_bits, value_bits, duplicate-heavy depths, write_keys
    ([0, 1, 2, 63, 64, 65, 0, 300, 1013, 2047, 2048, 0], 26, 20, False, True),
    ([2049, 5000, 0, 17, 20000, 4097], 26, 20, False, True),
    ([2049, 5000, 17, 9000], 26, 20, True, False),
    ([350] * 40 + [1400] * 3, 9, 20, True, True),
    ([500, 3000, 1], 0, 20, False, True),
    ([777, 2500, 64], 1, 31, True, True),
    ([1024, 6000, 2000], 32, 20, False, False),
    # more long segments than the launch's 1024 long-segment workgroups, so
    # that each takes several (some through the chunked global path)
    ([1025 + 150 * (i % 7) for i in range(1100)] + [3000] * 30 + [100] * 50, 26, 20, False, True),
]


@pytest.mark.parametrize("sizes,depth_bits,value_bits,dup,write_keys", SEGMENT_CASES)
def test_tile_segment_sort_matches_full_key_sort(sizes, depth_bits, value_bits, dup, write_keys, device):
    """gs_sort_tile_segments on tile-grouped keys gives the full (tile, depth,
    point) key order: tiles empty, tiny, ragged, exactly at and above the
    2048-key on-chip capacity (the chunked global path), more long tiles than
    long-segment workgroups, partial last digits, no depth bits, and
    duplicate-heavy depths (stability)."""
    lib = _lib.load()
    rng = np.random.default_rng(sum(sizes) * 7 + depth_bits)
    keys, ranges = _tile_sorted_keys(rng, sizes, depth_bits, value_bits, dup)
    n = keys.size
    kt = torch.from_numpy(keys.view(np.int64).copy()).to(device)
    alt = torch.full_like(kt, -1)
    rt = torch.from_numpy(ranges).to(device)
    pl = torch.full((n,), -7, dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    print(f"[segsort] n={n} tiles={len(sizes)} depth_bits={depth_bits} write_keys={write_keys}", flush=True)
    lib.call("gs_sort_tile_segments", n, kt.data_ptr(), alt.data_ptr(), len(sizes), rt.data_ptr(), value_bits,
             depth_bits, value_bits, pl.data_ptr(), int(write_keys), stream)
    torch.cuda.synchronize()
    expect = np.sort(keys)
    vmask = np.uint64((1 << value_bits) - 1)
    assert np.array_equal(pl.cpu().numpy(), (expect & vmask).astype(np.int32))
    got_keys = kt.cpu().numpy().view(np.uint64)
    if write_keys:
        assert np.array_equal(got_keys, expect)
    else:  # left in place, or (tiles above 2048 keys) permuted within their segment
        assert np.array_equal(np.sort(got_keys), expect)
        for (a, b) in ranges:
            assert np.array_equal(np.sort(got_keys[a:b]), expect[a:b])
