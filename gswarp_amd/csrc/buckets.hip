// Bucketed binning for heavy tile overlap (many tiles per Gaussian): the
// per-tile lists in (depth, point index) order without emitting and sorting
// one key per (Gaussian, tile) pair.
//
// The reference sorts the Gaussians by depth, emits a (tile, point) pair per
// covered tile in that order and sorts the pairs stably by tile
// (binning_ops.py:152-222, 297-343).  With tens of pairs per Gaussian that
// moves each pair through HBM several times.  Here:
//
//   1. depth order: the Gaussians with a valid cover word are sorted stably
//      by their depth bits (the others, keyed 0, come first and are skipped);
//   2. level 1, super-tiles (8 x 8 tiles): each Gaussian, in depth order,
//      yields one entry per super-tile its tile rectangle meets, holding the
//      point index and the 64-bit mask of the tiles it covers there;
//      a stable partition (a counting pass per chunk of 1024 Gaussians, a
//      scan, and a ranking pass) lists every super-tile's entries in depth
//      order;
//   3. level 2, tiles: per chunk of 1024 entries of one super-tile list, the
//      number of entries covering each of its 64 tiles, a prefix over the
//      chunks and a scan over the tiles give every tile's range and every
//      chunk's start in it; the chunk then writes its entries' point indices
//      into the lists of the tiles they cover, in order.
//
// Each pair is written once (4 bytes); entries are about one per Gaussian and
// super-tile.  Stability: chunks of one list are in depth order, a chunk is
// walked in order, and ranks within a wave follow lane order.
//
// The covered tiles of an entry come from the Gaussian's cover word: all
// tiles of its rectangle, the cells of its recorded mask, or the coverage
// bands of its conic (accutile_band, the function the preprocess counted
// with), which the ranking pass recomputes for the Gaussians that need them,
// 64 bands per step flattened over the wave's Gaussians.
#include "gs_common.h"
#include "gs_capi.h"

namespace gs {

constexpr int kL1Chunk = 256;            // depth positions per level-1 workgroup (one wave, 4 groups of 64)
constexpr int kL1Groups = kL1Chunk / 64;
constexpr int kL2Chunk = 1024;           // entries per level-2 workgroup (one wave)
constexpr int kStageRing = 32;           // level-2 staged pairs per tile (two flush blocks of 16)
constexpr int kMaxGridTiles = 255;       // cover words hold spans below 2^8: at most 32 x 32 super-tiles

__global__ __launch_bounds__(256) void bucket_zero_kernel(int n, int* __restrict__ p) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// Inclusive sum and maximum over the wave with DPP row shifts (rows of 16
// lanes, no LDS round trip) and the three row totals read back: about a
// dozen instructions and no memory latency.
__device__ __forceinline__ int wave_scan_add_dpp(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);  // row_shr:8
  const int lane = threadIdx.x & 63;
  const int r0 = __builtin_amdgcn_readlane(x, 15), r1 = __builtin_amdgcn_readlane(x, 31);
  const int r2 = __builtin_amdgcn_readlane(x, 47);
  return x + (lane >= 16 ? r0 : 0) + (lane >= 32 ? r1 : 0) + (lane >= 48 ? r2 : 0);
}

__device__ __forceinline__ int wave_scan_max_dpp(int x) {
  x = imax(x, __builtin_amdgcn_update_dpp(-1, x, 0x111, 0xF, 0xF, false));
  x = imax(x, __builtin_amdgcn_update_dpp(-1, x, 0x112, 0xF, 0xF, false));
  x = imax(x, __builtin_amdgcn_update_dpp(-1, x, 0x114, 0xF, 0xF, false));
  x = imax(x, __builtin_amdgcn_update_dpp(-1, x, 0x118, 0xF, 0xF, false));
  const int lane = threadIdx.x & 63;
  const int r0 = __builtin_amdgcn_readlane(x, 15), r1 = __builtin_amdgcn_readlane(x, 31);
  const int r2 = __builtin_amdgcn_readlane(x, 47);
  int before = -1;
  if (lane >= 16) before = r0;
  if (lane >= 32) before = imax(before, r1);
  if (lane >= 48) before = imax(before, r2);
  return imax(x, before);
}

// Sort key of the depth order: the float bits of the depth above the
// smallest visible depth's bits, plus one, for Gaussians with a valid cover
// word (positive depths order like their bits); 0 for the others.
__global__ __launch_bounds__(256) void bucket_depth_keys_kernel(int P, const int4* __restrict__ coverage,
                                                               const float* __restrict__ depths, unsigned depth_min,
                                                               unsigned* __restrict__ keys,
                                                               int* __restrict__ values) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= P) return;
  const bool valid = unpack_cover(coverage[i]).valid;
  keys[i] = valid ? __float_as_uint(depths[i]) - depth_min + 1u : 0u;
  values[i] = i;
}

// The cover word of depth position j of the valid part of the order (zero
// past V or for an out-of-range index), and the Gaussian's index.
__device__ __forceinline__ int4 gather_word(int j, int V, int first, int P, const int* __restrict__ order,
                                           const int4* __restrict__ coverage, int& idx) {
  idx = 0;
  if (j >= V) return make_int4(0, 0, 0, 0);
  const int i = order[first + j];
  if ((unsigned)i >= (unsigned)P) return make_int4(0, 0, 0, 0);  // never for a permutation
  idx = i;
  return coverage[i];
}

// Level-1 counts: chunk c (depth positions [c * kL1Chunk, ...) of the valid
// part of the order) counts its entries per super-tile into
// hist[bucket * nchunks + c], and stores its cover words and indices in
// depth order for the ranking pass.  The next group's gathers are issued
// before the current group is counted.
__global__ __launch_bounds__(64) void bucket_count_kernel(int V, int first, int P, const int* __restrict__ order,
                                                         const int4* __restrict__ coverage,
                                                         int4* __restrict__ cw_sorted, int* __restrict__ idx_sorted,
                                                         int nsx, int B, int nchunks, int* __restrict__ hist) {
  extern __shared__ int h[];  // B counters
  const int lane = threadIdx.x;
  const int c = blockIdx.x;
  for (int b = lane; b < B; b += 64) h[b] = 0;
  __syncthreads();
  int idx;
  int4 cw = gather_word(c * kL1Chunk + lane, V, first, P, order, coverage, idx);
  for (int g = 0; g < kL1Groups; ++g) {
    const int j = c * kL1Chunk + g * 64 + lane;
    int next_idx = 0;
    int4 next = make_int4(0, 0, 0, 0);
    if (g + 1 < kL1Groups) next = gather_word(j + 64, V, first, P, order, coverage, next_idx);
    if (j < V) {
      cw_sorted[j] = cw;
      idx_sorted[j] = idx;
    }
    const SuperRect r = super_rect(unpack_cover(cw));
    for (int sy = r.sy0; sy < r.sy0 + r.ny; ++sy)
      for (int sx = r.sx0; sx < r.sx0 + r.nx; ++sx) {
        const int b = sy * nsx + sx;
        if (b < B) atomicAdd(&h[b], 1);
      }
    cw = next;
    idx = next_idx;
  }
  __syncthreads();
  for (int b = lane; b < B; b += 64) hist[(size_t)b * nchunks + c] = h[b];
}

// The clipped extent of a cover word's rectangle in super-tile (sx, sy):
// tiles [x0, x1) x [y0, y1); empty when x1 <= x0 or y1 <= y0.
struct Clip {
  int bx, by, x0, x1, y0, y1;
};

__device__ __forceinline__ Clip clip_to_super(const CoverWord& w, int sx, int sy) {
  Clip k;
  k.bx = sx * kSuperTile;
  k.by = sy * kSuperTile;
  k.x0 = imax(w.rx, k.bx);
  k.x1 = imin(w.rx + w.span_x, k.bx + kSuperTile);
  k.y0 = imax(w.ry, k.by);
  k.y1 = imin(w.ry + w.span_y, k.by + kSuperTile);
  return k;
}

// Tiles of the super-tile covered by every tile of the rectangle.
__device__ __forceinline__ uint64_t mask_full(const Clip& k) {
  if (k.x1 <= k.x0 || k.y1 <= k.y0) return 0ull;
  const uint64_t row = low_bits64(k.x1 - k.x0) << (k.x0 - k.bx);
  const uint64_t rows = low_bits64(8 * (k.y1 - k.y0)) << (8 * (k.y0 - k.by));
  return (row * 0x0101010101010101ull) & rows;
}

// Tiles of the super-tile among a recorded mask's cells (band order:
// row-major over the rectangle, or column-major with `columns`).
__device__ __forceinline__ uint64_t mask_cells(const CoverWord& w, const Clip& k) {
  uint64_t m = 0ull;
  if (k.x1 <= k.x0 || k.y1 <= k.y0) return m;
  if (!w.columns) {
    for (int ty = k.y0; ty < k.y1; ++ty) {
      const uint64_t bits = (w.mask >> ((ty - w.ry) * w.span_x + (k.x0 - w.rx))) & low_bits64(k.x1 - k.x0);
      m |= bits << ((ty - k.by) * 8 + (k.x0 - k.bx));
    }
  } else {
    for (int tx = k.x0; tx < k.x1; ++tx) {
      uint64_t bits = (w.mask >> ((tx - w.rx) * w.span_y + (k.y0 - w.ry))) & low_bits64(k.y1 - k.y0);
      while (bits != 0ull) {
        const int r = __builtin_ctzll(bits);
        bits &= bits - 1ull;
        m |= 1ull << ((k.y0 - k.by + r) * 8 + (tx - k.bx));
      }
    }
  }
  return m;
}

// Tiles of the super-tile covered by the Gaussian's coverage bands: the
// stored bands when there are any, else each band recomputed from the conic
// (accutile_band with the arguments of the preprocess's count).  Band b of a
// row-band Gaussian is tile row ry + b ([lo, hi) in tile columns); of a
// column-band Gaussian, tile column rx + b ([lo, hi) in tile rows).
__device__ __forceinline__ uint64_t mask_bands(const CoverWord& w, const Clip& k,
                                               const unsigned* __restrict__ band_store, float px, float py,
                                               float ca, float cb, float cc, float thr) {
  uint64_t m = 0ull;
  if (k.x1 <= k.x0 || k.y1 <= k.y0) return m;
  const bool stored = w.band_off >= 0 && band_store != nullptr;
  if (!w.columns) {
#pragma unroll
    for (int i = 0; i < kSuperTile; ++i) {
      const int ty = k.y0 + i;
      if (ty < k.y1) {
        int lo, hi;
        if (stored) {
          const unsigned word = band_store[w.band_off + (ty - w.ry)];
          lo = (int)(word & 0xFFFFu);
          hi = (int)(word >> 16);
        } else {
          const int2 iv = accutile_band(px, py, ca, cb, cc, thr, ty, kBlockX, kBlockY, w.rx, w.rx + w.span_x);
          lo = iv.x;
          hi = iv.y;
        }
        lo = imax(lo, k.bx);
        hi = imin(hi, k.bx + kSuperTile);
        if (hi > lo) m |= low_bits64(hi - lo) << ((ty - k.by) * 8 + (lo - k.bx));
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < kSuperTile; ++i) {
      const int tx = k.x0 + i;
      if (tx < k.x1) {
        int lo, hi;
        if (stored) {
          const unsigned word = band_store[w.band_off + (tx - w.rx)];
          lo = (int)(word & 0xFFFFu);
          hi = (int)(word >> 16);
        } else {
          const int2 iv = accutile_band(py, px, cc, cb, ca, thr, tx, kBlockY, kBlockX, w.ry, w.ry + w.span_y);
          lo = iv.x;
          hi = iv.y;
        }
        lo = imax(lo, k.by);
        hi = imin(hi, k.by + kSuperTile);
        if (hi > lo)
          m |= (0x0101010101010101ull << (tx - k.bx)) & (low_bits64(8 * (hi - lo)) << (8 * (lo - k.by)));
      }
    }
  }
  return m;
}

// Lanes (among `valid` ones) whose value of the low `bits` bits of d equals this lane's.
__device__ __forceinline__ uint64_t match_bits(unsigned d, bool valid, int bits) {
  uint64_t peers = __ballot(valid);
  for (int b = 0; b < bits; ++b) {
    const unsigned s = (unsigned)__builtin_amdgcn_sbfe((int)d, b, 1);  // 0 or ~0
    const uint64_t m = __ballot(s != 0u);
    const unsigned lo = __builtin_amdgcn_bitop3_b32((unsigned)m, (unsigned)peers, s, 0x84);
    const unsigned hi = __builtin_amdgcn_bitop3_b32((unsigned)(m >> 32), (unsigned)(peers >> 32), s, 0x84);
    peers = ((uint64_t)hi << 32) | lo;
  }
  return peers;
}

// Level-1 ranking: chunk c walks its Gaussians in depth order, 64 at a time.
// Their entries (flat positions: Gaussian-major, super-tiles row-major within
// a Gaussian's super-rectangle) are taken 64 per round, one per lane: the
// lane finds its entry's Gaussian (the last lane whose first entry is at or
// before it: marks and a prefix maximum), reads that Gaussian's cover word and
// parameters from a per-group LDS table, computes the entry's tile mask
// (from the recorded mask, the full rectangle, or the coverage bands), and
// ranks the entry among the round's entries of the same super-tile (ballot
// matching, lane order) on top of the running per-super-tile positions, which
// start at the chunk's offsets from the scanned counts.
__global__ __launch_bounds__(64) void bucket_scatter_kernel(int V, const int4* __restrict__ cw_sorted,
                                                           const int* __restrict__ idx_sorted,
                                                           const unsigned* __restrict__ band_store,
                                                           const float4* __restrict__ records,
                                                           const int* __restrict__ hist_incl, int nchunks, int nsx,
                                                           int B, int bucket_bits, long long E,
                                                           int* __restrict__ e_idx,
                                                           unsigned long long* __restrict__ e_mask) {
  extern __shared__ int cnt[];  // B running positions
  __shared__ int4 s_own[64];    // per lane: first entry, super-rectangle width, sx0 | sy0 << 8 | height << 16, index
  __shared__ int4 s_cw[64];     // per lane: cover word
  __shared__ int s_mark[64];
  const int lane = threadIdx.x;
  const int c = blockIdx.x;
  for (int b = lane; b < B; b += 64) {
    const long long f = (long long)b * nchunks + c;
    cnt[b] = f > 0 ? hist_incl[f - 1] : 0;
  }
  __syncthreads();
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  int j = c * kL1Chunk + lane;
  int4 cwv = j < V ? cw_sorted[j] : make_int4(0, 0, 0, 0);
  int idx = j < V ? idx_sorted[j] : 0;
  for (int g = 0; g < kL1Groups; ++g, j += 64) {
    // the next group's loads go out first
    int4 next_cw = make_int4(0, 0, 0, 0);
    int next_idx = 0;
    if (g + 1 < kL1Groups && j + 64 < V) {
      next_cw = cw_sorted[j + 64];
      next_idx = idx_sorted[j + 64];
    }
    const SuperRect r = super_rect(unpack_cover(cwv));
    const int n = r.nx * r.ny;
    const int incl = wave_scan_add_dpp(n);
    const int total = __builtin_amdgcn_readlane(incl, 63);
    const int excl = incl - n;
    s_own[lane] = make_int4(excl, r.nx, r.sx0 | (r.sy0 << 8) | (r.ny << 16), idx);
    s_cw[lane] = cwv;
    __builtin_amdgcn_wave_barrier();
    for (int r0 = 0; r0 < total; r0 += 64) {
      s_mark[lane] = -1;
      __builtin_amdgcn_wave_barrier();
      if (n > 0 && excl < r0 && excl + n > r0) s_mark[0] = lane;  // a Gaussian carried in from before r0
      __builtin_amdgcn_wave_barrier();
      if (n > 0 && excl >= r0 && excl < r0 + 64) s_mark[excl - r0] = lane;
      __builtin_amdgcn_wave_barrier();
      const int owner = wave_scan_max_dpp(s_mark[lane]);
      const int slot = r0 + lane;
      const bool ok = slot < total && owner >= 0;
      const int4 own = s_own[ok ? owner : 0];
      const int u = slot - own.x;
      const int o_ny = own.z >> 16;
      const bool in_owner = ok && u >= 0 && u < own.y * o_ny;
      // u / width by a float reciprocal: exact for u < 2^16 and widths up to 32
      const int uy = in_owner ? (int)(((float)u + 0.5f) * __builtin_amdgcn_rcpf((float)own.y)) : 0;
      const int ux = u - uy * own.y;
      const int sx = (own.z & 0xFF) + ux, sy = ((own.z >> 8) & 0xFF) + uy;
      const int bucket = in_owner ? sy * nsx + sx : 0;
      const bool live = in_owner && ux >= 0 && ux < own.y && bucket >= 0 && bucket < B;
      uint64_t m = 0ull;
      if (live) {
        const CoverWord w = unpack_cover(s_cw[owner]);
        const Clip k = clip_to_super(w, sx, sy);
        if (w.has_mask) {
          m = mask_cells(w, k);
        } else if (w.full) {
          m = mask_full(k);
        } else {
          // the conic, for a banded Gaussian whose bands were not stored
          float px = 0.0f, py = 0.0f, ca = 0.0f, cb = 0.0f, cc = 0.0f, thr = 0.0f;
          if (w.band_off < 0 || band_store == nullptr) {
            const float4 r0v = records[3 * (size_t)own.w];
            const float4 r1v = records[3 * (size_t)own.w + 1];
            px = r0v.x;
            py = r0v.y;
            ca = r0v.z;
            cb = r0v.w;
            cc = r1v.x;
            thr = coverage_threshold(r1v.y);
          }
          m = mask_bands(w, k, band_store, px, py, ca, cb, cc, thr);
        }
      }
      const uint64_t peers = match_bits((unsigned)bucket, live, bucket_bits);
      const int base = live ? cnt[bucket] : 0;
      const long long pos = (long long)base + __popcll(peers & below);
      if (live && pos < E) {
        e_idx[pos] = own.w;
        e_mask[pos] = m;
      }
      __builtin_amdgcn_wave_barrier();
      // the highest lane of each super-tile's peers moves its position on
      if (live && (peers >> lane) == 1ull) cnt[bucket] = base + __popcll(peers);
      __builtin_amdgcn_wave_barrier();
    }
    cwv = next_cw;
    idx = next_idx;
  }
}

// Per super-tile: its entry list [list_start[s], list_start[s + 1]) from the
// scanned level-1 counts, and its level-2 chunks [chunk_start[s],
// chunk_start[s + 1]); chunk_start[B] is the number of level-2 chunks.
__global__ __launch_bounds__(256) void bucket_table_kernel(const int* __restrict__ hist_incl, int nchunks, int B,
                                                          int* __restrict__ list_start,
                                                          int* __restrict__ chunk_start) {
  __shared__ int s_tot[256 / 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int carry = 0;
  for (int s0 = 0; s0 < B; s0 += 256) {
    const int s = s0 + threadIdx.x;
    int nch = 0;
    if (s < B) {
      const int start = s > 0 ? hist_incl[(size_t)s * nchunks - 1] : 0;
      const int end = hist_incl[(size_t)(s + 1) * nchunks - 1];
      list_start[s] = start;
      if (s == B - 1) list_start[B] = end;
      nch = (end - start + kL2Chunk - 1) / kL2Chunk;
    }
    const int incl = wave_inclusive_scan_i32(nch);
    if (lane == 63) s_tot[wave] = incl;
    __syncthreads();
    int before = 0, all = 0;
    for (int k = 0; k < 256 / 64; ++k) {
      before += k < wave ? s_tot[k] : 0;
      all += s_tot[k];
    }
    if (s < B) chunk_start[s] = carry + before + incl - nch;
    carry += all;
    __syncthreads();
  }
  if (threadIdx.x == 0) chunk_start[B] = carry;
}

// Super-tile of level-2 chunk g: the last s with chunk_start[s] <= g.
__device__ __forceinline__ int chunk_super(const int* __restrict__ chunk_start, int B, int g) {
  int lo = 0, hi = B;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (chunk_start[mid] <= g) lo = mid;
    else hi = mid;
  }
  return lo;
}

// Whether tile lane (bit `lane` of the super-tile's masks) is set in m: the
// lane's half of the mask, shifted.
__device__ __forceinline__ unsigned mask_bit(unsigned long long m, int lane) {
  const unsigned half = lane < 32 ? (unsigned)m : (unsigned)(m >> 32);
  return (half >> (lane & 31)) & 1u;
}

// Level-2 counts: lane k of chunk g counts the chunk's entries covering tile k
// of its super-tile into cnt2[g * 64 + k].  The chunk's masks pass through
// LDS 64 at a time (one coalesced load each, the next one in flight) and
// every lane reads them all.
__global__ __launch_bounds__(64) void bucket_tile_count_kernel(const int* __restrict__ list_start,
                                                              const int* __restrict__ chunk_start, int B, int E,
                                                              const unsigned long long* __restrict__ e_mask,
                                                              int* __restrict__ cnt2) {
  __shared__ unsigned long long s_m[64];
  const int g = blockIdx.x;
  if (g >= chunk_start[B]) return;
  const int s = chunk_super(chunk_start, B, g);
  const int e0 = list_start[s] + (g - chunk_start[s]) * kL2Chunk;
  const int e1 = imin(imin(e0 + kL2Chunk, list_start[s + 1]), E);
  const int lane = threadIdx.x;
  int count = 0;
  unsigned long long cur = e0 + lane < e1 ? e_mask[e0 + lane] : 0ull;
  for (int eb = e0; eb < e1; eb += 64) {
    const unsigned long long next = eb + 64 + lane < e1 ? e_mask[eb + 64 + lane] : 0ull;
    s_m[lane] = cur;
    __builtin_amdgcn_wave_barrier();
    const int n = imin(64, e1 - eb);
#pragma unroll 8
    for (int i = 0; i < n; ++i) count += mask_bit(s_m[i], lane);
    __builtin_amdgcn_wave_barrier();
    cur = next;
  }
  cnt2[(size_t)g * 64 + lane] = count;
}

// Per super-tile: each chunk's count becomes its exclusive prefix over the
// super-tile's chunks, and the totals are the tiles' pair counts.
__global__ __launch_bounds__(64) void bucket_tile_prefix_kernel(const int* __restrict__ chunk_start, int nsx,
                                                               int grid_x, int grid_y, int nc2,
                                                               int* __restrict__ cnt2, int* __restrict__ tile_count) {
  const int s = blockIdx.x;
  const int lane = threadIdx.x;
  int run = 0;
  for (int g = chunk_start[s]; g < imin(chunk_start[s + 1], nc2); ++g) {
    int* p = cnt2 + (size_t)g * 64 + lane;
    const int v = *p;
    *p = run;
    run += v;
  }
  const int tx = (s % nsx) * kSuperTile + (lane & 7);
  const int ty = (s / nsx) * kSuperTile + (lane >> 3);
  if (tx < grid_x && ty < grid_y) tile_count[ty * grid_x + tx] = run;
}

// Tile ranges from the tile counts in tile order (one workgroup): [start,
// start + count) for a tile with pairs, [0, 0] for an empty one (the
// reference's cleared ranges).
__global__ __launch_bounds__(1024) void bucket_ranges_kernel(int T, const int* __restrict__ tile_count,
                                                            int2* __restrict__ ranges) {
  __shared__ int s_tot[1024 / 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int carry = 0;
  for (int t0 = 0; t0 < T; t0 += 1024) {
    const int t = t0 + threadIdx.x;
    const int v = t < T ? tile_count[t] : 0;
    const int incl = wave_inclusive_scan_i32(v);
    if (lane == 63) s_tot[wave] = incl;
    __syncthreads();
    int before = 0, all = 0;
    for (int k = 0; k < 1024 / 64; ++k) {
      before += k < wave ? s_tot[k] : 0;
      all += s_tot[k];
    }
    const int start = carry + before + incl - v;
    if (t < T) ranges[t] = v > 0 ? make_int2(start, start + v) : make_int2(0, 0);
    carry += all;
    __syncthreads();
  }
}

// Four consecutive ints at a dword-aligned address (one vector store).
typedef int int4_dw __attribute__((ext_vector_type(4), aligned(4)));

// Level-2 scatter: chunk g walks its entries in order, 64 at a time through
// LDS; lane k appends the point index of every entry covering tile k to its
// LDS ring (the store goes out for every entry, the ring position only moves
// on a hit), and every 16 entries the lanes with 16 staged pairs write them to
// their tile's list as four 16-byte stores; the rest follows at the end.
__global__ __launch_bounds__(64) void bucket_tile_scatter_kernel(const int* __restrict__ list_start,
                                                                const int* __restrict__ chunk_start, int B, int E,
                                                                int nsx, int grid_x, int grid_y,
                                                                const int* __restrict__ e_idx,
                                                                const unsigned long long* __restrict__ e_mask,
                                                                const int* __restrict__ cnt2,
                                                                const int2* __restrict__ ranges, long long R,
                                                                int* __restrict__ point_list) {
  __shared__ unsigned long long s_m[64];
  __shared__ int s_id[64];
  __shared__ int s_ring[kStageRing * 64];  // slot-major: slot q of tile k at q * 64 + k (conflict-free)
  const int g = blockIdx.x;
  if (g >= chunk_start[B]) return;
  const int s = chunk_super(chunk_start, B, g);
  const int e0 = list_start[s] + (g - chunk_start[s]) * kL2Chunk;
  const int e1 = imin(imin(e0 + kL2Chunk, list_start[s + 1]), E);
  const int lane = threadIdx.x;
  const int tx = (s % nsx) * kSuperTile + (lane & 7);
  const int ty = (s / nsx) * kSuperTile + (lane >> 3);
  const bool tile_ok = tx < grid_x && ty < grid_y;
  long long out = tile_ok ? (long long)ranges[ty * grid_x + tx].x + cnt2[(size_t)g * 64 + lane] : 0;
  // staged pairs [flushed, staged) in ring slots modulo kStageRing
  int staged = 0, flushed = 0;
  int* ring = s_ring + lane;
  unsigned long long cur_m = e0 + lane < e1 ? e_mask[e0 + lane] : 0ull;
  int cur_id = e0 + lane < e1 ? e_idx[e0 + lane] : 0;
  for (int eb = e0; eb < e1; eb += 64) {
    const bool more = eb + 64 + lane < e1;
    const unsigned long long next_m = more ? e_mask[eb + 64 + lane] : 0ull;
    const int next_id = more ? e_idx[eb + 64 + lane] : 0;
    s_m[lane] = cur_m;
    s_id[lane] = cur_id;
    __builtin_amdgcn_wave_barrier();
    const int n = imin(64, e1 - eb);
    for (int i0 = 0; i0 < n; i0 += 16) {
      const int i1 = imin(n, i0 + 16);
#pragma unroll 4
      for (int i = i0; i < i1; ++i) {
        ring[(staged & (kStageRing - 1)) * 64] = s_id[i];
        staged += (int)mask_bit(s_m[i], lane);
      }
      // 16 staged pairs (ring slots 0-15 or 16-31): one flush of four 16-byte stores
      if (staged - flushed >= 16) {
        const int* src = ring + (flushed & (kStageRing - 1)) * 64;
        if (out + flushed + 16 <= R) {
          int4_dw* dst = reinterpret_cast<int4_dw*>(point_list + out + flushed);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            int4_dw v;
            v.x = src[(4 * q) * 64];
            v.y = src[(4 * q + 1) * 64];
            v.z = src[(4 * q + 2) * 64];
            v.w = src[(4 * q + 3) * 64];
            dst[q] = v;
          }
        }
        flushed += 16;
      }
    }
    __builtin_amdgcn_wave_barrier();
    cur_m = next_m;
    cur_id = next_id;
  }
  for (int q = flushed; q < staged; ++q)
    if (out + q < R) point_list[out + q] = ring[(q & (kStageRing - 1)) * 64];
}

}  // namespace gs

// ---------------------------------------------------------------------------
// C ABI

static inline size_t bucket_align(size_t b) { return (b + 255) & ~(size_t)255; }

namespace {

struct BucketLayout {
  int grid_x, grid_y, num_tiles, nsx, nsy, B, nchunks, nc2_max;
  size_t off_keys, off_vals, off_keys_alt, off_vals_alt, off_sort, off_cw, off_idx, off_hist, off_hist_incl, off_scan,
      off_info, off_eidx, off_emask, off_list, off_chunk, off_cnt2, off_tiles, total;
};

int bucket_layout(int32_t P, int32_t V, int64_t E, int32_t W, int32_t H, BucketLayout& L) {
  if (P < 0 || V < 0 || V > P || E < 0 || W <= 0 || H <= 0) return GS_ERR_INVALID_ARGUMENT;
  if (E > 0x7fffffffLL) return GS_ERR_OVERFLOW;
  L.grid_x = (W + gs::kBlockX - 1) / gs::kBlockX;
  L.grid_y = (H + gs::kBlockY - 1) / gs::kBlockY;
  if (L.grid_x > gs::kMaxGridTiles || L.grid_y > gs::kMaxGridTiles) return GS_ERR_TOO_LARGE;
  L.num_tiles = L.grid_x * L.grid_y;
  L.nsx = (L.grid_x + gs::kSuperTile - 1) / gs::kSuperTile;
  L.nsy = (L.grid_y + gs::kSuperTile - 1) / gs::kSuperTile;
  L.B = L.nsx * L.nsy;
  L.nchunks = (V + gs::kL1Chunk - 1) / gs::kL1Chunk;
  L.nc2_max = (int)((E + gs::kL2Chunk - 1) / gs::kL2Chunk) + L.B;
  const size_t nh = (size_t)L.B * (size_t)(L.nchunks > 0 ? L.nchunks : 1);
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += bucket_align(bytes);
    return at;
  };
  L.off_keys = take((size_t)P * 4);
  L.off_vals = take((size_t)P * 4);
  L.off_keys_alt = take((size_t)P * 4);
  L.off_vals_alt = take((size_t)P * 4);
  L.off_sort = take(gs_sort_scratch_bytes(P));
  L.off_cw = take((size_t)V * 16);
  L.off_idx = take((size_t)V * 4);
  L.off_hist = take(nh * 4);
  L.off_hist_incl = take(nh * 4);
  L.off_scan = take(gs_scan_scratch_bytes((int32_t)nh));
  L.off_info = take(4 * sizeof(int64_t));
  L.off_eidx = take((size_t)E * 4);
  L.off_emask = take((size_t)E * 8);
  L.off_list = take((size_t)(L.B + 1) * 4);
  L.off_chunk = take((size_t)(L.B + 1) * 4);
  L.off_cnt2 = take((size_t)L.nc2_max * 64 * 4);
  L.off_tiles = take((size_t)L.num_tiles * 4);
  L.total = o;
  if (nh > 0x7fffffffULL) return GS_ERR_OVERFLOW;
  return GS_OK;
}

}  // namespace

extern "C" size_t gs_bin_buckets_workspace_bytes(int32_t P, int32_t num_valid, int64_t num_entries,
                                                 int32_t image_width, int32_t image_height) {
  BucketLayout L;
  if (bucket_layout(P, num_valid, num_entries, image_width, image_height, L) != GS_OK) return 0;
  return L.total;
}

extern "C" int gs_bin_buckets(int32_t P, int32_t num_valid, int64_t num_entries, int64_t num_rendered,
                              const float* depths, uint32_t depth_min, uint32_t depth_max, const int32_t* coverage,
                              const int32_t* band_store, const float* records, int32_t image_width,
                              int32_t image_height, void* workspace, size_t workspace_bytes, int32_t* ranges,
                              int32_t* point_list, void* const* stage_events, void* stream) {
  BucketLayout L;
  int st = bucket_layout(P, num_valid, num_entries, image_width, image_height, L);
  if (st != GS_OK) return st;
  if (num_rendered < 0) return GS_ERR_INVALID_ARGUMENT;
  if (num_rendered > 0x7fffffffLL) return GS_ERR_OVERFLOW;
  if (!ranges) return GS_ERR_INVALID_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  auto mark = [&](int k) {
    if (stage_events) (void)hipEventRecord((hipEvent_t)stage_events[k], s);
  };
  const int V = num_valid;
  const long long E = num_entries;
  if (V == 0 || E == 0 || num_rendered == 0) {
    const int n2 = 2 * L.num_tiles;
    mark(0);
    hipLaunchKernelGGL(gs::bucket_zero_kernel, dim3((n2 + 255) / 256), dim3(256), 0, s, n2, ranges);
    mark(1);
    mark(2);
    mark(3);
    return gs_status_from_hip(hipGetLastError());
  }
  if (!depths || !coverage || !records || !point_list || !workspace) return GS_ERR_INVALID_ARGUMENT;
  if ((reinterpret_cast<uintptr_t>(coverage) | reinterpret_cast<uintptr_t>(records) |
       reinterpret_cast<uintptr_t>(workspace)) & 15)
    return GS_ERR_MISALIGNED;
  if (workspace_bytes < L.total) return GS_ERR_SCRATCH_TOO_SMALL;
  if (depth_max < depth_min) return GS_ERR_INVALID_ARGUMENT;
  char* ws = static_cast<char*>(workspace);
  unsigned* keys = reinterpret_cast<unsigned*>(ws + L.off_keys);
  int* vals = reinterpret_cast<int*>(ws + L.off_vals);
  unsigned* keys_alt = reinterpret_cast<unsigned*>(ws + L.off_keys_alt);
  int* vals_alt = reinterpret_cast<int*>(ws + L.off_vals_alt);
  int4* cw_sorted = reinterpret_cast<int4*>(ws + L.off_cw);
  int* idx_sorted = reinterpret_cast<int*>(ws + L.off_idx);
  int* hist = reinterpret_cast<int*>(ws + L.off_hist);
  int* hist_incl = reinterpret_cast<int*>(ws + L.off_hist_incl);
  int64_t* info = reinterpret_cast<int64_t*>(ws + L.off_info);
  int* e_idx = reinterpret_cast<int*>(ws + L.off_eidx);
  unsigned long long* e_mask = reinterpret_cast<unsigned long long*>(ws + L.off_emask);
  int* list_start = reinterpret_cast<int*>(ws + L.off_list);
  int* chunk_start = reinterpret_cast<int*>(ws + L.off_chunk);
  int* cnt2 = reinterpret_cast<int*>(ws + L.off_cnt2);
  int* tile_count = reinterpret_cast<int*>(ws + L.off_tiles);
  const int4* cw = reinterpret_cast<const int4*>(coverage);

  // 1. depth order of the Gaussians with a valid cover word (they sort last)
  mark(0);
  const int key_bits = gs_bit_length((long long)(depth_max - depth_min) + 1);
  hipLaunchKernelGGL(gs::bucket_depth_keys_kernel, dim3((P + 255) / 256), dim3(256), 0, s, P, cw, depths, depth_min,
                     keys, vals);
  st = gs_sort_pairs_u32(P, 0, key_bits, keys, vals, keys_alt, vals_alt, ws + L.off_sort,
                         L.off_cw - L.off_sort, stream);
  if (st != GS_OK) return st;
  const int* order = gs_sort_num_passes(key_bits) % 2 ? vals_alt : vals;
  const int first = P - V;
  mark(1);

  // 2. level 1: entries per super-tile in depth order
  const int nh = L.B * L.nchunks;
  const size_t lds_b = (size_t)L.B * sizeof(int);
  hipLaunchKernelGGL(gs::bucket_count_kernel, dim3(L.nchunks), dim3(64), lds_b, s, V, first, P, order, cw,
                     cw_sorted, idx_sorted, L.nsx, L.B, L.nchunks, hist);
  st = gs_scan_tiles(nh, hist, nullptr, nullptr, nullptr, hist_incl, info, ws + L.off_scan,
                     L.off_info - L.off_scan, stream);
  if (st != GS_OK) return st;
  const int bucket_bits = gs_bit_length((long long)L.B - 1);
  hipLaunchKernelGGL(gs::bucket_scatter_kernel, dim3(L.nchunks), dim3(64), lds_b, s, V, cw_sorted, idx_sorted,
                     reinterpret_cast<const unsigned*>(band_store), reinterpret_cast<const float4*>(records),
                     hist_incl, L.nchunks, L.nsx, L.B, bucket_bits, E, e_idx, e_mask);
  mark(2);

  // 3. level 2: per-tile lists
  hipLaunchKernelGGL(gs::bucket_table_kernel, dim3(1), dim3(256), 0, s, hist_incl, L.nchunks, L.B, list_start,
                     chunk_start);
  hipLaunchKernelGGL(gs::bucket_tile_count_kernel, dim3(L.nc2_max), dim3(64), 0, s, list_start, chunk_start, L.B,
                     (int)E, e_mask, cnt2);
  hipLaunchKernelGGL(gs::bucket_tile_prefix_kernel, dim3(L.B), dim3(64), 0, s, chunk_start, L.nsx, L.grid_x,
                     L.grid_y, L.nc2_max, cnt2, tile_count);
  hipLaunchKernelGGL(gs::bucket_ranges_kernel, dim3(1), dim3(1024), 0, s, L.num_tiles, tile_count,
                     reinterpret_cast<int2*>(ranges));
  hipLaunchKernelGGL(gs::bucket_tile_scatter_kernel, dim3(L.nc2_max), dim3(64), 0, s, list_start, chunk_start, L.B,
                     (int)E, L.nsx, L.grid_x, L.grid_y, e_idx, e_mask, cnt2, reinterpret_cast<const int2*>(ranges),
                     (long long)num_rendered, point_list);
  mark(3);
  return gs_status_from_hip(hipGetLastError());
}
