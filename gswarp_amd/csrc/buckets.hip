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
//      a stable partition (a counting pass per chunk of kL1Chunk Gaussians,
//      a scan, and a ranking pass) lists every super-tile's entries in depth
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
constexpr int kFlushPairs = 16;          // level-2 pairs per tile written out at once (64 bytes)
constexpr int kStageRing = 2 * kFlushPairs;  // level-2 staged pairs per tile (two flush blocks)
constexpr int kMaxGridTiles = 255;       // cover words hold spans below 2^8: at most 32 x 32 super-tiles
constexpr int kMaxSuper = 32 * 32;       // super-tiles at most (kMaxGridTiles tiles a side)

__global__ __launch_bounds__(256) void bucket_zero_kernel(int n, int* __restrict__ p) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
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

// Level-1 counts: chunk c (depth positions [c * kL1Chunk, ...) of the valid
// part of the order) counts its entries per super-tile into
// hist[bucket * nchunks + c], and stores its cover words and indices in
// depth order for the ranking pass.  The chunk's indices are loaded in one
// batch, then its cover words in one batch (addresses clamped, no branches).
// A Gaussian's entries are the super-tiles of its super-rectangle, so the
// chunk counts them as a 2D difference array over the (nsx + 1) x (nsy + 1)
// corners (four LDS adds per Gaussian, whatever its size) and takes the
// counts as the array's 2D prefix sums.
__global__ __launch_bounds__(64) void bucket_count_kernel(int V, int first, int P, const int* __restrict__ order,
                                                         const int4* __restrict__ coverage,
                                                         int4* __restrict__ cw_sorted, int* __restrict__ idx_sorted,
                                                         int nsx, int nsy, int nchunks, int* __restrict__ hist) {
  extern __shared__ int h[];  // (nsy + 1) x (nsx + 1) difference counters
  const int lane = threadIdx.x;
  const int c = blockIdx.x;
  const int stride = nsx + 1;
  const int nd = (nsy + 1) * stride;
  int idx[kL1Groups];
#pragma unroll
  for (int g = 0; g < kL1Groups; ++g) idx[g] = order[first + imin(c * kL1Chunk + g * 64 + lane, V - 1)];
  for (int b = lane; b < nd; b += 64) h[b] = 0;
  int4 cw[kL1Groups];
#pragma unroll
  for (int g = 0; g < kL1Groups; ++g) cw[g] = coverage[(unsigned)idx[g] < (unsigned)P ? idx[g] : 0];
  __syncthreads();
#pragma unroll
  for (int g = 0; g < kL1Groups; ++g) {
    const int j = c * kL1Chunk + g * 64 + lane;
    // past V, or an out-of-range index (never for a permutation): no word
    const bool in = j < V && (unsigned)idx[g] < (unsigned)P;
    const int4 w = in ? cw[g] : make_int4(0, 0, 0, 0);
    if (j < V) {
      cw_sorted[j] = w;
      idx_sorted[j] = in ? idx[g] : 0;
    }
    const SuperRect r = super_rect(unpack_cover(w));
    const int x0 = imin(r.sx0, nsx), x1 = imin(r.sx0 + r.nx, nsx);
    const int y0 = imin(r.sy0, nsy), y1 = imin(r.sy0 + r.ny, nsy);
    if (x1 > x0 && y1 > y0) {
      atomicAdd(&h[y0 * stride + x0], 1);
      atomicAdd(&h[y0 * stride + x1], -1);
      atomicAdd(&h[y1 * stride + x0], -1);
      atomicAdd(&h[y1 * stride + x1], 1);
    }
  }
  __syncthreads();
  // prefix sums down the columns, then along the rows
  for (int x = lane; x <= nsx; x += 64) {
    int run = 0;
    for (int y = 0; y <= nsy; ++y) {
      run += h[y * stride + x];
      h[y * stride + x] = run;
    }
  }
  __syncthreads();
  for (int y = lane; y <= nsy; y += 64) {
    int run = 0;
    for (int x = 0; x <= nsx; ++x) {
      run += h[y * stride + x];
      h[y * stride + x] = run;
    }
  }
  __syncthreads();
  const int B = nsx * nsy;
  for (int b = lane; b < B; b += 64) hist[(size_t)c * B + b] = h[(b / nsx) * stride + b % nsx];
}

// Transpose of an int matrix through LDS, 64 x 64 elements per workgroup:
// out[c * rows + r] = flat[r * cols + c - shift] of the rows x cols input
// (0 where that index is negative), so that both sides are read and written
// in contiguous runs.  With shift 1 it turns an inclusive prefix into the
// exclusive one of the transposed layout.
__global__ __launch_bounds__(256) void bucket_transpose_kernel(const int* __restrict__ in, int rows, int cols,
                                                              int shift, int* __restrict__ out) {
  __shared__ int t[64][65];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  int v[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int r = r0 + ty + 4 * k, c = c0 + tx;
    const long long f = (long long)r * cols + c - shift;
    const bool ok = r < rows && c < cols && f >= 0;
    v[k] = in[ok ? f : 0];
    v[k] = ok ? v[k] : 0;
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) t[ty + 4 * k][tx] = v[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int c = c0 + ty + 4 * k, r = r0 + tx;
    if (c < cols && r < rows) out[(size_t)c * rows + r] = t[tx][ty + 4 * k];
  }
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

// Transpose of an 8 x 8 bit matrix held as 8 bytes (bit 8 r + c is entry
// (r, c)): three rounds of delta swaps.
__device__ __forceinline__ uint64_t transpose8x8(uint64_t x) {
  uint64_t t = (x ^ (x >> 7)) & 0x00AA00AA00AA00AAull;
  x = x ^ t ^ (t << 7);
  t = (x ^ (x >> 14)) & 0x0000CCCC0000CCCCull;
  x = x ^ t ^ (t << 14);
  t = (x ^ (x >> 28)) & 0x00000000F0F0F0F0ull;
  return x ^ t ^ (t << 28);
}

// The tile mask of an entry in one code path for every kind of coverage, so
// that a round's lanes do not diverge on it.  The super-tile's 8 lines are
// its tile rows, or its tile columns for column-oriented coverage (a
// column-major cell mask or column bands); line i's byte holds the covered
// tiles along it, taken (by selects) from the recorded cells of band
// (line - rect origin), from that band's interval in `bands` (LDS), or from
// the whole clipped rectangle; the bytes of a column-oriented entry are then
// transposed.  `bands` must be readable at [0, lines of the rectangle) for
// every kind (its words only count for banded coverage).
__device__ __forceinline__ uint64_t entry_mask(const CoverWord& w, const Clip& k, const unsigned* bands) {
  if (k.x1 <= k.x0 || k.y1 <= k.y0) return 0ull;
  const bool cols = w.columns;
  const int l0 = cols ? k.x0 : k.y0, l1 = cols ? k.x1 : k.y1;      // lines present, in tile coordinates
  const int lb = cols ? k.bx : k.by;                               // first line of the super-tile
  const int u0 = cols ? k.y0 : k.x0, u1 = cols ? k.y1 : k.x1;      // clipped extent along a line
  const int ub = cols ? k.by : k.bx;
  const int rl = cols ? w.rx : w.ry, ru = cols ? w.ry : w.rx;      // rectangle origin: band index, along a line
  const int span_u = cols ? w.span_y : w.span_x, span_l = cols ? w.span_x : w.span_y;
  const unsigned width = (1u << (u1 - u0)) - 1u;
  const unsigned full = width << (u0 - ub);
  uint64_t m = 0ull;
#pragma unroll
  for (int i = 0; i < kSuperTile; ++i) {
    const int line = l0 + i;
    const int b = line - rl;
    const unsigned from_cells = ((unsigned)(w.mask >> ((b * span_u + (u0 - ru)) & 63)) & width) << (u0 - ub);
    const unsigned word = bands[imin(b, span_l - 1)];
    const int lo = imax((int)(word & 0xFFFFu), ub), hi = imin((int)(word >> 16), ub + kSuperTile);
    const unsigned from_band = hi > lo ? ((1u << (hi - lo)) - 1u) << (lo - ub) : 0u;
    const unsigned byte = w.has_mask ? from_cells : (w.full ? full : from_band);
    m |= line < l1 ? (uint64_t)(byte & 0xFFu) << (8 * (line - lb)) : 0ull;
  }
  return cols ? transpose8x8(m) : m;
}

// Largest index g of a nondecreasing table of kL1Chunk values with t[g] <= v
// (0 when none), by binary search in LDS.
__device__ __forceinline__ int table_floor(const int* t, int v) {
  int lo = 0;
#pragma unroll
  for (int step = kL1Chunk / 2; step > 0; step >>= 1)
    if (t[lo + step] <= v) lo += step;
  return lo;
}

// Workgroups go round-robin to the eight XCDs (each with its own L2).  The
// level-1 ranking maps workgroup b to a chunk so that runs of kXcdRun
// consecutive chunks run on one XCD: consecutive chunks write adjacent pieces
// of every super-tile's list, which then meet in one L2 before they are
// written back; the runs still take turns over the XCDs, so the heavy chunks
// at the front of the depth order are spread over all of them.  Bijective on
// [0, n): workgroups past the last whole round of 8 runs keep their index.
constexpr int kXcdRun = 16;
__device__ __forceinline__ int xcd_run_chunk(int b, int n) {
  const int full = n / (8 * kXcdRun) * (8 * kXcdRun);
  if (b >= full) return b;
  const int k = b >> 3;  // the k-th workgroup on XCD b & 7
  return ((k / kXcdRun) * 8 + (b & 7)) * kXcdRun + k % kXcdRun;
}

constexpr int kL1BandCap = 1024;   // band words of a level-1 chunk held in LDS
constexpr int kL1OwnerCap = 1024;  // entries of a level-1 chunk whose Gaussian is looked up in a table

// Level-1 ranking.  Chunk c (kL1Chunk Gaussians in depth order) first loads
// the Gaussians' cover words and indices and the chunk's running
// per-super-tile positions (from the scanned counts) into LDS.  Its entries
// (flat positions: Gaussian-major, super-tiles row-major within a Gaussian's
// super-rectangle) are then handled in segments of whole Gaussians whose
// coverage bands fit an LDS buffer of kL1BandCap words: the segment's bands
// are staged (stored ones loaded, the others recomputed from the conic), and
// its entries are taken 64 per round, one per lane: the lane finds its
// entry's Gaussian (a per-entry table, or binary search over the Gaussians'
// first entries), computes the entry's tile mask and ranks the entry among
// the round's entries of the same super-tile (ballot matching, lane order) on
// top of the running position.  The rounds make no global loads, so no load
// waits behind their stores (one counter covers loads and stores); only a
// segment's staging does, once.
__global__ __launch_bounds__(64) void bucket_scatter_kernel(int V, const int4* __restrict__ cw_sorted,
                                                           const int* __restrict__ idx_sorted,
                                                           const unsigned* __restrict__ band_store,
                                                           const float4* __restrict__ records,
                                                           const int* __restrict__ pos_cm, int nchunks, int nsx,
                                                           int B, int bucket_bits, long long E,
                                                           int* __restrict__ e_idx,
                                                           unsigned long long* __restrict__ e_mask) {
  extern __shared__ int cnt[];  // B running positions
  __shared__ int4 s_cw[kL1Chunk];
  __shared__ int s_idx[kL1Chunk];
  __shared__ int s_excl[kL1Chunk];   // first entry of each Gaussian
  __shared__ int s_bexcl[kL1Chunk];  // first LDS band word of each Gaussian
  __shared__ unsigned s_band[kL1BandCap];
  __shared__ unsigned char s_owner[kL1OwnerCap];  // Gaussian of each entry, for chunks of few entries
  const int lane = threadIdx.x;
  const int c = xcd_run_chunk(blockIdx.x, nchunks);
  const int j0 = c * kL1Chunk;
  // loads: words, indices, positions, all issued (addresses clamped, no
  // branches) before the first LDS store, so the wave waits for memory once
  // per batch
  {
    int4 cwv[kL1Groups];
    int idv[kL1Groups];
#pragma unroll
    for (int q = 0; q < kL1Groups; ++q) {
      const int j = imin(j0 + q * 64 + lane, V - 1);
      cwv[q] = cw_sorted[j];
      idv[q] = idx_sorted[j];
    }
    constexpr int kPosBatch = 4;
    for (int b0 = 0; b0 < B; b0 += 64 * kPosBatch) {
      int v[kPosBatch];
#pragma unroll
      for (int q = 0; q < kPosBatch; ++q) v[q] = pos_cm[(size_t)c * B + imin(b0 + q * 64 + lane, B - 1)];
#pragma unroll
      for (int q = 0; q < kPosBatch; ++q)
        if (b0 + q * 64 + lane < B) cnt[b0 + q * 64 + lane] = v[q];
    }
#pragma unroll
    for (int q = 0; q < kL1Groups; ++q) {
      const bool in = j0 + q * 64 + lane < V;
      s_cw[q * 64 + lane] = in ? cwv[q] : make_int4(0, 0, 0, 0);
      s_idx[q * 64 + lane] = in ? idv[q] : 0;
    }
  }
  __syncthreads();
  // entries and coverage bands per Gaussian, scanned over the chunk
  int carry = 0, bcarry = 0;
#pragma unroll
  for (int q = 0; q < kL1Groups; ++q) {
    const CoverWord w = unpack_cover(s_cw[q * 64 + lane]);
    const SuperRect r = super_rect(w);
    const int n = r.nx * r.ny;
    const bool banded = w.valid && !w.has_mask && !w.full;
    const int nb = banded ? (w.columns ? w.span_x : w.span_y) : 0;
    const int incl = wave_scan_add_dpp(n), bincl = wave_scan_add_dpp(nb);
    s_excl[q * 64 + lane] = carry + incl - n;
    s_bexcl[q * 64 + lane] = bcarry + bincl - nb;
    carry += __builtin_amdgcn_readlane(incl, 63);
    bcarry += __builtin_amdgcn_readlane(bincl, 63);
  }
  const int total = carry;
  const int band_all = bcarry;
  __syncthreads();
  const bool owner_table = total <= kL1OwnerCap;
  if (owner_table) {
#pragma unroll
    for (int q = 0; q < kL1Groups; ++q) {
      const int g = q * 64 + lane;
      const int e0 = s_excl[g], e1 = g + 1 < kL1Chunk ? s_excl[g + 1] : total;
      for (int e = e0; e < e1; ++e) s_owner[e] = (unsigned char)g;
    }
  }
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  // Segments of whole Gaussians whose bands fit the LDS band buffer: each
  // segment's bands are staged (stored ones loaded, the others recomputed
  // from the conic), then its entries are ranked and written.
  for (int g0 = 0; g0 < kL1Chunk;) {
    const int b0 = s_bexcl[g0];
    // the segment [g0, g1) ends where its bands would pass the buffer: g1 is the
    // last Gaussian whose first band word still fits (every band span is < 256)
    int g1 = table_floor(s_bexcl, b0 + kL1BandCap);
    if (g1 == kL1Chunk - 1 && band_all <= b0 + kL1BandCap) g1 = kL1Chunk;
    if (g1 <= g0) g1 = g0 + 1;
    const int b1 = g1 < kL1Chunk ? s_bexcl[g1] : band_all;
    const int e_begin = s_excl[g0], e_end = g1 < kL1Chunk ? s_excl[g1] : total;
    __syncthreads();  // the previous segment's rounds are done with s_band
    // batches of kBandBatch words per lane: the stored words' loads are all
    // issued before the first of them is used; the words to recompute are
    // handled after, one at a time
    constexpr int kBandBatch = 4;
    for (int tb = b0; tb < b1; tb += 64 * kBandBatch) {
      unsigned word[kBandBatch];
      unsigned recompute = 0;  // bit q: word q has no stored copy
#pragma unroll
      for (int q = 0; q < kBandBatch; ++q) {
        const int t = imin(tb + q * 64 + lane, b1 - 1);
        const int g = table_floor(s_bexcl, t);
        const CoverWord w = unpack_cover(s_cw[g]);
        const bool stored = w.band_off >= 0 && band_store != nullptr;
        word[q] = stored ? band_store[w.band_off + (t - s_bexcl[g])] : 0u;
        recompute |= stored || tb + q * 64 + lane >= b1 ? 0u : 1u << q;
      }
#pragma unroll
      for (int q = 0; q < kBandBatch; ++q) {
        const int t = tb + q * 64 + lane;
        if (t < b1 && !((recompute >> q) & 1u)) s_band[t - b0] = word[q];
      }
#pragma unroll 1
      for (int q = 0; q < kBandBatch; ++q) {
        if (!((recompute >> q) & 1u)) continue;
        const int t = tb + q * 64 + lane;
        const int g = table_floor(s_bexcl, t);
        const CoverWord w = unpack_cover(s_cw[g]);
        const int b = t - s_bexcl[g];
        const int idx = s_idx[g];
        const float4 r0v = records[3 * (size_t)idx];
        const float4 r1v = records[3 * (size_t)idx + 1];
        const float thr = coverage_threshold(r1v.y);
        const int2 iv = w.columns ? accutile_band(r0v.y, r0v.x, r1v.x, r0v.w, r0v.z, thr, w.rx + b, kBlockY,
                                                  kBlockX, w.ry, w.ry + w.span_y)
                                  : accutile_band(r0v.x, r0v.y, r0v.z, r0v.w, r1v.x, thr, w.ry + b, kBlockX,
                                                  kBlockY, w.rx, w.rx + w.span_x);
        s_band[t - b0] = (unsigned)iv.x | ((unsigned)iv.y << 16);
      }
    }
    __syncthreads();
    for (int r0 = e_begin; r0 < e_end; r0 += 64) {
      const int slot = r0 + lane;
      const bool ok = slot < e_end;
      const int g = owner_table ? (ok ? (int)s_owner[slot] : g0) : table_floor(s_excl, slot);
      const CoverWord w = unpack_cover(s_cw[g]);
      const SuperRect r = super_rect(w);
      const int u = slot - s_excl[g];
      const bool in_owner = ok && u >= 0 && u < r.nx * r.ny;
      // u / width by a float reciprocal: exact for u < 2^16 and widths up to 32
      const int uy = in_owner ? (int)(((float)u + 0.5f) * __builtin_amdgcn_rcpf((float)r.nx)) : 0;
      const int ux = u - uy * r.nx;
      const int sx = r.sx0 + ux, sy = r.sy0 + uy;
      const int bucket = in_owner ? sy * nsx + sx : 0;
      // (a rectangle inside the grid, as the preprocess writes them, meets only
      // super-tiles with sx < nsx; the counts clip likewise)
      const bool live = in_owner && ux >= 0 && ux < r.nx && sx < nsx && bucket >= 0 && bucket < B;
      const bool banded = w.valid && !w.has_mask && !w.full;
      // a banded Gaussian's words in this segment's buffer (kept in bounds
      // whatever the word says); other kinds read any words and ignore them
      const int nb = w.columns ? w.span_x : w.span_y;
      const int boff = banded ? imax(0, imin(s_bexcl[g] - b0, kL1BandCap - nb)) : 0;
      const uint64_t m = live ? entry_mask(w, clip_to_super(w, sx, sy), s_band + boff) : 0ull;
      const uint64_t peers = match_bits((unsigned)bucket, live, bucket_bits);
      const int base = live ? cnt[bucket] : 0;
      const long long pos = (long long)base + __popcll(peers & below);
      if (live && pos < E) {
        e_idx[pos] = s_idx[g];
        e_mask[pos] = m;
      }
      __builtin_amdgcn_wave_barrier();
      // the highest lane of each super-tile's peers moves its position on
      if (live && (peers >> lane) == 1ull) cnt[bucket] = base + __popcll(peers);
      __builtin_amdgcn_wave_barrier();
    }
    g0 = g1;
  }
}

// Per super-tile: its entry list [list_start[s], list_start[s + 1]) from the
// scanned level-1 counts, and its level-2 chunks [chunk_start[s],
// chunk_start[s + 1]); chunk_start[B] is the number of level-2 chunks.  Each
// chunk g < nc2_max gets chunk_info[g] = (s, first entry, end entry), or
// (-1, 0, 0) past the last chunk, so that a chunk's wave finds its entries
// with one load.  Every workgroup scans the super-tiles itself (at most
// kMaxSuper, four per thread) and fills 256 chunks, each finding its
// super-tile by binary search; workgroup 0 also writes the two tables.
__global__ __launch_bounds__(256) void bucket_table_kernel(const int* __restrict__ hist_incl, int nchunks, int B,
                                                          int nc2_max, int* __restrict__ list_start,
                                                          int* __restrict__ chunk_start,
                                                          int4* __restrict__ chunk_info) {
  constexpr int kPer = kMaxSuper / 256;
  __shared__ int s_ls[kMaxSuper + 1], s_cs[kMaxSuper + 1];
  __shared__ int s_tot[256 / 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int start[kPer], end[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int s = k * 256 + threadIdx.x;
    start[k] = s > 0 && s < B ? hist_incl[(size_t)s * nchunks - 1] : 0;
    end[k] = s < B ? hist_incl[(size_t)(s + 1) * nchunks - 1] : 0;
  }
  int carry = 0;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    if (k * 256 >= B) break;
    const int s = k * 256 + threadIdx.x;
    const int nch = s < B ? (end[k] - start[k] + kL2Chunk - 1) / kL2Chunk : 0;
    const int incl = wave_inclusive_scan_i32(nch);
    if (lane == 63) s_tot[wave] = incl;
    __syncthreads();
    int before = 0, all = 0;
    for (int w = 0; w < 256 / 64; ++w) {
      before += w < wave ? s_tot[w] : 0;
      all += s_tot[w];
    }
    if (s < B) {
      s_ls[s] = start[k];
      s_cs[s] = carry + before + incl - nch;
      if (s == B - 1) s_ls[B] = end[k];
    }
    carry += all;
    __syncthreads();
  }
  if (threadIdx.x == 0) s_cs[B] = carry;
  __syncthreads();
  if (blockIdx.x == 0) {
    for (int s = threadIdx.x; s <= B; s += 256) {
      list_start[s] = s_ls[s];
      chunk_start[s] = s_cs[s];
    }
  }
  const int g = blockIdx.x * 256 + threadIdx.x;
  if (g >= nc2_max) return;
  if (g >= carry) {
    chunk_info[g] = make_int4(-1, 0, 0, 0);
    return;
  }
  int lo = 0, hi = B - 1;  // the last super-tile whose chunks start at or before g
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (s_cs[mid] <= g) lo = mid;
    else hi = mid - 1;
  }
  const int e0 = s_ls[lo] + (g - s_cs[lo]) * kL2Chunk;
  chunk_info[g] = make_int4(lo, e0, imin(e0 + kL2Chunk, s_ls[lo + 1]), 0);
}

// Copies the entries [e0, e0 + n) (1 <= n <= kL2Chunk) of a level-2 chunk
// into LDS, zero past n up to the next multiple of 16.  Every load of the
// lane is issued before its first LDS store (addresses clamped into the
// chunk, no branches), so the wave waits for memory once.
__device__ __forceinline__ void stage_chunk(int e0, int n, int lane, const unsigned long long* __restrict__ e_mask,
                                            const int* __restrict__ e_idx, unsigned long long* s_m, int* s_id) {
  constexpr int kQ = kL2Chunk / 64;
  unsigned long long m[kQ];
  int id[kQ];
#pragma unroll
  for (int q = 0; q < kQ; ++q) {
    const int e = e0 + imin(q * 64 + lane, n - 1);
    m[q] = e_mask[e];
    id[q] = e_idx[e];
  }
  const int n16 = (n + 15) & ~15;
#pragma unroll
  for (int q = 0; q < kQ; ++q) {
    const int i = q * 64 + lane;
    if (i < n16) {
      s_m[i] = i < n ? m[q] : 0ull;
      s_id[i] = i < n ? id[q] : 0;
    }
  }
}

// Carry-save addition of three bit vectors: per bit, a + b + c = 2 hi + lo.
__device__ __forceinline__ void csa(unsigned& hi, unsigned& lo, unsigned a, unsigned b, unsigned c) {
  const unsigned u = a ^ b;
  hi = (a & b) | (u & c);
  lo = u ^ c;
}

// One step of the wave's bit transpose inside each 32-bit word: lane L and
// lane L ^ S swap the bits k of L's word with (k & S) != 0 (L below its
// partner) for the bits k - S of the partner's word, and so on mirrored.
template <int S>
__device__ __forceinline__ unsigned transpose_step(unsigned x, unsigned keep, unsigned rot) {
  const unsigned p = (unsigned)__builtin_amdgcn_ds_swizzle((int)x, (S << 10) | 0x1f);  // lane ^ S
  return (keep & x) | (~keep & __builtin_amdgcn_alignbit(p, p, rot));
}

// Transposes the 64 x 64 bit matrix whose row j is lane j's 64-bit word
// (lo, hi): afterwards bit j of lane k's word is bit k of lane j's word.
// Recursive block swap: halves across lanes L and L ^ 32 (one lane permute),
// then quarters, ..., single bits inside each word (lane swizzles).
__device__ __forceinline__ void wave_bit_transpose(unsigned& lo, unsigned& hi, int lane) {
  const bool up = lane >= 32;
  const unsigned recv = (unsigned)__builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, (int)(up ? lo : hi));
  if (up) lo = recv;
  else hi = recv;
#define GS_TRANSPOSE_STEP(S, MASK)                                   \
  {                                                                  \
    const bool u = (lane & (S)) != 0;                                \
    const unsigned keep = u ? ~(unsigned)(MASK) : (unsigned)(MASK);  \
    const unsigned rot = u ? (S) : 32 - (S);                         \
    lo = transpose_step<S>(lo, keep, rot);                           \
    hi = transpose_step<S>(hi, keep, rot);                           \
  }
  GS_TRANSPOSE_STEP(16, 0x0000ffffu)
  GS_TRANSPOSE_STEP(8, 0x00ff00ffu)
  GS_TRANSPOSE_STEP(4, 0x0f0f0f0fu)
  GS_TRANSPOSE_STEP(2, 0x33333333u)
  GS_TRANSPOSE_STEP(1, 0x55555555u)
#undef GS_TRANSPOSE_STEP
}

// Level-2 counts: lane k of chunk g counts the chunk's entries covering tile k
// of its super-tile into cnt2[g * 64 + k].  Lane j loads the masks of entries
// j, 64 + j, ..., adds its 16 masks bit-sliced (carry-save adders: five bit
// planes of the per-tile counts 0..16), and the wave transposes each plane,
// so that lane k's popcounts of the planes are tile k's count.
// chunk_info[g] = (super-tile, first entry, end entry), super-tile -1 past the
// last chunk.
__global__ __launch_bounds__(64) void bucket_tile_count_kernel(const int4* __restrict__ chunk_info, int E,
                                                              const unsigned long long* __restrict__ e_mask,
                                                              int* __restrict__ cnt2) {
  constexpr int kQ = kL2Chunk / 64;
  static_assert(kQ == 16, "sixteen masks per lane");
  const int g = blockIdx.x;
  const int lane = threadIdx.x;
  const int4 ci = chunk_info[g];
  if (ci.x < 0) return;
  const int e0 = ci.y, n = imin(ci.z, E) - e0;
  if (n <= 0) {
    cnt2[(size_t)g * 64 + lane] = 0;
    return;
  }
  unsigned long long m[kQ];
#pragma unroll
  for (int q = 0; q < kQ; ++q) m[q] = e_mask[e0 + imin(q * 64 + lane, n - 1)];
#pragma unroll
  for (int q = 0; q < kQ; ++q)
    if (q * 64 + lane >= n) m[q] = 0ull;
  unsigned plane_lo[5], plane_hi[5];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    unsigned a[kQ];
#pragma unroll
    for (int q = 0; q < kQ; ++q) a[q] = h ? (unsigned)(m[q] >> 32) : (unsigned)m[q];
    unsigned ones = 0, twos = 0, fours = 0, eights = 0, sixteens, tA, tB, fA, fB, eA, eB;
    csa(tA, ones, ones, a[0], a[1]);
    csa(tB, ones, ones, a[2], a[3]);
    csa(fA, twos, twos, tA, tB);
    csa(tA, ones, ones, a[4], a[5]);
    csa(tB, ones, ones, a[6], a[7]);
    csa(fB, twos, twos, tA, tB);
    csa(eA, fours, fours, fA, fB);
    csa(tA, ones, ones, a[8], a[9]);
    csa(tB, ones, ones, a[10], a[11]);
    csa(fA, twos, twos, tA, tB);
    csa(tA, ones, ones, a[12], a[13]);
    csa(tB, ones, ones, a[14], a[15]);
    csa(fB, twos, twos, tA, tB);
    csa(eB, fours, fours, fA, fB);
    csa(sixteens, eights, eights, eA, eB);
    unsigned* pl = h ? plane_hi : plane_lo;
    pl[0] = ones;
    pl[1] = twos;
    pl[2] = fours;
    pl[3] = eights;
    pl[4] = sixteens;
  }
  int count = 0;
#pragma unroll
  for (int pidx = 0; pidx < 5; ++pidx) {
    unsigned lo = plane_lo[pidx], hi = plane_hi[pidx];
    wave_bit_transpose(lo, hi, lane);
    count += (__popc(lo) + __popc(hi)) << pidx;
  }
  cnt2[(size_t)g * 64 + lane] = count;
}

// Per super-tile: each chunk's count becomes its exclusive prefix over the
// super-tile's chunks, and the totals are the tiles' pair counts.  The
// super-tile's chunks are split into 16 consecutive runs, one per wave: each
// wave sums its run, the waves' sums are scanned in LDS, and each wave walks
// its run again writing the prefixes (a sixteenth of the serial walk).
__global__ __launch_bounds__(1024) void bucket_tile_prefix_kernel(const int* __restrict__ chunk_start, int nsx,
                                                                 int grid_x, int grid_y, int nc2,
                                                                 int* __restrict__ cnt2, int* __restrict__ tile_count) {
  constexpr int kWaves = 1024 / 64;
  constexpr int kBatch = 16;  // chunks whose counts are loaded together
  __shared__ int s_tot[kWaves][64];
  const int s = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g0 = chunk_start[s], g1 = imin(chunk_start[s + 1], nc2);
  const int per = imax(g1 - g0 + kWaves - 1, 0) / kWaves;
  const int a = g0 + wave * per, b = imin(a + per, g1);
  int sum = 0;
  for (int g = a; g < b; g += kBatch) {
    int v[kBatch];
#pragma unroll
    for (int q = 0; q < kBatch; ++q) v[q] = cnt2[(size_t)imin(g + q, b - 1) * 64 + lane];
#pragma unroll
    for (int q = 0; q < kBatch; ++q) sum += g + q < b ? v[q] : 0;
  }
  s_tot[wave][lane] = sum;
  __syncthreads();
  int run = 0;
  for (int w = 0; w < wave; ++w) run += s_tot[w][lane];
  for (int g = a; g < b; g += kBatch) {
    int v[kBatch];
#pragma unroll
    for (int q = 0; q < kBatch; ++q) v[q] = cnt2[(size_t)imin(g + q, b - 1) * 64 + lane];
#pragma unroll
    for (int q = 0; q < kBatch; ++q) {
      if (g + q < b) {
        cnt2[(size_t)(g + q) * 64 + lane] = run;
        run += v[q];
      }
    }
  }
  const int tx = (s % nsx) * kSuperTile + (lane & 7);
  const int ty = (s / nsx) * kSuperTile + (lane >> 3);
  if (wave == kWaves - 1 && tx < grid_x && ty < grid_y) tile_count[ty * grid_x + tx] = run;
}

// Tile ranges from the tile counts in tile order (one workgroup): [start,
// start + count) for a tile with pairs, [0, 0] for an empty one (the
// reference's cleared ranges).  Eight rounds of 1024 tiles are loaded
// together, then scanned round by round.
__global__ __launch_bounds__(1024) void bucket_ranges_kernel(int T, const int* __restrict__ tile_count,
                                                            int2* __restrict__ ranges) {
  constexpr int kRounds = 8;
  __shared__ int s_tot[1024 / 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int carry = 0;
  for (int t0 = 0; t0 < T; t0 += 1024 * kRounds) {
    int v[kRounds];
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
      const int t = t0 + r * 1024 + threadIdx.x;
      v[r] = t < T ? tile_count[t] : 0;
    }
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
      if (t0 + r * 1024 >= T) break;
      const int t = t0 + r * 1024 + threadIdx.x;
      const int incl = wave_inclusive_scan_i32(v[r]);
      if (lane == 63) s_tot[wave] = incl;
      __syncthreads();
      int before = 0, all = 0;
      for (int k = 0; k < 1024 / 64; ++k) {
        before += k < wave ? s_tot[k] : 0;
        all += s_tot[k];
      }
      const int start = carry + before + incl - v[r];
      if (t < T) ranges[t] = v[r] > 0 ? make_int2(start, start + v[r]) : make_int2(0, 0);
      carry += all;
      __syncthreads();
    }
  }
}

// Four consecutive ints at a dword-aligned address (one vector store).
typedef int int4_dw __attribute__((ext_vector_type(4), aligned(4)));

// Level-2 scatter: chunk g first copies its entries (masks and point indices)
// into LDS, so that no load waits behind the stores that follow, then walks
// them in order; lane k appends the point index of every entry covering tile
// k to its LDS ring (the store goes out for every entry, the ring position
// only moves on a hit).  Every 16 entries a lane writes out the staged pairs
// up to the next 64-byte boundary of its tile's list once (the head), and
// after that whole 64-byte blocks of 16 as four 16-byte stores, so the list
// is written in full HBM sectors; the rest follows at the end.
__global__ __launch_bounds__(64) void bucket_tile_scatter_kernel(const int4* __restrict__ chunk_info, int E,
                                                                int nsx, int grid_x, int grid_y,
                                                                const int* __restrict__ e_idx,
                                                                const unsigned long long* __restrict__ e_mask,
                                                                const int* __restrict__ cnt2,
                                                                const int2* __restrict__ ranges, long long R,
                                                                int* __restrict__ point_list) {
  __shared__ __align__(16) unsigned long long s_m[kL2Chunk];
  __shared__ __align__(16) int s_id[kL2Chunk];
  __shared__ int s_ring[kStageRing * 64];  // slot-major: slot q of tile k at q * 64 + k (conflict-free)
  static_assert(kFlushPairs == 16, "four lanes of four pairs per block");
  const int g = blockIdx.x;
  const int lane = threadIdx.x;
  const int4 ci = chunk_info[g];
  const int s = ci.x;
  if (s < 0) return;
  const int e0 = ci.y;
  const int n = imin(ci.z, E) - e0;
  if (n <= 0) return;
  const int n16 = (n + 15) & ~15;  // entries past n have no tile: zero masks
  const int tx = (s % nsx) * kSuperTile + (lane & 7);
  const int ty = (s / nsx) * kSuperTile + (lane >> 3);
  const bool tile_ok = tx < grid_x && ty < grid_y;
  // the tile's list start and the chunk's offset in it, loaded with the chunk
  const int start = ranges[tile_ok ? ty * grid_x + tx : 0].x;
  const int before = cnt2[(size_t)g * 64 + lane];
  stage_chunk(e0, n, lane, e_mask, e_idx, s_m, s_id);
  const long long out = tile_ok ? (long long)start + before : 0;
  int head = (int)((kFlushPairs - (out & (kFlushPairs - 1))) & (kFlushPairs - 1));  // pairs before the next block boundary
  // staged pairs [flushed, staged) in ring slots modulo kStageRing
  int staged = 0, flushed = 0;
  int* ring = s_ring + lane;
  // Each lane reads only its half of the masks, and keeps its ring position
  // as the byte offset of its slot row (staged << 8), so that an entry costs
  // one bit extract, one add and one and-or for the ring address.
  const unsigned* s_half = reinterpret_cast<const unsigned*>(s_m) + (lane >> 5);
  const unsigned lbit = lane & 31;
  const int lane4 = lane << 2;
  char* ring_b = reinterpret_cast<char*>(s_ring);
  int pos = 0;
  __syncthreads();
  for (int i0 = 0; i0 < n16; i0 += 16) {
    // 16 entries: all their LDS reads first, then the ring positions in
    // registers, then the ring writes, so no write waits on a read
    unsigned h[16];
    int id[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) h[q] = s_half[2 * (i0 + q)];
#pragma unroll
    for (int q = 0; q < 16; q += 4) {
      const int4 v = *reinterpret_cast<const int4*>(s_id + i0 + q);
      id[q] = v.x;
      id[q + 1] = v.y;
      id[q + 2] = v.z;
      id[q + 3] = v.w;
    }
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      *reinterpret_cast<int*>(ring_b + ((pos & ((kStageRing - 1) << 8)) | lane4)) = id[q];
      pos += (int)__builtin_amdgcn_ubfe(h[q], lbit, 1u) << 8;
    }
    staged = pos >> 8;
    if (head > 0 && staged - flushed >= head) {
      for (int q = 0; q < head; ++q)
        if (out + flushed + q < R) point_list[out + flushed + q] = ring[((flushed + q) & (kStageRing - 1)) * 64];
      flushed += head;
      head = 0;
    }
    // Whole blocks, written four lanes to a block: each lane with a block to
    // write sends its tile (lane), the block's ring slot and its start (-1
    // past R) to the first lane of a quad (a forward lane permute, then a
    // quad broadcast), and lane 4 j + h stores part h (one 16-byte store) of
    // the j-th block, so that one store instruction writes sixteen blocks'
    // 64-byte sectors whole.
    const bool fl = head == 0 && staged - flushed >= kFlushPairs;
    const uint64_t fmask = __ballot(fl);
    if (fmask != 0) {
      const int rank = (int)__builtin_amdgcn_mbcnt_hi((unsigned)(fmask >> 32),
                                                      __builtin_amdgcn_mbcnt_lo((unsigned)fmask, 0u));
      const int nfl = __popcll(fmask);
      const int info_x = lane | ((flushed & (kStageRing - 1)) << 8);
      const int info_y = out + flushed + kFlushPairs <= R ? (int)(out + flushed) : -1;
      for (int p0 = 0; p0 < nfl; p0 += 16) {
        // this pass's blocks go to lanes 0, 4, ..., 60; every other lane
        // sends to lane 1, whose value no lane reads
        const bool mine = fl && rank >= p0 && rank < p0 + 16;
        const int to = (mine ? 4 * (rank - p0) : 1) * 4;
        int x = __builtin_amdgcn_ds_permute(to, info_x);
        int y = __builtin_amdgcn_ds_permute(to, info_y);
        x = __builtin_amdgcn_update_dpp(0, x, 0x00, 0xF, 0xF, false);  // quad_perm [0,0,0,0]
        y = __builtin_amdgcn_update_dpp(0, y, 0x00, 0xF, 0xF, false);
        if (p0 + (lane >> 2) < nfl) {
          const int t = x & 63, slot = (x >> 8) + 4 * (lane & 3);
          int4_dw v;
          v.x = s_ring[(slot & (kStageRing - 1)) * 64 + t];
          v.y = s_ring[((slot + 1) & (kStageRing - 1)) * 64 + t];
          v.z = s_ring[((slot + 2) & (kStageRing - 1)) * 64 + t];
          v.w = s_ring[((slot + 3) & (kStageRing - 1)) * 64 + t];
          if (y >= 0) *reinterpret_cast<int4_dw*>(point_list + y + 4 * (lane & 3)) = v;
        }
      }
      if (fl) flushed += kFlushPairs;
    }
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
  size_t off_keys, off_vals, off_keys_alt, off_vals_alt, off_sort, off_cw, off_idx, off_hist, off_hist_incl, off_pos,
      off_scan,
      off_info, off_eidx, off_emask, off_list, off_chunk, off_cinfo, off_cnt2, off_tiles, total;
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
  L.off_pos = take(nh * 4);
  L.off_scan = take(gs_scan_scratch_bytes((int32_t)nh));
  L.off_info = take(4 * sizeof(int64_t));
  L.off_eidx = take((size_t)E * 4);
  L.off_emask = take((size_t)E * 8);
  L.off_list = take((size_t)(L.B + 1) * 4);
  L.off_chunk = take((size_t)(L.B + 1) * 4);
  L.off_cinfo = take((size_t)L.nc2_max * 16);
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
  int* pos_cm = reinterpret_cast<int*>(ws + L.off_pos);
  int64_t* info = reinterpret_cast<int64_t*>(ws + L.off_info);
  int* e_idx = reinterpret_cast<int*>(ws + L.off_eidx);
  unsigned long long* e_mask = reinterpret_cast<unsigned long long*>(ws + L.off_emask);
  int* list_start = reinterpret_cast<int*>(ws + L.off_list);
  int* chunk_start = reinterpret_cast<int*>(ws + L.off_chunk);
  int4* chunk_info = reinterpret_cast<int4*>(ws + L.off_cinfo);
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
  const size_t lds_d = (size_t)(L.nsx + 1) * (L.nsy + 1) * sizeof(int);
  // counts chunk-major (each chunk writes one contiguous row), transposed to
  // super-tile-major for the scan, and the scanned positions transposed back
  // so that each ranking chunk reads one contiguous row
  hipLaunchKernelGGL(gs::bucket_count_kernel, dim3(L.nchunks), dim3(64), lds_d, s, V, first, P, order, cw,
                     cw_sorted, idx_sorted, L.nsx, L.nsy, L.nchunks, pos_cm);
  hipLaunchKernelGGL(gs::bucket_transpose_kernel, dim3((L.B + 63) / 64, (L.nchunks + 63) / 64), dim3(256), 0, s,
                     pos_cm, L.nchunks, L.B, 0, hist);
  st = gs_scan_tiles(nh, hist, nullptr, nullptr, nullptr, hist_incl, info, ws + L.off_scan,
                     L.off_info - L.off_scan, stream);
  if (st != GS_OK) return st;
  hipLaunchKernelGGL(gs::bucket_transpose_kernel, dim3((L.nchunks + 63) / 64, (L.B + 63) / 64), dim3(256), 0, s,
                     hist_incl, L.B, L.nchunks, 1, pos_cm);
  const int bucket_bits = gs_bit_length((long long)L.B - 1);
  hipLaunchKernelGGL(gs::bucket_scatter_kernel, dim3(L.nchunks), dim3(64), lds_b, s, V, cw_sorted, idx_sorted,
                     reinterpret_cast<const unsigned*>(band_store), reinterpret_cast<const float4*>(records),
                     pos_cm, L.nchunks, L.nsx, L.B, bucket_bits, E, e_idx, e_mask);
  mark(2);

  // 3. level 2: per-tile lists
  hipLaunchKernelGGL(gs::bucket_table_kernel, dim3((L.nc2_max + 255) / 256), dim3(256), 0, s, hist_incl, L.nchunks,
                     L.B, L.nc2_max, list_start, chunk_start, chunk_info);
  hipLaunchKernelGGL(gs::bucket_tile_count_kernel, dim3(L.nc2_max), dim3(64), 0, s, chunk_info, (int)E, e_mask, cnt2);
  hipLaunchKernelGGL(gs::bucket_tile_prefix_kernel, dim3(L.B), dim3(1024), 0, s, chunk_start, L.nsx, L.grid_x,
                     L.grid_y, L.nc2_max, cnt2, tile_count);
  hipLaunchKernelGGL(gs::bucket_ranges_kernel, dim3(1), dim3(1024), 0, s, L.num_tiles, tile_count,
                     reinterpret_cast<int2*>(ranges));
  hipLaunchKernelGGL(gs::bucket_tile_scatter_kernel, dim3(L.nc2_max), dim3(64), 0, s, chunk_info, (int)E, L.nsx,
                     L.grid_x, L.grid_y, e_idx, e_mask, cnt2, reinterpret_cast<const int2*>(ranges),
                     (long long)num_rendered, point_list);
  mark(3);
  return gs_status_from_hip(hipGetLastError());
}
