// Tile binning: depth sort keys, tile-count prefix sum, duplicate-with-keys,
// tile ranges.  Two dataflows produce identical per-tile lists:
//
// * depth then tile (the reference's default, binning_ops.py:152-222 and
//   297-343): the N Gaussians are sorted stably by depth bits (culled ones
//   first with key 0), the tile counts are scanned in that order, each
//   Gaussian emits (tile id, index) pairs at its offset, and a stable sort of
//   the R tile ids (ceil(log2 T) bits) orders pairs by (tile, depth, index).
// * one 64-bit key (the reference's packed "warp_radix" mode): pairs are
//   emitted in point-index order as
//     key = ((tile << depth_bits) | (float_bits(depth) - depth_min)) << value_bits | point
//   and sorted once on the tile and depth fields.  Subtracting the smallest
//   visible depth's bits keeps the order and drops the bits all depths share;
//   the point index rides in the low value_bits bits when the fields fit in
//   64 bits, so the sort moves 8 bytes per pair.
// Depths of binned Gaussians are positive, so their float bits order like the
// depths; both stable sorts therefore give (tile, depth, point index) order.
#include <mutex>

#include "gs_common.h"
#include "gs_capi.h"

namespace gs {

constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;
constexpr int kScanTile = kScanThreads * kScanItems;

__device__ __forceinline__ long long wave_inclusive_scan_i64(long long v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const long long n = __shfl_up(v, off, 64);
    if (lane >= off) v += n;
  }
  return v;
}

// Block-wide exclusive scan of one int64 per thread (256 threads); returns the
// exclusive prefix and writes the block total to *total.
__device__ __forceinline__ long long block_exclusive_scan_i64(long long v, long long* lds4, long long* total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const long long inc = wave_inclusive_scan_i64(v);
  if (lane == 63) lds4[wave] = inc;
  __syncthreads();
  long long wave_off = 0;
  long long tot = 0;
#pragma unroll
  for (int w = 0; w < kScanThreads / 64; ++w) {
    const long long s = lds4[w];
    if (w < wave) wave_off += s;
    tot += s;
  }
  *total = tot;
  __syncthreads();
  return wave_off + inc - v;
}

__device__ __forceinline__ unsigned wave_min_u32(unsigned v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const unsigned o = __shfl_xor(v, off, 64);
    v = o < v ? o : v;
  }
  return v;
}

__device__ __forceinline__ unsigned wave_max_u32(unsigned v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const unsigned o = __shfl_xor(v, off, 64);
    v = o > v ? o : v;
  }
  return v;
}

// The scan runs in two passes over blocks of kScanTile = 4096 Gaussians.
// Thread t of a block owns elements 4t .. 4t + 3 of each of its four
// 1024-element chunks, so every load and store of a wave covers 1 KB of
// consecutive elements (16-byte vector accesses when nothing is gathered).
constexpr int kScanChunk = kScanThreads * 4;
static_assert(kScanTile == 4 * kScanChunk, "four chunks of four elements per thread");

// The four elements of thread t in chunk k of block `base`, gathered through
// order when there is one; elements past n are 0.
__device__ __forceinline__ void scan_load4(const int* __restrict__ in, const int* __restrict__ order, long long i0,
                                           long long n, bool vec, int (&v)[4], int (&src)[4]) {
  if (vec && i0 + 3 < n) {
    const int4 o = order ? *reinterpret_cast<const int4*>(order + i0) : make_int4(0, 0, 0, 0);
    src[0] = order ? o.x : (int)i0;
    src[1] = order ? o.y : (int)i0 + 1;
    src[2] = order ? o.z : (int)i0 + 2;
    src[3] = order ? o.w : (int)i0 + 3;
    if (!order) {
      const int4 x = *reinterpret_cast<const int4*>(in + i0);
      v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
      return;
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) src[j] = i0 + j < n ? (order ? order[i0 + j] : (int)(i0 + j)) : -1;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = src[j] >= 0 ? in[src[j]] : 0;
}

// Per block: the tile-count sum, and the smallest and largest depth bits of
// the Gaussians with radius > 0 (min ~0u / max 0 when there are none), packed
// as max << 32 | min.  With an order, the counts are gathered through it and
// also stored contiguously in `gathered` (when given), so that the apply pass
// reads them without a second gather.
__global__ __launch_bounds__(kScanThreads) void scan_reduce_kernel(int n, const int* __restrict__ in,
                                                                  const int* __restrict__ order,
                                                                  const int* __restrict__ radii,
                                                                  const float* __restrict__ depths,
                                                                  long long* __restrict__ block_sums,
                                                                  unsigned long long* __restrict__ block_range,
                                                                  int* __restrict__ gathered, int vec,
                                                                  const int4* __restrict__ coverage,
                                                                  long long* __restrict__ block_ev) {
  __shared__ long long lds4[kScanThreads / 64];
  __shared__ unsigned s_min[kScanThreads / 64], s_max[kScanThreads / 64];
  const long long base = (long long)blockIdx.x * kScanTile;
  long long s = 0;
  unsigned dmin = ~0u, dmax = 0u;
  long long units = 0;  // with coverage: super-tile units of the block's valid words
  int valid = 0, bad = 0;  // valid words; Gaussians with tiles but no valid word
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const long long i0 = base + k * kScanChunk + 4 * threadIdx.x;
    int v[4], src[4];
    scan_load4(in, order, i0, n, vec != 0, v, src);
    if (coverage) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (i0 + j < n) {
          const CoverWord w = unpack_cover(coverage[i0 + j]);
          const int u = super_units(w);
          units += u;
          valid += w.valid;
          bad |= (v[j] > 0 && !w.valid) ? 1 : 0;
        }
      }
    }
    if (gathered) {
      if (vec && i0 + 3 < n) {
        *reinterpret_cast<int4*>(gathered + i0) = make_int4(v[0], v[1], v[2], v[3]);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (i0 + j < n) gathered[i0 + j] = v[j];
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      s += v[j];
      if (radii && src[j] >= 0 && radii[src[j]] > 0) {
        const unsigned bits = __float_as_uint(depths[src[j]]);
        dmin = bits < dmin ? bits : dmin;
        dmax = bits > dmax ? bits : dmax;
      }
    }
  }
  dmin = wave_min_u32(dmin);
  dmax = wave_max_u32(dmax);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s_min[wave] = dmin;
    s_max[wave] = dmax;
  }
  long long total;
  block_exclusive_scan_i64(s, lds4, &total);  // its barriers also order s_min / s_max
  if (coverage) {
    long long units_total, valid_total, bad_total;
    block_exclusive_scan_i64(units, lds4, &units_total);
    block_exclusive_scan_i64(valid, lds4, &valid_total);
    block_exclusive_scan_i64(bad, lds4, &bad_total);
    if (threadIdx.x == 0) {
      block_ev[2 * blockIdx.x] = bad_total > 0 ? -1 : units_total;
      block_ev[2 * blockIdx.x + 1] = valid_total;
    }
  }
  if (threadIdx.x == 0) {
    block_sums[blockIdx.x] = total;
    unsigned mn = ~0u, mx = 0u;
#pragma unroll
    for (int w = 0; w < kScanThreads / 64; ++w) {
      mn = s_min[w] < mn ? s_min[w] : mn;
      mx = s_max[w] > mx ? s_max[w] : mx;
    }
    block_range[blockIdx.x] = ((unsigned long long)mx << 32) | mn;
  }
}

// Inclusive prefix sums of the block's elements: its offset is the sum of the
// preceding blocks' sums (each block adds them up itself, so no pass runs
// between the two), then each chunk is scanned and carried into the next.
// The last block also stores the total pair count in info[0] and the visible
// depth-bit range (max << 32 | min, or 0 when nothing is visible) in
// info[1].  Offsets are int32 (meaningful when the total fits).  With
// block_ev (the reduce pass's per-block super-tile units and valid words) it
// also stores info[2] = the total units (-1 when a Gaussian with tiles has no
// valid cover word) and info[3] = the number of valid words.
__global__ __launch_bounds__(kScanThreads) void scan_apply_kernel(int n, int nb, const int* __restrict__ in,
                                                                 const int* __restrict__ order,
                                                                 const long long* __restrict__ block_sums,
                                                                 const unsigned long long* __restrict__ block_range,
                                                                 int* __restrict__ out, long long* __restrict__ info,
                                                                 int vec, const long long* __restrict__ block_ev) {
  __shared__ long long lds4[kScanThreads / 64];
  __shared__ unsigned s_min[kScanThreads / 64], s_max[kScanThreads / 64];
  const int b = blockIdx.x;
  const bool last = b == nb - 1;
  long long pre = 0;
  unsigned dmin = ~0u, dmax = 0u;
  for (int j = threadIdx.x; j < (last ? nb : b); j += kScanThreads) {
    if (j < b) pre += block_sums[j];
    if (last) {
      const unsigned long long r = block_range[j];
      const unsigned mn = (unsigned)r, mx = (unsigned)(r >> 32);
      dmin = mn < dmin ? mn : dmin;
      dmax = mx > dmax ? mx : dmax;
    }
  }
  long long pre_total;
  block_exclusive_scan_i64(pre, lds4, &pre_total);
  if (last) {
    dmin = wave_min_u32(dmin);
    dmax = wave_max_u32(dmax);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
      s_min[wave] = dmin;
      s_max[wave] = dmax;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      unsigned mn = ~0u, mx = 0u;
#pragma unroll
      for (int w = 0; w < kScanThreads / 64; ++w) {
        mn = s_min[w] < mn ? s_min[w] : mn;
        mx = s_max[w] > mx ? s_max[w] : mx;
      }
      info[0] = pre_total + block_sums[b];
      info[1] = mx >= mn ? (long long)(((unsigned long long)mx << 32) | mn) : 0;
    }
    if (block_ev) {
      long long units = 0, valid = 0, bad = 0;
      for (int j = threadIdx.x; j < nb; j += kScanThreads) {
        const long long u = block_ev[2 * j];
        bad += u < 0 ? 1 : 0;
        units += u < 0 ? 0 : u;
        valid += block_ev[2 * j + 1];
      }
      long long units_total, valid_total, bad_total;
      block_exclusive_scan_i64(units, lds4, &units_total);
      block_exclusive_scan_i64(valid, lds4, &valid_total);
      block_exclusive_scan_i64(bad, lds4, &bad_total);
      if (threadIdx.x == 0) {
        info[2] = bad_total > 0 ? -1 : units_total;
        info[3] = valid_total;
      }
    }
  }
  long long carry = pre_total;
  const long long base = (long long)b * kScanTile;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const long long i0 = base + k * kScanChunk + 4 * threadIdx.x;
    int v[4], src[4];
    scan_load4(in, order, i0, n, vec != 0, v, src);
    v[1] += v[0];
    v[2] += v[1];
    v[3] += v[2];
    long long chunk_total;
    const long long run = carry + block_exclusive_scan_i64(v[3], lds4, &chunk_total);
    if (vec && i0 + 3 < n) {
      *reinterpret_cast<int4*>(out + i0) =
          make_int4((int)(run + v[0]), (int)(run + v[1]), (int)(run + v[2]), (int)(run + v[3]));
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (i0 + j < n) out[i0 + j] = (int)(run + v[j]);
    }
    carry += chunk_total;
  }
}

// Visits one Gaussian's covered tiles in the enumeration order of
// the coverage count (binning_kernels.py:127-216 semantics), calling
// f(tile_id) for each.
template <typename F>
__device__ __forceinline__ void for_each_covered_tile(float px, float py, float ca, float cb, float cc,
                                                      float opacity, float cov_aa, float cov_cc, int radius,
                                                      int grid_x, int grid_y, int mode, F&& f) {
  const int4 rect = snugbox_rect(px, py, cov_aa, cov_cc, opacity, radius, grid_x, grid_y);
  const int span_x = rect.z - rect.x;
  const int span_y = rect.w - rect.y;
  const int area = span_x * span_y;
  if (area <= 1 || mode == kCoverageSnugbox) {
    for (int ty = rect.y; ty < rect.w; ++ty)
      for (int tx = rect.x; tx < rect.z; ++tx) f(ty * grid_x + tx);
    return;
  }
  const float threshold = coverage_threshold(opacity);
  if (mode == kCoverageConicRect && area <= kConicMaskMaxTiles) {
    for (int ty = rect.y; ty < rect.w; ++ty)
      for (int tx = rect.x; tx < rect.z; ++tx)
        if (conic_rect_intersects_tile(px, py, ca, cb, cc, threshold, tx, ty)) f(ty * grid_x + tx);
    return;
  }
  if (span_y <= span_x) {
    for (int ty = rect.y; ty < rect.w; ++ty) {
      const int2 iv = accutile_band(px, py, ca, cb, cc, threshold, ty, kBlockX, kBlockY, rect.x, rect.z);
      for (int tx = iv.x; tx < iv.y; ++tx) f(ty * grid_x + tx);
    }
  } else {
    for (int tx = rect.x; tx < rect.z; ++tx) {
      const int2 iv = accutile_band(py, px, cc, cb, ca, threshold, tx, kBlockY, kBlockX, rect.y, rect.w);
      for (int ty = iv.x; ty < iv.y; ++ty) f(ty * grid_x + tx);
    }
  }
}

// Emission is balanced per wave: a lane emits its own Gaussian's pairs when
// it covers at most kLaneEmitMax tiles; the wave then takes its larger
// Gaussians one at a time and emits each with its lanes in parallel, one
// lane per band of the coverage walk (one tile row or column, whose interval
// is computed exactly as the serial walk computes it) with a wave prefix sum
// of the band lengths as output offsets, or one lane per tile of the
// conic-rect masked case (at most 64 tiles).  The pairs land where the
// serial walk of for_each_covered_tile puts them.  With the heavy tail of
// large splats (a few hundred tiles each) a serial walk holds a whole wave
// for the longest of its Gaussians.
constexpr int kLaneEmitMax = 32;
constexpr int kMaskLaneEmitMax = 8;  // the same threshold for Gaussians emitted from a cover mask

__device__ __forceinline__ float bcast_f(float v, int src) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
}


// One Gaussian's pairs written by the whole wave (all lanes hold the same
// arguments).  write(position, tile id) stores one pair; positions start at
// off and stop at limit.  Band tiles are first placed in the wave's LDS
// window (stage, kEmitWindow entries) at their output positions, then
// written out with consecutive lanes on consecutive positions, so each store
// instruction covers a contiguous run instead of one cache line per lane.
constexpr int kEmitWindow = 1024;

template <typename W>
__device__ __forceinline__ void wave_emit_gaussian(float px, float py, float ca, float cb, float cc, float opacity,
                                                   float cov_aa, float cov_cc, int radius, int grid_x, int grid_y,
                                                   int mode, long long off, long long limit, int* stage,
                                                   W&& write) {
  const int lane = threadIdx.x & 63;
  const int4 rect = snugbox_rect(px, py, cov_aa, cov_cc, opacity, radius, grid_x, grid_y);
  const int span_x = rect.z - rect.x;
  const int span_y = rect.w - rect.y;
  const int area = span_x * span_y;
  const float threshold = coverage_threshold(opacity);
  if (area > 1 && mode == kCoverageConicRect && area <= kConicMaskMaxTiles) {
    // rect tiles in row-major order, one per lane; hits are compacted in lane order
    const int tx = rect.x + (span_x > 0 ? lane % span_x : 0);
    const int ty = rect.y + (span_x > 0 ? lane / span_x : 0);
    const bool hit = lane < area && conic_rect_intersects_tile(px, py, ca, cb, cc, threshold, tx, ty);
    const uint64_t m = __ballot(hit);
    const long long pos = off + __popcll(m & ((lane == 0) ? 0ull : (~0ull >> (64 - lane))));
    if (hit && pos < limit) write(pos, ty * grid_x + tx);
    return;
  }
  // bands: rows of the rect (full rect or AccuTile rows) or AccuTile columns
  const bool full = area <= 1 || mode == kCoverageSnugbox;
  const bool columns = !full && span_y > span_x;
  const int nb = columns ? span_x : span_y;
  long long base = off;
  for (int b0 = 0; b0 < nb; b0 += 64) {
    const int b = b0 + lane;
    int lo = 0, hi = 0;
    if (b < nb) {
      if (full) {
        lo = rect.x;
        hi = rect.z;
      } else if (!columns) {
        const int2 iv = accutile_band(px, py, ca, cb, cc, threshold, rect.y + b, kBlockX, kBlockY, rect.x, rect.z);
        lo = iv.x;
        hi = iv.y;
      } else {
        const int2 iv = accutile_band(py, px, cc, cb, ca, threshold, rect.x + b, kBlockY, kBlockX, rect.y, rect.w);
        lo = iv.x;
        hi = iv.y;
      }
    }
    const int len = imax(0, hi - lo);
    const int incl = wave_inclusive_scan_i32(len);
    const int excl = incl - len;
    const int total = __builtin_amdgcn_readlane(incl, 63);
    // windows [w0, w0 + kEmitWindow) of this band chunk's total positions
    for (int w0 = 0; w0 < total; w0 += kEmitWindow) {
      const int k_begin = imax(0, w0 - excl);
      const int k_end = imin(len, w0 + kEmitWindow - excl);
      for (int k = k_begin; k < k_end; ++k) {
        const int t = lo + k;
        stage[excl + k - w0] = columns ? t * grid_x + (rect.x + b) : (rect.y + b) * grid_x + t;
      }
      __builtin_amdgcn_wave_barrier();
      const int n = imin(kEmitWindow, total - w0);
      for (int i = lane; i < n; i += 64) {
        const long long pos = base + w0 + i;
        if (pos < limit) write(pos, stage[i]);
      }
      __builtin_amdgcn_wave_barrier();
    }
    base += total;
  }
}

// Emission from a cover mask recorded by the preprocess: a lane walks the
// set bits of its Gaussian's mask (the order of the coverage walk), or the
// wave writes a larger Gaussian's cells one per lane, each hit at the
// position given by the hits below it.
template <typename W>
__device__ __forceinline__ void emit_mask_lane(const CoverWord& c, int grid_x, long long off, long long limit,
                                               W&& write) {
  const float rcp_span_u = __builtin_amdgcn_rcpf((float)(c.columns ? c.span_y : c.span_x));
  uint64_t m = c.mask;
  long long pos = off;
  while (m != 0) {
    const int k = __builtin_ctzll(m);
    m &= m - 1;
    if (pos < limit) write(pos, cover_cell_tile(c, rcp_span_u, k, grid_x));
    ++pos;
  }
}

template <typename W>
__device__ __forceinline__ void wave_emit_mask(const CoverWord& c, int grid_x, long long off, long long limit,
                                               W&& write) {
  const int lane = threadIdx.x & 63;
  const float rcp_span_u = __builtin_amdgcn_rcpf((float)(c.columns ? c.span_y : c.span_x));
  const bool hit = ((c.mask >> lane) & 1ull) != 0;
  const long long pos = off + __popcll(c.mask & low_bits64(lane));
  if (hit && pos < limit) write(pos, cover_cell_tile(c, rcp_span_u, lane, grid_x));
}

// Per wave: small Gaussians by their own lanes, then large ones by the wave.
// `count` is the Gaussian's pair count (0 for lanes without one).
// write_own(pos, tile) stores a pair of the calling lane's Gaussian;
// write_from(src, pos, tile) one of lane src's Gaussian (src wave-uniform).
// `cover_w` is the Gaussian's packed cover word (zero: none recorded), and a
// recorded mask replaces the coverage walk.
template <typename WO, typename WF>
__device__ __forceinline__ void emit_balanced(bool active, int count, float px, float py, float ca, float cb,
                                              float cc, float opacity, float cov_aa, float cov_cc, int radius,
                                              int grid_x, int grid_y, int mode, int4 cover_w, long long off,
                                              long long limit, WO&& write_own, WF&& write_from) {
  __shared__ int s_stage[256 / 64][kEmitWindow];  // one window per wave of the 256-thread workgroup
  int* stage = s_stage[threadIdx.x >> 6];
  const CoverWord cw = unpack_cover(cover_w);
  const bool large = active && count > (cw.has_mask ? kMaskLaneEmitMax : kLaneEmitMax);
  if (active && !large) {
    if (cw.has_mask) {
      emit_mask_lane(cw, grid_x, off, limit, write_own);
    } else {
      long long pos = off;
      for_each_covered_tile(px, py, ca, cb, cc, opacity, cov_aa, cov_cc, radius, grid_x, grid_y, mode,
                            [&](int tile) {
                              if (pos < limit) write_own(pos, tile);
                              ++pos;
                            });
    }
  }
  uint64_t todo = __ballot(large);
  while (todo != 0) {
    const int src = __builtin_ctzll(todo);
    todo &= todo - 1;
    const long long soff = ((long long)__builtin_amdgcn_readlane((int)(off >> 32), src) << 32) |
                           (unsigned)__builtin_amdgcn_readlane((int)off, src);
    const CoverWord sc = unpack_cover(make_int4(
        __builtin_amdgcn_readlane(cover_w.x, src), __builtin_amdgcn_readlane(cover_w.y, src),
        __builtin_amdgcn_readlane(cover_w.z, src), __builtin_amdgcn_readlane(cover_w.w, src)));
    auto write = [&](long long pos, int tile) { write_from(src, pos, tile); };
    if (sc.has_mask) {
      wave_emit_mask(sc, grid_x, soff, limit, write);
    } else {
      wave_emit_gaussian(bcast_f(px, src), bcast_f(py, src), bcast_f(ca, src), bcast_f(cb, src),
                         bcast_f(cc, src), bcast_f(opacity, src), bcast_f(cov_aa, src), bcast_f(cov_cc, src),
                         __builtin_amdgcn_readlane(radius, src), grid_x, grid_y, mode, soff, limit, stage, write);
    }
  }
}

__global__ __launch_bounds__(256) void duplicate_keys_kernel(int P, const int* __restrict__ radii,
                                                            const float4* __restrict__ records,
                                                            const float* __restrict__ cov2d,
                                                            const int4* __restrict__ coverage,
                                                            const float* __restrict__ depths,
                                                            const int* __restrict__ offsets, int grid_x,
                                                            int grid_y, int mode, long long limit,
                                                            unsigned depth_min, int depth_bits, int value_bits,
                                                            unsigned long long* __restrict__ keys,
                                                            int* __restrict__ values) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  const int radius = idx < P ? radii[idx] : 0;
  const bool active = radius > 0;
  long long off = 0;
  int count = 0;
  float4 r0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), r1 = r0;
  float cov_aa = 0.0f, cov_cc = 0.0f;
  int4 cover_w = make_int4(0, 0, 0, 0);
  unsigned long long field = 0;
  if (active) {
    off = idx > 0 ? (long long)offsets[idx - 1] : 0;
    count = (int)((long long)offsets[idx] - off);
    if (coverage) cover_w = coverage[idx];
    float depth;
    if (!unpack_cover(cover_w).has_mask) {
      r0 = records[3 * (size_t)idx + 0];
      r1 = records[3 * (size_t)idx + 1];
      cov_aa = cov2d[3 * idx + 0];
      cov_cc = cov2d[3 * idx + 2];
      depth = r1.z;
    } else {
      // the record's depth, from the contiguous copy when there is one
      depth = depths ? depths[idx] : records[3 * (size_t)idx + 1].z;
    }
    const unsigned long long doff = (unsigned long long)(__float_as_uint(depth) - depth_min);
    field = (doff << value_bits) | (value_bits > 0 ? (unsigned long long)idx : 0ull);
  }
  const int tile_shift = depth_bits + value_bits;
  const bool with_values = value_bits == 0;
  emit_balanced(
      active, count, r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, cov_aa, cov_cc, radius, grid_x, grid_y, mode, cover_w, off,
      limit,
      [&](long long pos, int tile) {
        keys[pos] = ((unsigned long long)tile << tile_shift) | field;
        if (with_values) values[pos] = idx;
      },
      [&](int src, long long pos, int tile) {
        const unsigned long long f = ((unsigned long long)(unsigned)__builtin_amdgcn_readlane((int)(field >> 32), src)
                                      << 32) |
                                     (unsigned)__builtin_amdgcn_readlane((int)field, src);
        keys[pos] = ((unsigned long long)tile << tile_shift) | f;
        if (with_values) values[pos] = __builtin_amdgcn_readlane(idx, src);
      });
}

// Depth-sort input (binning_kernels.py:27-40 semantics): key = float bits of
// the depth for Gaussians with radius > 0 (positive floats order like their
// bits), 0 for culled ones; value = point index.
__global__ __launch_bounds__(256) void depth_keys_kernel(int P, const int* __restrict__ radii,
                                                        const float* __restrict__ depths,
                                                        unsigned* __restrict__ keys, int* __restrict__ values) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= P) return;
  keys[i] = radii[i] > 0 ? __float_as_uint(depths[i]) : 0u;
  values[i] = i;
}

// Emission in depth order: thread j emits the tiles of Gaussian order[j] at
// offsets[j-1] as (tile id, point index) pairs (binning_kernels.py:411-451).
__global__ __launch_bounds__(256) void duplicate_tiles_kernel(int P, const int* __restrict__ order,
                                                             const int* __restrict__ radii,
                                                             const float4* __restrict__ records,
                                                             const float* __restrict__ cov2d,
                                                             const int4* __restrict__ coverage,
                                                             const int* __restrict__ offsets, int grid_x,
                                                             int grid_y, int mode, long long limit,
                                                             unsigned* __restrict__ tiles,
                                                             int* __restrict__ values) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  int idx = j < P ? order[j] : -1;
  if ((unsigned)idx >= (unsigned)P) idx = -1;  // never taken for a permutation
  const int radius = idx >= 0 ? radii[idx] : 0;
  const bool active = radius > 0;
  long long off = 0;
  int count = 0;
  float4 r0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), r1 = r0;
  float cov_aa = 0.0f, cov_cc = 0.0f;
  int4 cover_w = make_int4(0, 0, 0, 0);
  if (active) {
    off = j > 0 ? (long long)offsets[j - 1] : 0;
    count = (int)((long long)offsets[j] - off);
    if (coverage) cover_w = coverage[idx];
    if (!unpack_cover(cover_w).has_mask) {
      r0 = records[3 * (size_t)idx + 0];
      r1 = records[3 * (size_t)idx + 1];
      cov_aa = cov2d[3 * idx + 0];
      cov_cc = cov2d[3 * idx + 2];
    }
  }
  emit_balanced(
      active, count, r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, cov_aa, cov_cc, radius, grid_x, grid_y, mode, cover_w, off,
      limit,
      [&](long long pos, int tile) {
        tiles[pos] = (unsigned)tile;
        values[pos] = idx;
      },
      [&](int src, long long pos, int tile) {
        tiles[pos] = (unsigned)tile;
        values[pos] = __builtin_amdgcn_readlane(idx, src);
      });
}

// Tile boundaries of sorted tile ids, kRangeItems consecutive pairs per
// thread (vector loads; the pair before the thread's run is one extra load):
// at a change from tile a to tile b at position i, ranges[a].y = i and
// ranges[b].x = i; the first pair starts its tile at 0 and the last ends its
// tile at n.
constexpr int kRangeItems = 8;

__device__ __forceinline__ void mark_ranges(long long i0, int cnt, const unsigned (&t)[kRangeItems], unsigned prev,
                                            long long n, int num_tiles, int2* __restrict__ ranges) {
#pragma unroll
  for (int k = 0; k < kRangeItems; ++k) {
    if (k < cnt) {
      const long long i = i0 + k;
      const unsigned tile = t[k];
      if (tile < (unsigned)num_tiles) {  // always true for ids from the emission kernels
        if (i == 0) {
          ranges[tile].x = 0;
        } else if (tile != prev) {
          if (prev < (unsigned)num_tiles) ranges[prev].y = (int)i;
          ranges[tile].x = (int)i;
        }
        if (i == n - 1) ranges[tile].y = (int)n;
      }
      prev = tile;
    }
  }
}

__global__ __launch_bounds__(256) void tile_ranges_u32_kernel(long long n, const unsigned* __restrict__ tiles,
                                                             int num_tiles, int2* __restrict__ ranges) {
  const long long i0 = ((long long)blockIdx.x * blockDim.x + threadIdx.x) * kRangeItems;
  if (i0 >= n) return;
  const int cnt = (int)(n - i0 < kRangeItems ? n - i0 : kRangeItems);
  unsigned t[kRangeItems];
  if (cnt == kRangeItems) {
    const uint4 a = reinterpret_cast<const uint4*>(tiles + i0)[0];
    const uint4 b = reinterpret_cast<const uint4*>(tiles + i0)[1];
    t[0] = a.x; t[1] = a.y; t[2] = a.z; t[3] = a.w;
    t[4] = b.x; t[5] = b.y; t[6] = b.z; t[7] = b.w;
  } else {
#pragma unroll
    for (int k = 0; k < kRangeItems; ++k) t[k] = k < cnt ? tiles[i0 + k] : 0u;
  }
  const unsigned prev = i0 > 0 ? tiles[i0 - 1] : 0xFFFFFFFFu;
  mark_ranges(i0, cnt, t, prev, n, num_tiles, ranges);
}

__global__ void zero_info_kernel(long long* p) {
  if (threadIdx.x < 2) p[threadIdx.x] = 0;
}

__global__ __launch_bounds__(256) void zero_ranges_kernel(int n2, int* __restrict__ ranges) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n2) ranges[i] = 0;
}

// ranges[t] = [start, end) of tile t in the sorted keys (tile = key >> tile_shift);
// with value_bits > 0 and point_list given also unpacks point_list[i] = low
// value_bits of key i.  kRangeItems keys per thread, as above.
__global__ __launch_bounds__(256) void tile_ranges_kernel(long long n, const unsigned long long* __restrict__ keys,
                                                         int tile_shift, int value_bits, int num_tiles,
                                                         int2* __restrict__ ranges, int* __restrict__ point_list) {
  const long long i0 = ((long long)blockIdx.x * blockDim.x + threadIdx.x) * kRangeItems;
  if (i0 >= n) return;
  const int cnt = (int)(n - i0 < kRangeItems ? n - i0 : kRangeItems);
  unsigned long long k64[kRangeItems];
  if (cnt == kRangeItems) {
#pragma unroll
    for (int q = 0; q < kRangeItems / 2; ++q) {
      const ulonglong2 v = reinterpret_cast<const ulonglong2*>(keys + i0)[q];
      k64[2 * q] = v.x;
      k64[2 * q + 1] = v.y;
    }
  } else {
#pragma unroll
    for (int k = 0; k < kRangeItems; ++k) k64[k] = k < cnt ? keys[i0 + k] : 0ull;
  }
  // tile ids as 32-bit values; ids too large for the grid map above num_tiles
  unsigned t[kRangeItems];
#pragma unroll
  for (int k = 0; k < kRangeItems; ++k) {
    const unsigned long long tile = k64[k] >> tile_shift;
    t[k] = tile < (unsigned long long)num_tiles ? (unsigned)tile : 0xFFFFFFFFu;
  }
  if (value_bits > 0 && point_list != nullptr) {
    const unsigned long long vmask = (1ull << value_bits) - 1ull;
#pragma unroll
    for (int k = 0; k < kRangeItems; ++k)
      if (k < cnt) point_list[i0 + k] = (int)(k64[k] & vmask);
  }
  unsigned prev = 0xFFFFFFFFu;
  if (i0 > 0) {
    const unsigned long long ptile = keys[i0 - 1] >> tile_shift;
    prev = ptile < (unsigned long long)num_tiles ? (unsigned)ptile : 0xFFFFFFFFu;
  }
  mark_ranges(i0, cnt, t, prev, n, num_tiles, ranges);
}

}  // namespace gs

extern "C" int gs_version(void) { return 10000; }

extern "C" const char* gs_status_string(int status) {
  switch (status) {
    case GS_OK:
      return "ok";
    case GS_ERR_INVALID_ARGUMENT:
      return "invalid argument";
    case GS_ERR_MISALIGNED:
      return "pointer not 16-byte aligned";
    case GS_ERR_SCRATCH_TOO_SMALL:
      return "scratch buffer too small";
    case GS_ERR_OVERFLOW:
      return "size exceeds the int32 index range";
    case GS_ERR_TOO_LARGE:
      return "size exceeds the fixed scratch of an allocation-free entry point";
    default:
      return status > 0 ? hipGetErrorString((hipError_t)status) : "unknown error";
  }
}

static inline int gs_scan_blocks(int32_t P) { return (P + gs::kScanTile - 1) / gs::kScanTile; }

// 16-byte vector accesses need every contiguous array 16-byte aligned.
static inline int gs_scan_vec(const void* in, const void* order, const void* out, const void* gathered) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(order) |
                      reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(gathered);
  return (a & 15) == 0 ? 1 : 0;
}

// Scratch: the block sums and depth ranges, then room for the counts
// gathered in the given order.
static inline size_t gs_scan_block_bytes(int32_t P) {
  return ((size_t)gs_scan_blocks(P) * 2 * sizeof(long long) + 255) & ~(size_t)255;
}
extern "C" size_t gs_scan_scratch_bytes(int32_t P) {
  if (P <= 0) return 0;
  return gs_scan_block_bytes(P) + (((size_t)P * sizeof(int) + 255) & ~(size_t)255);
}

extern "C" int gs_scan_tiles(int32_t P, const int32_t* tiles_touched, const int32_t* order, const int32_t* radii,
                             const float* depths, int32_t* offsets, int64_t* info_dev, void* scratch,
                             size_t scratch_bytes, void* stream) {
  if (P < 0 || !info_dev) return GS_ERR_INVALID_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  if (P == 0) {
    hipLaunchKernelGGL(gs::zero_info_kernel, dim3(1), dim3(64), 0, s, reinterpret_cast<long long*>(info_dev));
    return gs_status_from_hip(hipGetLastError());
  }
  if (!tiles_touched || !offsets || !scratch || (radii == nullptr) != (depths == nullptr))
    return GS_ERR_INVALID_ARGUMENT;
  if (scratch_bytes < gs_scan_scratch_bytes(P)) return GS_ERR_SCRATCH_TOO_SMALL;
  const int nb = gs_scan_blocks(P);
  long long* block_sums = reinterpret_cast<long long*>(scratch);
  unsigned long long* block_range = reinterpret_cast<unsigned long long*>(block_sums + nb);
  int* gathered = order ? reinterpret_cast<int*>(static_cast<char*>(scratch) + gs_scan_block_bytes(P)) : nullptr;
  const int vec = gs_scan_vec(tiles_touched, order, offsets, gathered);
  hipLaunchKernelGGL(gs::scan_reduce_kernel, dim3(nb), dim3(gs::kScanThreads), 0, s, P, tiles_touched, order,
                     radii, depths, block_sums, block_range, gathered, vec, nullptr, nullptr);
  hipLaunchKernelGGL(gs::scan_apply_kernel, dim3(nb), dim3(gs::kScanThreads), 0, s, P, nb,
                     gathered ? gathered : tiles_touched, nullptr, block_sums, block_range, offsets,
                     reinterpret_cast<long long*>(info_dev), vec, nullptr);
  return gs_status_from_hip(hipGetLastError());
}

// The point-order scan with the bucketed binning's sizes: the reduce pass
// also sums each valid cover word's super-tile count and counts the valid
// words (block_ev, 16 bytes per block, in the scratch region that the
// point-order scan leaves unused), and the apply pass's last block totals
// them into info[2] and info[3].
extern "C" int gs_scan_tiles_entries(int32_t P, const int32_t* tiles_touched, const int32_t* radii,
                                     const float* depths, const int32_t* coverage, int32_t* offsets,
                                     int64_t* info_dev, void* scratch, size_t scratch_bytes, void* stream) {
  if (P < 0 || !info_dev) return GS_ERR_INVALID_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  if (P == 0) {
    hipLaunchKernelGGL(gs::zero_info_kernel, dim3(1), dim3(64), 0, s, reinterpret_cast<long long*>(info_dev));
    hipLaunchKernelGGL(gs::zero_info_kernel, dim3(1), dim3(64), 0, s, reinterpret_cast<long long*>(info_dev) + 2);
    return gs_status_from_hip(hipGetLastError());
  }
  if (!tiles_touched || !offsets || !scratch || !coverage || (radii == nullptr) != (depths == nullptr))
    return GS_ERR_INVALID_ARGUMENT;
  if (reinterpret_cast<uintptr_t>(coverage) & 15) return GS_ERR_MISALIGNED;
  if (scratch_bytes < gs_scan_scratch_bytes(P)) return GS_ERR_SCRATCH_TOO_SMALL;
  const int nb = gs_scan_blocks(P);
  // block sums and ranges, then the per-block units and valid counts; the
  // scratch has room for them: gs_scan_scratch_bytes(P) >= 32 bytes per block
  long long* block_sums = reinterpret_cast<long long*>(scratch);
  unsigned long long* block_range = reinterpret_cast<unsigned long long*>(block_sums + nb);
  long long* block_ev = reinterpret_cast<long long*>(static_cast<char*>(scratch) + gs_scan_block_bytes(P));
  const int vec = gs_scan_vec(tiles_touched, nullptr, offsets, nullptr);
  hipLaunchKernelGGL(gs::scan_reduce_kernel, dim3(nb), dim3(gs::kScanThreads), 0, s, P, tiles_touched, nullptr,
                     radii, depths, block_sums, block_range, nullptr, vec,
                     reinterpret_cast<const int4*>(coverage), block_ev);
  hipLaunchKernelGGL(gs::scan_apply_kernel, dim3(nb), dim3(gs::kScanThreads), 0, s, P, nb, tiles_touched, nullptr,
                     block_sums, block_range, offsets, reinterpret_cast<long long*>(info_dev), vec, block_ev);
  return gs_status_from_hip(hipGetLastError());
}

extern "C" int gs_info_readback(const int64_t* info_dev, int64_t* info_host_pinned, int32_t count, void* stream) {
  if (!info_dev || !info_host_pinned || count < 1 || count > 16) return GS_ERR_INVALID_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e =
      hipMemcpyAsync(info_host_pinned, info_dev, (size_t)count * sizeof(int64_t), hipMemcpyDeviceToHost, s);
  if (e != hipSuccess) return (int)e;
  return gs_status_from_hip(hipStreamSynchronize(s));
}

// ---------------------------------------------------------------------------
// gs_scan_tiles_static: the same scan with its scratch in a file-scope
// device array instead of a caller buffer, for callers that cannot allocate.
// The scratch holds the per-block sums and depth ranges (16 bytes per block
// of kScanTile Gaussians); the reduce pass writes every entry the later
// passes read, so nothing has to start at zero.  With an order the counts are
// gathered through it in both passes (the caller-scratch variant stages the
// gathered counts in its scratch instead).

constexpr int32_t kStaticScanMaxPoints = 1 << 26;  // 64 Mi Gaussians
constexpr size_t kStaticScanScratchBytes =
    (((size_t)kStaticScanMaxPoints / gs::kScanTile) * 2 * sizeof(long long) + 255) & ~(size_t)255;  // 256 KiB

static __device__ __align__(256) unsigned char scratch[kStaticScanScratchBytes];

// Device address of `scratch` on each device, looked up once per device with
// that device current (the host-side symbol is not a device address).
constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mutex;
static void* g_scratch_ptr[kMaxScratchDevices] = {};

static int static_scan_scratch(hipStream_t s, void** out) {
  int dev = 0;
  hipError_t e = s ? hipStreamGetDevice(s, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxScratchDevices) return GS_ERR_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    int current = 0;
    e = hipGetDevice(&current);
    if (e != hipSuccess) return (int)e;
    if (current != dev && (e = hipSetDevice(dev)) != hipSuccess) return (int)e;
    void* p = nullptr;
    const hipError_t lookup = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (current != dev && (e = hipSetDevice(current)) != hipSuccess) return (int)e;
    if (lookup != hipSuccess) return (int)lookup;
    if (p == nullptr) return GS_ERR_INVALID_ARGUMENT;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return GS_OK;
}

extern "C" int32_t gs_scan_tiles_static_max_points(void) { return kStaticScanMaxPoints; }

extern "C" int gs_scan_tiles_static(int32_t P, const int32_t* tiles_touched, const int32_t* order,
                                    const int32_t* radii, const float* depths, int32_t* offsets, int64_t* info_dev,
                                    void* stream) {
  if (P < 0 || !info_dev) return GS_ERR_INVALID_ARGUMENT;
  if (P > kStaticScanMaxPoints) return GS_ERR_TOO_LARGE;
  hipStream_t s = (hipStream_t)stream;
  if (P == 0) {
    hipLaunchKernelGGL(gs::zero_info_kernel, dim3(1), dim3(64), 0, s, reinterpret_cast<long long*>(info_dev));
    return gs_status_from_hip(hipGetLastError());
  }
  if (!tiles_touched || !offsets || (radii == nullptr) != (depths == nullptr)) return GS_ERR_INVALID_ARGUMENT;
  void* base = nullptr;
  const int st = static_scan_scratch(s, &base);
  if (st != GS_OK) return st;
  const int nb = gs_scan_blocks(P);
  long long* block_sums = static_cast<long long*>(base);
  unsigned long long* block_range = reinterpret_cast<unsigned long long*>(block_sums + nb);
  const int vec = gs_scan_vec(tiles_touched, order, offsets, nullptr);
  hipLaunchKernelGGL(gs::scan_reduce_kernel, dim3(nb), dim3(gs::kScanThreads), 0, s, P, tiles_touched, order,
                     radii, depths, block_sums, block_range, nullptr, vec, nullptr, nullptr);
  hipLaunchKernelGGL(gs::scan_apply_kernel, dim3(nb), dim3(gs::kScanThreads), 0, s, P, nb, tiles_touched, order,
                     block_sums, block_range, offsets, reinterpret_cast<long long*>(info_dev), vec, nullptr);
  return gs_status_from_hip(hipGetLastError());
}

extern "C" int gs_num_rendered_readback(const int64_t* info_dev, int64_t* info_host_pinned, void* stream) {
  if (!info_dev || !info_host_pinned) return GS_ERR_INVALID_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = hipMemcpyAsync(info_host_pinned, info_dev, 2 * sizeof(int64_t), hipMemcpyDeviceToHost, s);
  if (e != hipSuccess) return (int)e;
  return gs_status_from_hip(hipStreamSynchronize(s));
}

extern "C" int gs_duplicate_keys(int32_t P, const int32_t* radii, const float* records,
                                 const float* conic_2d_inv, const int32_t* coverage, const float* depths,
                                 const int32_t* offsets, int32_t image_width,
                                 int32_t image_height, int32_t coverage_mode, int64_t num_rendered,
                                 uint32_t depth_min, int32_t depth_bits, int32_t value_bits, uint64_t* keys_out,
                                 int32_t* values_out, void* stream) {
  if (P < 0 || image_width <= 0 || image_height <= 0 || coverage_mode < 0 || coverage_mode > 2)
    return GS_ERR_INVALID_ARGUMENT;
  if (depth_bits < 0 || depth_bits > 32 || value_bits < 0 || value_bits > 31) return GS_ERR_INVALID_ARGUMENT;
  const int grid_x = (image_width + gs::kBlockX - 1) / gs::kBlockX;
  const int grid_y = (image_height + gs::kBlockY - 1) / gs::kBlockY;
  const int tile_bits = gs_bit_length(grid_x * grid_y - 1);
  if (tile_bits + depth_bits + value_bits > 64) return GS_ERR_INVALID_ARGUMENT;
  if (value_bits > 0 && gs_bit_length(P - 1) > value_bits) return GS_ERR_INVALID_ARGUMENT;
  if (P == 0 || num_rendered <= 0) return GS_OK;
  if (!radii || !records || !conic_2d_inv || !offsets || !keys_out || (value_bits == 0 && !values_out))
    return GS_ERR_INVALID_ARGUMENT;
  if ((reinterpret_cast<uintptr_t>(records) | reinterpret_cast<uintptr_t>(coverage)) & 15) return GS_ERR_MISALIGNED;
  hipLaunchKernelGGL(gs::duplicate_keys_kernel, dim3((P + 255) / 256), dim3(256), 0, (hipStream_t)stream, P,
                     radii, reinterpret_cast<const float4*>(records), conic_2d_inv,
                     reinterpret_cast<const int4*>(coverage), depths, offsets, grid_x, grid_y,
                     coverage_mode, (long long)num_rendered, depth_min, depth_bits, value_bits,
                     reinterpret_cast<unsigned long long*>(keys_out), values_out);
  return gs_status_from_hip(hipGetLastError());
}

// Tile ranges, with the clearing of ranges left out when the caller has
// already cleared them on the stream.
static int tile_ranges_impl(int64_t n, const uint64_t* sorted_keys, int32_t tile_shift, int32_t value_bits,
                            int32_t num_tiles, int32_t* ranges, int32_t* point_list, bool cleared, hipStream_t s) {
  if (n < 0 || num_tiles <= 0 || !ranges) return GS_ERR_INVALID_ARGUMENT;
  if (tile_shift < 0 || tile_shift > 63 || value_bits < 0 || value_bits > 31 || value_bits > tile_shift)
    return GS_ERR_INVALID_ARGUMENT;
  if (n > 0x7fffffffLL) return GS_ERR_OVERFLOW;
  const int n2 = 2 * num_tiles;
  if (!cleared) hipLaunchKernelGGL(gs::zero_ranges_kernel, dim3((n2 + 255) / 256), dim3(256), 0, s, n2, ranges);
  if (n > 0) {
    if (!sorted_keys || (value_bits > 0 && !point_list)) return GS_ERR_INVALID_ARGUMENT;
    const long long threads = (n + gs::kRangeItems - 1) / gs::kRangeItems;
    hipLaunchKernelGGL(gs::tile_ranges_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, (long long)n,
                       reinterpret_cast<const unsigned long long*>(sorted_keys), tile_shift, value_bits, num_tiles,
                       reinterpret_cast<int2*>(ranges), point_list);
  }
  return gs_status_from_hip(hipGetLastError());
}

extern "C" int gs_tile_ranges(int64_t n, const uint64_t* sorted_keys, int32_t tile_shift, int32_t value_bits,
                              int32_t num_tiles, int32_t* ranges, int32_t* point_list, void* stream) {
  return tile_ranges_impl(n, sorted_keys, tile_shift, value_bits, num_tiles, ranges, point_list, false,
                          (hipStream_t)stream);
}

extern "C" int gs_depth_keys(int32_t P, const int32_t* radii, const float* depths, uint32_t* keys_out,
                             int32_t* values_out, void* stream) {
  if (P < 0) return GS_ERR_INVALID_ARGUMENT;
  if (P == 0) return GS_OK;
  if (!radii || !depths || !keys_out || !values_out) return GS_ERR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(gs::depth_keys_kernel, dim3((P + 255) / 256), dim3(256), 0, (hipStream_t)stream, P, radii,
                     depths, keys_out, values_out);
  return gs_status_from_hip(hipGetLastError());
}

extern "C" int gs_duplicate_tiles(int32_t P, const int32_t* order, const int32_t* radii, const float* records,
                                  const float* conic_2d_inv, const int32_t* coverage, const int32_t* offsets,
                                  int32_t image_width,
                                  int32_t image_height, int32_t coverage_mode, int64_t num_rendered,
                                  uint32_t* tiles_out, int32_t* values_out, void* stream) {
  if (P < 0 || image_width <= 0 || image_height <= 0 || coverage_mode < 0 || coverage_mode > 2)
    return GS_ERR_INVALID_ARGUMENT;
  if (P == 0 || num_rendered <= 0) return GS_OK;
  if (!order || !radii || !records || !conic_2d_inv || !offsets || !tiles_out || !values_out)
    return GS_ERR_INVALID_ARGUMENT;
  if ((reinterpret_cast<uintptr_t>(records) | reinterpret_cast<uintptr_t>(coverage)) & 15) return GS_ERR_MISALIGNED;
  const int grid_x = (image_width + gs::kBlockX - 1) / gs::kBlockX;
  const int grid_y = (image_height + gs::kBlockY - 1) / gs::kBlockY;
  hipLaunchKernelGGL(gs::duplicate_tiles_kernel, dim3((P + 255) / 256), dim3(256), 0, (hipStream_t)stream, P, order,
                     radii, reinterpret_cast<const float4*>(records), conic_2d_inv,
                     reinterpret_cast<const int4*>(coverage), offsets, grid_x, grid_y,
                     coverage_mode, (long long)num_rendered, tiles_out, values_out);
  return gs_status_from_hip(hipGetLastError());
}

extern "C" int gs_tile_ranges_u32(int64_t n, const uint32_t* sorted_tiles, int32_t num_tiles, int32_t* ranges,
                                  void* stream) {
  if (n < 0 || num_tiles <= 0 || !ranges) return GS_ERR_INVALID_ARGUMENT;
  if (n > 0x7fffffffLL) return GS_ERR_OVERFLOW;
  hipStream_t s = (hipStream_t)stream;
  const int n2 = 2 * num_tiles;
  hipLaunchKernelGGL(gs::zero_ranges_kernel, dim3((n2 + 255) / 256), dim3(256), 0, s, n2, ranges);
  if (n > 0) {
    if (!sorted_tiles) return GS_ERR_INVALID_ARGUMENT;
    const long long threads = (n + gs::kRangeItems - 1) / gs::kRangeItems;
    hipLaunchKernelGGL(gs::tile_ranges_u32_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s,
                       (long long)n, sorted_tiles, num_tiles, reinterpret_cast<int2*>(ranges));
  }
  return gs_status_from_hip(hipGetLastError());
}

// Packed-key binning after the pair count is known, as one host call so that
// its launches follow each other without host round trips: emission, the
// stable sort on the tile field, tile ranges and the per-tile depth sort.
static inline size_t gs_align256(size_t b) { return (b + 255) & ~(size_t)255; }

extern "C" size_t gs_bin_packed_workspace_bytes(int64_t num_rendered) {
  if (num_rendered <= 0) return 0;
  return 2 * gs_align256((size_t)num_rendered * sizeof(uint64_t)) + gs_align256(gs_sort_scratch_bytes(num_rendered));
}

static int bin_packed_impl(int32_t P, const int32_t* radii, const float* records, const float* conic_2d_inv,
                           const int32_t* coverage, const float* depths, const int32_t* offsets, int32_t image_width,
                           int32_t image_height, int32_t coverage_mode, int64_t num_rendered, uint32_t depth_min,
                           int32_t depth_bits, int32_t value_bits, void* workspace, size_t workspace_bytes,
                           int32_t* ranges, int32_t* point_list, uint64_t* sorted_keys_out,
                           void* const* stage_events, void* stream, bool ranges_cleared) {
  if (P < 0 || num_rendered < 0 || image_width <= 0 || image_height <= 0 || value_bits < 1 || value_bits > 31 ||
      depth_bits < 0 || depth_bits > 32)
    return GS_ERR_INVALID_ARGUMENT;
  if (num_rendered > 0x7fffffffLL) return GS_ERR_OVERFLOW;
  const int grid_x = (image_width + gs::kBlockX - 1) / gs::kBlockX;
  const int grid_y = (image_height + gs::kBlockY - 1) / gs::kBlockY;
  const int num_tiles = grid_x * grid_y;
  const int tile_bits = gs_bit_length(num_tiles - 1);
  const int tile_shift = depth_bits + value_bits;
  if (tile_shift + tile_bits > 64) return GS_ERR_INVALID_ARGUMENT;
  if (!ranges) return GS_ERR_INVALID_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  if (num_rendered == 0)
    return tile_ranges_impl(0, nullptr, tile_shift, 0, num_tiles, ranges, nullptr, ranges_cleared, s);
  if (!workspace || !point_list) return GS_ERR_INVALID_ARGUMENT;
  if (workspace_bytes < gs_bin_packed_workspace_bytes(num_rendered)) return GS_ERR_SCRATCH_TOO_SMALL;
  const size_t key_bytes = gs_align256((size_t)num_rendered * sizeof(uint64_t));
  uint64_t* keys = reinterpret_cast<uint64_t*>(workspace);
  uint64_t* keys_alt = reinterpret_cast<uint64_t*>(reinterpret_cast<char*>(workspace) + key_bytes);
  void* scratch = reinterpret_cast<char*>(workspace) + 2 * key_bytes;
  const size_t scratch_bytes = workspace_bytes - 2 * key_bytes;
  // Optional profiling: events recorded before emission and after each stage.
  auto mark = [&](int k) {
    if (stage_events) (void)hipEventRecord((hipEvent_t)stage_events[k], s);
  };
  mark(0);
  int st = gs_duplicate_keys(P, radii, records, conic_2d_inv, coverage, depths, offsets, image_width, image_height,
                             coverage_mode, num_rendered, depth_min, depth_bits, value_bits, keys, nullptr, stream);
  if (st != GS_OK) return st;
  mark(1);
  st = gs_sort_keys_u64(num_rendered, tile_shift, tile_bits, keys, keys_alt, scratch, scratch_bytes, stream);
  if (st != GS_OK) return st;
  mark(2);
  if (gs_sort_num_passes(tile_bits) % 2) {
    uint64_t* t = keys;
    keys = keys_alt;
    keys_alt = t;
  }
  st = tile_ranges_impl(num_rendered, keys, tile_shift, 0, num_tiles, ranges, nullptr, ranges_cleared, s);
  if (st != GS_OK) return st;
  mark(3);
  st = gs_sort_tile_segments(num_rendered, keys, keys_alt, num_tiles, ranges, value_bits, depth_bits, value_bits,
                             point_list, sorted_keys_out != nullptr, stream);
  if (st != GS_OK) return st;
  mark(4);
  if (sorted_keys_out) {
    const hipError_t e = hipMemcpyAsync(sorted_keys_out, keys, (size_t)num_rendered * sizeof(uint64_t),
                                        hipMemcpyDeviceToDevice, s);
    if (e != hipSuccess) return (int)e;
  }
  return GS_OK;
}

extern "C" int gs_bin_packed(int32_t P, const int32_t* radii, const float* records, const float* conic_2d_inv,
                             const int32_t* coverage, const float* depths, const int32_t* offsets,
                             int32_t image_width,
                             int32_t image_height,
                             int32_t coverage_mode, int64_t num_rendered, uint32_t depth_min, int32_t depth_bits,
                             int32_t value_bits, void* workspace, size_t workspace_bytes, int32_t* ranges,
                             int32_t* point_list, uint64_t* sorted_keys_out, void* const* stage_events,
                             void* stream) {
  return bin_packed_impl(P, radii, records, conic_2d_inv, coverage, depths, offsets, image_width, image_height,
                         coverage_mode, num_rendered, depth_min, depth_bits, value_bits, workspace, workspace_bytes,
                         ranges, point_list, sorted_keys_out, stage_events, stream, false);
}

// The forward's read-back of the pair count followed, without returning to the
// caller, by the packed-key binning into buffers the caller allocated for up to
// `capacity` pairs before the count was known.  The key layout and the
// dataflow are the caller's rules (key_layout and the default sort mode):
//   tile_bits = bit length of T - 1, depth_bits = bit length of the visible
//   depth-bit range, value_bits = max(1, bit length of P - 1), and the packed
//   dataflow applies when the three fit in 64 bits and, if max_pairs_per_point
//   > 0, num_rendered <= max_pairs_per_point * P.
// result[0] = num_rendered, result[1] = depth_min, result[2] = depth_bits,
// result[3] = value_bits, result[4] = 1 if the binning was launched, 0 if the
// caller must bin itself (count outside [0, 2^31 - 1], over capacity, or
// another dataflow), result[5] = 1 if the standard forward render was
// launched too (out_color given).
extern "C" int gs_readback_bin_packed(const int64_t* info_dev, int64_t* info_host_pinned, int32_t P,
                                      const int32_t* radii, const float* records, const float* conic_2d_inv,
                                      const int32_t* coverage, const float* depths, const int32_t* offsets,
                                      int32_t image_width, int32_t image_height,
                                      int32_t coverage_mode, int32_t max_pairs_per_point, int64_t capacity,
                                      void* workspace, size_t workspace_bytes, int32_t* ranges, int32_t* point_list,
                                      const float* background, int32_t compute_depth, float* out_color,
                                      float* out_depth, float* out_alpha, int32_t* n_contrib,
                                      void* const* stage_events, int64_t* result, void* stream) {
  if (!result || P < 0 || capacity < 0 || image_width <= 0 || image_height <= 0) return GS_ERR_INVALID_ARGUMENT;
  // The ranges are cleared before the read-back, while the stream would
  // otherwise wait for the host.
  const bool clear_first = ranges != nullptr && capacity > 0;
  if (clear_first) {
    const int n2 =
        2 * ((image_width + gs::kBlockX - 1) / gs::kBlockX) * ((image_height + gs::kBlockY - 1) / gs::kBlockY);
    hipLaunchKernelGGL(gs::zero_ranges_kernel, dim3((n2 + 255) / 256), dim3(256), 0, (hipStream_t)stream, n2, ranges);
  }
  int st = gs_num_rendered_readback(info_dev, info_host_pinned, stream);
  if (st != GS_OK) return st;
  const int64_t R = info_host_pinned[0];
  const uint64_t range = (uint64_t)info_host_pinned[1];
  const uint32_t depth_min = (uint32_t)(range & 0xFFFFFFFFull);
  const uint32_t depth_max = (uint32_t)(range >> 32);
  const int depth_bits = depth_max >= depth_min ? gs_bit_length((long long)(depth_max - depth_min)) : 0;
  int value_bits = gs_bit_length((long long)P - 1);
  if (value_bits < 1) value_bits = 1;
  const int grid_x = (image_width + gs::kBlockX - 1) / gs::kBlockX;
  const int grid_y = (image_height + gs::kBlockY - 1) / gs::kBlockY;
  const int tile_bits = gs_bit_length((long long)grid_x * grid_y - 1);
  result[0] = R;
  result[1] = depth_min;
  result[2] = depth_bits;
  result[3] = value_bits;
  result[4] = 0;
  result[5] = 0;
  if (R <= 0 || R > 0x7fffffffLL || R > capacity) return GS_OK;
  if (tile_bits + depth_bits + value_bits > 64 || value_bits > 31) return GS_OK;
  if (max_pairs_per_point > 0 && R > (int64_t)max_pairs_per_point * P) return GS_OK;
  st = bin_packed_impl(P, radii, records, conic_2d_inv, coverage, depths, offsets, image_width, image_height,
                       coverage_mode, R, depth_min, depth_bits, value_bits, workspace, workspace_bytes, ranges,
                       point_list, nullptr, stage_events, stream, clear_first);
  if (st != GS_OK) return st;
  result[4] = 1;
  if (out_color) {
    st = gs_render_fwd(image_width, image_height, P, R, ranges, point_list, records, background, compute_depth,
                       out_color, out_depth, out_alpha, n_contrib, stream);
    if (st != GS_OK) return st;
    if (stage_events) (void)hipEventRecord((hipEvent_t)stage_events[5], (hipStream_t)stream);
    result[5] = 1;
  }
  return GS_OK;
}
