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
#include <atomic>
#include <cstring>
#include <mutex>
#include <sched.h>

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

// All kScanTile elements of the block at `base` (thread t: elements 4t ..
// 4t + 3 of each chunk), gathered through order when there is one.  A full
// block with 16-byte aligned arrays (the block-uniform common case) issues
// its vector loads (and then its gathers) without a branch between them, so
// they are all in flight together; the last, partial block takes
// scan_load4 per chunk.
__device__ __forceinline__ void scan_load_block(const int* __restrict__ in, const int* __restrict__ order,
                                                long long base, long long n, bool vec, int (&v)[4][4],
                                                int (&src)[4][4]) {
  if (vec && base + kScanTile <= n) {
    int4 x[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      x[k] = *reinterpret_cast<const int4*>((order ? order : in) + base + k * kScanChunk + 4 * threadIdx.x);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int i0 = (int)(base + k * kScanChunk + 4 * threadIdx.x);
      if (order) {
        src[k][0] = x[k].x; src[k][1] = x[k].y; src[k][2] = x[k].z; src[k][3] = x[k].w;
      } else {
        src[k][0] = i0; src[k][1] = i0 + 1; src[k][2] = i0 + 2; src[k][3] = i0 + 3;
        v[k][0] = x[k].x; v[k][1] = x[k].y; v[k][2] = x[k].z; v[k][3] = x[k].w;
      }
    }
    if (order) {
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j) v[k][j] = in[src[k][j]];
    }
    return;
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) scan_load4(in, order, base + k * kScanChunk + 4 * threadIdx.x, n, vec, v[k], src[k]);
}

// Per block: the tile-count sum, and the smallest and largest depth bits of
// the Gaussians with radius > 0 (min ~0u / max 0 when there are none), packed
// as max << 32 | min.  With an order, the counts are gathered through it and
// also stored contiguously in `gathered` (when given), so that the apply pass
// reads them without a second gather.  With coverage it also stores the
// block's super-tile units of valid cover words (-1 when a Gaussian with
// tiles has no valid word) and its valid words in block_ev.  Every load of
// the block is issued before any is used (the radii and depths as 16-byte
// vectors on the identity order, vec_rd), and the block's totals take one
// barrier.
__global__ __launch_bounds__(kScanThreads) void scan_reduce_kernel(int n, const int* __restrict__ in,
                                                                  const int* __restrict__ order,
                                                                  const int* __restrict__ radii,
                                                                  const float* __restrict__ depths,
                                                                  long long* __restrict__ block_sums,
                                                                  unsigned long long* __restrict__ block_range,
                                                                  int* __restrict__ gathered, int vec, int vec_rd,
                                                                  const int4* __restrict__ coverage,
                                                                  long long* __restrict__ block_ev) {
  constexpr int kWaves = kScanThreads / 64;
  __shared__ long long s_sum[kWaves], s_units[kWaves];
  __shared__ int s_valid[kWaves], s_bad[kWaves];
  __shared__ unsigned s_min[kWaves], s_max[kWaves];
  const long long base = (long long)blockIdx.x * kScanTile;
  int v[4][4], src[4][4];
  scan_load_block(in, order, base, n, vec != 0, v, src);
  int r[4][4];
  float d[4][4];
  if (radii) {
    if (vec_rd && base + kScanTile <= n) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const long long i0 = base + k * kScanChunk + 4 * threadIdx.x;
        const int4 r4 = *reinterpret_cast<const int4*>(radii + i0);
        const float4 d4 = *reinterpret_cast<const float4*>(depths + i0);
        r[k][0] = r4.x; r[k][1] = r4.y; r[k][2] = r4.z; r[k][3] = r4.w;
        d[k][0] = d4.x; d[k][1] = d4.y; d[k][2] = d4.z; d[k][3] = d4.w;
      }
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          r[k][j] = src[k][j] >= 0 ? radii[src[k][j]] : 0;
          d[k][j] = src[k][j] >= 0 ? depths[src[k][j]] : 0.0f;
        }
    }
  }
  long long s = 0;
  unsigned dmin = ~0u, dmax = 0u;
  long long units = 0;
  int valid = 0, bad = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const long long i0 = base + k * kScanChunk + 4 * threadIdx.x;
    if (coverage) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (i0 + j < n) {
          const CoverWord w = unpack_cover(coverage[i0 + j]);
          units += super_units(w);
          valid += w.valid;
          bad |= (v[k][j] > 0 && !w.valid) ? 1 : 0;
        }
      }
    }
    if (gathered) {
      if (vec && i0 + 3 < n) {
        *reinterpret_cast<int4*>(gathered + i0) = make_int4(v[k][0], v[k][1], v[k][2], v[k][3]);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (i0 + j < n) gathered[i0 + j] = v[k][j];
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      s += v[k][j];
      if (radii && r[k][j] > 0) {
        const unsigned bits = __float_as_uint(d[k][j]);
        dmin = bits < dmin ? bits : dmin;
        dmax = bits > dmax ? bits : dmax;
      }
    }
  }
  s = wave_sum_i64(s);
  dmin = wave_min_u32(dmin);
  dmax = wave_max_u32(dmax);
  if (coverage) {
    units = wave_sum_i64(units);
    valid = (int)wave_sum_i64(valid);
    bad = (int)wave_sum_i64(bad);
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s_sum[wave] = s;
    s_min[wave] = dmin;
    s_max[wave] = dmax;
    s_units[wave] = units;
    s_valid[wave] = valid;
    s_bad[wave] = bad;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    long long total = 0, units_total = 0, valid_total = 0, bad_total = 0;
    unsigned mn = ~0u, mx = 0u;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      total += s_sum[w];
      mn = s_min[w] < mn ? s_min[w] : mn;
      mx = s_max[w] > mx ? s_max[w] : mx;
      units_total += s_units[w];
      valid_total += s_valid[w];
      bad_total += s_bad[w];
    }
    block_sums[blockIdx.x] = total;
    block_range[blockIdx.x] = ((unsigned long long)mx << 32) | mn;
    if (coverage) {
      block_ev[2 * blockIdx.x] = bad_total > 0 ? -1 : units_total;
      block_ev[2 * blockIdx.x + 1] = valid_total;
    }
  }
}

// Inclusive prefix sums of the block's elements: its offset is the sum of the
// preceding blocks' sums (each block adds them up itself, so no pass runs
// between the two).  The block's elements are loaded first; each thread's
// four chunks are scanned by one wave scan each and one exchange of the
// waves' chunk totals (the chunk sums fit int32 whenever the offsets do).
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
  constexpr int kWaves = kScanThreads / 64;
  __shared__ long long s_pre[kWaves];
  __shared__ int s_tot[kWaves][4];
  __shared__ long long s_units[kWaves], s_valid[kWaves];
  __shared__ int s_bad[kWaves];
  __shared__ unsigned s_min[kWaves], s_max[kWaves];
  const int b = blockIdx.x;
  const long long base = (long long)b * kScanTile;
  int v[4][4], src[4][4];
  scan_load_block(in, order, base, n, vec != 0, v, src);
  long long pre = 0;
  for (int j = threadIdx.x; j < b; j += kScanThreads) pre += block_sums[j];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int t[4], inc[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    v[k][1] += v[k][0];
    v[k][2] += v[k][1];
    v[k][3] += v[k][2];
    t[k] = v[k][3];
    inc[k] = wave_scan_add_dpp(t[k]);
  }
  pre = wave_sum_i64(pre);
  if (lane == 63) {
#pragma unroll
    for (int k = 0; k < 4; ++k) s_tot[wave][k] = inc[k];
  }
  if (lane == 0) s_pre[wave] = pre;
  __syncthreads();
  long long pre_total = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) pre_total += s_pre[w];
  long long run = pre_total;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const long long i0 = base + k * kScanChunk + 4 * threadIdx.x;
    int before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const int x = s_tot[w][k];
      all += x;
      before += w < wave ? x : 0;
    }
    const long long off = run + before + (inc[k] - t[k]);
    if (vec && i0 + 3 < n) {
      *reinterpret_cast<int4*>(out + i0) =
          make_int4((int)(off + v[k][0]), (int)(off + v[k][1]), (int)(off + v[k][2]), (int)(off + v[k][3]));
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (i0 + j < n) out[i0 + j] = (int)(off + v[k][j]);
    }
    run += all;
  }
  if (b != nb - 1) return;
  // The last block: the pair total, the visible depth range and the sizes of
  // the bucketed binning.
  unsigned dmin = ~0u, dmax = 0u;
  long long units = 0, valid = 0;
  int bad = 0;
  for (int j = threadIdx.x; j < nb; j += kScanThreads) {
    const unsigned long long r = block_range[j];
    const unsigned mn = (unsigned)r, mx = (unsigned)(r >> 32);
    dmin = mn < dmin ? mn : dmin;
    dmax = mx > dmax ? mx : dmax;
    if (block_ev) {
      const long long u = block_ev[2 * j];
      bad |= u < 0 ? 1 : 0;
      units += u < 0 ? 0 : u;
      valid += block_ev[2 * j + 1];
    }
  }
  dmin = wave_min_u32(dmin);
  dmax = wave_max_u32(dmax);
  units = wave_sum_i64(units);
  valid = wave_sum_i64(valid);
  bad = (int)wave_sum_i64(bad);
  if (lane == 0) {
    s_min[wave] = dmin;
    s_max[wave] = dmax;
    s_units[wave] = units;
    s_valid[wave] = valid;
    s_bad[wave] = bad;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned mn = ~0u, mx = 0u;
    long long units_total = 0, valid_total = 0;
    int bad_total = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      mn = s_min[w] < mn ? s_min[w] : mn;
      mx = s_max[w] > mx ? s_max[w] : mx;
      units_total += s_units[w];
      valid_total += s_valid[w];
      bad_total += s_bad[w];
    }
    info[0] = pre_total + block_sums[b];
    info[1] = mx >= mn ? (long long)(((unsigned long long)mx << 32) | mn) : 0;
    if (block_ev) {
      info[2] = bad_total > 0 ? -1 : units_total;
      info[3] = valid_total;
    }
  }
}

// ---------------------------------------------------------------------------
// One-pass scan (decoupled look-back) in point order.  Its state holds the
// per-256-Gaussian aggregates of store_scan_aggregates (kScanAggWords words
// each; depth range, super-tile units, valid cover words), which the
// preprocess (or gs_scan_state_prepare) writes, then per block of kScanTile
// counts a status word (flag in the top two bits: 0 unpublished, kStatusAgg
// the block's own sum, kStatusIncl the sum of all counts up to its end; value
// in the low 62 bits) and kPublishedWords published words (kPublished |
// value: the block's depth range as two words, its units (-1 when a Gaussian
// with tiles has no valid cover word), its valid words), which must hold
// zeros when the kernel starts (the same writer clears them).  Each block
// loads its counts and its 16 aggregates once, publishes its sum and its
// aggregates, walks back over the preceding status words 256 at a time,
// adding sums up to the nearest inclusive word, and stores its inclusive
// word before writing its offsets.  Every word is published on its own (no
// store waits for another) and crosses blocks through coherent (agent-scope
// atomic) accesses (a release store would write back the whole L2 of the
// XCD).  Block nb - 1 stores the pair total in info[0] and, once every
// block's words are published, totals info[1..3].  Blocks start in index
// order, so every word a block waits for belongs to a block that is running
// or done; each wait is nevertheless bounded by spin_limit sleeps: a block
// whose look-back times out adds up the counts before it directly (slow,
// same offsets), and a final wait that times out stores the widest depth
// range (every positive float) and no sizes (info[2] = -1, info[3] = 0),
// which the callers treat as a Gaussian without a valid cover word.
constexpr unsigned long long kStatusAgg = 1ull << 62;
constexpr unsigned long long kStatusIncl = 2ull << 62;
constexpr unsigned long long kStatusValue = (1ull << 62) - 1;
constexpr unsigned long long kPublished = 1ull << 63;
constexpr int kPublishedWords = 4;
constexpr int kAggPerBlock = kScanTile / kScanAggGaussians;  // 16
static_assert(kAggPerBlock <= 64, "one lane per aggregate");

// A published word holds a value in [-2^62, 2^62) below its flag bit.
__device__ __forceinline__ unsigned long long publish(long long v) {
  return kPublished | ((unsigned long long)v & ~kPublished);
}

__device__ __forceinline__ long long published_value(unsigned long long w) {
  return (long long)(w << 1) >> 1;  // sign-extends bit 62
}

// Agent-scope relaxed atomic accesses: coherent across the XCDs' L2s.
__device__ __forceinline__ unsigned long long status_load(const unsigned long long* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void status_store(unsigned long long* p, unsigned long long v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned long long wave_sum_u64(unsigned long long v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Aggregates of 256 consecutive Gaussians for the one-pass scan (the
// preprocess writes the same from its registers), and the cleared status and
// published words (fewer than this grid's threads).
__global__ __launch_bounds__(kScanAggGaussians) void scan_prepare_kernel(int n, const int* __restrict__ tiles,
                                                                        const int* __restrict__ radii,
                                                                        const float* __restrict__ depths,
                                                                        const int4* __restrict__ coverage,
                                                                        unsigned long long* agg,
                                                                        unsigned long long* status,
                                                                        int clear_words) {
  __shared__ ScanAggLds s_agg;
  const int i = blockIdx.x * kScanAggGaussians + threadIdx.x;
  if (i < clear_words) status[i] = 0ull;
  const bool in_range = i < n;
  bool visible = false;
  float depth = 0.0f;
  int units = 0, valid = 0, bad = 0;
  if (in_range) {
    visible = radii != nullptr && radii[i] > 0;
    depth = visible ? depths[i] : 0.0f;
    if (coverage) {
      const CoverWord w = unpack_cover(coverage[i]);
      units = super_units(w);
      valid = w.valid;
      bad = (tiles[i] > 0 && !w.valid) ? 1 : 0;
    }
  }
  store_scan_aggregates(visible, depth, units, valid, bad, s_agg, agg);
}

__global__ __launch_bounds__(kScanThreads) void scan_onepass_kernel(int n, int nb, const int* __restrict__ in,
                                                                   const unsigned long long* __restrict__ agg,
                                                                   int n_agg, int sized,
                                                                   unsigned long long* status,
                                                                   unsigned long long* pub, int* __restrict__ out,
                                                                   long long* __restrict__ info, int vec,
                                                                   int spin_limit) {
  constexpr int kWaves = kScanThreads / 64;
  __shared__ int s_tot[kWaves][4];
  __shared__ long long s_sum[kWaves], s_units[kWaves], s_valid[kWaves];
  __shared__ int s_bad[kWaves];
  __shared__ unsigned s_min[kWaves], s_max[kWaves];
  __shared__ unsigned long long s_incl[kWaves], s_ready[kWaves], s_part[kWaves];
  const int b = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const long long base = (long long)b * kScanTile;
  int v[4][4], src[4][4];
  scan_load_block(in, nullptr, base, n, vec != 0, v, src);
  // lane l < kAggPerBlock of the first wave: the block's aggregate l
  const int ai = b * kAggPerBlock + lane;
  const bool has_agg = wave == 0 && lane < kAggPerBlock && ai < n_agg;
  unsigned long long g0 = 0, g1 = 0, g2 = 0;
  if (has_agg) {
    g0 = agg[kScanAggWords * ai];
    g1 = agg[kScanAggWords * ai + 1];
    g2 = agg[kScanAggWords * ai + 2];
  }
  long long s = 0;
  int t[4], inc[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
#pragma unroll
    for (int j = 0; j < 4; ++j) s += v[k][j];
    v[k][1] += v[k][0];
    v[k][2] += v[k][1];
    v[k][3] += v[k][2];
    t[k] = v[k][3];
    inc[k] = wave_scan_add_dpp(t[k]);
  }
  s = wave_sum_i64(s);
  if (lane == 63) {
#pragma unroll
    for (int k = 0; k < 4; ++k) s_tot[wave][k] = inc[k];
  }
  if (lane == 0) s_sum[wave] = s;
  __syncthreads();
  long long total = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) total += s_sum[w];
  if (wave == 0) {
    const unsigned lo = wave_min_u32(has_agg ? (unsigned)g0 : ~0u);
    const unsigned hi = wave_max_u32(has_agg ? (unsigned)(g0 >> 32) : 0u);
    const long long units = wave_sum_i64(has_agg && (long long)g1 >= 0 ? (long long)g1 : 0);
    const long long bad = wave_sum_i64(has_agg && (long long)g1 < 0 ? 1 : 0);
    const long long valid = wave_sum_i64(has_agg ? (long long)g2 : 0);
    if (lane == 0) {
      status_store(status + b, (b == 0 ? kStatusIncl : kStatusAgg) | ((unsigned long long)total & kStatusValue));
      unsigned long long* q = pub + kPublishedWords * b;
      status_store(q, publish(lo));
      status_store(q + 1, publish(hi));
      status_store(q + 2, publish(bad ? -1 : units));
      status_store(q + 3, publish(valid));
    }
  }
  // Look-back by the whole block, 256 preceding words per round (thread t:
  // block j - t), adding sums up to the nearest inclusive word.  Every
  // decision is block-uniform (taken from the waves' ballots in LDS).
  unsigned long long prefix = 0;
  if (b > 0) {
    int j = b - 1, spins = 0;
    bool timed_out = false;
    while (true) {
      const int idx = j - (int)threadIdx.x;
      const unsigned long long w = idx >= 0 ? status_load(status + idx) : kStatusIncl;
      const unsigned long long flag = w & ~kStatusValue;
      const uint64_t incl = __ballot(flag == kStatusIncl);
      const uint64_t ready = __ballot(flag != 0);
      if (lane == 0) {
        s_incl[wave] = incl;
        s_ready[wave] = ready;
      }
      __syncthreads();
      // first: the thread of the nearest inclusive word (kScanThreads: none
      // in this window); every word up to it must be published
      int first = kScanThreads;
      bool all_ready = true;
#pragma unroll
      for (int q = 0; q < kWaves; ++q) {
        const uint64_t iq = s_incl[q], rq = s_ready[q];
        if (first < kScanThreads) continue;
        if (iq != 0) {
          const int f = __builtin_ctzll(iq);
          const uint64_t need = f == 63 ? ~0ull : ((2ull << f) - 1);
          all_ready = all_ready && (rq & need) == need;
          first = q * 64 + f;
        } else {
          all_ready = all_ready && rq == ~0ull;
        }
      }
      if (!all_ready) {
        __syncthreads();  // every thread has read the ballots before they are rewritten
        if (++spins > spin_limit) {
          timed_out = true;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
        continue;
      }
      const unsigned long long part = wave_sum_u64((int)threadIdx.x <= first ? (w & kStatusValue) : 0ull);
      if (lane == 0) s_part[wave] = part;
      __syncthreads();
#pragma unroll
      for (int q = 0; q < kWaves; ++q) prefix += s_part[q];
      const bool found = first < kScanThreads;
      __syncthreads();  // s_part and the ballots are read before the next round rewrites them
      if (found) break;
      j -= kScanThreads;
    }
    if (timed_out) {
      // the counts before the block, added up by the block (four loads in
      // flight per thread)
      long long a0 = 0, a1 = 0, a2 = 0, a3 = 0;
      long long i = threadIdx.x;
      for (; i + 3 * kScanThreads < base; i += 4 * kScanThreads) {
        a0 += in[i];
        a1 += in[i + kScanThreads];
        a2 += in[i + 2 * kScanThreads];
        a3 += in[i + 3 * kScanThreads];
      }
      for (; i < base; i += kScanThreads) a0 += in[i];
      const long long direct = wave_sum_i64((a0 + a1) + (a2 + a3));
      if (lane == 0) s_part[wave] = (unsigned long long)direct;
      __syncthreads();
      prefix = 0;
#pragma unroll
      for (int q = 0; q < kWaves; ++q) prefix += s_part[q];
    }
    if (threadIdx.x == 0) status_store(status + b, kStatusIncl | ((prefix + (unsigned long long)total) & kStatusValue));
  }
  long long run = (long long)prefix;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const long long i0 = base + k * kScanChunk + 4 * threadIdx.x;
    int before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const int x = s_tot[w][k];
      all += x;
      before += w < wave ? x : 0;
    }
    const long long off = run + before + (inc[k] - t[k]);
    if (vec && i0 + 3 < n) {
      *reinterpret_cast<int4*>(out + i0) =
          make_int4((int)(off + v[k][0]), (int)(off + v[k][1]), (int)(off + v[k][2]), (int)(off + v[k][3]));
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (i0 + j < n) out[i0 + j] = (int)(off + v[k][j]);
    }
    run += all;
  }
  if (b != nb - 1) return;
  // Block nb - 1: the pair total, and every block's published words.
  int spins = 0;
  bool timed_out = false;
  unsigned mn = ~0u, mx = 0u;
  long long units = 0, valid = 0;
  int bad = 0;
  while (true) {
    int ready = 1;
    mn = ~0u;
    mx = 0u;
    units = valid = 0;
    bad = 0;
    // four blocks' words per thread in flight at once
    for (int i0 = threadIdx.x; i0 < nb; i0 += 4 * kScanThreads) {
      unsigned long long w[4][kPublishedWords];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int idx = i0 + r * kScanThreads;
#pragma unroll
        for (int c = 0; c < kPublishedWords; ++c)
          w[r][c] = idx < nb ? status_load(pub + kPublishedWords * idx + c) : kPublished | 0xffffffffull;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (i0 + r * kScanThreads >= nb) continue;
        ready &= ((w[r][0] & w[r][1] & w[r][2] & w[r][3]) & kPublished) != 0 ? 1 : 0;
        const unsigned lo = (unsigned)published_value(w[r][0]), hi = (unsigned)published_value(w[r][1]);
        mn = lo < mn ? lo : mn;
        mx = hi > mx ? hi : mx;
        const long long u = published_value(w[r][2]);
        bad |= u < 0 ? 1 : 0;
        units += u < 0 ? 0 : u;
        valid += published_value(w[r][3]);
      }
    }
    if (__syncthreads_and(ready)) break;
    if (++spins > spin_limit) {
      timed_out = true;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  mn = wave_min_u32(mn);
  mx = wave_max_u32(mx);
  units = wave_sum_i64(units);
  valid = wave_sum_i64(valid);
  bad = (int)wave_sum_i64(bad);
  if (lane == 0) {
    s_min[wave] = mn;
    s_max[wave] = mx;
    s_units[wave] = units;
    s_valid[wave] = valid;
    s_bad[wave] = bad;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned lo = ~0u, hi = 0u;
    long long units_all = 0, valid_all = 0;
    int bad_all = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      lo = s_min[w] < lo ? s_min[w] : lo;
      hi = s_max[w] > hi ? s_max[w] : hi;
      units_all += s_units[w];
      valid_all += s_valid[w];
      bad_all |= s_bad[w];
    }
    info[0] = (long long)(prefix + (unsigned long long)total);
    if (timed_out) {
      info[1] = (long long)(((unsigned long long)0x7f7fffffu << 32) | 0u);
      if (sized) {
        info[2] = -1;
        info[3] = 0;
      }
    } else {
      info[1] = hi >= lo ? (long long)(((unsigned long long)hi << 32) | lo) : 0;
      if (sized) {
        info[2] = bad_all ? -1 : units_all;
        info[3] = valid_all;
      }
    }
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
                                                            int* __restrict__ values,
                                                            const long long* __restrict__ dev_info,
                                                            int* __restrict__ clear, int clear_count) {
  // clear: an int array the grid sets to 0 on the way (the tile ranges of the
  // binning that follows), clear_count ints.
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < clear_count; i += gridDim.x * blockDim.x) clear[i] = 0;
  // With dev_info (the scan's pair count and visible depth range) the key
  // layout is taken from device memory, as the host would compute it after
  // reading the same words back: depth_min the range's low bits, depth_bits
  // the bit length of the range's width, at most dev_info[0] keys.  A layout
  // wider than 64 bits, which the host declines, writes nothing.
  if (dev_info) {
    const unsigned long long range = (unsigned long long)dev_info[1];
    const unsigned dmin = (unsigned)range, dmax = (unsigned)(range >> 32);
    depth_min = dmin;
    depth_bits = dmax >= dmin ? 32 - __clz((int)(dmax - dmin)) : 0;
    limit = dev_info[0] < limit ? dev_info[0] : limit;
    const int tile_bits = 32 - __clz(grid_x * grid_y - 1);
    if (depth_bits + value_bits + tile_bits > 64) limit = 0;
  }
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  // The Gaussian's radius, offsets and cover word are loaded together (index
  // clamped, no branch between them), so the wave waits for memory once
  // before the cover word decides which further words it needs.
  const int ic = imin(idx, P - 1);
  const int radius_in = radii[ic];
  const int off_prev = offsets[imax(ic - 1, 0)];
  const int off_cur = offsets[ic];
  const int4 cover_in = coverage ? coverage[ic] : make_int4(0, 0, 0, 0);
  const int radius = idx < P ? radius_in : 0;
  const bool active = radius > 0;
  long long off = 0;
  int count = 0;
  float4 r0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), r1 = r0;
  float cov_aa = 0.0f, cov_cc = 0.0f;
  int4 cover_w = make_int4(0, 0, 0, 0);
  unsigned long long field = 0;
  if (active) {
    off = idx > 0 ? (long long)off_prev : 0;
    count = (int)((long long)off_cur - off);
    cover_w = cover_in;
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

// Publishes count info words to a slot of coherent pinned host memory and
// then raises the slot's flag (its last word) to seq with a system-scope
// release store, after which the host may read the words.  One wave.
__global__ __launch_bounds__(64) void publish_info_kernel(const int64_t* info, int count, int64_t* slot,
                                                         int flag_word, int64_t seq) {
  const int i = threadIdx.x;
  if (i < count) slot[i] = info[i];
  if (i == 0) __hip_atomic_store(slot + flag_word, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

}  // namespace gs

extern "C" int gs_version(void) { return 10200; }

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

// Radii and depths as 16-byte vectors: the identity order and both arrays
// 16-byte aligned.
static inline int gs_scan_vec_rd(const void* order, const void* radii, const void* depths) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(radii) | reinterpret_cast<uintptr_t>(depths);
  return order == nullptr && radii != nullptr && (a & 15) == 0 ? 1 : 0;
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
                     radii, depths, block_sums, block_range, gathered, vec, gs_scan_vec_rd(order, radii, depths),
                     nullptr, nullptr);
  hipLaunchKernelGGL(gs::scan_apply_kernel, dim3(nb), dim3(gs::kScanThreads), 0, s, P, nb,
                     gathered ? gathered : tiles_touched, nullptr, block_sums, block_range, offsets,
                     reinterpret_cast<long long*>(info_dev), vec, nullptr);
  return gs_status_from_hip(hipGetLastError());
}

// One-pass scan state: the aggregates of every 256 Gaussians, then per block
// of kScanTile counts a status word and the published words (zero when the
// scan starts).
static inline int64_t gs_scan_agg_words(int32_t P) {
  return (int64_t)((P + gs::kScanAggGaussians - 1) / gs::kScanAggGaussians) * gs::kScanAggWords;
}
extern "C" int64_t gs_scan_state_status_offset(int32_t P) { return P <= 0 ? 0 : gs_scan_agg_words(P); }
extern "C" int64_t gs_scan_state_status_words(int32_t P) {
  return P <= 0 ? 0 : (int64_t)gs_scan_blocks(P) * (1 + gs::kPublishedWords);
}
extern "C" size_t gs_scan_state_bytes(int32_t P) {
  return P <= 0 ? 0
                : ((((size_t)gs_scan_agg_words(P) + (size_t)gs_scan_state_status_words(P)) * sizeof(long long) +
                    255) &
                   ~(size_t)255);
}

extern "C" int gs_scan_state_prepare(int32_t P, const int32_t* tiles_touched, const int32_t* radii,
                                     const float* depths, const int32_t* coverage, void* state, size_t state_bytes,
                                     void* stream) {
  if (P < 0) return GS_ERR_INVALID_ARGUMENT;
  if (P == 0) return GS_OK;
  if (!state || (radii == nullptr) != (depths == nullptr) || (coverage != nullptr && tiles_touched == nullptr))
    return GS_ERR_INVALID_ARGUMENT;
  if ((reinterpret_cast<uintptr_t>(coverage) & 15) || (reinterpret_cast<uintptr_t>(state) & 7))
    return GS_ERR_MISALIGNED;
  if (state_bytes < gs_scan_state_bytes(P)) return GS_ERR_SCRATCH_TOO_SMALL;
  unsigned long long* agg = static_cast<unsigned long long*>(state);
  hipLaunchKernelGGL(gs::scan_prepare_kernel, dim3((P + gs::kScanAggGaussians - 1) / gs::kScanAggGaussians),
                     dim3(gs::kScanAggGaussians), 0, (hipStream_t)stream, P, tiles_touched, radii, depths,
                     reinterpret_cast<const int4*>(coverage), agg, agg + gs_scan_agg_words(P),
                     (int)gs_scan_state_status_words(P));
  return gs_status_from_hip(hipGetLastError());
}

extern "C" int gs_scan_tiles_onepass(int32_t P, const int32_t* tiles_touched, int32_t* offsets, int64_t* info_dev,
                                     void* state, size_t state_bytes, int32_t sized, int32_t spin_limit,
                                     void* stream) {
  if (P < 0 || !info_dev || spin_limit < 0) return GS_ERR_INVALID_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  if (P == 0) {
    hipLaunchKernelGGL(gs::zero_info_kernel, dim3(1), dim3(64), 0, s, reinterpret_cast<long long*>(info_dev));
    if (sized)
      hipLaunchKernelGGL(gs::zero_info_kernel, dim3(1), dim3(64), 0, s, reinterpret_cast<long long*>(info_dev) + 2);
    return gs_status_from_hip(hipGetLastError());
  }
  if (!tiles_touched || !offsets || !state) return GS_ERR_INVALID_ARGUMENT;
  if (reinterpret_cast<uintptr_t>(state) & 7) return GS_ERR_MISALIGNED;
  if (state_bytes < gs_scan_state_bytes(P)) return GS_ERR_SCRATCH_TOO_SMALL;
  const int nb = gs_scan_blocks(P);
  unsigned long long* agg = static_cast<unsigned long long*>(state);
  unsigned long long* status = agg + gs_scan_agg_words(P);
  const int vec = gs_scan_vec(tiles_touched, nullptr, offsets, nullptr);
  hipLaunchKernelGGL(gs::scan_onepass_kernel, dim3(nb), dim3(gs::kScanThreads), 0, s, P, nb, tiles_touched, agg,
                     (P + gs::kScanAggGaussians - 1) / gs::kScanAggGaussians, sized ? 1 : 0, status, status + nb,
                     offsets,
                     reinterpret_cast<long long*>(info_dev), vec, spin_limit);
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
                     radii, depths, block_sums, block_range, nullptr, vec, gs_scan_vec_rd(nullptr, radii, depths),
                     reinterpret_cast<const int4*>(coverage), block_ev);
  hipLaunchKernelGGL(gs::scan_apply_kernel, dim3(nb), dim3(gs::kScanThreads), 0, s, P, nb, tiles_touched, nullptr,
                     block_sums, block_range, offsets, reinterpret_cast<long long*>(info_dev), vec, block_ev);
  return gs_status_from_hip(hipGetLastError());
}

// Read-back of a few info words without a device-to-host copy and a blocking
// stream synchronisation.  The caller owns the slot: kReadbackSlotWords int64
// of host memory, the info words first and the flag in the last word, which
// the device can write (coherent pinned memory: hipHostMalloc with
// hipHostMallocPortable | hipHostMallocMapped | hipHostMallocCoherent), and a
// sequence number seq > 0 that the slot's flag does not hold yet (the caller
// counts its uses of the slot).  publish_info_kernel writes the words into
// the slot and raises its flag to seq; the host spins on the flag (acquire
// order, so the words are read after it).  A slot serves one call at a time:
// the words stay in it for the caller to read.  Every 1024 spins the stream
// is polled: an error ends the wait, and a drained stream whose flag is still
// down (a launch that did not run) falls back to a copy.  A slot the device
// cannot address (pageable memory) is filled by a copy and a stream
// synchronisation.  The library keeps no state between calls.  (Publishing
// from a side stream made to wait on the caller's stream with an event was
// tried: the cross-stream wait cost more than the kernel it took off the
// caller's stream.)
namespace {
constexpr int kReadbackSlotWords = 32;  // up to 16 info words; the flag in the last word
constexpr int kReadbackFlagWord = kReadbackSlotWords - 1;

struct ReadbackTicket {
  int64_t* slot = nullptr;
  int64_t seq = 0;
  bool flagged = false;  // publish_info_kernel was launched: wait on the flag
};

// Enqueues the publication of count words at info_dev into slot on s.
int readback_begin(const int64_t* info_dev, int count, int64_t* slot, int64_t seq, hipStream_t s,
                   ReadbackTicket* t) {
  t->slot = slot;
  t->seq = seq;
  t->flagged = false;
  if (seq <= 0 || __atomic_load_n(slot + kReadbackFlagWord, __ATOMIC_ACQUIRE) == seq)
    return GS_ERR_INVALID_ARGUMENT;  // a flag that already holds seq would end the wait at once
  void* dslot = nullptr;
  if (hipHostGetDevicePointer(&dslot, slot, 0) != hipSuccess || dslot == nullptr) {
    (void)hipGetLastError();  // not device-mapped: the wait copies instead
    return GS_OK;
  }
  hipLaunchKernelGGL(gs::publish_info_kernel, dim3(1), dim3(64), 0, s, info_dev, count,
                     static_cast<int64_t*>(dslot), kReadbackFlagWord, seq);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  t->flagged = true;
  return GS_OK;
}

// Waits until the words of readback_begin are in slot[0, count).
int readback_wait(const ReadbackTicket& t, const int64_t* info_dev, int count, hipStream_t s) {
  if (t.flagged) {
    const int64_t* flag = t.slot + kReadbackFlagWord;
    for (uint64_t spin = 1;; ++spin) {
      if (__atomic_load_n(flag, __ATOMIC_ACQUIRE) == t.seq) return GS_OK;
      if ((spin & 1023) == 0) {
        const hipError_t q = hipStreamQuery(s);
        if (q == hipErrorNotReady) {
          // past the first ~10^4 spins, give the core to other runnable threads now and then
          if (spin >= 16384 && (spin & 4095) == 0) sched_yield();
          continue;
        }
        if (q != hipSuccess) return (int)q;
        if (__atomic_load_n(flag, __ATOMIC_ACQUIRE) == t.seq) continue;  // read at the loop's top
        break;  // drained without the flag: copy below
      }
#if defined(__x86_64__) || defined(__i386__)
      __builtin_ia32_pause();
#endif
    }
  }
  const hipError_t e =
      hipMemcpyAsync(t.slot, info_dev, (size_t)count * sizeof(int64_t), hipMemcpyDeviceToHost, s);
  if (e != hipSuccess) return (int)e;
  return gs_status_from_hip(hipStreamSynchronize(s));
}
}  // namespace

extern "C" size_t gs_readback_slot_bytes(void) { return (size_t)kReadbackSlotWords * sizeof(int64_t); }

extern "C" int gs_info_readback(const int64_t* info_dev, int64_t* slot, int64_t seq, int32_t count, void* stream) {
  if (!info_dev || !slot || count < 1 || count > 16) return GS_ERR_INVALID_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  ReadbackTicket t;
  const int st = readback_begin(info_dev, count, slot, seq, s, &t);
  if (st != GS_OK) return st;
  return readback_wait(t, info_dev, count, s);
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
                     radii, depths, block_sums, block_range, nullptr, vec, gs_scan_vec_rd(order, radii, depths),
                     nullptr, nullptr);
  hipLaunchKernelGGL(gs::scan_apply_kernel, dim3(nb), dim3(gs::kScanThreads), 0, s, P, nb, tiles_touched, order,
                     block_sums, block_range, offsets, reinterpret_cast<long long*>(info_dev), vec, nullptr);
  return gs_status_from_hip(hipGetLastError());
}

extern "C" int gs_num_rendered_readback(const int64_t* info_dev, int64_t* slot, int64_t seq, void* stream) {
  return gs_info_readback(info_dev, slot, seq, 2, stream);
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
                     reinterpret_cast<unsigned long long*>(keys_out), values_out, nullptr, nullptr, 0);
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
                           void* const* stage_events, void* stream, bool ranges_cleared,
                           bool keys_emitted = false, int32_t* tile_order = nullptr) {
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
  int st = GS_OK;
  if (!keys_emitted) {  // (else the caller has emitted them into the workspace and marked the stage)
    mark(0);
    st = gs_duplicate_keys(P, radii, records, conic_2d_inv, coverage, depths, offsets, image_width, image_height,
                           coverage_mode, num_rendered, depth_min, depth_bits, value_bits, keys, nullptr, stream);
    if (st != GS_OK) return st;
    mark(1);
  }
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
  // With a tile order buffer (when the order pays) the tiles are ordered
  // longest list first here, for the segment sort and then the render.
  const bool ordered = tile_order != nullptr && gs::tile_order_pays(num_rendered, P, num_tiles);
  if (ordered) {
    st = gs_tile_order(num_tiles, ranges, tile_order, stream);
    if (st != GS_OK) return st;
  }
  st = gs_sort_tile_segments_ordered(num_rendered, keys, keys_alt, num_tiles, ranges, value_bits, depth_bits,
                                     value_bits, point_list, sorted_keys_out != nullptr,
                                     ordered ? tile_order : nullptr, stream);
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
extern "C" int gs_readback_bin_packed(const int64_t* info_dev, int64_t* slot, int64_t seq, int32_t P,
                                      const int32_t* radii, const float* records, const float* conic_2d_inv,
                                      const int32_t* coverage, const float* depths, const int32_t* offsets,
                                      int32_t image_width, int32_t image_height,
                                      int32_t coverage_mode, int32_t max_pairs_per_point, int64_t capacity,
                                      void* workspace, size_t workspace_bytes, int32_t* ranges, int32_t* point_list,
                                      const float* background, int32_t compute_depth, float* out_color,
                                      float* out_depth, float* out_alpha, int32_t* n_contrib, float* grad_clear,
                                      int64_t grad_clear_floats, void* const* stage_events, int64_t* result,
                                      int32_t* tile_order, void* stream) {
  if (!info_dev || !slot || !result || P < 0 || capacity < 0 || image_width <= 0 || image_height <= 0)
    return GS_ERR_INVALID_ARGUMENT;
  // The ranges are cleared while the host waits for the count: the clearing
  // is enqueued after the count's publication, so it runs during the wait
  // instead of delaying it (by the key emission when there is one).
  hipStream_t hs = (hipStream_t)stream;
  ReadbackTicket ticket;
  int st = readback_begin(info_dev, 2, slot, seq, hs, &ticket);
  if (st != GS_OK) return st;
  const bool clear_first = ranges != nullptr && capacity > 0;
  const int grid_x = (image_width + gs::kBlockX - 1) / gs::kBlockX;
  const int grid_y = (image_height + gs::kBlockY - 1) / gs::kBlockY;
  const int tile_bits = gs_bit_length((long long)grid_x * grid_y - 1);
  int value_bits = gs_bit_length((long long)P - 1);
  if (value_bits < 1) value_bits = 1;
  const int n2 = 2 * grid_x * grid_y;  // range words
  // The keys are emitted before the count is known, into the start of the
  // workspace (where the binning keeps them), with the key layout and the
  // count read from info_dev by the kernel and at most capacity keys
  // written: the emission runs while the host waits for the count and
  // launches the sort.  When the host then declines the packed binning the
  // keys are not used.  The same kernel clears the tile ranges.
  bool emitted = false;
  if (capacity > 0 && P > 0 && workspace && workspace_bytes >= (size_t)capacity * sizeof(uint64_t) && radii &&
      records && conic_2d_inv && offsets && point_list && value_bits <= 31 && coverage_mode >= 0 &&
      coverage_mode <= 2 && ((reinterpret_cast<uintptr_t>(records) | reinterpret_cast<uintptr_t>(coverage)) & 15) == 0) {
    if (stage_events) (void)hipEventRecord((hipEvent_t)stage_events[0], hs);
    hipLaunchKernelGGL(gs::duplicate_keys_kernel, dim3((P + 255) / 256), dim3(256), 0, hs, P, radii,
                       reinterpret_cast<const float4*>(records), conic_2d_inv, reinterpret_cast<const int4*>(coverage),
                       depths, offsets, grid_x, grid_y, coverage_mode, (long long)capacity, 0u, 0, value_bits,
                       reinterpret_cast<unsigned long long*>(workspace), nullptr,
                       reinterpret_cast<const long long*>(info_dev), clear_first ? ranges : nullptr,
                       clear_first ? n2 : 0);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    if (stage_events) (void)hipEventRecord((hipEvent_t)stage_events[1], hs);
    emitted = true;
  } else if (clear_first) {
    hipLaunchKernelGGL(gs::zero_ranges_kernel, dim3((n2 + 255) / 256), dim3(256), 0, hs, n2, ranges);
  }
  st = readback_wait(ticket, info_dev, 2, hs);
  if (st != GS_OK) return st;
  const int64_t R = slot[0];
  const uint64_t range = (uint64_t)slot[1];
  const uint32_t depth_min = (uint32_t)(range & 0xFFFFFFFFull);
  const uint32_t depth_max = (uint32_t)(range >> 32);
  const int depth_bits = depth_max >= depth_min ? gs_bit_length((long long)(depth_max - depth_min)) : 0;
  result[0] = R;
  result[1] = depth_min;
  result[2] = depth_bits;
  result[3] = value_bits;
  result[4] = 0;
  result[5] = 0;
  if (R <= 0 || R > 0x7fffffffLL || R > capacity) return GS_OK;
  if (tile_bits + depth_bits + value_bits > 64 || value_bits > 31) return GS_OK;
  if (max_pairs_per_point > 0 && R > (int64_t)max_pairs_per_point * P) return GS_OK;
  // the render's tile order is written by the binning (before its segment sort)
  int32_t* order = out_color ? tile_order : nullptr;
  st = bin_packed_impl(P, radii, records, conic_2d_inv, coverage, depths, offsets, image_width, image_height,
                       coverage_mode, R, depth_min, depth_bits, value_bits, workspace, workspace_bytes, ranges,
                       point_list, nullptr, stage_events, stream, clear_first, emitted, order);
  if (st != GS_OK) return st;
  result[4] = 1;
  if (out_color) {
    st = gs_render_fwd_clear_ordered(image_width, image_height, P, R, ranges, point_list, records, background,
                                     compute_depth, out_color, out_depth, out_alpha, n_contrib, grad_clear,
                                     grad_clear_floats, order, true, stream);
    if (st != GS_OK) return st;
    if (stage_events) (void)hipEventRecord((hipEvent_t)stage_events[5], (hipStream_t)stream);
    result[5] = 1;
  }
  return GS_OK;
}
