// Tile binning: tile-count prefix sum, duplicate-with-keys, tile ranges.
//
// The reference builds its per-tile lists with two stable sorts: all N
// Gaussians by depth (binning_ops.py:152-222), then the R emitted
// (tile, point) pairs by tile (binning_ops.py:297-343).  Here the pairs are
// emitted once in point-index order with a 64-bit key tile<<32 | depth bits
// and sorted once (sort.hip).  A stable sort of that key orders pairs by
// (tile, depth bits, point index), which is exactly the order the
// reference's depth-then-tile sorts produce, so point lists and tile ranges
// are identical.
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

__global__ __launch_bounds__(kScanThreads) void scan_reduce_kernel(int n, const int* __restrict__ in,
                                                                  long long* __restrict__ block_sums) {
  __shared__ long long lds4[kScanThreads / 64];
  const long long base = (long long)blockIdx.x * kScanTile;
  long long s = 0;
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    const long long idx = base + (long long)i * kScanThreads + threadIdx.x;
    if (idx < n) s += in[idx];
  }
  long long total;
  block_exclusive_scan_i64(s, lds4, &total);
  if (threadIdx.x == 0) block_sums[blockIdx.x] = total;
}

// Single-workgroup exclusive scan of the block sums; also stores the total.
__global__ __launch_bounds__(kScanThreads) void scan_blocks_kernel(int nb, long long* __restrict__ block_sums,
                                                                  long long* __restrict__ total_out) {
  __shared__ long long lds4[kScanThreads / 64];
  long long carry = 0;
  for (int base = 0; base < nb; base += kScanThreads) {
    const int i = base + threadIdx.x;
    const long long v = i < nb ? block_sums[i] : 0;
    long long tot;
    const long long ex = block_exclusive_scan_i64(v, lds4, &tot);
    if (i < nb) block_sums[i] = carry + ex;
    carry += tot;
  }
  if (threadIdx.x == 0) *total_out = carry;
}

__global__ __launch_bounds__(kScanThreads) void scan_apply_kernel(int n, const int* __restrict__ in,
                                                                 const long long* __restrict__ block_offsets,
                                                                 int* __restrict__ out) {
  __shared__ long long lds4[kScanThreads / 64];
  const long long base = (long long)blockIdx.x * kScanTile + (long long)threadIdx.x * kScanItems;
  int v[kScanItems];
  long long s = 0;
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    const long long idx = base + i;
    v[i] = idx < n ? in[idx] : 0;
    s += v[i];
  }
  long long total;
  long long run = block_offsets[blockIdx.x] + block_exclusive_scan_i64(s, lds4, &total);
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    const long long idx = base + i;
    run += v[i];
    if (idx < n) out[idx] = (int)run;
  }
}

// Emission of one Gaussian's covered tiles, in the same enumeration as
// count_covered_tiles (binning_kernels.py:127-216 semantics).
__device__ __forceinline__ void emit_tiles(float px, float py, float ca, float cb, float cc, float opacity,
                                           float cov_aa, float cov_cc, int radius, int grid_x, int grid_y,
                                           int mode, uint32_t depth_bits, int point_id, long long off,
                                           long long limit, unsigned long long* __restrict__ keys,
                                           int* __restrict__ values) {
  const int4 rect = snugbox_rect(px, py, cov_aa, cov_cc, opacity, radius, grid_x, grid_y);
  const int span_x = rect.z - rect.x;
  const int span_y = rect.w - rect.y;
  const int area = span_x * span_y;
  const unsigned long long dk = (unsigned long long)depth_bits;
  if (area <= 1 || mode == kCoverageSnugbox) {
    for (int ty = rect.y; ty < rect.w; ++ty)
      for (int tx = rect.x; tx < rect.z; ++tx) {
        if (off < limit) {
          keys[off] = ((unsigned long long)(ty * grid_x + tx) << 32) | dk;
          values[off] = point_id;
        }
        ++off;
      }
    return;
  }
  const float threshold = coverage_threshold(opacity);
  if (mode == kCoverageConicRect && area <= kConicMaskMaxTiles) {
    for (int ty = rect.y; ty < rect.w; ++ty)
      for (int tx = rect.x; tx < rect.z; ++tx)
        if (conic_rect_intersects_tile(px, py, ca, cb, cc, threshold, tx, ty)) {
          if (off < limit) {
            keys[off] = ((unsigned long long)(ty * grid_x + tx) << 32) | dk;
            values[off] = point_id;
          }
          ++off;
        }
    return;
  }
  if (span_y <= span_x) {
    for (int ty = rect.y; ty < rect.w; ++ty) {
      const int2 iv = accutile_band(px, py, ca, cb, cc, threshold, ty, kBlockX, kBlockY, rect.x, rect.z);
      for (int tx = iv.x; tx < iv.y; ++tx) {
        if (off < limit) {
          keys[off] = ((unsigned long long)(ty * grid_x + tx) << 32) | dk;
          values[off] = point_id;
        }
        ++off;
      }
    }
  } else {
    for (int tx = rect.x; tx < rect.z; ++tx) {
      const int2 iv = accutile_band(py, px, cc, cb, ca, threshold, tx, kBlockY, kBlockX, rect.y, rect.w);
      for (int ty = iv.x; ty < iv.y; ++ty) {
        if (off < limit) {
          keys[off] = ((unsigned long long)(ty * grid_x + tx) << 32) | dk;
          values[off] = point_id;
        }
        ++off;
      }
    }
  }
}

__global__ __launch_bounds__(256) void duplicate_keys_kernel(int P, const int* __restrict__ radii,
                                                            const float4* __restrict__ records,
                                                            const float* __restrict__ cov2d,
                                                            const int* __restrict__ offsets, int grid_x,
                                                            int grid_y, int mode, long long limit,
                                                            unsigned long long* __restrict__ keys,
                                                            int* __restrict__ values) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= P) return;
  const int radius = radii[idx];
  if (radius <= 0) return;
  const long long off = idx > 0 ? (long long)offsets[idx - 1] : 0;
  const float4 r0 = records[3 * (size_t)idx + 0];
  const float4 r1 = records[3 * (size_t)idx + 1];
  const float cov_aa = cov2d[3 * idx + 0];
  const float cov_cc = cov2d[3 * idx + 2];
  emit_tiles(r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, cov_aa, cov_cc, radius, grid_x, grid_y, mode,
             __float_as_uint(r1.z), idx, off, limit, keys, values);
}

__global__ void zero_i64_kernel(long long* p) {
  if (threadIdx.x == 0) *p = 0;
}

__global__ __launch_bounds__(256) void zero_ranges_kernel(int n2, int* __restrict__ ranges) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n2) ranges[i] = 0;
}

__global__ __launch_bounds__(256) void tile_ranges_kernel(long long n, const unsigned long long* __restrict__ keys,
                                                         int num_tiles, int2* __restrict__ ranges) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const unsigned tile = (unsigned)(keys[i] >> 32);
  if (tile >= (unsigned)num_tiles) return;  // never taken for keys from gs_duplicate_keys
  if (i == 0) {
    ranges[tile].x = 0;
  } else {
    const unsigned prev = (unsigned)(keys[i - 1] >> 32);
    if (tile != prev) {
      if (prev < (unsigned)num_tiles) ranges[prev].y = (int)i;
      ranges[tile].x = (int)i;
    }
  }
  if (i == n - 1) ranges[tile].y = (int)n;
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
    default:
      return status > 0 ? hipGetErrorString((hipError_t)status) : "unknown error";
  }
}

static inline int gs_scan_blocks(int32_t P) { return (P + gs::kScanTile - 1) / gs::kScanTile; }

extern "C" size_t gs_scan_scratch_bytes(int32_t P) {
  if (P <= 0) return 0;
  return ((size_t)gs_scan_blocks(P) * sizeof(long long) + 255) & ~(size_t)255;
}

extern "C" int gs_scan_tiles(int32_t P, const int32_t* tiles_touched, int32_t* offsets, int64_t* total_dev,
                             void* scratch, size_t scratch_bytes, void* stream) {
  if (P < 0 || !total_dev) return GS_ERR_INVALID_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  if (P == 0) {
    hipLaunchKernelGGL(gs::zero_i64_kernel, dim3(1), dim3(64), 0, s, reinterpret_cast<long long*>(total_dev));
    return gs_status_from_hip(hipGetLastError());
  }
  if (!tiles_touched || !offsets || !scratch) return GS_ERR_INVALID_ARGUMENT;
  if (scratch_bytes < gs_scan_scratch_bytes(P)) return GS_ERR_SCRATCH_TOO_SMALL;
  const int nb = gs_scan_blocks(P);
  long long* block_sums = reinterpret_cast<long long*>(scratch);
  hipLaunchKernelGGL(gs::scan_reduce_kernel, dim3(nb), dim3(gs::kScanThreads), 0, s, P, tiles_touched,
                     block_sums);
  hipLaunchKernelGGL(gs::scan_blocks_kernel, dim3(1), dim3(gs::kScanThreads), 0, s, nb, block_sums,
                     reinterpret_cast<long long*>(total_dev));
  hipLaunchKernelGGL(gs::scan_apply_kernel, dim3(nb), dim3(gs::kScanThreads), 0, s, P, tiles_touched,
                     block_sums, offsets);
  return gs_status_from_hip(hipGetLastError());
}

extern "C" int gs_num_rendered_readback(const int64_t* total_dev, int64_t* total_host_pinned, void* stream) {
  if (!total_dev || !total_host_pinned) return GS_ERR_INVALID_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = hipMemcpyAsync(total_host_pinned, total_dev, sizeof(int64_t), hipMemcpyDeviceToHost, s);
  if (e != hipSuccess) return (int)e;
  return gs_status_from_hip(hipStreamSynchronize(s));
}

extern "C" int gs_duplicate_keys(int32_t P, const int32_t* radii, const float* records,
                                 const float* conic_2d_inv, const int32_t* offsets, int32_t image_width,
                                 int32_t image_height, int32_t coverage_mode, int64_t num_rendered,
                                 uint64_t* keys_out, int32_t* values_out, void* stream) {
  if (P < 0 || image_width <= 0 || image_height <= 0 || coverage_mode < 0 || coverage_mode > 2)
    return GS_ERR_INVALID_ARGUMENT;
  if (P == 0 || num_rendered <= 0) return GS_OK;
  if (!radii || !records || !conic_2d_inv || !offsets || !keys_out || !values_out)
    return GS_ERR_INVALID_ARGUMENT;
  if (reinterpret_cast<uintptr_t>(records) & 15) return GS_ERR_MISALIGNED;
  const int grid_x = (image_width + gs::kBlockX - 1) / gs::kBlockX;
  const int grid_y = (image_height + gs::kBlockY - 1) / gs::kBlockY;
  hipLaunchKernelGGL(gs::duplicate_keys_kernel, dim3((P + 255) / 256), dim3(256), 0, (hipStream_t)stream, P,
                     radii, reinterpret_cast<const float4*>(records), conic_2d_inv, offsets, grid_x, grid_y,
                     coverage_mode, (long long)num_rendered, reinterpret_cast<unsigned long long*>(keys_out),
                     values_out);
  return gs_status_from_hip(hipGetLastError());
}

extern "C" int gs_tile_ranges(int64_t n, const uint64_t* sorted_keys, int32_t num_tiles, int32_t* ranges,
                              void* stream) {
  if (n < 0 || num_tiles <= 0 || !ranges) return GS_ERR_INVALID_ARGUMENT;
  if (n > 0x7fffffffLL) return GS_ERR_OVERFLOW;
  hipStream_t s = (hipStream_t)stream;
  const int n2 = 2 * num_tiles;
  hipLaunchKernelGGL(gs::zero_ranges_kernel, dim3((n2 + 255) / 256), dim3(256), 0, s, n2, ranges);
  if (n > 0) {
    if (!sorted_keys) return GS_ERR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(gs::tile_ranges_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, (long long)n,
                       reinterpret_cast<const unsigned long long*>(sorted_keys), num_tiles,
                       reinterpret_cast<int2*>(ranges));
  }
  return gs_status_from_hip(hipGetLastError());
}
