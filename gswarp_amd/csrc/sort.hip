// Stable LSD radix sort of (uint64 key, int32 value) pairs for gfx950.
//
// Per 8-bit digit pass (reduce-then-scan):
//   1. upsweep:   each 4096-element block histograms its digits in LDS
//                 (one 256-bin histogram per wave) -> hist[digit][block].
//   2. rowscan:   one workgroup per digit scans hist[digit][*] across blocks
//                 (exclusive) and records the digit total.
//   3. downsweep: each block ranks its elements stably with 64-lane ballot
//                 matching (8 ballots per item give the set of lanes holding
//                 the same digit), stages them in LDS in digit order, and
//                 writes them out so that consecutive lanes store consecutive
//                 addresses within each digit run.
// Element e of block b is handled by wave w = (e / 1024), item slot
// i = (e % 1024) / 64, lane = e % 64, so processing slots in order with a
// per-wave running counter preserves the input order among equal digits.
#include "gs_capi.h"

namespace gs_sort {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kItems = 16;
constexpr int kTile = kThreads * kItems;  // 4096
constexpr int kRadix = 256;

typedef unsigned long long u64;

__device__ __forceinline__ unsigned block_exclusive_scan_u32(unsigned v, unsigned* lds_w, unsigned* total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  unsigned inc = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const unsigned n = __shfl_up(inc, off, 64);
    if (lane >= off) inc += n;
  }
  if (lane == 63) lds_w[wave] = inc;
  __syncthreads();
  unsigned wave_off = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const unsigned s = lds_w[w];
    if (w < wave) wave_off += s;
    tot += s;
  }
  *total = tot;
  __syncthreads();
  return wave_off + inc - v;
}

__global__ __launch_bounds__(kThreads) void upsweep_kernel(const u64* __restrict__ keys, long long n, int shift,
                                                          int nb, unsigned* __restrict__ hist) {
  __shared__ unsigned wh[kWaves][kRadix];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int i = threadIdx.x; i < kWaves * kRadix; i += kThreads) (&wh[0][0])[i] = 0;
  __syncthreads();
  const long long base = (long long)blockIdx.x * kTile + wave * (64 * kItems) + lane;
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const long long idx = base + i * 64;
    if (idx < n) {
      const unsigned d = (unsigned)(keys[idx] >> shift) & (kRadix - 1);
      atomicAdd(&wh[wave][d], 1u);
    }
  }
  __syncthreads();
  const int d = threadIdx.x;
  const unsigned c = wh[0][d] + wh[1][d] + wh[2][d] + wh[3][d];
  hist[(size_t)d * nb + blockIdx.x] = c;
}

__global__ __launch_bounds__(kThreads) void rowscan_kernel(int nb, unsigned* __restrict__ hist,
                                                          unsigned* __restrict__ digit_totals) {
  __shared__ unsigned lds_w[kWaves];
  unsigned* row = hist + (size_t)blockIdx.x * nb;
  unsigned carry = 0;
  for (int base = 0; base < nb; base += kThreads) {
    const int i = base + threadIdx.x;
    const unsigned v = i < nb ? row[i] : 0u;
    unsigned tot;
    const unsigned ex = block_exclusive_scan_u32(v, lds_w, &tot);
    if (i < nb) row[i] = carry + ex;
    carry += tot;
  }
  if (threadIdx.x == 0) digit_totals[blockIdx.x] = carry;
}

__global__ __launch_bounds__(kThreads) void downsweep_kernel(const u64* __restrict__ keys_in,
                                                            const int* __restrict__ vals_in,
                                                            u64* __restrict__ keys_out, int* __restrict__ vals_out,
                                                            long long n, int shift, int nb,
                                                            const unsigned* __restrict__ hist,
                                                            const unsigned* __restrict__ digit_totals) {
  __shared__ u64 s_keys[kTile];
  __shared__ int s_vals[kTile];
  __shared__ unsigned s_wcount[kWaves][kRadix];
  __shared__ unsigned s_dstart[kRadix];
  __shared__ long long s_gbase[kRadix];
  __shared__ unsigned s_lds_w[kWaves];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const long long block_base = (long long)blockIdx.x * kTile;
  const long long wave_base = block_base + wave * (64 * kItems) + lane;
  const int block_count = (int)((n - block_base) < kTile ? (n - block_base) : kTile);

#pragma unroll
  for (int i = threadIdx.x; i < kWaves * kRadix; i += kThreads) (&s_wcount[0][0])[i] = 0;

  u64 key[kItems];
  int val[kItems];
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const long long idx = wave_base + i * 64;
    if (idx < n) {
      key[i] = keys_in[idx];
      val[i] = vals_in[idx];
    } else {
      key[i] = 0;
      val[i] = 0;
    }
  }
  __syncthreads();

  const u64 lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  unsigned rank[kItems];
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const bool valid = (wave_base + i * 64) < n;
    const unsigned d = (unsigned)(key[i] >> shift) & (kRadix - 1);
    u64 peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const bool bit = (d >> b) & 1u;
      const u64 m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    unsigned before = 0;
    if (valid) before = s_wcount[wave][d];
    __builtin_amdgcn_wave_barrier();
    const unsigned below = (unsigned)__popcll(peers & lt_mask);
    const bool leader = valid && below == 0;
    if (leader) s_wcount[wave][d] = before + (unsigned)__popcll(peers);
    __builtin_amdgcn_wave_barrier();
    rank[i] = before + below;
  }
  __syncthreads();

  // Per digit: exclusive offsets of each wave, block-local digit start, and
  // the global base such that global position = s_gbase[d] + local position.
  {
    const int d = threadIdx.x;
    unsigned run = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const unsigned c = s_wcount[w][d];
      s_wcount[w][d] = run;
      run += c;
    }
    unsigned tot;
    const unsigned dstart = block_exclusive_scan_u32(run, s_lds_w, &tot);
    unsigned gtot;
    const unsigned gstart = block_exclusive_scan_u32(digit_totals[d], s_lds_w, &gtot);
    s_dstart[d] = dstart;
    s_gbase[d] = (long long)gstart + (long long)hist[(size_t)d * nb + blockIdx.x] - (long long)dstart;
  }
  __syncthreads();

#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const bool valid = (wave_base + i * 64) < n;
    if (valid) {
      const unsigned d = (unsigned)(key[i] >> shift) & (kRadix - 1);
      const unsigned lp = s_dstart[d] + s_wcount[wave][d] + rank[i];
      s_keys[lp] = key[i];
      s_vals[lp] = val[i];
    }
  }
  __syncthreads();

#pragma unroll
  for (int j = 0; j < kItems; ++j) {
    const int p = j * kThreads + threadIdx.x;
    if (p < block_count) {
      const u64 k = s_keys[p];
      const unsigned d = (unsigned)(k >> shift) & (kRadix - 1);
      const long long gp = s_gbase[d] + p;
      if (gp >= 0 && gp < n) {  // always true for a consistent histogram
        keys_out[gp] = k;
        vals_out[gp] = s_vals[p];
      }
    }
  }
}

static inline int num_blocks(long long n) { return (int)((n + kTile - 1) / kTile); }

}  // namespace gs_sort

extern "C" int gs_sort_num_passes(int32_t key_bits) { return gs_passes_for_bits(key_bits); }

extern "C" size_t gs_sort_scratch_bytes(int64_t n) {
  if (n <= 0) return 0;
  const size_t nb = (size_t)gs_sort::num_blocks(n);
  const size_t bytes = (nb * gs_sort::kRadix + gs_sort::kRadix) * sizeof(unsigned);
  return (bytes + 255) & ~(size_t)255;
}

extern "C" int gs_sort_pairs_u64(int64_t n, int32_t key_bits, uint64_t* keys, int32_t* values,
                                 uint64_t* keys_alt, int32_t* values_alt, void* scratch, size_t scratch_bytes,
                                 void* stream) {
  if (n < 0 || key_bits < 0 || key_bits > 64) return GS_ERR_INVALID_ARGUMENT;
  if (n > 0x7fffffffLL) return GS_ERR_OVERFLOW;
  if (n == 0 || key_bits == 0) return GS_OK;
  if (!keys || !values || !keys_alt || !values_alt || !scratch) return GS_ERR_INVALID_ARGUMENT;
  if (scratch_bytes < gs_sort_scratch_bytes(n)) return GS_ERR_SCRATCH_TOO_SMALL;
  hipStream_t s = (hipStream_t)stream;
  const int nb = gs_sort::num_blocks(n);
  unsigned* hist = reinterpret_cast<unsigned*>(scratch);
  unsigned* digit_totals = hist + (size_t)nb * gs_sort::kRadix;
  const int passes = gs_passes_for_bits(key_bits);
  gs_sort::u64* kin = reinterpret_cast<gs_sort::u64*>(keys);
  gs_sort::u64* kout = reinterpret_cast<gs_sort::u64*>(keys_alt);
  int* vin = values;
  int* vout = values_alt;
  for (int pass = 0; pass < passes; ++pass) {
    const int shift = pass * 8;
    hipLaunchKernelGGL(gs_sort::upsweep_kernel, dim3(nb), dim3(gs_sort::kThreads), 0, s, kin, (long long)n, shift,
                       nb, hist);
    hipLaunchKernelGGL(gs_sort::rowscan_kernel, dim3(gs_sort::kRadix), dim3(gs_sort::kThreads), 0, s, nb, hist,
                       digit_totals);
    hipLaunchKernelGGL(gs_sort::downsweep_kernel, dim3(nb), dim3(gs_sort::kThreads), 0, s, kin, vin, kout, vout,
                       (long long)n, shift, nb, hist, digit_totals);
    gs_sort::u64* tk = kin;
    kin = kout;
    kout = tk;
    int* tv = vin;
    vin = vout;
    vout = tv;
  }
  return gs_status_from_hip(hipGetLastError());
}
