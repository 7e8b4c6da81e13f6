// Stable LSD radix sort of uint32 or uint64 keys (optionally with int32
// values) for gfx950, on a bit field [lo_bit, lo_bit + key_bits) of the key.
//
// Per digit pass (reduce-then-scan; digits of at most 8 bits, the field split
// evenly over ceil(bits / 8) passes):
//   1. upsweep:   each 4096-element block counts its digits -> hist[digit][block].
//   2. rowscan:   one workgroup per digit scans hist[digit][*] across blocks
//                 (exclusive) and records the digit total.
//   3. downsweep: each block ranks its elements stably, stages them in LDS in
//                 digit order, and writes them out so that consecutive lanes
//                 store consecutive addresses within each digit run.
// The downsweep ranks with ballot matching: 8 ballots give each lane the set
// of lanes holding its digit, the lane's rank among them is a popcount, and
// only the lowest such lane updates the wave's counter, so ranks are stable
// and keys whose digits take few values (the exponent bits of depths, the
// high bits of tile ids) cause no LDS serialisation.
// Element e of block b is handled by wave w = (e / 1024), item slot
// i = (e % 1024) / 64, lane = e % 64, so processing slots in order with a
// per-wave running counter preserves the input order among equal digits.
#include "gs_capi.h"

namespace gs_sort {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
// Keys per thread of the radix passes: 16 (4096 per workgroup), or 32 for
// sorts of at least kLargeSortKeys keys whose workgroup tile fits in 64 KB of
// LDS, where the longer per-digit runs of each workgroup's scatter outweigh
// the lower occupancy (and the halved number of histogram columns shortens
// the digit-row scans).
constexpr int kItems = 16;
constexpr int kItemsLarge = 32;
constexpr long long kLargeSortKeys = 1ll << 24;
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

// Digit of a pass: bits [shift, shift + width) of the key, dmask = 2^width - 1
// (bits above the pass's digit take no part).
template <typename K>
__device__ __forceinline__ unsigned digit_of(K key, int shift, unsigned dmask) {
  return (unsigned)(key >> shift) & dmask;
}

// Digit width of pass `pass` of `passes`: the key_bits are split as evenly as
// possible (13 bits: 7 + 6, 26: 7 + 7 + 6 + 6), never above 8.  Narrow
// digits mean fewer destination runs per block in the scatter, and the
// passes with wide digits are the ones whose writes scatter the most.
static inline int pass_digit_bits(int key_bits, int passes, int pass) {
  return key_bits / passes + (pass < key_bits % passes ? 1 : 0);
}

// Lanes of the wave holding the same digit d as this lane (among valid lanes).
// Per bit b: s = bit b of d sign-extended (0 or ~0, one v_bfe_i32), m = ballot
// of that bit, and the lanes agreeing with this lane's bit are ~(m ^ s).  The
// update peers &= ~(m ^ s) is one v_bitop3_b32 per 32-bit half with truth
// table 0x84 = S1 & ~(S0 ^ S2) (peers as S1; symmetric in S0 and S2).
__device__ __forceinline__ u64 match_digit(unsigned d, bool valid) {
  const u64 v = __ballot(valid);
  unsigned lo = (unsigned)v, hi = (unsigned)(v >> 32);
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    const unsigned s = (unsigned)__builtin_amdgcn_sbfe((int)d, b, 1);
    const u64 m = __ballot(s != 0u);
    lo = __builtin_amdgcn_bitop3_b32((unsigned)m, lo, s, 0x84);
    hi = __builtin_amdgcn_bitop3_b32((unsigned)(m >> 32), hi, s, 0x84);
  }
  return ((u64)hi << 32) | lo;
}

// Digit counts of one block.  Counting needs no stable order, so lanes add
// into one of kCopies histogram copies chosen by lane % kCopies with LDS
// atomics; copies sit kRadix + 1 words apart, so equal digits in different
// copies fall in different banks and a wave whose lanes share one digit
// serialises 64 / kCopies deep instead of 64.
constexpr int kCopies = 8;
constexpr int kCopyStride = kRadix + 1;

template <typename K, int kIt>
__global__ __launch_bounds__(kThreads) void upsweep_kernel(const K* __restrict__ keys, long long n, int shift,
                                                          unsigned dmask, int nb, unsigned* __restrict__ hist) {
  constexpr int kTile = kThreads * kIt;
  __shared__ unsigned h[kCopies * kCopyStride];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  for (int i = threadIdx.x; i < kCopies * kCopyStride; i += kThreads) h[i] = 0;
  const long long base = (long long)blockIdx.x * kTile + wave * (64 * kIt) + lane;
  K key[kIt];
#pragma unroll
  for (int i = 0; i < kIt; ++i) {
    const long long idx = base + i * 64;
    key[i] = idx < n ? keys[idx] : K(0);
  }
  __syncthreads();
  unsigned* mine = h + (lane & (kCopies - 1)) * kCopyStride;
#pragma unroll
  for (int i = 0; i < kIt; ++i)
    if (base + i * 64 < n) atomicAdd(mine + digit_of(key[i], shift, dmask), 1u);
  __syncthreads();
  const int d = threadIdx.x;
  unsigned c = 0;
#pragma unroll
  for (int k = 0; k < kCopies; ++k) c += h[k * kCopyStride + d];
  if ((unsigned)d <= dmask) hist[(size_t)d * nb + blockIdx.x] = c;
}

// One workgroup per digit row: hist[d][*] becomes its exclusive prefix over
// blocks and digit_totals[d] the row total.  The row is scanned in chunks of
// kRowChunk entries, thread t owning kRowItems consecutive entries of a
// chunk, so the workgroup reads and writes each chunk as one contiguous
// span: per-thread sums, one block scan, the prefixes written back, the
// chunk total carried.  The next chunk is loaded before the current one is
// scanned, so its loads overlap the scan.
constexpr int kRowItems = 8;
constexpr int kRowChunk = kThreads * kRowItems;
__global__ __launch_bounds__(kThreads) void rowscan_kernel(int nb, unsigned* __restrict__ hist,
                                                          unsigned* __restrict__ digit_totals) {
  __shared__ unsigned s_lds_w[kWaves];
  unsigned* row = hist + (size_t)blockIdx.x * nb;
  const int t0 = threadIdx.x * kRowItems;
  unsigned cur[kRowItems], nxt[kRowItems];
#pragma unroll
  for (int k = 0; k < kRowItems; ++k) cur[k] = t0 + k < nb ? row[t0 + k] : 0u;
  unsigned carry = 0;
  for (int base = 0; base < nb; base += kRowChunk) {
#pragma unroll
    for (int k = 0; k < kRowItems; ++k) {
      const int i = base + kRowChunk + t0 + k;
      nxt[k] = i < nb ? row[i] : 0u;
    }
    unsigned sum = 0;
#pragma unroll
    for (int k = 0; k < kRowItems; ++k) sum += cur[k];
    unsigned total;
    unsigned run = carry + block_exclusive_scan_u32(sum, s_lds_w, &total);
#pragma unroll
    for (int k = 0; k < kRowItems; ++k) {
      const int i = base + t0 + k;
      if (i < nb) row[i] = run;
      run += cur[k];
      cur[k] = nxt[k];
    }
    carry += total;
  }
  if (threadIdx.x == 0) digit_totals[blockIdx.x] = carry;
}

template <typename K, bool kValues, int kIt>
__global__ __launch_bounds__(kThreads) void downsweep_kernel(const K* __restrict__ keys_in,
                                                            const int* __restrict__ vals_in,
                                                            K* __restrict__ keys_out, int* __restrict__ vals_out,
                                                            long long n, int shift, unsigned dmask, int nb,
                                                            const unsigned* __restrict__ hist,
                                                            const unsigned* __restrict__ digit_totals) {
  constexpr int kTile = kThreads * kIt;
  __shared__ K s_keys[kTile];
  __shared__ int s_vals[kValues ? kTile : 1];
  __shared__ unsigned s_wcount[kWaves][kRadix];
  __shared__ unsigned s_dstart[kRadix];
  __shared__ long long s_gbase[kRadix];
  __shared__ unsigned s_lds_w[kWaves];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const long long block_base = (long long)blockIdx.x * kTile;
  const long long wave_base = block_base + wave * (64 * kIt) + lane;
  const int block_count = (int)((n - block_base) < kTile ? (n - block_base) : kTile);

#pragma unroll
  for (int i = threadIdx.x; i < kWaves * kRadix; i += kThreads) (&s_wcount[0][0])[i] = 0;

  K key[kIt];
  int val[kIt];
#pragma unroll
  for (int i = 0; i < kIt; ++i) {
    const long long idx = wave_base + i * 64;
    const bool in = idx < n;
    key[i] = in ? keys_in[idx] : K(0);
    if (kValues) val[i] = in ? vals_in[idx] : 0;
  }
  __syncthreads();

  const u64 lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  unsigned rank[kIt];
#pragma unroll
  for (int i = 0; i < kIt; ++i) {
    const bool valid = (wave_base + i * 64) < n;
    const unsigned d = digit_of(key[i], shift, dmask);
    const u64 peers = match_digit(d, valid);
    unsigned before = 0;
    if (valid) before = s_wcount[wave][d];
    __builtin_amdgcn_wave_barrier();
    const unsigned below = (unsigned)__popcll(peers & lt_mask);
    if (valid && below == 0) s_wcount[wave][d] = before + (unsigned)__popcll(peers);
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
    // digits above dmask do not occur in this pass (no table rows exist)
    const bool used = (unsigned)d <= dmask;
    unsigned gtot;
    const unsigned gstart = block_exclusive_scan_u32(used ? digit_totals[d] : 0u, s_lds_w, &gtot);
    s_dstart[d] = dstart;
    s_gbase[d] = (long long)gstart + (long long)(used ? hist[(size_t)d * nb + blockIdx.x] : 0u) - (long long)dstart;
  }
  __syncthreads();

#pragma unroll
  for (int i = 0; i < kIt; ++i) {
    const bool valid = (wave_base + i * 64) < n;
    if (valid) {
      const unsigned d = digit_of(key[i], shift, dmask);
      const unsigned lp = s_dstart[d] + s_wcount[wave][d] + rank[i];
      s_keys[lp] = key[i];
      if (kValues) s_vals[lp] = val[i];
    }
  }
  __syncthreads();

#pragma unroll
  for (int j = 0; j < kIt; ++j) {
    const int p = j * kThreads + threadIdx.x;
    if (p < block_count) {
      const K k = s_keys[p];
      const long long gp = s_gbase[digit_of(k, shift, dmask)] + p;
      if (gp >= 0 && gp < n) {  // always true for a consistent histogram
        keys_out[gp] = k;
        if (kValues) vals_out[gp] = s_vals[p];
      }
    }
  }
}

static inline int items_for(long long n, size_t key_bytes, bool values) {
  const size_t tile_bytes = (size_t)kThreads * kItemsLarge * (key_bytes + (values ? sizeof(int) : 0));
  return (n >= kLargeSortKeys && tile_bytes <= 65536) ? kItemsLarge : kItems;
}
static inline int num_blocks(long long n, int items = kItems) {
  const long long tile = (long long)kThreads * items;
  return (int)((n + tile - 1) / tile);
}

template <typename K, bool kValues>
static int sort_impl(int64_t n, int32_t lo_bit, int32_t key_bits, K* kin, K* kout, int* vin, int* vout,
                     void* scratch, size_t scratch_bytes, hipStream_t s);

}  // namespace gs_sort

extern "C" int gs_sort_num_passes(int32_t key_bits) { return gs_passes_for_bits(key_bits); }

extern "C" size_t gs_sort_scratch_bytes(int64_t n) {
  if (n <= 0) return 0;
  const size_t nb = (size_t)gs_sort::num_blocks(n);
  const size_t bytes = (nb * gs_sort::kRadix + gs_sort::kRadix) * sizeof(unsigned);
  return (bytes + 255) & ~(size_t)255;
}

template <typename K, bool kValues>
static int gs_sort::sort_impl(int64_t n, int32_t lo_bit, int32_t key_bits, K* kin, K* kout, int* vin,
                              int* vout, void* scratch, size_t scratch_bytes, hipStream_t s) {
  if (n < 0 || lo_bit < 0 || key_bits < 0 || lo_bit + key_bits > (int)(8 * sizeof(K)))
    return GS_ERR_INVALID_ARGUMENT;
  if (n > 0x7fffffffLL) return GS_ERR_OVERFLOW;
  if (n == 0 || key_bits == 0) return GS_OK;
  if (!kin || !kout || !scratch || (kValues && (!vin || !vout))) return GS_ERR_INVALID_ARGUMENT;
  if (scratch_bytes < gs_sort_scratch_bytes(n)) return GS_ERR_SCRATCH_TOO_SMALL;
  // the scratch query counts 16-key tiles, the most histogram columns
  const int items = items_for(n, sizeof(K), kValues);
  const int nb = num_blocks(n, items);
  unsigned* hist = reinterpret_cast<unsigned*>(scratch);
  unsigned* digit_totals = hist + (size_t)nb * kRadix;
  const int passes = gs_passes_for_bits(key_bits);
  int shift = lo_bit;
  for (int pass = 0; pass < passes; ++pass) {
    const int bits = pass_digit_bits(key_bits, passes, pass);
    const unsigned dmask = (1u << bits) - 1u;
    if (items == kItemsLarge) {
      hipLaunchKernelGGL((upsweep_kernel<K, kItemsLarge>), dim3(nb), dim3(kThreads), 0, s, kin, (long long)n, shift,
                         dmask, nb, hist);
    } else {
      hipLaunchKernelGGL((upsweep_kernel<K, kItems>), dim3(nb), dim3(kThreads), 0, s, kin, (long long)n, shift,
                         dmask, nb, hist);
    }
    hipLaunchKernelGGL(rowscan_kernel, dim3(dmask + 1), dim3(kThreads), 0, s, nb, hist, digit_totals);
    if (items == kItemsLarge) {
      hipLaunchKernelGGL((downsweep_kernel<K, kValues, kItemsLarge>), dim3(nb), dim3(kThreads), 0, s, kin, vin,
                         kout, vout, (long long)n, shift, dmask, nb, hist, digit_totals);
    } else {
      hipLaunchKernelGGL((downsweep_kernel<K, kValues, kItems>), dim3(nb), dim3(kThreads), 0, s, kin, vin, kout,
                         vout, (long long)n, shift, dmask, nb, hist, digit_totals);
    }
    shift += bits;
    K* tk = kin;
    kin = kout;
    kout = tk;
    int* tv = vin;
    vin = vout;
    vout = tv;
  }
  return gs_status_from_hip(hipGetLastError());
}

extern "C" int gs_sort_pairs_u64(int64_t n, int32_t key_bits, uint64_t* keys, int32_t* values,
                                 uint64_t* keys_alt, int32_t* values_alt, void* scratch, size_t scratch_bytes,
                                 void* stream) {
  return gs_sort::sort_impl<gs_sort::u64, true>(n, 0, key_bits, reinterpret_cast<gs_sort::u64*>(keys),
                                  reinterpret_cast<gs_sort::u64*>(keys_alt), values, values_alt, scratch,
                                  scratch_bytes, (hipStream_t)stream);
}

extern "C" int gs_sort_keys_u64(int64_t n, int32_t lo_bit, int32_t key_bits, uint64_t* keys, uint64_t* keys_alt,
                                void* scratch, size_t scratch_bytes, void* stream) {
  return gs_sort::sort_impl<gs_sort::u64, false>(n, lo_bit, key_bits, reinterpret_cast<gs_sort::u64*>(keys),
                                   reinterpret_cast<gs_sort::u64*>(keys_alt), nullptr, nullptr, scratch,
                                   scratch_bytes, (hipStream_t)stream);
}

extern "C" int gs_sort_pairs_u32(int64_t n, int32_t lo_bit, int32_t key_bits, uint32_t* keys, int32_t* values,
                                 uint32_t* keys_alt, int32_t* values_alt, void* scratch, size_t scratch_bytes,
                                 void* stream) {
  return gs_sort::sort_impl<unsigned, true>(n, lo_bit, key_bits, keys, keys_alt, values, values_alt, scratch,
                                            scratch_bytes, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// Per-tile segment sort.  After the packed (tile, depth, point) keys have been
// sorted stably by their tile field alone, each tile's keys are contiguous and
// still in point order.  One 256-thread workgroup per tile then sorts its
// segment stably by the depth field [lo_bit, lo_bit + key_bits) with 8-bit LSD
// passes, which yields the (depth, point) order of a full key sort, and writes
// point_list = the low value_bits of each key (and, on request, the sorted keys
// back in place).
//
// Segments of up to kSmallCap keys are sorted by one wave each
// (small_segment_sort); longer ones by a 256-thread workgroup
// (long_segment_sort), both in one launch (segment_sort_kernel).  There,
// segments of up to kCap keys are sorted on
// chip: each thread holds up to
// kSlots keys in registers, ranks them with the same ballot-matched stable
// ranking as the downsweep above, scatters them into one LDS buffer and
// reloads them in element order for the next pass.  Longer segments are
// sorted through global memory, ping-ponging between their ranges of keys and
// keys_alt: a counting pass per digit, then chunks of kCap keys ranked on chip
// and scattered behind the running digit offsets.
namespace gs_seg {

using gs_sort::u64;
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kSlots = 8;
constexpr int kCap = kThreads * kSlots;  // 2048 keys
constexpr int kRadix = 256;

struct Shared {
  u64 buf[kCap];
  unsigned wc[2][kWaves][kRadix];
  unsigned base[kRadix];
  unsigned lds_w[kWaves];
};

// Stable ranks of this wave's keys among the keys of equal digit: slot by
// slot, lanes in order, continuing this wave's per-digit counters wc.
__device__ __forceinline__ void rank_slots(const u64 (&key)[kSlots], const bool (&valid)[kSlots], int nslots,
                                           int shift, unsigned dmask, unsigned* wc, unsigned (&rank)[kSlots]) {
  const int lane = threadIdx.x & 63;
  const u64 lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
  for (int i = 0; i < kSlots; ++i) {
    rank[i] = 0;
    if (i < nslots) {
      const unsigned d = gs_sort::digit_of(key[i], shift, dmask);
      const u64 peers = gs_sort::match_digit(d, valid[i]);
      unsigned before = 0;
      if (valid[i]) before = wc[d];
      __builtin_amdgcn_wave_barrier();
      const unsigned below = (unsigned)__popcll(peers & lt_mask);
      if (valid[i] && below == 0) wc[d] = before + (unsigned)__popcll(peers);
      __builtin_amdgcn_wave_barrier();
      rank[i] = before + below;
    }
  }
}

// Element e of a chunk of cnt keys belongs to wave e / cw, slot (e % cw) / 64,
// lane e % 64, with cw = 64 * ceil(cnt / 256): waves take contiguous runs, so
// processing waves, slots and lanes in order is processing elements in order.
__device__ __forceinline__ int chunk_wave_span(int cnt) { return 64 * ((cnt + kThreads - 1) / kThreads); }

// Segments of up to kSmallCap keys: one wave per tile, no workgroup barriers.
// Lane l holds keys 64 i + l (i < kSmallSlots) in registers; 9-bit digits
// (three passes over a 26-bit depth field) with 512 per-digit counters in LDS,
// scanned by the wave with lane l owning counters 8 l .. 8 l + 7.  The wave's
// LDS accesses execute in issue order, so the wave_barrier() compiler fences
// are all the ordering the counter and buffer updates need.
constexpr int kSmallSlots = 16;
constexpr int kSmallCap = 64 * kSmallSlots;  // 1024 keys
constexpr int kSmallDigitBits = 9;
constexpr int kSmallRadix = 1 << kSmallDigitBits;

// Lanes of the wave holding the same kBits-bit digit d (among valid lanes);
// the same per-bit ballot filtering as gs_sort::match_digit.
template <int kBits>
__device__ __forceinline__ u64 match_bits(unsigned d, bool valid) {
  const u64 v = __ballot(valid);
  unsigned lo = (unsigned)v, hi = (unsigned)(v >> 32);
#pragma unroll
  for (int b = 0; b < kBits; ++b) {
    const unsigned sb = (unsigned)__builtin_amdgcn_sbfe((int)d, b, 1);
    const u64 m = __ballot(sb != 0u);
    lo = __builtin_amdgcn_bitop3_b32((unsigned)m, lo, sb, 0x84);
    hi = __builtin_amdgcn_bitop3_b32((unsigned)(m >> 32), hi, sb, 0x84);
  }
  return ((u64)hi << 32) | lo;
}

// Inclusive prefix sum over the 64 lanes: Hillis-Steele within each row of
// 16 lanes by DPP row shifts (lanes shifted in from outside the row read 0),
// then the totals of the rows below added from three lane reads.
__device__ __forceinline__ unsigned wave_inclusive_scan_u32(unsigned x) {
  x += (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xF, 0xF, true);  // row_shr:1
  x += (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xF, 0xF, true);  // row_shr:2
  x += (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xF, 0xF, true);  // row_shr:4
  x += (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xF, 0xF, true);  // row_shr:8
  const unsigned r0 = (unsigned)__builtin_amdgcn_readlane((int)x, 15);
  const unsigned r1 = (unsigned)__builtin_amdgcn_readlane((int)x, 31);
  const unsigned r2 = (unsigned)__builtin_amdgcn_readlane((int)x, 47);
  const int row = (threadIdx.x & 63) >> 4;
  return x + (row >= 1 ? r0 : 0u) + (row >= 2 ? r1 : 0u) + (row >= 3 ? r2 : 0u);
}

// The wave's LDS for one short segment.
struct SmallShared {
  u64 buf[kSmallCap];
  uint4 wc4[kSmallRadix / 4];
};

__device__ __forceinline__ void small_segment_sort(long long n, u64* __restrict__ keys, int2 rg, int lo_bit,
                                                   int key_bits, int value_bits, int* __restrict__ point_list,
                                                   int write_keys, SmallShared& sh) {
  u64* const s_buf = sh.buf;
  uint4* const s_wc4 = sh.wc4;
  unsigned* s_wc = reinterpret_cast<unsigned*>(s_wc4);
  const int lane = threadIdx.x & 63;
  const long long start = rg.x < 0 ? 0 : (rg.x > n ? n : rg.x);
  const long long end = rg.y < start ? start : (rg.y > n ? n : rg.y);
  const int cnt = (int)(end - start);
  if (cnt <= 0 || cnt > kSmallCap) return;
  const int nslots = (cnt + 63) >> 6;
  const u64 vmask = (1ull << value_bits) - 1ull;
  const u64 lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  u64 key[kSmallSlots];
  bool valid[kSmallSlots];
#pragma unroll
  for (int i = 0; i < kSmallSlots; ++i) {
    valid[i] = i < nslots && 64 * i + lane < cnt;
    key[i] = valid[i] ? keys[start + 64 * i + lane] : 0ull;
  }
  const uint4 zero4 = make_uint4(0u, 0u, 0u, 0u);
  s_wc4[2 * lane] = zero4;
  s_wc4[2 * lane + 1] = zero4;
  __builtin_amdgcn_wave_barrier();
  const int passes = (key_bits + kSmallDigitBits - 1) / kSmallDigitBits;
  for (int pass = 0; pass < passes; ++pass) {
    const int shift = lo_bit + kSmallDigitBits * pass;
    const int bits = key_bits - kSmallDigitBits * pass < kSmallDigitBits ? key_bits - kSmallDigitBits * pass
                                                                         : kSmallDigitBits;
    const unsigned dmask = (1u << bits) - 1u;
    unsigned rank[kSmallSlots];
#pragma unroll
    for (int i = 0; i < kSmallSlots; ++i) {
      rank[i] = 0;
      if (i < nslots) {
        const unsigned d = (unsigned)(key[i] >> shift) & dmask;
        const u64 peers = match_bits<kSmallDigitBits>(d, valid[i]);
        unsigned before = 0;
        if (valid[i]) before = s_wc[d];
        __builtin_amdgcn_wave_barrier();
        const unsigned below = (unsigned)__popcll(peers & lt_mask);
        if (valid[i] && below == 0) s_wc[d] = before + (unsigned)__popcll(peers);
        __builtin_amdgcn_wave_barrier();
        rank[i] = before + below;
      }
    }
    // counters -> exclusive digit starts
    {
      const uint4 a = s_wc4[2 * lane];
      const uint4 b = s_wc4[2 * lane + 1];
      const unsigned t = a.x + a.y + a.z + a.w + b.x + b.y + b.z + b.w;
      unsigned e = wave_inclusive_scan_u32(t) - t;
      uint4 ea, eb;
      ea.x = e; e += a.x;
      ea.y = e; e += a.y;
      ea.z = e; e += a.z;
      ea.w = e; e += a.w;
      eb.x = e; e += b.x;
      eb.y = e; e += b.y;
      eb.z = e; e += b.z;
      eb.w = e;
      s_wc4[2 * lane] = ea;
      s_wc4[2 * lane + 1] = eb;
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < kSmallSlots; ++i) {
      if (valid[i]) s_buf[s_wc[(unsigned)(key[i] >> shift) & dmask] + rank[i]] = key[i];
    }
    __builtin_amdgcn_wave_barrier();
    s_wc4[2 * lane] = zero4;
    s_wc4[2 * lane + 1] = zero4;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < kSmallSlots; ++i)
      if (valid[i]) key[i] = s_buf[64 * i + lane];
    __builtin_amdgcn_wave_barrier();
  }
#pragma unroll
  for (int i = 0; i < kSmallSlots; ++i) {
    if (valid[i]) {
      point_list[start + 64 * i + lane] = (int)(key[i] & vmask);
      if (write_keys) keys[start + 64 * i + lane] = key[i];
    }
  }
}

__device__ __forceinline__ void long_segment_sort(long long n, u64* __restrict__ keys, u64* __restrict__ keys_alt,
                                                  int2 rg, int lo_bit, int key_bits, int value_bits,
                                                  int* __restrict__ point_list, int write_keys, Shared& s) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const long long start = rg.x < 0 ? 0 : (rg.x > n ? n : rg.x);
  const long long end = rg.y < start ? start : (rg.y > n ? n : rg.y);
  const int cnt_all = (int)(end - start);
  if (cnt_all <= kSmallCap) return;  // small_segment_sort's
  const u64 vmask = (1ull << value_bits) - 1ull;
  const int passes = (key_bits + 7) / 8;

  if (cnt_all <= kCap) {
    const int cw = chunk_wave_span(cnt_all);
    const int nslots = cw / 64;
    u64 key[kSlots];
    bool valid[kSlots];
    int elem[kSlots];
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      elem[i] = wave * cw + 64 * i + lane;
      valid[i] = i < nslots && elem[i] < cnt_all;
      key[i] = valid[i] ? keys[start + elem[i]] : 0ull;
    }
    for (int i = tid; i < kWaves * kRadix; i += kThreads) (&s.wc[0][0][0])[i] = 0;
    __syncthreads();
    for (int pass = 0; pass < passes; ++pass) {
      const int b = pass & 1;
      const int shift = lo_bit + 8 * pass;
      const unsigned dmask = key_bits - 8 * pass >= 8 ? 0xFFu : ((1u << (key_bits - 8 * pass)) - 1u);
      unsigned rank[kSlots];
      rank_slots(key, valid, nslots, shift, dmask, s.wc[b][wave], rank);
      __syncthreads();
      {
        const int d = tid;
        unsigned run = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
          const unsigned c = s.wc[b][w][d];
          s.wc[b][w][d] = run;
          s.wc[b ^ 1][w][d] = 0;
          run += c;
        }
        unsigned tot;
        s.base[d] = gs_sort::block_exclusive_scan_u32(run, s.lds_w, &tot);
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < kSlots; ++i) {
        if (valid[i]) {
          const unsigned d = gs_sort::digit_of(key[i], shift, dmask);
          s.buf[s.base[d] + s.wc[b][wave][d] + rank[i]] = key[i];
        }
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < kSlots; ++i)
        if (valid[i]) key[i] = s.buf[elem[i]];
    }
    // key[i] is now sorted element elem[i]; waves cover contiguous runs.
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      if (valid[i]) {
        point_list[start + elem[i]] = (int)(key[i] & vmask);
        if (write_keys) keys[start + elem[i]] = key[i];
      }
    }
    return;
  }

  // Long segment: ping-pong through global memory.
  u64* src = keys + start;
  u64* dst = keys_alt + start;
  unsigned* cnt = &s.wc[1][0][0];
  for (int pass = 0; pass < passes; ++pass) {
    const int shift = lo_bit + 8 * pass;
    const unsigned dmask = key_bits - 8 * pass >= 8 ? 0xFFu : ((1u << (key_bits - 8 * pass)) - 1u);
    cnt[tid] = 0;
    for (int w = 0; w < kWaves; ++w) s.wc[0][w][tid] = 0;
    __syncthreads();
    for (int e = tid; e < cnt_all; e += kThreads) atomicAdd(&cnt[gs_sort::digit_of(src[e], shift, dmask)], 1u);
    __syncthreads();
    {
      unsigned tot;
      s.base[tid] = gs_sort::block_exclusive_scan_u32(cnt[tid], s.lds_w, &tot);
    }
    __syncthreads();
    for (int c0 = 0; c0 < cnt_all; c0 += kCap) {
      const int ccnt = cnt_all - c0 < kCap ? cnt_all - c0 : kCap;
      const int cw = chunk_wave_span(ccnt);
      const int nslots = cw / 64;
      u64 key[kSlots];
      bool valid[kSlots];
#pragma unroll
      for (int i = 0; i < kSlots; ++i) {
        const int e = wave * cw + 64 * i + lane;
        valid[i] = i < nslots && e < ccnt;
        key[i] = valid[i] ? src[c0 + e] : 0ull;
      }
      unsigned rank[kSlots];
      rank_slots(key, valid, nslots, shift, dmask, s.wc[0][wave], rank);
      __syncthreads();
      unsigned run = 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const unsigned c = s.wc[0][w][tid];
        s.wc[0][w][tid] = run;
        run += c;
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < kSlots; ++i) {
        if (valid[i]) {
          const unsigned d = gs_sort::digit_of(key[i], shift, dmask);
          dst[s.base[d] + s.wc[0][wave][d] + rank[i]] = key[i];
        }
      }
      __syncthreads();
      s.base[tid] += run;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) s.wc[0][w][tid] = 0;
      __threadfence_block();
      __syncthreads();
    }
    u64* t = src;
    src = dst;
    dst = t;
  }
  for (int e = tid; e < cnt_all; e += kThreads) {
    const u64 k = src[e];
    point_list[start + e] = (int)(k & vmask);
    if (write_keys && src != keys + start) keys[start + e] = k;
  }
}

// One launch for every segment.  The grid's first min(num_tiles,
// kLongWorkgroups) workgroups take the segments longer than kSmallCap, one
// 256-thread workgroup at a time, tiles b, b + kLongWorkgroups, ... (the
// others are skipped at once), so that the long sorts start first and run
// beside the short ones; the rest of the grid takes the short segments four
// at a time, one wave each (its path has no workgroup barrier).  With an order
// (longest list first) the long segments come first and a workgroup's four
// short ones are of about one length, so its waves finish together.
constexpr int kLongWorkgroups = 1024;

__global__ __launch_bounds__(kThreads) void segment_sort_kernel(long long n, u64* __restrict__ keys,
                                                               u64* __restrict__ keys_alt, int num_tiles,
                                                               const int2* __restrict__ ranges, int lo_bit,
                                                               int key_bits, int value_bits,
                                                               int* __restrict__ point_list, int write_keys,
                                                               const int* __restrict__ order) {
  __shared__ union Lds {
    Shared big;
    SmallShared small[kWaves];
  } lds;
  const int long_wgs = min(num_tiles, kLongWorkgroups);
  if ((int)blockIdx.x < long_wgs) {
    for (int b = blockIdx.x; b < num_tiles; b += long_wgs) {
      const int tile = order ? max(0, min(order[b], num_tiles - 1)) : b;
      long_segment_sort(n, keys, keys_alt, ranges[tile], lo_bit, key_bits, value_bits, point_list, write_keys,
                        lds.big);
      __syncthreads();  // the next segment reuses the LDS
    }
    return;
  }
  const int wave = threadIdx.x >> 6;
  const int slot = ((int)blockIdx.x - long_wgs) * kWaves + wave;
  if (slot >= num_tiles) return;
  const int tile = order ? max(0, min(order[slot], num_tiles - 1)) : slot;
  small_segment_sort(n, keys, ranges[tile], lo_bit, key_bits, value_bits, point_list, write_keys, lds.small[wave]);
}

}  // namespace gs_seg

int gs_sort_tile_segments_ordered(int64_t n, uint64_t* keys, uint64_t* keys_alt, int32_t num_tiles,
                                  const int32_t* ranges, int32_t lo_bit, int32_t key_bits, int32_t value_bits,
                                  int32_t* point_list, int32_t write_keys, const int32_t* order, void* stream) {
  if (n < 0 || num_tiles < 0 || key_bits < 0 || value_bits < 1 || value_bits > 31 || lo_bit < value_bits ||
      lo_bit + key_bits > 64)
    return GS_ERR_INVALID_ARGUMENT;
  if (n > 0x7fffffffLL) return GS_ERR_OVERFLOW;
  if (n == 0 || num_tiles == 0) return GS_OK;
  if (!keys || !keys_alt || !ranges || !point_list) return GS_ERR_INVALID_ARGUMENT;
  const int grid = std::min(num_tiles, gs_seg::kLongWorkgroups) + (num_tiles + gs_seg::kWaves - 1) / gs_seg::kWaves;
  hipLaunchKernelGGL(gs_seg::segment_sort_kernel, dim3(grid), dim3(gs_seg::kThreads), 0, (hipStream_t)stream,
                     (long long)n, reinterpret_cast<gs_sort::u64*>(keys), reinterpret_cast<gs_sort::u64*>(keys_alt),
                     num_tiles, reinterpret_cast<const int2*>(ranges), lo_bit, key_bits, value_bits, point_list,
                     write_keys, order);
  return gs_status_from_hip(hipGetLastError());
}

extern "C" int gs_sort_tile_segments(int64_t n, uint64_t* keys, uint64_t* keys_alt, int32_t num_tiles,
                                     const int32_t* ranges, int32_t lo_bit, int32_t key_bits, int32_t value_bits,
                                     int32_t* point_list, int32_t write_keys, void* stream) {
  return gs_sort_tile_segments_ordered(n, keys, keys_alt, num_tiles, ranges, lo_bit, key_bits, value_bits, point_list,
                                       write_keys, nullptr, stream);
}
