// Shared device-side definitions for the gfx950 Gaussian-splatting rasterizer.
//
// Everything here that feeds an integer decision (radius, tile rectangle,
// tile coverage, alpha >= 1/255, transmittance cut-off) is written as plain
// IEEE-754 binary32 arithmetic in a fixed evaluation order.  The library is
// compiled with -ffp-contract=off and correctly rounded fp32 divide/sqrt, so
// every such decision is reproducible bit-for-bit by a host compiler that
// evaluates the same expressions with the same flags.
//
// Reference semantics followed (file:line into fancifulland2718/gswarp 1.1.0):
//   constants           gswarp/_internal/backends/warp/constants.py:5-45
//   tile rect           gswarp/_internal/backends/warp/math_kernels.py:137-148
//   SnugBox rect        gswarp/_internal/backends/warp/math_kernels.py:151-194
//   conic-rect test     gswarp/_internal/backends/warp/math_kernels.py:197-240
//   AccuTile band       gswarp/_internal/backends/warp/math_kernels.py:243-303
//   tile count          gswarp/_internal/backends/warp/math_kernels.py:306-390
//   NDC -> pixel        gswarp/_internal/backends/warp/math_kernels.py:86-87
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#pragma clang fp contract(off)

namespace gs {

constexpr int kBlockX = 16;
constexpr int kBlockY = 16;
constexpr int kTilePixels = kBlockX * kBlockY;
constexpr int kChannels = 3;

// Real spherical-harmonics constants of the 3DGS convention, rounded to fp32.
constexpr float kShC0 = 0.28209479177387814f;
constexpr float kShC1 = 0.4886025119029199f;
constexpr float kShC2_0 = 1.0925484305920792f;
constexpr float kShC2_1 = -1.0925484305920792f;
constexpr float kShC2_2 = 0.31539156525252005f;
constexpr float kShC2_3 = -1.0925484305920792f;
constexpr float kShC2_4 = 0.5462742152960396f;
constexpr float kShC3_0 = -0.5900435899266435f;
constexpr float kShC3_1 = 2.890611442640554f;
constexpr float kShC3_2 = -0.4570457994644658f;
constexpr float kShC3_3 = 0.3731763325901154f;
constexpr float kShC3_4 = -0.4570457994644658f;
constexpr float kShC3_5 = 1.445305721320277f;
constexpr float kShC3_6 = -0.5900435899266435f;

constexpr float kNearPlane = 0.2f;
constexpr float kFovClamp = 1.3f;
constexpr float kDetEps = 1.0e-7f;
constexpr float kOneMinusAlphaMin = 1.0e-5f;
constexpr float kSnugPad = 1.0f;
constexpr float kQEps = 1.0e-4f;
constexpr float kFloatMax = 3.402823466e38f;
constexpr float kAlphaMin = 1.0f / 255.0f;
constexpr float kTransmittanceMin = 0.0001f;
constexpr float kAlphaMax = 0.99f;

// Comparison predicates of the lane-mask compare builtins
// (__builtin_amdgcn_fcmpf / sicmp; LLVM's predicate codes).
constexpr int kCmpOEQ = 1, kCmpOGE = 3, kCmpOLT = 4, kCmpOLE = 5, kCmpULT = 36, kCmpSLT = 40;

constexpr int kCoverageSnugbox = 0;
constexpr int kCoverageAccutile = 1;
constexpr int kCoverageConicRect = 2;
constexpr int kConicMaskMaxTiles = 64;

// Per-Gaussian render record, 48 bytes = three float4:
//   r0 = (x, y, conic_a, conic_b)
//   r1 = (conic_c, opacity, depth, qcut)
//   r2 = (r, g, b, extents): extents = record_extents(r0, r1), two binary16
// The blend loops evaluate the Gaussian exponent of a pixel at offset
// (dx, dy) = (x - px, y - py) as power = -0.5 q with the quadratic form
//   q = fma(fma(c, dy, 2 b dx), dy, a dx dx)        (conic_q_px below)
// and qcut = -2 power_cutoff (quad_cutoff()): a pixel with q > qcut has an
// alpha provably below 1/255, so the loops skip its exponential without
// changing any decision; 0 <= q <= qcut is the candidate test.
constexpr int kRecordFloats = 12;

__host__ __device__ __forceinline__ float fminr(float a, float b) { return a < b ? a : b; }
__host__ __device__ __forceinline__ float fmaxr(float a, float b) { return a > b ? a : b; }
__host__ __device__ __forceinline__ int imin(int a, int b) { return a < b ? a : b; }
__host__ __device__ __forceinline__ int imax(int a, int b) { return a > b ? a : b; }
__host__ __device__ __forceinline__ float clampr(float x, float lo, float hi) {
  return x < lo ? lo : (x > hi ? hi : x);
}

// Truncating float -> int32 conversion with defined results everywhere:
// NaN -> 0, saturation at the int32 range (the semantics of the hardware
// conversion instruction, made explicit so host code can reproduce it).
__host__ __device__ __forceinline__ int f2i(float f) {
  if (!(f == f)) return 0;
  if (f >= 2147483648.0f) return 2147483647;
  if (f <= -2147483648.0f) return (-2147483647 - 1);
  return (int)f;
}

// Software exponential of the blend loops.  exp(x), x <= 0, is defined as
// Cody-Waite range reduction x = n ln2 + r, |r| <= ln2/2, with n the integer
// nearest to x log2(e) (one fused multiply-add onto 1.5 * 2^23, which leaves
// n in the low mantissa bits, then one exact subtraction) and ln2 split into
// an exact 9-bit head and a tail; then a degree-6 minimax polynomial of e^r
// (relative error 3.6e-9 on |r| <= ln2/2; coefficients from Lawson's
// iteration, rounded to float) in Horner form and an exact scaling by 2^n:
//   t = fma(x, log2e, 1.5*2^23), n = t - 1.5*2^23,
//   r = fma(n, -ln2_lo, fma(n, -ln2_hi, x)),
//   p = fma(...fma(fma(c6, r, c5), r, c4)..., r, 1), exp = p 2^n.
// Every step is one correctly rounded operation, so a host evaluating the same
// sequence reproduces the result bit for bit; against a long double exp it is
// within 0.9 ulp at every float of [-87, 0].  Below -87 it is defined as 0
// (the result would be below 1.7e-38 and only ever feeds an alpha < 1/255
// decision), and the loops never evaluate it there.
//
// exp_sw_q(q) evaluates exp(-q/2) of the loops' quadratic forms, q in
// [-0, 174] (they need it only where 0 <= q <= qcut, and qcut = -2
// power_cutoff <= 174), by the same operations on q = -2x with every
// intermediate scaled by a power of two, which commutes with each rounding:
// the product q (-log2(e)/2), the reduced argument carried as rho = -2r and
// the polynomial in rho with the coefficients c_k (-1/2)^k.  2^n is applied
// by adding n << 23 to the exponent field (t's bits << 23 equal n << 23
// modulo 2^32, since 1.5 * 2^23 contributes only bits at or above 2^45); for
// q <= 174 the result is a normal number, so this is exact.  The result is
// bit-identical to the x form at x = -q/2 (checked at every float of
// [-87, 0]) and needs no conversion, rounding or ldexp instruction.  For q
// outside the range the value is unspecified; the loops mask such lanes out.
constexpr float kExpMagic = 12582912.0f;  // 1.5 * 2^23
constexpr float kExpLog2e = 1.44269504088896341f;
constexpr float kExpLn2Hi = 0.693359375f;
constexpr float kExpLn2Lo = -2.12194440e-4f;
constexpr float kExpC2 = 0x1.fffffcp-2f, kExpC3 = 0x1.555492p-3f, kExpC4 = 0x1.5558f2p-5f, kExpC5 = 0x1.123a2p-7f,
                kExpC6 = 0x1.6a23dp-10f;

__device__ __forceinline__ float exp_sw_q(float q) {
  const float t = fmaf(q, -0.5f * kExpLog2e, kExpMagic);
  const float n = t - kExpMagic;
  float rho = fmaf(n, 2.0f * kExpLn2Hi, q);
  rho = fmaf(n, 2.0f * kExpLn2Lo, rho);
  float p = fmaf(kExpC6 * (1.0f / 64.0f), rho, kExpC5 * (-1.0f / 32.0f));
  p = fmaf(p, rho, kExpC4 * (1.0f / 16.0f));
  p = fmaf(p, rho, kExpC3 * (-1.0f / 8.0f));
  p = fmaf(p, rho, kExpC2 * (1.0f / 4.0f));
  p = fmaf(p, rho, -0.5f);
  p = fmaf(p, rho, 1.0f);
  return __uint_as_float(__float_as_uint(p) + (__float_as_uint(t) << 23));
}

// ln(y) for finite y > 0: y = m * 2^e with m in [sqrt(1/2), sqrt(2)), then
// ln(m) = 2*atanh(s), s = (m-1)/(m+1), |s| <= 0.1716, by its odd series to
// s^11.  ln2 is split into a head with trailing zero bits and a tail so that
// e*ln2_hi is exact.
__device__ __forceinline__ float log_sw(float y) {
  int e;
  float m = frexpf(y, &e);
  if (m < 0.70710678118654752f) {
    m = m * 2.0f;
    e = e - 1;
  }
  const float s = (m - 1.0f) / (m + 1.0f);
  const float s2 = s * s;
  float p = 0.0909090909f;           // 1/11
  p = p * s2 + 0.111111111f;         // 1/9
  p = p * s2 + 0.142857143f;         // 1/7
  p = p * s2 + 0.2f;                 // 1/5
  p = p * s2 + 0.333333333f;         // 1/3
  const float lnm = 2.0f * s + (2.0f * s) * (s2 * p);
  const float ef = (float)e;
  return ef * 0.693145751953125f + (lnm + ef * 1.42860677e-6f);
}

// Largest exponent below which o*exp(power) < 1/255 holds for every power,
// with a 1e-3 margin that covers exp_sw_q and product rounding (relative error
// < 1e-6).  Returns FLT_MAX when the Gaussian can never reach the alpha
// cut-off.  Never below -87: the software exponential is 0 there, so alpha is 0 and skipping
// those exponents changes no decision either.
__device__ __forceinline__ float power_cutoff(float opacity) {
  const float o255 = 255.0f * opacity;
  if (!(o255 > 1.0f)) return kFloatMax;
  if (o255 > 1.0e37f) return -87.0f;
  return fmaxr(-log_sw(o255) - 1.0e-3f, -87.0f);
}

// Whether a render record can pass the blend loops' candidate test
// 0 <= q <= qcut at any pixel centre near its mean.  The candidate set is the
// ellipse
//   Q(d) = a dx^2 + 2 b dx dy + c dy^2 <= qcut,
// whose bounding box has half-widths sqrt(qcut c / det) and
// sqrt(qcut a / det), det = a c - b^2.  The loops evaluate q in fp32 with
// two fused multiply-adds over per-lane products: every rounding is
// relative to a term of magnitude at most qcut * (a c / det) inside the box,
// so the fp32 q can pass the test only where the exact Q <= qcut
// (1 + 4 * 2^-24 * 3 * ac/det).  The half-widths are computed in double (a c
// and b^2 are exact there) for qcut inflated ten times that bound, plus
// 0.02 px; conics that are not positive definite or so elongated
// (ac/det >= 1e5) that the bound is weak are never culled (infinite
// half-widths), and a record that no pixel can blend (qcut < 0) gets
// negative infinite ones.  The preprocess stores them in the record's last
// word (record_extents), so the blend kernels test a batch against a pixel
// rectangle with a few fp32 operations (extents_meet) instead of evaluating
// the box per batch.  Meeting is always safe to report: it only costs the
// per-pixel test.

// x >= 0 (or +inf) as binary16, rounded up.
__device__ __forceinline__ unsigned half_bits_up(float x) {
  const _Float16 h = (_Float16)x;  // round to nearest (overflow: +inf)
  unsigned bits = (unsigned)__builtin_bit_cast(unsigned short, h);
  if ((float)h < x) bits += 1u;  // the next binary16 above (0x7bff + 1 = +inf)
  return bits;
}

// The record's candidate half-widths (ex, ey) about its mean (r0.x, r0.y),
// as two binary16 rounded up, ex in the low half: widened by 1/64 px, which
// covers the fp32 rounding of extents_meet's sums for coordinates below
// 2^16 (beyond that the widths are infinite).  Never-culled conics: +inf;
// records that no pixel blends: -inf.
__device__ __forceinline__ unsigned record_extents(float4 r0, float4 r1) {
  const unsigned kInf = 0x7C00u, kNegInf = 0xFC00u;
  const float qcut = r1.w;
  if (qcut < 0.0f) return kNegInf | (kNegInf << 16);  // alpha < 1/255 at every exponent <= 0
  const double a = r0.z, b = r0.w, c = r1.x;
  const double ac = a * c;
  const double det = ac - b * b;
  if (!(a > 0.0 && c > 0.0 && det > 0.0 && ac < 1.0e5 * det)) return kInf | (kInf << 16);
  const double q = (double)qcut * (1.0 + 8.0e-6 * (ac / det)) + 1.0e-6;
  const double ex = sqrt(q * c / det) + 0.02 + 1.0 / 64.0;
  const double ey = sqrt(q * a / det) + 0.02 + 1.0 / 64.0;
  const double far = 65536.0;
  if (!(fabs((double)r0.x) + ex < far && fabs((double)r0.y) + ey < far)) return kInf | (kInf << 16);
  // double -> float rounded up, then -> binary16 rounded up
  float fx = (float)ex, fy = (float)ey;  // positive and finite here
  if ((double)fx < ex) fx = __uint_as_float(__float_as_uint(fx) + 1u);
  if ((double)fy < ey) fy = __uint_as_float(__float_as_uint(fy) + 1u);
  return half_bits_up(fx) | (half_bits_up(fy) << 16);
}

// Whether a record with half-widths word w about (cx, cy) may meet the pixel
// rectangle [x0, x1] x [y0, y1] (pixel centres).
__device__ __forceinline__ bool extents_meet(float cx, float cy, unsigned w, float x0, float x1, float y0,
                                             float y1) {
  const float ex = (float)__builtin_bit_cast(_Float16, (unsigned short)(w & 0xFFFFu));
  const float ey = (float)__builtin_bit_cast(_Float16, (unsigned short)(w >> 16));
  return cx + ex >= x0 && cx - ex <= x1 && cy + ey >= y0 && cy - ey <= y1;
}

// Largest quadratic form q at which alpha can still reach 1/255:
// -2 * power_cutoff (exact scaling); -inf when it never can.
__device__ __forceinline__ float quad_cutoff(float opacity) { return -2.0f * power_cutoff(opacity); }

// The blend loops' quadratic form of a pixel offset, from the per-lane
// adxx = (a dx) dx and b2dx = (b dx) 2 shared by a lane's pixels:
// q = fma(fma(c, dy, b2dx), dy, adxx); the exponent is -0.5 q (exact).
__device__ __forceinline__ float conic_q_px(float adxx, float b2dx, float c, float dy) {
  return fmaf(fmaf(c, dy, b2dx), dy, adxx);
}

// The candidate test 0 <= q <= qcut as one unsigned compare of q's bits: for
// q >= +0 (sign bit clear) bits(q) < cand_threshold(qcut) exactly when
// q <= qcut; negative q, -0 and NaN have larger bits, and a negative or NaN
// qcut allows nothing (0).  q = -0 passes the float test but not this one; it
// needs a <= 0 (adxx = (a dx) dx is then -0 for dx = 0), so the loops add the
// q == 0 lanes only for batches holding such a conic.
__device__ __forceinline__ unsigned cand_threshold(float qcut) {
  return qcut >= 0.0f ? __float_as_uint(qcut) + 1u : 0u;
}

// A render record as the blend kernels load it: three float4.
struct RecordRegs {
  float4 r0, r1, r2;
};

__device__ __forceinline__ RecordRegs load_record(const float4* records, int id) {
  const float4* rec = records + 3 * (size_t)id;
  RecordRegs r;
  r.r0 = rec[0];
  r.r1 = rec[1];
  r.r2 = rec[2];
  return r;
}

// A list entry's Gaussian index, 0 for an index outside [0, num_points)
// (which only inconsistent caller input can hold).
__device__ __forceinline__ int checked_point(int id, int num_points) {
  return (unsigned)id < (unsigned)num_points ? id : 0;
}

// The entry of lane `lane` in the batch [first, first + cnt) of a list of n
// >= 1 entries.  Lanes past the batch read its first entry, and an empty
// batch reads a valid one, so the blend kernels can issue the load
// unconditionally: nothing merges the loaded value with another, and so no
// wait for it comes before it is used, a batch later.
__device__ __forceinline__ int batch_entry(const int* list, int first, int cnt, int n, int lane) {
  return list[imax(0, imin(first + imin(lane, imax(cnt, 1) - 1), n - 1))];
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

__device__ __forceinline__ long long wave_sum_i64(long long v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// The one-pass scan's aggregates of kScanAggGaussians consecutive Gaussians
// (one 256-thread workgroup, thread t: Gaussian 256 b + t): the smallest
// and largest float bits of the depths of the visible ones (radius > 0;
// ~0u / 0 when there are none), the super-tile units of the valid cover
// words, their number, and whether a Gaussian with tiles has no valid word.
// Stored as kScanAggWords words at agg + kScanAggWords * b: max << 32 | min,
// the units (-1 in the last case) and the valid words.  Every thread of the
// workgroup calls it (it holds a barrier).
constexpr int kScanAggGaussians = 256;
constexpr int kScanAggWords = 3;

struct ScanAggLds {
  unsigned mn[4], mx[4];
  long long units[4];
  int valid[4], bad[4];
};

__device__ __forceinline__ void store_scan_aggregates(bool visible, float depth, int units, int valid, int bad,
                                                      ScanAggLds& lds, unsigned long long* agg) {
  const unsigned bits = __float_as_uint(depth);
  const unsigned mn = wave_min_u32(visible ? bits : ~0u);
  const unsigned mx = wave_max_u32(visible ? bits : 0u);
  const long long u = wave_sum_i64(units);
  const long long v = wave_sum_i64(valid);
  const long long bd = wave_sum_i64(bad);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    lds.mn[wave] = mn;
    lds.mx[wave] = mx;
    lds.units[wave] = u;
    lds.valid[wave] = (int)v;
    lds.bad[wave] = (int)bd;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned lo = ~0u, hi = 0u;
    long long units_all = 0, valid_all = 0;
    int bad_all = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      lo = lds.mn[w] < lo ? lds.mn[w] : lo;
      hi = lds.mx[w] > hi ? lds.mx[w] : hi;
      units_all += lds.units[w];
      valid_all += lds.valid[w];
      bad_all |= lds.bad[w];
    }
    unsigned long long* q = agg + (size_t)kScanAggWords * blockIdx.x;
    q[0] = ((unsigned long long)hi << 32) | lo;
    q[1] = bad_all ? ~0ull : (unsigned long long)units_all;
    q[2] = (unsigned long long)valid_all;
  }
}

// Inclusive sum over the wave with DPP row shifts (rows of 16 lanes, no LDS
// round trip) and the three row totals read back: about a dozen
// instructions and no memory latency.
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

// Workgroups are dispatched round-robin over the eight XCDs (each with its
// own L2).  Mapping workgroup b to tile start(b % 8) + b / 8 gives every XCD
// one contiguous band of tiles, so neighbouring tiles, which share most of
// their Gaussians, hit the same L2.  Bijective on [0, num_tiles).
__device__ __forceinline__ int xcd_tile(int b, int num_tiles) {
  const int q = num_tiles >> 3;
  const int r = num_tiles & 7;
  const int xcd = b & 7;
  return xcd * q + (xcd < r ? xcd : r) + (b >> 3);
}

// The tile kernels deal their work units (a tile, or one slice of a tile;
// the units of a tile are consecutive) to the XCDs in chunks of kXcdChunk
// consecutive units: chunk j runs on XCD j % 8.  Each XCD then gets runs of
// horizontally neighbouring tiles, which share most of their Gaussians in its
// L2, from every part of the image, so the eight XCDs carry nearly equal
// work.  (With one contiguous band of the image per XCD, xcd_tile, the bands
// through the image centre, where the Gaussians concentrate, carried up to
// 1.4 times the mean work of a band.)  kXcdChunk 0 selects the banding.
#ifndef GS_XCD_CHUNK
#define GS_XCD_CHUNK 32
#endif
constexpr int kXcdChunk = GS_XCD_CHUNK;

// Workgroups to launch for num_units units (whole chunks for every XCD);
// xcd_unit returns >= num_units for the padding workgroups.
__host__ __device__ __forceinline__ int xcd_grid(int num_units) {
  if (kXcdChunk <= 0) return (num_units + 7) & ~7;
  const int span = 8 * kXcdChunk;
  return (num_units + span - 1) / span * span;
}

// Unit of workgroup b (dispatched to XCD b % 8), a bijection of
// [0, xcd_grid(num_units)).
__device__ __forceinline__ int xcd_unit(int b, int num_units) {
  if (kXcdChunk <= 0) return xcd_tile(b, xcd_grid(num_units));
  const int u = b >> 3;  // this workgroup's position among its XCD's workgroups
  return ((u / kXcdChunk) * 8 + (b & 7)) * kXcdChunk + u % kXcdChunk;
}

// The blend kernels take the tiles longest list first (gs_tile_order) when
// the lists hold at most 4 pairs per Gaussian (the backward's halves; the
// heavier lists of its whole-tile walk measured faster in the XCD tile
// order, whose neighbouring tiles share the large Gaussians' records in L2)
// and at least 192 pairs per tile on average: below that the walks are
// short and the order's own launch (about 5 us) costs more than the tail it
// removes (100k Gaussians at 800x800, 95 pairs a tile: 8 us slower).  A
// forward given an order buffer writes the order into it under this
// condition; the backward, given the same buffer, reads it under the same
// condition of the same arguments.
inline bool tile_order_pays(int64_t num_rendered, int64_t num_points, int64_t num_tiles) {
  return num_rendered > 0 && num_rendered <= 4 * num_points && num_rendered >= 192 * num_tiles;
}

__device__ __forceinline__ float lane_f(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

__device__ __forceinline__ int lane_i(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }

__device__ __forceinline__ float ndc_to_pix(float v, int size) {
  return ((v + 1.0f) * (float)size - 1.0f) * 0.5f;
}

// Tile rectangle of the 3-sigma square (truncating casts, clamped to grid).
__device__ __forceinline__ int4 tile_rect(float px, float py, int rx, int ry, int grid_x, int grid_y) {
  int4 r;
  r.x = imin(grid_x, imax(0, f2i((px - (float)rx) / (float)kBlockX)));
  r.y = imin(grid_y, imax(0, f2i((py - (float)ry) / (float)kBlockY)));
  r.z = imin(grid_x, imax(0, f2i((px + (float)rx + (float)(kBlockX - 1)) / (float)kBlockX)));
  r.w = imin(grid_y, imax(0, f2i((py + (float)ry + (float)(kBlockY - 1)) / (float)kBlockY)));
  return r;
}

// Alpha-cutoff threshold of the conic quadratic form: 2*ln(max(255*o, 1)).
__device__ __forceinline__ float coverage_threshold(float opacity) {
  return 2.0f * log_sw(fmaxr(255.0f * opacity, 1.0f));
}

// Padded SnugBox (1/255 cut-off + one pixel) intersected with the 3-sigma rect.
__device__ __forceinline__ int4 snugbox_rect(float px, float py, float cov_aa, float cov_cc, float opacity,
                                             int cuda_radius, int grid_x, int grid_y) {
  const int4 c = tile_rect(px, py, cuda_radius, cuda_radius, grid_x, grid_y);
  const float t = coverage_threshold(opacity);
  if (t <= 0.0f) return make_int4(0, 0, 0, 0);
  const int rx = f2i(ceilf(sqrtf(fmaxr(t * cov_aa, 0.0f)) + kSnugPad));
  const int ry = f2i(ceilf(sqrtf(fmaxr(t * cov_cc, 0.0f)) + kSnugPad));
  const int4 s = tile_rect(px, py, rx, ry, grid_x, grid_y);
  return make_int4(imax(c.x, s.x), imax(c.y, s.y), imin(c.z, s.z), imin(c.w, s.w));
}

__device__ __forceinline__ float conic_q(float x, float y, float a, float b, float c) {
  return a * x * x + 2.0f * b * x * y + c * y * y;
}

__device__ __forceinline__ bool conic_rect_intersects_tile(float px, float py, float a, float b, float c,
                                                           float threshold, int tile_x, int tile_y) {
  const float det = a * c - b * b;
  if (a <= 0.0f || c <= 0.0f || det <= kDetEps) return true;
  const float x0 = (float)(tile_x * kBlockX) - px;
  const float x1 = (float)(tile_x * kBlockX + kBlockX - 1) - px;
  const float y0 = (float)(tile_y * kBlockY) - py;
  const float y1 = (float)(tile_y * kBlockY + kBlockY - 1) - py;
  if (x0 <= 0.0f && x1 >= 0.0f && y0 <= 0.0f && y1 >= 0.0f) return true;
  float qmin = kFloatMax;
  float y = clampr(-b * x0 / c, y0, y1);
  qmin = fminr(qmin, conic_q(x0, y, a, b, c));
  y = clampr(-b * x1 / c, y0, y1);
  qmin = fminr(qmin, conic_q(x1, y, a, b, c));
  float x = clampr(-b * y0 / a, x0, x1);
  qmin = fminr(qmin, conic_q(x, y0, a, b, c));
  x = clampr(-b * y1 / a, x0, x1);
  qmin = fminr(qmin, conic_q(x, y1, a, b, c));
  return qmin <= threshold + kQEps;
}

// Exact conic-ellipse interval along the u axis for one band of tiles at
// tile_v, returned as a half-open tile range clamped to [u_min, u_max].
__device__ __forceinline__ int2 accutile_band(float pu, float pv, float cuu, float cuv, float cvv,
                                              float threshold, int tile_v, int block_u, int block_v,
                                              int rect_u_min, int rect_u_max) {
  const float det = cuu * cvv - cuv * cuv;
  if (cuu <= 0.0f || cvv <= 0.0f || det <= kDetEps) return make_int2(rect_u_min, rect_u_max);
  const float ts = threshold + kQEps;
  const float v0 = (float)(tile_v * block_v) - pv;
  const float v1 = (float)(tile_v * block_v + block_v - 1) - pv;
  float umin = kFloatMax;
  float umax = -kFloatMax;
  bool found = false;
  float disc = cuu * ts - det * v0 * v0;
  if (disc >= -kQEps) {
    const float half = sqrtf(fmaxr(disc, 0.0f)) / cuu;
    const float center = -cuv * v0 / cuu;
    umin = fminr(umin, center - half);
    umax = fmaxr(umax, center + half);
    found = true;
  }
  disc = cuu * ts - det * v1 * v1;
  if (disc >= -kQEps) {
    const float half = sqrtf(fmaxr(disc, 0.0f)) / cuu;
    const float center = -cuv * v1 / cuu;
    umin = fminr(umin, center - half);
    umax = fmaxr(umax, center + half);
    found = true;
  }
  const float ext = sqrtf(fmaxr(ts * cvv / det, 0.0f));
  const float v_at_min = cuv * ext / cvv;
  if (v_at_min >= v0 - kQEps && v_at_min <= v1 + kQEps) {
    umin = fminr(umin, -ext);
    umax = fmaxr(umax, -ext);
    found = true;
  }
  const float v_at_max = -cuv * ext / cvv;
  if (v_at_max >= v0 - kQEps && v_at_max <= v1 + kQEps) {
    umin = fminr(umin, ext);
    umax = fmaxr(umax, ext);
    found = true;
  }
  if (!found) return make_int2(rect_u_min, rect_u_min);
  const int tmin = f2i(floorf((pu + umin) / (float)block_u));
  const int tmax = f2i(floorf((pu + umax) / (float)block_u)) + 1;
  return make_int2(imax(rect_u_min, imin(rect_u_max, tmin)), imax(rect_u_min, imin(rect_u_max, tmax)));
}

// Covered tiles of a Gaussian whose tile rectangle has at most
// kCoverMaskCells cells, as a mask in the order of the coverage walk: bit k
// is the k-th cell of the rectangle in band order (row-major for row bands
// and the full or conic-rect walks, column-major for column bands), set when
// the walk emits that tile.  The preprocess records it beside the count, so
// that the emission reads the tiles instead of re-deriving the bands.
constexpr int kCoverMaskCells = 64;

struct TileCover {
  int4 rect;       // tile rectangle [x, z) x [y, w)
  int columns;     // 1: bands are tile columns (column-major mask)
  int valid;       // non-empty rectangle that fits the packed word (origin < 2^16, spans < 2^8)
  int has_mask;    // valid, with at most kCoverMaskCells cells
  int full;        // every tile of the rectangle is covered (area <= 1 or the SnugBox mode)
  int band_off;    // banded (valid, neither mask nor full): index of its stored bands, or -1
  uint64_t mask;
};

// Band store: the coverage bands of a valid Gaussian with neither a mask nor
// a full rectangle, one word per band (interval [lo, hi) of tile columns for
// a row band, of tile rows for a column band: lo | hi << 16), in band order.
// Wave w of a preprocess launch owns words [w kBandSlots, (w + 1) kBandSlots)
// and fills them in lane order; a Gaussian whose bands do not fit its wave's
// region is not stored (band_off -1) and its consumers recompute its bands.
constexpr int kBandSlots = 512;

__device__ __forceinline__ uint64_t low_bits64(int n) { return n >= 64 ? ~0ull : ((1ull << n) - 1ull); }

// Packed per-Gaussian coverage word:
//   x = rect.x | rect.y << 16,
//   y = span_x | span_y << 8 | columns << 16 | has_mask << 17 | valid << 18 | full << 19,
//   z / w = mask low / high with has_mask; else z = the band store index
//   (band_off, -1 when not stored) for a banded Gaussian, and w = 0.
// The word is all zero unless the Gaussian covers a valid rectangle.  Which
// tiles of a valid rectangle are covered follows from the word: all of them
// (full), the mask's cells (has_mask), or else the coverage bands (tile rows,
// or tile columns with `columns`) of the Gaussian's conic.
__device__ __forceinline__ int4 pack_cover(const TileCover& c) {
  const int span_x = c.rect.z - c.rect.x, span_y = c.rect.w - c.rect.y;
  if (!c.valid) return make_int4(0, 0, 0, 0);
  return make_int4(c.rect.x | (c.rect.y << 16),
                   span_x | (span_y << 8) | (c.columns << 16) | (c.has_mask << 17) | (1 << 18) | (c.full << 19),
                   c.has_mask ? (int)(unsigned)c.mask : (c.full ? 0 : c.band_off),
                   c.has_mask ? (int)(unsigned)(c.mask >> 32) : 0);
}

struct CoverWord {
  int rx, ry, span_x, span_y, columns, has_mask, valid, full;
  uint64_t mask;  // with has_mask
  int band_off;   // banded: index into the band store, or -1
};

__device__ __forceinline__ CoverWord unpack_cover(int4 w) {
  CoverWord c;
  c.rx = w.x & 0xffff;
  c.ry = (unsigned)w.x >> 16;
  c.span_x = w.y & 0xff;
  c.span_y = (w.y >> 8) & 0xff;
  c.columns = (w.y >> 16) & 1;
  c.has_mask = (w.y >> 17) & 1;
  c.valid = (w.y >> 18) & 1;
  c.full = (w.y >> 19) & 1;
  c.mask = ((uint64_t)(unsigned)w.w << 32) | (unsigned)w.z;
  c.band_off = w.z;
  return c;
}

// Super-tiles: squares of kSuperTile x kSuperTile tiles, numbered row-major
// over the grid (ceil(grid_x / 8) per row).  A tile's cells within its
// super-tile are bit (ty % 8) * 8 + (tx % 8) of a 64-bit mask.  super_rect
// gives the super-tiles met by a valid cover word's rectangle: nx x ny of
// them from (sx0, sy0); none for an invalid word.
constexpr int kSuperTile = 8;

struct SuperRect {
  int sx0, sy0, nx, ny;
};

__device__ __forceinline__ SuperRect super_rect(const CoverWord& w) {
  SuperRect r;
  r.sx0 = w.rx / kSuperTile;
  r.sy0 = w.ry / kSuperTile;
  r.nx = w.valid ? (w.rx + w.span_x - 1) / kSuperTile - r.sx0 + 1 : 0;
  r.ny = w.valid ? (w.ry + w.span_y - 1) / kSuperTile - r.sy0 + 1 : 0;
  return r;
}

__device__ __forceinline__ int super_units(const CoverWord& w) {
  const SuperRect r = super_rect(w);
  return r.nx * r.ny;
}

// Tile id of cell k of a packed rectangle in band order.  k / span is
// floor((k + 0.5) * rcp(span)): for k < 64 and span <= 64 the quotient is at
// least 0.5 / span away from an integer, far beyond the float error.
__device__ __forceinline__ int cover_cell_tile(const CoverWord& c, float rcp_span_u, int k, int grid_x) {
  const int span_u = c.columns ? c.span_y : c.span_x;
  const int band = (int)(((float)k + 0.5f) * rcp_span_u);
  const int u = k - band * span_u;
  return c.columns ? (c.ry + u) * grid_x + (c.rx + band) : (c.ry + band) * grid_x + (c.rx + u);
}

// Inclusive sum and maximum over the lanes of a wave (every lane active).
__device__ __forceinline__ int wave_inclusive_scan_i32(int x) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  return x;
}

__device__ __forceinline__ int wave_inclusive_max_i32(int x) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x = y > x ? y : x;
  }
  return x;
}

// Per-wave LDS for wave_count_covered_tiles.
struct CoverCountLds {
  int mark[64];
  unsigned count[64];
  unsigned long long mask[64];
};

// Number of tiles each lane's Gaussian is binned to under the given coverage
// mode (active lanes; inactive ones get 0), and its cover mask when the
// rectangle is small enough; every lane of the wave must call it.
// Mode kCoverageConicRect counts tiles exactly only up to kConicMaskMaxTiles
// candidate tiles and falls back to AccuTile beyond that, which is the
// effective behaviour of the reference binning stage for that mode.
// The AccuTile bands of the wave's Gaussians (one tile row or column each,
// rows when span_y <= span_x) are walked flattened over the lanes, 64 bands
// per step, so a step costs one band interval whatever the mix of small and
// large Gaussians: a band's owner is the last lane whose first band is at
// or before it (marks in LDS and a prefix maximum), the owner's parameters
// come by lane shuffle, and each band adds its length and mask bits to its
// owner's LDS accumulators.  The counts and masks are those of the serial
// walk band by band (count_covered_tiles semantics of binning_kernels.py).
// With band_store, the bands of the wave's banded Gaussians are also stored
// in the wave's region starting at band_base (see kBandSlots).
__device__ __forceinline__ int wave_count_covered_tiles(bool active, float px, float py, float cov_aa, float cov_cc,
                                                        float ca, float cb, float cc, float opacity, int cuda_radius,
                                                        int grid_x, int grid_y, int mode, TileCover& cover,
                                                        CoverCountLds& lds, unsigned* band_store = nullptr,
                                                        int band_base = 0) {
  static_assert(kBlockX == kBlockY, "row and column bands share one band routine");
  const int lane = threadIdx.x & 63;
  int count = 0;
  int nbands = 0;
  float threshold = 0.0f;
  cover.rect = make_int4(0, 0, 0, 0);
  cover.columns = 0;
  cover.valid = 0;
  cover.has_mask = 0;
  cover.full = 0;
  cover.band_off = -1;
  cover.mask = 0;
  if (active) {
    const int4 rect = snugbox_rect(px, py, cov_aa, cov_cc, opacity, cuda_radius, grid_x, grid_y);
    const int span_x = rect.z - rect.x;
    const int span_y = rect.w - rect.y;
    const int area = span_x * span_y;
    cover.rect = rect;
    cover.valid = span_x > 0 && span_y > 0 && span_x <= 0xff && span_y <= 0xff && rect.x <= 0xffff &&
                  rect.y <= 0xffff;
    cover.has_mask = cover.valid && area <= kCoverMaskCells;
    if (area <= 1 || mode == kCoverageSnugbox) {
      cover.full = 1;
      count = area;
      if (cover.has_mask) cover.mask = low_bits64(area);
    } else {
      threshold = coverage_threshold(opacity);
      if (mode == kCoverageConicRect && area <= kConicMaskMaxTiles) {
        for (int ty = rect.y; ty < rect.w; ++ty)
          for (int tx = rect.x; tx < rect.z; ++tx)
            if (conic_rect_intersects_tile(px, py, ca, cb, cc, threshold, tx, ty)) {
              ++count;
              if (cover.has_mask) cover.mask |= 1ull << ((ty - rect.y) * span_x + (tx - rect.x));
            }
      } else {
        cover.columns = span_y > span_x;
        nbands = imax(0, cover.columns ? span_x : span_y);
      }
    }
  }
  const int incl = wave_inclusive_scan_i32(nbands);
  const int excl = incl - nbands;
  const int total = __builtin_amdgcn_readlane(incl, 63);
  if (band_store != nullptr) {  // uniform
    const int stored = cover.valid && !cover.has_mask ? nbands : 0;
    const int sincl = wave_inclusive_scan_i32(stored);
    if (stored > 0 && sincl <= kBandSlots) cover.band_off = band_base + sincl - stored;
  }
  lds.count[lane] = 0u;
  lds.mask[lane] = 0ull;
  // the owner's view, gathered once per step by lane shuffle
  const float pu = cover.columns ? py : px, pv = cover.columns ? px : py;
  const float cuu = cover.columns ? cc : ca, cvv = cover.columns ? ca : cc;
  const int v0 = cover.columns ? cover.rect.x : cover.rect.y;
  const int u_min = cover.columns ? cover.rect.y : cover.rect.x;
  const int u_max = cover.columns ? cover.rect.w : cover.rect.z;
  const int mask_span = cover.has_mask ? u_max - u_min : -1;  // -1: no mask
  for (int t0 = 0; t0 < total; t0 += 64) {
    lds.mark[lane] = -1;
    __builtin_amdgcn_wave_barrier();
    if (nbands > 0 && excl < t0 && incl > t0) lds.mark[0] = lane;  // bands carried in from the last step
    __builtin_amdgcn_wave_barrier();
    if (nbands > 0 && excl >= t0 && excl < t0 + 64) lds.mark[excl - t0] = lane;
    __builtin_amdgcn_wave_barrier();
    const int f = t0 + lane;
    const bool valid = f < total;
    const int owner = wave_inclusive_max_i32(lds.mark[lane]);  // every lane takes part
    const int o = (valid && owner >= 0) ? owner : lane;  // every valid position has an owner
    const int b = f - __shfl(excl, o, 64);
    const float o_pu = __shfl(pu, o, 64), o_pv = __shfl(pv, o, 64);
    const float o_cuu = __shfl(cuu, o, 64), o_cuv = __shfl(cb, o, 64), o_cvv = __shfl(cvv, o, 64);
    const float o_thr = __shfl(threshold, o, 64);
    const int o_v0 = __shfl(v0, o, 64), o_umin = __shfl(u_min, o, 64), o_umax = __shfl(u_max, o, 64);
    const int o_mspan = __shfl(mask_span, o, 64);
    const int o_boff = __shfl(cover.band_off, o, 64);
    if (valid) {
      const int2 iv = accutile_band(o_pu, o_pv, o_cuu, o_cuv, o_cvv, o_thr, o_v0 + b, kBlockX, kBlockY, o_umin,
                                    o_umax);
      if (o_boff >= 0) band_store[o_boff + b] = (unsigned)iv.x | ((unsigned)iv.y << 16);
      const int len = imax(0, iv.y - iv.x);
      if (len > 0) {
        atomicAdd(&lds.count[o], (unsigned)len);
        if (o_mspan >= 0) atomicOr(&lds.mask[o], low_bits64(len) << (b * o_mspan + (iv.x - o_umin)));
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
  if (nbands > 0) {
    count += (int)lds.count[lane];
    cover.mask |= lds.mask[lane];
  }
  return count;
}

}  // namespace gs
