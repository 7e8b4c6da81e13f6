// Forward render: each 16x16 tile is covered by 4/kPix independent wave64
// workgroups, each owning a slice of 64 kPix pixels: an 8x8 quadrant for
// one pixel per lane (8x16 halves for two, the whole tile for four); lane l
// owns the pixels of column l % w in rows l / w + (64 / w) k of its slice,
// w its width.  Square slices are visited by fewer Gaussians than 16-wide
// rows of the same size (the footprints are small and round).  The flow
// variant keeps 16-wide rows (16 x 4 kPix slices): its per-pixel top-K
// planes are written in rows of w consecutive floats, and 8-float rows
// leave half of each cache line to another wave.  Pixels of a
// lane share dx to a Gaussian, so a*dx*dx and b*dx are evaluated once per
// lane, exactly as the per-pixel expression would round them.  The tile's
// sorted Gaussians are fetched 64 at a time, one packed 48-byte record per
// lane, with the next batch prefetched into registers while the current one
// is blended from a per-wave LDS slot (the record's three float4 adjacent,
// so one address register serves its broadcast reads; no barriers since
// each workgroup is one wave).  Each batch is
// first tested lane-parallel against the slice rectangle (record_may_touch)
// and only records that may touch the slice are visited.  Per Gaussian the
// per-pixel work is branch-free (select-based updates inside one wave-uniform
// "any candidate" branch) so the pixels' exponential chains interleave.  A
// wave-wide ballot ends the slice once every one of its pixels is done.
//
// Semantics follow render_kernels.py:16-147 (and flow_kernels.py:31-176 for
// the flow variant):
//   power > 0 skipped; alpha = min(0.99, o*exp(power)); alpha < 1/255 skipped;
//   (power = -0.5 q with the record's quadratic form q, see gs_common.h)
//   T*(1-alpha) < 1e-4 ends the pixel without blending that Gaussian;
//   colour += f*alpha*T, alpha_out = sum alpha*T, depth = sum z*alpha*T
//   (colour and depth accumulated with one fused multiply-add per Gaussian);
//   n_contrib = 1-based list index of the last blended Gaussian.
// Quadratic forms above the record's qcut are skipped without evaluating
// exp: their alpha is provably below 1/255, so no decision changes.
#include "gs_common.h"
#include "gs_capi.h"

namespace gs {

#ifndef GS_FWD_PIX
#define GS_FWD_PIX 1
#endif
constexpr int kFwdPix = GS_FWD_PIX;  // pixels per lane: 1, 2 or 4

struct RenderFwdParams {
  int W, H, grid_x, num_tiles;
  int num_points;
  int num_rendered;
  const int2* ranges;
  const int* point_list;
  const float4* records;
  const float* bg;
  int compute_depth;
  float* out_color;
  float* out_depth;
  float* out_alpha;
  int* n_contrib;
  int write_aux, top_k;
  int* gs_per_pixel;
  float* weight;
  float* x_mu;
  // optional: the tiles in the order the workgroups take them (gs_tile_order),
  // null: in tile order
  const int* tile_order;
  int masked;  // blend updates under the exec mask of the blending lanes (render_fwd_tile)
  // optional: clear_floats floats at clear (16-byte aligned) set to 0 by the
  // grid on the way, the backward's gradient accumulator
  float* clear;
  long long clear_floats;
};

// Workgroup blockIdx.x's share of the optional buffer to zero, float4 stores
// issued after its last image store: no later load of the wave waits for them
// (the vector memory counter covers stores too), and the stores of a finished
// workgroup overlap the blending of the others.
__device__ __forceinline__ void clear_share(const RenderFwdParams& p, int lane) {
  if (!p.clear) return;
  const long long n4 = p.clear_floats >> 2;
  const long long per = (n4 + gridDim.x - 1) / gridDim.x;
  const long long b0 = (long long)blockIdx.x * per;
  const long long b1 = b0 + per < n4 ? b0 + per : n4;
  float4* c4 = reinterpret_cast<float4*>(p.clear);
  for (long long i = b0 + lane; i < b1; i += 64) c4[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (blockIdx.x == 0 && lane < (int)(p.clear_floats & 3)) p.clear[(n4 << 2) + lane] = 0.0f;
}

// Top-K auxiliaries of up to this many slots are staged in LDS (below).
constexpr int kMaxStagedTopK = 64;

// Slot s of a staged pixel's top-K: the Gaussian id, its weight (alpha T)
// and its offset (dx, dy) from the pixel, recomputed from the id by the
// walk's own operations (so bit for bit the walk's values), with Tw the
// transmittance in front of it, which the call advances; id < 0 gives the
// unused slot's -1 / 0 / 0 / 0.
__device__ __forceinline__ void topk_slot(int id, const float4& r0, const float4& r1, float pfx, float pfy,
                                          float& Tw, float& w, float& dx, float& dy) {
  w = dx = dy = 0.0f;
  if (id < 0) return;
  dx = r0.x - pfx;
  dy = r0.y - pfy;
  const float adxx = r0.z * dx * dx;
  const float b2dx = (2.0f * r0.w) * dx;
  const float q = conic_q_px(adxx, b2dx, r1.x, dy);
  const float alpha = fminf(kAlphaMax, r1.y * exp_sw_q(q));
  w = alpha * Tw;
  Tw = Tw * (1.0f - alpha);
}

// Tiles with fewer pairs than this stage their top-K as 16-bit list positions.
constexpr int kStagedMaxList = 1 << 16;

// kStaged (flow with K <= kMaxStagedTopK): the walk only records where each
// pixel's first K blended Gaussians are in the tile's list, as 16-bit
// positions in LDS (slot-major, 64 K kPix of them in dynamic LDS: 2.5 KB at
// K = 20, so the LDS keeps about seven waves per SIMD resident); after the
// walk every lane writes all K slots of its pixel plane by plane, so that
// each store instruction writes whole rows of 16 consecutive pixels of one
// plane (64-byte segments) instead of one scattered word per blended
// Gaussian, and the unused slots in the same stores.  Larger K, and tiles
// of kStagedMaxList pairs or more, keep the direct stores during the walk.
//
// kMasked: a pixel's blend updates run under the exec mask of the lanes that
// blend (a visit with none skips them), which replaces three selects (four-
// cycle instructions) per visit and the record's colour read of visits
// without a blend by a scalar branch.  That branch and its mask sit on the
// walk's serial path, so it pays where the kernel is bound by its issue rate
// (config 2 render 0.230 -> 0.223 ms, config 4 0.256 -> 0.252) and not where
// a few long walks bound it (config 1: 12% slower); the host takes it under
// the tile order's condition (tile_order_pays: lists of 192 pairs a tile or
// more on average).  (Choosing per tile, selects for lists over four times
// the mean, kept config 1 2.5% slower and config 4 1.3% slower.)
template <bool kFlow, bool kDepth, int kPixPerLane, bool kStaged, bool kMasked>
__device__ __forceinline__ void render_fwd_tile(const RenderFwdParams& p, float4* s_rec, int* s_id,
                                                unsigned short* s_pos, int lane, int2 ts) {
  const int tile = ts.x;
  const int tx = tile % p.grid_x;
  const int ty = tile / p.grid_x;
  // The wave's slice: kSliceW x kSliceH pixels, lane l at column l % kSliceW
  // and rows l / kSliceW + kRowStep k of it.
  constexpr int kSliceW = (kFlow || kPixPerLane == 4) ? 16 : 8;
  constexpr int kSliceH = 64 * kPixPerLane / kSliceW;
  constexpr int kRowStep = 64 / kSliceW;
  constexpr int kAcross = kBlockX / kSliceW;  // slices side by side in a tile
  const int sx0 = tx * kBlockX + (ts.y % kAcross) * kSliceW;
  const int sy0 = ty * kBlockY + (ts.y / kAcross) * kSliceH;
  const int px = sx0 + (lane % kSliceW);
  const int py0 = sy0 + lane / kSliceW;
  const int P = p.W * p.H;
  const float pfx = (float)px;
  const float rx0 = (float)sx0, rx1 = (float)(sx0 + kSliceW - 1);
  const float ry0 = (float)sy0, ry1 = (float)(sy0 + kSliceH - 1);
  int2 rg = p.ranges[tile];
  rg.x = imax(0, imin(rg.x, p.num_rendered));
  rg.y = imax(rg.x, imin(rg.y, p.num_rendered));
  const int n = rg.y - rg.x;
  const bool aux = kFlow && p.write_aux != 0;
  const bool staged = kStaged && n < kStagedMaxList;  // uniform per workgroup

  // live_lanes[k]: the wave's lanes whose pixel k is still blending, kept as
  // a lane mask in scalar registers (pixels outside the image start
  // finished); T is the pixel's transmittance, finished or not.
  float T[kPixPerLane], c0[kPixPerLane], c1[kPixPerLane], c2[kPixPerLane], ws[kPixPerLane], da[kPixPerLane];
  float pfy[kPixPerLane];
  int last[kPixPerLane], nsucc[kPixPerLane];
  uint64_t live_lanes[kPixPerLane];
#pragma unroll
  for (int k = 0; k < kPixPerLane; ++k) {
    const int py = py0 + kRowStep * k;
    pfy[k] = (float)py;
    T[k] = 1.0f;
    live_lanes[k] = __ballot(px < p.W && py < p.H);
    c0[k] = c1[k] = c2[k] = ws[k] = da[k] = 0.0f;
    last[k] = 0;
    nsucc[k] = 0;
  }

  // Batches of 64 list entries, front to back.  The loads run ahead: a
  // batch's records were requested during the batch before it, from indices
  // requested one batch earlier still, so no wave waits for memory but at a
  // batch's start, for loads issued a whole batch before.  The loads are
  // unconditional (in-bounds entries for lanes past the list).
  const int* const list = p.point_list + rg.x;
  int id = 0, id_ahead = 0;
  RecordRegs next;
  next.r0 = next.r1 = next.r2 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (n > 0) {
    id = checked_point(batch_entry(list, 0, imin(64, n), n, lane), p.num_points);
    id_ahead = batch_entry(list, 64, imin(64, n - 64), n, lane);
    next = load_record(p.records, id);
  }
  for (int base = 0; base < n; base += 64) {
    uint64_t live = 0;
#pragma unroll
    for (int k = 0; k < kPixPerLane; ++k) live |= live_lanes[k];
    if (live == 0) break;
    const int cnt = imin(64, n - base);
    // One wave per workgroup: LDS writes and the broadcast reads below are
    // ordered by the wave's own in-order LDS queue, no barrier needed.  The
    // LDS copy holds 2b in r0.w (the visits need b only as 2 b dx, and
    // (2b) dx rounds exactly as (b dx) 2) and qcut as its bound on q's bits
    // in r1.w (cand_threshold).
    s_rec[3 * lane] = make_float4(next.r0.x, next.r0.y, next.r0.z, 2.0f * next.r0.w);
    s_rec[3 * lane + 1] = make_float4(next.r1.x, next.r1.y, next.r1.z, __uint_as_float(cand_threshold(next.r1.w)));
    s_rec[3 * lane + 2] = next.r2;
    if (kFlow) s_id[lane] = id;
    // A conic with a <= 0 can give q = -0 (adxx = (a dx) dx = -0), which the
    // 0 <= q test takes and the bit compare does not; batches with such a
    // record add the q == 0 lanes to the candidates.
    const bool signed_zero = __ballot(lane < cnt && !(next.r0.z > 0.0f)) != 0;
    uint64_t todo = __ballot(lane < cnt && extents_meet(next.r0.x, next.r0.y, __float_as_uint(next.r2.w), rx0, rx1,
                                                        ry0, ry1));
    // the next batch's records and the indices of the one after it
    id = checked_point(id_ahead, p.num_points);
    next = load_record(p.records, id);
    id_ahead = batch_entry(list, base + 128, imin(64, n - base - 128), n, lane);
    while (todo != 0) {
      const int j = __builtin_ctzll(todo);
      todo &= todo - 1;
      const float4 a = s_rec[3 * j];
      const float4 b = s_rec[3 * j + 1];
      const float dx = a.x - pfx;
      const float adxx = a.z * dx * dx;
      const float b2dx = a.w * dx;  // a.w = 2b
      const unsigned thr = __float_as_uint(b.w);
      float q[kPixPerLane], dy[kPixPerLane];
      uint64_t cand_lanes[kPixPerLane];  // live && 0 <= q <= qcut, as lane masks
      uint64_t any = 0;
#pragma unroll
      for (int k = 0; k < kPixPerLane; ++k) {
        dy[k] = a.y - pfy[k];
        q[k] = conic_q_px(adxx, b2dx, b.x, dy[k]);  // exponent = -0.5 q
        cand_lanes[k] = live_lanes[k] & __builtin_amdgcn_uicmp(__float_as_uint(q[k]), thr, kCmpULT);
        if (signed_zero) cand_lanes[k] |= live_lanes[k] & __builtin_amdgcn_fcmpf(q[k], 0.0f, kCmpOEQ);
        any |= cand_lanes[k];
      }
      if (any == 0) continue;
      const float4 f = s_rec[3 * j + 2];
#pragma unroll
      for (int k = 0; k < kPixPerLane; ++k) {
        // Every lane evaluates the exponential; the result only counts for
        // candidate lanes (0 <= q), where the argument is non-positive.  For
        // the others it may be anything, including inf or NaN, and every
        // decision below masks it out.  o * exp <= o <= 1, so the minimum
        // needs no NaN rule of its own.
        const float alpha = fminf(kAlphaMax, b.y * exp_sw_q(q[k]));
        // The blend decisions as lane masks: scalar ANDs of the comparisons.
        const uint64_t ok_lanes = cand_lanes[k] & __builtin_amdgcn_fcmpf(alpha, kAlphaMin, kCmpOGE);
        const float test_T = T[k] * (1.0f - alpha);
        const uint64_t fin_lanes = ok_lanes & __builtin_amdgcn_fcmpf(test_T, kTransmittanceMin, kCmpOLT);
        live_lanes[k] &= ~fin_lanes;
        const bool blend = __builtin_amdgcn_inverse_ballot_w64(ok_lanes & ~fin_lanes);
        if constexpr (kMasked) {
          if (blend) {
            const float contribution = alpha * T[k];
            c0[k] = fmaf(f.x, contribution, c0[k]);
            c1[k] = fmaf(f.y, contribution, c1[k]);
            c2[k] = fmaf(f.z, contribution, c2[k]);
            ws[k] = ws[k] + contribution;
            if (kDepth) da[k] = fmaf(b.z, contribution, da[k]);
            if (staged) {
              if (aux && nsucc[k] < p.top_k)
                s_pos[(nsucc[k] * kPixPerLane + k) * 64 + lane] = (unsigned short)(base + j);
            } else if (aux && nsucc[k] < p.top_k) {
              const size_t pix = (size_t)(py0 + kRowStep * k) * p.W + px;
              const size_t ai = (size_t)nsucc[k] * P + pix;
              p.gs_per_pixel[ai] = s_id[j];
              p.weight[ai] = contribution;
              p.x_mu[ai] = dx;
              p.x_mu[(size_t)p.top_k * P + ai] = dy[k];
            }
            if (kFlow) nsucc[k] += 1;
            T[k] = test_T;
            last[k] = base + j + 1;
          }
        } else {
          // A pixel that does not blend adds a contribution of exactly +0
          // (the sums are unchanged bit for bit), which replaces per-output
          // selects.
          const float contribution = blend ? alpha * T[k] : 0.0f;
          c0[k] = fmaf(f.x, contribution, c0[k]);
          c1[k] = fmaf(f.y, contribution, c1[k]);
          c2[k] = fmaf(f.z, contribution, c2[k]);
          ws[k] = ws[k] + contribution;
          if (kDepth) da[k] = fmaf(b.z, contribution, da[k]);
          if (staged) {
            if (aux && blend && nsucc[k] < p.top_k)
              s_pos[(nsucc[k] * kPixPerLane + k) * 64 + lane] = (unsigned short)(base + j);
          } else if (aux && blend && nsucc[k] < p.top_k) {
            const size_t pix = (size_t)(py0 + kRowStep * k) * p.W + px;
            const size_t ai = (size_t)nsucc[k] * P + pix;
            p.gs_per_pixel[ai] = s_id[j];
            p.weight[ai] = contribution;
            p.x_mu[ai] = dx;
            p.x_mu[(size_t)p.top_k * P + ai] = dy[k];
          }
          if (kFlow) nsucc[k] += blend ? 1 : 0;
          T[k] = blend ? test_T : T[k];
          last[k] = blend ? base + j + 1 : last[k];
        }
      }
    }
  }

#pragma unroll
  for (int k = 0; k < kPixPerLane; ++k) {
    const int py = py0 + kRowStep * k;
    const bool in_image = px < p.W && py < p.H;
    const int pix = py * p.W + px;
    if (in_image) {
      const float Tk = T[k];
      p.n_contrib[pix] = last[k];
      p.out_color[pix] = c0[k] + Tk * p.bg[0];
      p.out_color[P + pix] = c1[k] + Tk * p.bg[1];
      p.out_color[2 * P + pix] = c2[k] + Tk * p.bg[2];
      p.out_alpha[pix] = ws[k];
      p.out_depth[pix] = da[k];
    }
    if (staged && aux) {
      // Slots in plane order: the list entry of slot s + 2 and the record of
      // slot s + 1 are loaded before slot s's arithmetic.
      float Tw = 1.0f;
      const unsigned short* pos = s_pos + k * 64 + lane;
      const int used = imin(nsucc[k], p.top_k);
      auto list_id = [&](int s) {
        if (s >= used) return -1;
        int id = p.point_list[rg.x + pos[s * kPixPerLane * 64]];
        return (unsigned)id < (unsigned)p.num_points ? id : 0;  // as checked_point
      };
      int id_a = list_id(0);
      int id_b = list_id(1);
      float4 r0a = make_float4(0.0f, 0.0f, 0.0f, 0.0f), r1a = r0a;
      if (id_a >= 0) {
        r0a = p.records[3 * (size_t)id_a];
        r1a = p.records[3 * (size_t)id_a + 1];
      }
      for (int s = 0; s < p.top_k; ++s) {
        const int id = id_a;
        const float4 r0 = r0a, r1 = r1a;
        id_a = id_b;
        if (id_a >= 0) {
          r0a = p.records[3 * (size_t)id_a];
          r1a = p.records[3 * (size_t)id_a + 1];
        }
        id_b = list_id(s + 2);
        float w, sdx, sdy;
        topk_slot(id, r0, r1, pfx, pfy[k], Tw, w, sdx, sdy);
        if (in_image) {
          const size_t ai = (size_t)s * P + pix;
          p.gs_per_pixel[ai] = id;
          p.weight[ai] = w;
          p.x_mu[ai] = sdx;
          p.x_mu[(size_t)p.top_k * P + ai] = sdy;
        }
      }
    } else if (aux) {
      // Unused slots, plane by plane for the whole wave, so that each store
      // covers the wave's pixels of one plane (rows of kSliceW consecutive
      // pixels) rather than one plane per lane.
      int s_from = in_image ? nsucc[k] : p.top_k;
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) s_from = imin(s_from, __shfl_xor(s_from, off, 64));
      for (int s = s_from; s < p.top_k; ++s) {
        if (in_image && s >= nsucc[k]) {
          const size_t ai = (size_t)s * P + pix;
          p.gs_per_pixel[ai] = -1;
          p.weight[ai] = 0.0f;
          p.x_mu[ai] = 0.0f;
          p.x_mu[(size_t)p.top_k * P + ai] = 0.0f;
        }
      }
    }
  }
}

template <bool kFlow, bool kDepth, int kPixPerLane, bool kStaged, bool kMasked>
__global__ __launch_bounds__(64) void render_fwd_kernel(RenderFwdParams p) {
  constexpr int kSubs = 4 / kPixPerLane;
  __shared__ float4 s_rec[3 * 64];  // record j at s_rec[3 j .. 3 j + 2]
  __shared__ int s_id[kFlow ? 64 : 1];
  extern __shared__ unsigned short s_pos[];  // kStaged: slot s of pixel k at [(s kPix + k) 64 + lane]
  const int lane = threadIdx.x;
  const int unit = xcd_unit(blockIdx.x, p.num_tiles * kSubs);
  if (unit < p.num_tiles * kSubs) {  // else grid padding
    const int2 ts = make_int2(p.tile_order ? p.tile_order[unit / kSubs] : unit / kSubs, unit % kSubs);
    render_fwd_tile<kFlow, kDepth, kPixPerLane, kStaged, kMasked>(p, s_rec, s_id, s_pos, lane, ts);
  }
  clear_share(p, lane);
}

// The order in which the blend kernels take the tiles: longest list first,
// by a counting sort over 256 classes of the list length (4 pairs wide
// below 512, 64 wide above, the last class open; one workgroup).  The
// longest walks then start first and the end of the grid is made of short
// ones: in tile order the long lists at the image's centre start half way
// through the grid and the last of them finish well after the rest.
// Ordering groups of 4 x 4 tiles instead, to keep neighbours (which share
// Gaussians) together in one XCD's L2, measured slower at configs 2 and 4.
__device__ __forceinline__ int tile_length_class(int2 r) {
  const int len = imax(0, r.y - r.x);
  const int c = len < 512 ? len >> 2 : 128 + imin(127, (len - 512) >> 6);
  return 255 - c;  // longest first
}

// Up to kOrderRegTiles tiles per thread keep their classes in registers
// between the two passes (images of up to 16384 tiles); beyond, the second
// pass reads the ranges again.
constexpr int kOrderRegTiles = 16;

__global__ __launch_bounds__(1024) void tile_order_kernel(int T, const int2* __restrict__ ranges,
                                                         int* __restrict__ order) {
  __shared__ __align__(16) int s_count[256];
  const int t0 = threadIdx.x;
  if (t0 < 256) s_count[t0] = 0;
  int2 rr[kOrderRegTiles];
  int cls[kOrderRegTiles];
#pragma unroll
  for (int i = 0; i < kOrderRegTiles; ++i) rr[i] = ranges[imin(t0 + 1024 * i, T - 1)];
#pragma unroll
  for (int i = 0; i < kOrderRegTiles; ++i) cls[i] = tile_length_class(rr[i]);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kOrderRegTiles; ++i)
    if (t0 + 1024 * i < T) atomicAdd(&s_count[cls[i]], 1);
  for (int t = t0 + 1024 * kOrderRegTiles; t < T; t += 1024) atomicAdd(&s_count[tile_length_class(ranges[t])], 1);
  __syncthreads();
  if (t0 < 64) {  // exclusive prefix over the 256 classes, four per lane
    const int4 c = reinterpret_cast<const int4*>(s_count)[t0];
    const int sum = c.x + c.y + c.z + c.w;
    int incl = sum;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int o = __shfl_up(incl, off, 64);
      if (t0 >= off) incl += o;
    }
    const int e = incl - sum;
    reinterpret_cast<int4*>(s_count)[t0] = make_int4(e, e + c.x, e + c.x + c.y, e + c.x + c.y + c.z);
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kOrderRegTiles; ++i) {
    const int t = t0 + 1024 * i;
    if (t < T) order[atomicAdd(&s_count[cls[i]], 1)] = t;
  }
  for (int t = t0 + 1024 * kOrderRegTiles; t < T; t += 1024)
    order[atomicAdd(&s_count[tile_length_class(ranges[t])], 1)] = t;
}

// One launch of render_fwd_kernel with the template arguments of p's flags.
template <bool kFlow, bool kDepth, bool kStaged>
static void launch_render_fwd_as(const RenderFwdParams& p, dim3 grid, size_t lds, hipStream_t s) {
  if (p.masked)
    hipLaunchKernelGGL((render_fwd_kernel<kFlow, kDepth, kFwdPix, kStaged, true>), grid, dim3(64), lds, s, p);
  else
    hipLaunchKernelGGL((render_fwd_kernel<kFlow, kDepth, kFwdPix, kStaged, false>), grid, dim3(64), lds, s, p);
}

static int launch_render_fwd(const RenderFwdParams& p, bool flow, hipStream_t s) {
  const dim3 grid(gs::xcd_grid(p.num_tiles * (4 / kFwdPix)));
  if (flow && p.write_aux && p.top_k <= kMaxStagedTopK) {
    const size_t lds = (size_t)p.top_k * kFwdPix * 64 * sizeof(unsigned short);
    if (p.compute_depth)
      launch_render_fwd_as<true, true, true>(p, grid, lds, s);
    else
      launch_render_fwd_as<true, false, true>(p, grid, lds, s);
  } else if (flow) {
    if (p.compute_depth)
      launch_render_fwd_as<true, true, false>(p, grid, 0, s);
    else
      launch_render_fwd_as<true, false, false>(p, grid, 0, s);
  } else {
    if (p.compute_depth)
      launch_render_fwd_as<false, true, false>(p, grid, 0, s);
    else
      launch_render_fwd_as<false, false, false>(p, grid, 0, s);
  }
  return gs_status_from_hip(hipGetLastError());
}

}  // namespace gs

static int gs_render_fwd_common(int32_t W, int32_t H, int32_t num_points, int64_t num_rendered,
                                const int32_t* ranges, const int32_t* point_list, const float* records,
                                const float* background, int32_t compute_depth, int32_t write_aux, int32_t top_k,
                                float* out_color, float* out_depth, float* out_alpha, int32_t* n_contrib,
                                int32_t* gs_per_pixel, float* weight, float* x_mu, bool flow, void* stream,
                                int32_t* tile_order, float* clear = nullptr, int64_t clear_floats = 0,
                                bool order_ready = false) {
  if (W <= 0 || H <= 0 || (long long)W * H > 0x7fffffffLL) return GS_ERR_INVALID_ARGUMENT;
  if (clear_floats < 0 || (clear_floats > 0 && !clear)) return GS_ERR_INVALID_ARGUMENT;
  if (reinterpret_cast<uintptr_t>(clear) & 15) return GS_ERR_MISALIGNED;
  if (num_points <= 0 || num_rendered < 0) return GS_ERR_INVALID_ARGUMENT;
  if (num_rendered > 0x7fffffffLL) return GS_ERR_OVERFLOW;
  if (!ranges || !point_list || !records || !background || !out_color || !out_depth || !out_alpha || !n_contrib)
    return GS_ERR_INVALID_ARGUMENT;
  if (reinterpret_cast<uintptr_t>(records) & 15) return GS_ERR_MISALIGNED;
  if (flow && write_aux && (top_k <= 0 || !gs_per_pixel || !weight || !x_mu)) return GS_ERR_INVALID_ARGUMENT;
  gs::RenderFwdParams p;
  p.W = W;
  p.H = H;
  p.grid_x = (W + gs::kBlockX - 1) / gs::kBlockX;
  p.num_tiles = p.grid_x * ((H + gs::kBlockY - 1) / gs::kBlockY);
  p.num_points = num_points;
  p.num_rendered = (int)num_rendered;
  p.ranges = reinterpret_cast<const int2*>(ranges);
  p.point_list = point_list;
  p.records = reinterpret_cast<const float4*>(records);
  p.bg = background;
  p.compute_depth = compute_depth;
  p.out_color = out_color;
  p.out_depth = out_depth;
  p.out_alpha = out_alpha;
  p.n_contrib = n_contrib;
  p.write_aux = flow ? write_aux : 0;
  p.top_k = top_k;
  p.gs_per_pixel = gs_per_pixel;
  p.weight = weight;
  p.x_mu = x_mu;
  p.clear = clear_floats > 0 ? clear : nullptr;
  p.clear_floats = clear_floats;
  p.masked = gs::tile_order_pays(num_rendered, num_points, p.num_tiles) ? 1 : 0;
  p.tile_order = nullptr;
  if (tile_order && gs::tile_order_pays(num_rendered, num_points, p.num_tiles)) {
    if (!order_ready) {
      const int st = gs_tile_order(p.num_tiles, ranges, tile_order, stream);
      if (st != GS_OK) return st;
    }
    p.tile_order = tile_order;
  }
  return gs::launch_render_fwd(p, flow, (hipStream_t)stream);
}

extern "C" int gs_tile_order(int32_t num_tiles, const int32_t* ranges, int32_t* order, void* stream) {
  if (num_tiles < 0 || (num_tiles > 0 && (!ranges || !order))) return GS_ERR_INVALID_ARGUMENT;
  if (num_tiles == 0) return GS_OK;
  hipLaunchKernelGGL(gs::tile_order_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, num_tiles,
                     reinterpret_cast<const int2*>(ranges), order);
  return gs_status_from_hip(hipGetLastError());
}

extern "C" int gs_render_fwd(int32_t image_width, int32_t image_height, int32_t num_points, int64_t num_rendered,
                             const int32_t* ranges, const int32_t* point_list, const float* records,
                             const float* background, int32_t compute_depth, float* out_color, float* out_depth,
                             float* out_alpha, int32_t* n_contrib, int32_t* tile_order, void* stream) {
  return gs_render_fwd_common(image_width, image_height, num_points, num_rendered, ranges, point_list, records,
                              background, compute_depth, 0, 0, out_color, out_depth, out_alpha, n_contrib, nullptr,
                              nullptr, nullptr, false, stream, tile_order);
}

extern "C" int gs_render_fwd_clear(int32_t image_width, int32_t image_height, int32_t num_points,
                                   int64_t num_rendered, const int32_t* ranges, const int32_t* point_list,
                                   const float* records, const float* background, int32_t compute_depth,
                                   float* out_color, float* out_depth, float* out_alpha, int32_t* n_contrib,
                                   float* clear, int64_t clear_floats, int32_t* tile_order, void* stream) {
  return gs_render_fwd_common(image_width, image_height, num_points, num_rendered, ranges, point_list, records,
                              background, compute_depth, 0, 0, out_color, out_depth, out_alpha, n_contrib, nullptr,
                              nullptr, nullptr, false, stream, tile_order, clear, clear_floats);
}

int gs_render_fwd_clear_ordered(int32_t image_width, int32_t image_height, int32_t num_points, int64_t num_rendered,
                                const int32_t* ranges, const int32_t* point_list, const float* records,
                                const float* background, int32_t compute_depth, float* out_color, float* out_depth,
                                float* out_alpha, int32_t* n_contrib, float* clear, int64_t clear_floats,
                                int32_t* tile_order, bool order_ready, void* stream) {
  return gs_render_fwd_common(image_width, image_height, num_points, num_rendered, ranges, point_list, records,
                              background, compute_depth, 0, 0, out_color, out_depth, out_alpha, n_contrib, nullptr,
                              nullptr, nullptr, false, stream, tile_order, clear, clear_floats, order_ready);
}

extern "C" int gs_render_fwd_flow(int32_t image_width, int32_t image_height, int32_t num_points,
                                  int64_t num_rendered, const int32_t* ranges, const int32_t* point_list,
                                  const float* records, const float* background, int32_t compute_depth,
                                  int32_t write_aux, int32_t top_k, float* out_color, float* out_depth,
                                  float* out_alpha, int32_t* n_contrib, int32_t* gs_per_pixel,
                                  float* weight_per_gs_pixel, float* x_mu, int32_t* tile_order, void* stream) {
  return gs_render_fwd_common(image_width, image_height, num_points, num_rendered, ranges, point_list, records,
                              background, compute_depth, write_aux, top_k, out_color, out_depth, out_alpha,
                              n_contrib, gs_per_pixel, weight_per_gs_pixel, x_mu, true, stream, tile_order);
}
