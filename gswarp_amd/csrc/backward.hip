// Manual backward for gfx950.
//
// render_bwd: wave64 workgroups each own a slice of a tile (an 8x16 half,
// two pixels per lane; the whole tile, four pixels per lane, when the
// Gaussians are large; one 8x8 quadrant for tiles whose list is more than
// four times the mean) and walk the tile's list back to front from the
// largest n_contrib of their pixels
// (backward_kernels.py:539-707 semantics: T starts at 1 - alpha_out and is
// divided by max(1-alpha, 1e-5) per blended Gaussian, reverse recurrences for
// colour, depth and alpha, the background term).  Per Gaussian each lane
// sums its pixels' pixel moments and colour / depth terms; the wave reduces
// them through LDS (a transposed store and per-column sums for one-column
// slices, two lane-swap folds for the whole tile) into a per-wave slot, which
// is reduced and sent to global memory with one float atomic per component
// at the next Gaussian (skipped for a zero sum).
// The blend decisions are exactly the forward's (exp_sw is evaluated only in
// a thin band above the record's power cutoff where the decision needs it);
// gradient values use the hardware exponential and reciprocal.
//
// preprocess_bwd: one thread per Gaussian forming the xy and conic render
// gradients from the moments (the W/2, H/2 and -1/2 factors of
// backward_kernels.py:678-685 with the record's conic and opacity), fusing
// the SH colour backward
// (backward_kernels.py:298-536), the projected-mean / depth backward
// (backward_kernels.py:89-112), the cov2D -> cov3D -> scale/rotation backward
// (backward_kernels.py:114-287) and the accumulation (backward_kernels.py:289-295).
// cov3D is recomputed from scale and rotation with the forward's exact
// expression instead of being stored by the forward pass.
#include <type_traits>

#include "gs_common.h"
#include "gs_capi.h"

namespace gs {

constexpr int kGradFloats = 10;  // dx, dy, conic a, b, c, opacity, r, g, b, depth
constexpr float kSureMargin = 2.0e-3f;  // exponents this far above the cutoff always blend
constexpr float kLog2e = 1.44269504088896341f;
constexpr int64_t kLongTileFactor = 4;  // long tile: list longer than this many times the mean

template <int kCtrl, int kRowMask>
__device__ __forceinline__ float dpp_mov(float src) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(src), kCtrl, kRowMask, 0xF, false));
}

// v_permlane32_swap exchanges lanes 32-63 of a with lanes 0-31 of b, so the
// sum of the two results holds a[l] + a[l+32] in lanes 0-31 and
// b[l-32] + b[l] in lanes 32-63: two half-wave partial sums for one add.
__device__ __forceinline__ float fold32(float a, float b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// v_permlane16_swap exchanges the odd rows of a with the even rows of b: the
// sum holds a folded over row pairs (0,1) and (2,3) in rows 0 and 2 and b
// folded the same way in rows 1 and 3.
__device__ __forceinline__ float fold16(float a, float b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Partial transposed reduction of ten per-lane values: two lane-swap folds
// leave three registers in which row r (lanes 16 r .. 16 r + 15) of
// register i holds 16 partial sums (over 4 lanes each) of component
// slot_component(4 i + r); the duplicated rows of the third register are
// unused.
__device__ __forceinline__ void wave_fold10(const float (&g)[10], float (&m)[3]) {
  const float h0 = fold32(g[0], g[5]);
  const float h1 = fold32(g[1], g[6]);
  const float h2 = fold32(g[2], g[7]);
  const float h3 = fold32(g[3], g[8]);
  const float h4 = fold32(g[4], g[9]);
  m[0] = fold16(h0, h1);
  m[1] = fold16(h2, h3);
  m[2] = fold16(h4, h4);
}

// Per-wave LDS slot of a Gaussian's gradient partial sums.  It holds, for
// the 12 (register, row) positions p = 4 i + r of wave_fold10's output, the
// 16 partial sums of lanes 16 r .. 16 r + 15: float p * 16 + lane % 16, so
// the three registers are stored at float offsets 0, 64 and 128 from
// slot + lane (plain stores: the slot belongs to one wave).  The slot of the
// previous Gaussian is reduced (one float4 and a quad sum per position) and
// sent to global memory with one atomic per component just before the next
// Gaussian's sums are stored, and at the end of the slice: a whole
// Gaussian's work lies between a store and its read-back, and the slot's
// address is the same for every Gaussian.
constexpr int kSlotFloats = 12 * 16;
constexpr int kSlotPad = 64 * 4 - kSlotFloats;  // a whole wave's float4 read of the slot

// The address of Gaussian gid's (wave-uniform) row of grad_gauss, formed on
// the scalar unit.
__device__ __forceinline__ uint64_t grad_row(float* grad_gauss, int gid) {
  return reinterpret_cast<uint64_t>(grad_gauss) +
         (uint64_t)(unsigned)__builtin_amdgcn_readfirstlane(gid) * (kGradFloats * sizeof(float));
}

// Adds v to component comp of a grad_gauss row, no value returned: a vector
// memory atomic in its scalar-base form (the row address in scalar
// registers, each lane's 32-bit byte offset in a vector register).  Written
// as one instruction because the compiler otherwise forms every lane's
// 64-bit address with a vector 64-bit add at each flush.  Its completion is
// counted by the same in-order vector memory counter as the compiler's own
// loads, so any wait the compiler places for a load issued before it also
// covers it; nothing in the kernel reads grad_gauss.
__device__ __forceinline__ void global_add(uint64_t row, unsigned comp, float v) {
  asm volatile("global_atomic_add_f32 %0, %1, %2" : : "v"(comp * 4u), "v"(v), "s"(row) : "memory");
}

// Component at slot position p (-1: a duplicated row): {0, 1, 5, 6, 2, 3, 7,
// 8, 4, -1, 9, -1}.
__device__ __forceinline__ int slot_component(int p) {
  const int i = p >> 2, r = p & 3;
  if (i < 2) return 2 * i + (r & 1) + 5 * (r >> 1);
  return (r & 1) ? -1 : 4 + 5 * (r >> 1);
}

// Reduces the slot and adds its components to grad_gauss[gid]: lane l reads
// float4 l of the slot (position l / 4 for l < 48), sums it, and each quad
// of lanes sums its position's four float4 sums; the quad's first lane
// issues the atomic of a used, non-zero component.
__device__ __forceinline__ void flush_slot(const float* slot, int gid, int lane, int comp, float* grad_gauss) {
  // Every lane reads a float4 (the slot is padded so that lanes 48-63 stay
  // inside it); those lanes hold no component.
  const float4 v = reinterpret_cast<const float4*>(slot)[lane];
  float t = (v.x + v.y) + (v.z + v.w);
  t = t + dpp_mov<0xB1, 0xF>(t);  // quad_perm [1,0,3,2]
  t = t + dpp_mov<0x4E, 0xF>(t);  // quad_perm [2,3,0,1]
  const uint64_t row = grad_row(grad_gauss, gid);
  if ((lane & 3) == 0 && comp >= 0 && t != 0.0f) global_add(row, (unsigned)comp, t);
}

// Column-slice reduction through LDS (kCols == 1: a lane's pixels lie in the
// column lane % 8 and share its dx).  Cross-lane VALU moves are the slow
// part of a wave-wide sum (a v_permlane swap costs four fast adds), so the
// wave transposes its sums through LDS instead.  The seven per-lane sums
// (v, v dy, v dy^2 and the three colour and the depth terms) are stored so
// that the eight lanes of one column hold a contiguous group of 8 floats:
// component c of lane l at float
//   c * 64 + col * 8 + ((row + 4 (col / 4)) % 8),   col = l % 8, row = l / 8
// (the rotation by 4 (col / 4) puts each half-wave's 32 stores on 32 banks).
// Lane 8 c + col (c < 7; lanes 56-63 repeat c = 6) reads its group as two
// float4 and adds them: the column sum S of component c; with the column's
// dx it forms S dx and S dx^2, the dx moments (used for c = 0 and 1).  These
// go to the slot: S at float lane, S dx at 64 + lane, S dx^2 at 128 + lane.
// The slot is reduced at the next Gaussian, or at the slice's end: lane
// 2 k + h (k < 10) reads the float4 of columns 4 h .. 4 h + 3 of output k and
// adds it, the lane pair adds its two sums (one DPP add) and the even lane
// sends output k with one atomic.  Outputs 0-6 are the column sums (grad
// components 5, 1, 4, 6, 7, 8, 9), 7 sum v dx (component 0), 8 sum v dy dx
// (3) and 9 sum v dx^2 (2).
constexpr int kColSlotFloats = 3 * 64;
constexpr int kColRawFloats = 7 * 64;

__device__ __forceinline__ int col_raw_offset(int lane) {
  const int col = lane & 7, row = lane >> 3;
  return col * 8 + ((row + 4 * (col >> 2)) & 7);
}

// float4 index (in the raw area) of the first of a lane's two groups
__device__ __forceinline__ int col_group_index(int lane) {
  return imin(lane >> 3, 6) * 16 + (lane & 7) * 2;
}

// float4 index (in the slot) that lane 2 k + h reads for output k
__device__ __forceinline__ int col_flush_index(int lane) {
  const int k = lane >> 1, h = lane & 1;
  if (k >= 10) return 0;
  const int f = k < 7 ? 8 * k : (k == 7 ? 64 : (k == 8 ? 72 : 128));
  return (f >> 2) + h;
}

// grad component that lane 2 k sends (-1: none), stored in the nibbles of a constant
__device__ __forceinline__ int col_flush_component(int lane) {
  if (lane >= 20 || (lane & 1)) return -1;
  return (int)((0x2309876415ull >> (4 * (lane >> 1))) & 15);
}

__device__ __forceinline__ void flush_col_slot(float4 v, int gid, int comp, float* grad_gauss) {
  float t = (v.x + v.y) + (v.z + v.w);
  t = t + dpp_mov<0xB1, 0xF>(t);  // quad_perm [1,0,3,2]: the pair partner's sum
  // The Gaussian's row is wave-uniform: its address is formed on the scalar
  // unit, and each lane adds only its component's offset.
  const uint64_t row = grad_row(grad_gauss, gid);
  if (comp >= 0 && t != 0.0f) global_add(row, (unsigned)comp, t);
}

// The wave's LDS besides the records: the fold slot of wave_fold10, or the
// column slot and the transposed sums.
constexpr int kSlotLdsFloats =
    (kSlotFloats + kSlotPad) > (kColSlotFloats + kColRawFloats) ? (kSlotFloats + kSlotPad)
                                                                : (kColSlotFloats + kColRawFloats);

// A record's pixel classes as thresholds on the bits of q: for q >= +0 (sign
// bit clear) bits(q) < cand exactly when q <= qcut (a candidate) and
// bits(q) < sure exactly when q <= qcut - 2 kSureMargin (surely blends);
// negative q, -0 and NaN have larger bits, and a negative threshold allows
// nothing (0).  Both are computed from the record's qcut as the visits'
// float compares would.
struct BlendThresholds {
  unsigned cand, sure;
};

__device__ __forceinline__ BlendThresholds blend_thresholds(float qcut) {
  const float qsure = qcut - 2.0f * kSureMargin;
  BlendThresholds t;
  t.cand = cand_threshold(qcut);
  t.sure = cand_threshold(qsure);
  return t;
}

__device__ __forceinline__ int wave_max_i32(int v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const int o = __shfl_xor(v, off, 64);
    v = v > o ? v : o;
  }
  return v;
}

struct RenderBwdParams {
  int W, H, grid_x, num_tiles;
  int num_points;
  int num_rendered;
  const int2* ranges;
  const int* point_list;
  const float4* records;
  const float* bg;
  const float* out_alpha;
  const int* n_contrib;
  const float* grad_color;
  const float* grad_depth;
  const float* grad_alpha;
  int compute_depth;
  int long_tile;  // list length above which a tile is walked by four one-pixel-per-lane slices
  float* grad_gauss;
  const int* tile_order;  // the tiles in the order the workgroups take them (gs_tile_order), null: tile order
};

// One wave walks a slice of kPix blocks of 8x8 pixels, kCols blocks wide:
// lane l owns pixel (l % 8, l / 8) of every block, block k lying at
// ((k % kCols) 8, (k / kCols) 8) from the slice's origin.  Slice `sub` of a
// tile: with four blocks (kCols 2) the whole tile; with two stacked blocks
// the left (0) or right (1) half; with one block the quadrant sub (0 / 1
// the upper left / right, 2 / 3 the lower ones).  Pixels of a lane in one
// column of blocks share dx to a Gaussian.
//
// Per pixel the reverse blend keeps two running values: 1 / T, T the
// transmittance in front of the current Gaussian (the reference's division
// T <- T / (1 - alpha) becomes the product 1/T <- (1/T) (1 - alpha), one
// fused multiply-add, and T = rcp(1/T)), and S = U . acc, the upstream gradient
// U = (dL/dr, dL/dg, dL/db, dL/ddepth, dL/dalpha) dotted with the
// accumulated features behind it, acc = (colour, depth, alpha) of everything
// behind, each Gaussian adding F = (r, g, b, depth, 1) as
//   acc <- alpha F + (1 - alpha) acc   =>   S <- alpha (F.U) + (1 - alpha) S.
// The reference's per-channel sum  sum_ch (F_ch - acc_ch) U_ch  is F.U - S,
// and its background term -T_final / (1 - alpha) (bg . dL/dcolour) is the
// same recurrence started from S = bg . dL/dcolour instead of 0 (the
// background is an opaque layer behind the last Gaussian; 1 - alpha >= 0.01
// since alpha <= 0.99, so the 1e-5 floor never applies to it).  Per
// Gaussian each lane then sums, with v = G * dL/dalpha_hat per pixel, the
// moments (v dx, v dy, v dx^2, v dx dy, v dy^2, v) over its pixels (per
// column of blocks, whose pixels share dx) and the colour and depth terms
// alpha T dL/dpixel; the ten per-lane components are summed over the wave
// and added to grad_gauss.
// The per-Gaussian backward forms the reference's per-pixel expressions
// summed over pixels from the moments:
//   dL/dxy    = -(W/2, H/2) * o * (a sum(v dx) + b sum(v dy), c sum(v dy) + b sum(v dx)),
//   dL/dconic = -1/2 * o * (sum(v dx^2), sum(v dx dy), sum(v dy^2)),
//   dL/dopacity = sum(v).  Each batch of 64
// records is first tested lane-parallel against the slice (one bounding box
// per record, record_box), and only records that may touch it are visited;
// with kBlockCull each block is tested, and a record's visit skips the
// blocks its box misses (worth its branches when a slice has four blocks).
// The batch's LDS copy of a record carries the candidate and sure-blend
// thresholds of blend_thresholds in the words the records leave unused, so
// a visit classifies a pixel with two unsigned compares of q's bits.
// s_rec (3 x 64 float4) and s_slot (kSlotLdsFloats floats, 16-byte aligned)
// are the wave's LDS.
template <bool kDepth, int kPix, int kCols, bool kBlockCull>
__device__ __forceinline__ void render_bwd_slice(const RenderBwdParams& p, int tile, int sub, float4* s_rec,
                                                 float* s_slot) {
  static_assert(kPix % kCols == 0 && 8 * kCols <= kBlockX && 8 * (kPix / kCols) <= kBlockY, "slice in a tile");
  constexpr int kSliceW = 8 * kCols;
  constexpr int kSliceH = 8 * (kPix / kCols);
  constexpr int kAcross = kBlockX / kSliceW;
  const int lane = threadIdx.x;
  const int tx = tile % p.grid_x;
  const int ty = tile / p.grid_x;
  const int sx0 = tx * kBlockX + (sub % kAcross) * kSliceW;
  const int sy0 = ty * kBlockY + (sub / kAcross) * kSliceH;
  const int P = p.W * p.H;
  float pfx[kCols];
#pragma unroll
  for (int c = 0; c < kCols; ++c) pfx[c] = (float)(sx0 + 8 * c + (lane & 7));
  int2 rg = p.ranges[tile];
  // The pixels' loads are issued with the range's, at addresses clamped into
  // the image and with no branch between them, so the wave waits for memory
  // once; pixels outside the image (or of an empty tile) then take the
  // values of a pixel that blends nothing.
  const float bg0 = p.bg[0], bg1 = p.bg[1], bg2 = p.bg[2];
  float pfy[kPix], Ti[kPix], S[kPix], gp0[kPix], gp1[kPix], gp2[kPix], gpd[kPix], gpa[kPix];
  float a_out[kPix];
  int last[kPix];
#pragma unroll
  for (int k = 0; k < kPix; ++k) {
    const int px = sx0 + 8 * (k % kCols) + (lane & 7);
    const int py = sy0 + 8 * (k / kCols) + (lane >> 3);
    pfy[k] = (float)py;
    const int pix = imin(py, p.H - 1) * p.W + imin(px, p.W - 1);
    a_out[k] = p.out_alpha[pix];
    last[k] = p.n_contrib[pix];
    gp0[k] = gp1[k] = gp2[k] = gpd[k] = gpa[k] = 0.0f;
    // absent upstream gradients (null) are zero
    if (p.grad_color) {
      gp0[k] = p.grad_color[pix];
      gp1[k] = p.grad_color[P + pix];
      gp2[k] = p.grad_color[2 * P + pix];
    }
    if (kDepth && p.grad_depth) gpd[k] = p.grad_depth[pix];
    if (p.grad_alpha) gpa[k] = p.grad_alpha[pix];
  }
  rg.x = imax(0, imin(rg.x, p.num_rendered));
  rg.y = imax(rg.x, imin(rg.y, p.num_rendered));
  const int n = rg.y - rg.x;
  int lmax = 0;
#pragma unroll
  for (int k = 0; k < kPix; ++k) {
    const int px = sx0 + 8 * (k % kCols) + (lane & 7);
    const int py = sy0 + 8 * (k / kCols) + (lane >> 3);
    const float T0 = 1.0f - a_out[k];
    // With T = 0 every term of the pixel is an exact zero, as for a pixel
    // that blends nothing (and 1/T would be infinite).
    const bool live = px < p.W && py < p.H && n > 0;
    last[k] = live && T0 != 0.0f ? imax(0, imin(last[k], n)) : 0;
    Ti[k] = live && T0 != 0.0f ? 1.0f / T0 : 1.0f;
    gp0[k] = live ? gp0[k] : 0.0f;
    gp1[k] = live ? gp1[k] : 0.0f;
    gp2[k] = live ? gp2[k] : 0.0f;
    gpd[k] = live ? gpd[k] : 0.0f;
    gpa[k] = live ? gpa[k] : 0.0f;
    S[k] = live ? fmaf(bg2, gp2[k], fmaf(bg1, gp1[k], bg0 * gp0[k])) : 0.0f;
    lmax = imax(lmax, last[k]);
  }
  const int max_lc = __builtin_amdgcn_readfirstlane(wave_max_i32(lmax));
  if (max_lc == 0) return;
  const int flush_comp = lane < kSlotFloats / 4 ? slot_component(lane >> 2) : -1;  // kCols == 2
  float* const col_raw = s_slot + kColSlotFloats;  // kCols == 1: the column slot, then the sums
  const int raw_ofs = col_raw_offset(lane);
  const int raw_grp = col_group_index(lane);
  const int col_fidx = col_flush_index(lane);
  const int col_fcomp = col_flush_component(lane);
  int slot_gid = -1;  // Gaussian whose sums the slot holds (wave-uniform), -1: none

  // Batches of 64 list entries, back to front: [bs, batch_end).  The loads
  // run ahead: a batch's records were requested during the batch before it,
  // from indices requested one batch earlier still, so the only wait for
  // memory is the one at each batch's start (which also covers the
  // flushes' atomics: one counter tracks every vector memory operation).
  // The loads are unconditional (in-bounds entries for lanes past a batch),
  // which leaves the compiler nothing to merge, and so nothing to wait for,
  // right after them.
  const int* const list = p.point_list + rg.x;
  int bs = imax(0, max_lc - 64);
  int id = checked_point(batch_entry(list, bs, max_lc - bs, max_lc, lane), p.num_points);
  int id_ahead = batch_entry(list, imax(0, bs - 64), bs - imax(0, bs - 64), max_lc, lane);
  RecordRegs next = load_record(p.records, id);
  for (int batch_end = max_lc; batch_end > 0; batch_end = bs, bs = imax(0, bs - 64)) {
    const int cnt = batch_end - bs;
    // One wave per workgroup: its LDS queue orders these writes before the
    // broadcast reads below.  In the LDS copy r1.w (qcut, which the visits
    // only need as a threshold) and r2.w (the culling half-widths, used
    // above) carry the thresholds, and r0.w holds 2b (the visits need b only as 2 b dx, and
    // (2b) dx rounds exactly as (b dx) 2).
    {
      const BlendThresholds th = blend_thresholds(next.r1.w);
      s_rec[3 * lane] = make_float4(next.r0.x, next.r0.y, next.r0.z, 2.0f * next.r0.w);
      s_rec[3 * lane + 1] = make_float4(next.r1.x, next.r1.y, next.r1.z, __uint_as_float(th.cand));
      s_rec[3 * lane + 2] = make_float4(next.r2.x, next.r2.y, next.r2.z, __uint_as_float(th.sure));
    }
    const int batch_id = id;  // lane j: Gaussian of record j
    // A conic with a <= 0 can give q = -0 (adxx = (a dx) dx = -0), which
    // the forward's 0 <= q test takes and the bit compares do not; batches
    // with such a record add the q == 0 lanes to the candidates.
    const bool signed_zero = __ballot(lane < cnt && !(next.r0.z > 0.0f)) != 0;
    // blk[k]: the batch's records that may touch block k (with kBlockCull;
    // otherwise those that may touch the slice, for every block)
    uint64_t blk[kPix], todo = 0;
    {
      const bool live = lane < cnt;
      const unsigned ext = __float_as_uint(next.r2.w);
      if constexpr (kBlockCull) {
#pragma unroll
        for (int k = 0; k < kPix; ++k) {
          const float x0 = (float)(sx0 + 8 * (k % kCols)), y0 = (float)(sy0 + 8 * (k / kCols));
          blk[k] = __ballot(live && extents_meet(next.r0.x, next.r0.y, ext, x0, x0 + 7.0f, y0, y0 + 7.0f));
          todo |= blk[k];
        }
      } else {
        todo = __ballot(live && extents_meet(next.r0.x, next.r0.y, ext, (float)sx0, (float)(sx0 + kSliceW - 1),
                                             (float)sy0, (float)(sy0 + kSliceH - 1)));
#pragma unroll
        for (int k = 0; k < kPix; ++k) blk[k] = todo;
      }
    }
    // the next batch [bs - 64, bs): its records; and the indices of the one
    // after it (either may be empty: the loads then read a valid entry)
    {
      const int nbs = imax(0, bs - 64), nnbs = imax(0, nbs - 64);
      id = checked_point(id_ahead, p.num_points);
      next = load_record(p.records, id);
      id_ahead = batch_entry(list, nnbs, nbs - nnbs, max_lc, lane);
    }
    // Pixel k is active at list position pos when pos < last[k].  The
    // lanes whose pixel is active at every position of the batch (last >=
    // batch_end) form one mask per pixel; only a batch in which some pixel's
    // last contributor lies (bs < last < batch_end) has its visits compare
    // positions.  The walk is instantiated for both cases.
    uint64_t act_all[kPix];
    bool partial = false;
#pragma unroll
    for (int k = 0; k < kPix; ++k) {
      act_all[k] = __ballot(last[k] >= batch_end);
      partial |= __ballot(last[k] > bs && last[k] < batch_end) != 0;
    }
    auto walk = [&](auto partial_tag) {
      constexpr bool kPartial = decltype(partial_tag)::value;
      while (todo != 0) {
        const int jj = 63 - __builtin_clzll(todo);
        todo ^= 1ull << jj;
        const int pos = bs + jj;
        const float4 a = s_rec[3 * jj];
        const float4 b = s_rec[3 * jj + 1];
        const float4 f = s_rec[3 * jj + 2];
        const unsigned thr_cand = __float_as_uint(b.w), thr_sure = __float_as_uint(f.w);
        float dx[kCols], adxx[kCols], b2dx[kCols];
#pragma unroll
        for (int c = 0; c < kCols; ++c) {
          dx[c] = a.x - pfx[c];
          adxx[c] = a.z * dx[c] * dx[c];
          b2dx[c] = a.w * dx[c];  // a.w = 2b
        }
        float q[kPix], dy[kPix];
        uint64_t cand_lanes[kPix];  // the wave's lanes whose pixel k is a candidate
        uint64_t sure_lanes[kPix];  // ... and surely blends
        uint64_t any_lanes = 0, band = 0;  // band: lanes with a candidate that is not sure
#pragma unroll
        for (int k = 0; k < kPix; ++k) {
          q[k] = dy[k] = 0.0f;
          cand_lanes[k] = 0;
          if (kBlockCull && !((blk[k] >> jj) & 1)) continue;  // the record's box misses block k
          const int c = k % kCols;
          dy[k] = a.y - pfy[k];
          q[k] = conic_q_px(adxx[c], b2dx[c], b.x, dy[k]);  // exponent = -0.5 q
          // Lane masks of pos < last and 0 <= q <= qcut (the bit compare of
          // blend_thresholds), ANDed in scalar registers.
          const uint64_t act = kPartial ? __builtin_amdgcn_sicmp(pos, last[k], kCmpSLT) : act_all[k];
          cand_lanes[k] = act & __builtin_amdgcn_uicmp(__float_as_uint(q[k]), thr_cand, kCmpULT);
          if (signed_zero) cand_lanes[k] |= act & __builtin_amdgcn_fcmpf(q[k], 0.0f, kCmpOEQ);
          any_lanes |= cand_lanes[k];
        }
        if (any_lanes == 0) continue;
        // ... and 0 <= q <= qsure, only for visits with a candidate
#pragma unroll
        for (int k = 0; k < kPix; ++k) {
          sure_lanes[k] = cand_lanes[k] & __builtin_amdgcn_uicmp(__float_as_uint(q[k]), thr_sure, kCmpULT);
          band |= cand_lanes[k] & ~sure_lanes[k];
        }
        // Blend decisions, identical to the forward's: with the exponent above
        // power_cutoff + 2e-3 (q <= qcut - 4e-3) the forward's alpha is provably
        // >= 1/255 (the cutoff sits 1e-3 below -ln(255 o) and exp_sw / log_sw
        // err by < 1e-6 relative), above qcut provably < 1/255; only the thin
        // band between (and q = -0) needs exp_sw.  e = log2 of the Gaussian
        // value G for pixels that blend, -inf (G = 0) for the others.
        float e[kPix];
#pragma unroll
        for (int k = 0; k < kPix; ++k)
          e[k] = __builtin_amdgcn_inverse_ballot_w64(sure_lanes[k]) ? q[k] * (-0.5f * kLog2e) : -__builtin_inff();
        if (band != 0) {
#pragma unroll
          for (int k = 0; k < kPix; ++k) {
            // in the band 0 <= q, so the exponential's argument is non-positive;
            // on other lanes its value (inf or NaN included) is masked out
            const uint64_t band_lanes = cand_lanes[k] & ~sure_lanes[k];
            const float a_sw = fminf(kAlphaMax, b.y * exp_sw_q(q[k]));
            const bool blends = __builtin_amdgcn_inverse_ballot_w64(
                band_lanes & __builtin_amdgcn_fcmpf(a_sw, kAlphaMin, kCmpOGE));
            e[k] = blends ? q[k] * (-0.5f * kLog2e) : e[k];
          }
        }
        // -0 is the additive identity of every float, so the first terms
        // enter the sums exactly (and the compiler drops the additions).
        float sv[kCols], svy[kCols];
#pragma unroll
        for (int c = 0; c < kCols; ++c) sv[c] = svy[c] = -0.0f;
        float svyy = -0.0f, sr = -0.0f, sg = -0.0f, sb = -0.0f, sd = -0.0f;
        // One pixel's terms; the sums start at -0, the additive identity of
        // every float, so the first pixel's terms enter them exactly.
        auto blend = [&](int k) {
          const int c = k % kCols;
          // Gradient values use the hardware exponential (v_exp_f32): they only
          // need the 1e-3 gradient tolerance, the decisions above are exact.
          // A pixel that does not blend this Gaussian gets G = 2^-inf = 0, so
          // alpha = 0, 1/T is unchanged (an exact fma), S is unchanged and it
          // adds exact zeros.
          const float G = __builtin_amdgcn_exp2f(e[k]);
          const float alpha = fminf(kAlphaMax, b.y * G);
          // 1/T in front of this Gaussian: (1/T behind it) (1 - alpha), with
          // 1 - alpha >= 1 - kAlphaMax (the reference's 1e-5 floor never applies)
          const float tin = fmaf(-alpha, Ti[k], Ti[k]);
          const float Tn = __builtin_amdgcn_rcpf(tin);
          float fu = fmaf(f.z, gp2[k], fmaf(f.y, gp1[k], fmaf(f.x, gp0[k], gpa[k])));
          if (kDepth) fu = fmaf(b.z, gpd[k], fu);
          const float d = fu - S[k];
          const float v = G * (Tn * d);
          const float dch = alpha * Tn;
          const float vdy = v * dy[k];
          sv[c] += v;
          svy[c] += vdy;
          svyy = fmaf(vdy, dy[k], svyy);
          sr = fmaf(dch, gp0[k], sr);
          sg = fmaf(dch, gp1[k], sg);
          sb = fmaf(dch, gp2[k], sb);
          if (kDepth) sd = fmaf(dch, gpd[k], sd);
          // this Gaussian joins what lies behind the next (nearer) one:
          // alpha fu + (1 - alpha) S = S + alpha (fu - S)
          S[k] = fmaf(alpha, d, S[k]);
          Ti[k] = tin;
        };
        // A block with no candidate in the whole wave is skipped: there G = 0
        // for every lane, which leaves 1/T, S and the sums unchanged.  (Giving
        // the two blocks of a half their own paths, so that a visit skipping
        // the first one computes no -0 starting values, made the compiler
        // copy the four carried pixel states between registers on every
        // visit and took 79 VGPRs instead of 72: 1-2% slower.)
#pragma unroll
        for (int k = 0; k < kPix; ++k)
          if (cand_lanes[k] != 0) blend(k);
        // Pixel moments of v about the Gaussian's mean; the conic, opacity
        // and W/2, H/2 factors are per Gaussian and applied once, when the
        // per-Gaussian backward turns the sums into 2D gradients.
        if constexpr (kCols == 1) {
          // The transposed store of this Gaussian's sums, then (the wave's LDS
          // operations complete in order) the reads of the previous Gaussian's
          // slot and of this Gaussian's column groups, and the new slot after
          // the flush.
          col_raw[raw_ofs] = sv[0];
          col_raw[64 + raw_ofs] = svy[0];
          col_raw[128 + raw_ofs] = svyy;
          col_raw[192 + raw_ofs] = sr;
          col_raw[256 + raw_ofs] = sg;
          col_raw[320 + raw_ofs] = sb;
          col_raw[384 + raw_ofs] = sd;
          const float4 prev = reinterpret_cast<const float4*>(s_slot)[col_fidx];
          const float4 ga = reinterpret_cast<const float4*>(col_raw)[raw_grp];
          const float4 gb = reinterpret_cast<const float4*>(col_raw)[raw_grp + 1];
          if (slot_gid >= 0) flush_col_slot(prev, slot_gid, col_fcomp, p.grad_gauss);
          slot_gid = __builtin_amdgcn_readlane(batch_id, jj);
          const float col_sum = ((ga.x + ga.y) + (ga.z + ga.w)) + ((gb.x + gb.y) + (gb.z + gb.w));
          const float col_dx = col_sum * dx[0];
          s_slot[lane] = col_sum;
          s_slot[64 + lane] = col_dx;
          s_slot[128 + lane] = col_dx * dx[0];
        } else {
          float m[3];
          float g[kGradFloats];
          float vdx = sv[0] * dx[0];
          g[0] = vdx;               // sum v dx
          g[1] = svy[0];            // sum v dy
          g[2] = vdx * dx[0];       // sum v dx^2
          g[3] = svy[0] * dx[0];    // sum v dx dy
          g[5] = sv[0];             // dL/dopacity
#pragma unroll
          for (int c = 1; c < kCols; ++c) {
            vdx = sv[c] * dx[c];
            g[0] += vdx;
            g[1] += svy[c];
            g[2] = fmaf(vdx, dx[c], g[2]);
            g[3] = fmaf(svy[c], dx[c], g[3]);
            g[5] += sv[c];
          }
          g[4] = svyy;              // sum v dy^2
          g[6] = sr;
          g[7] = sg;
          g[8] = sb;
          g[9] = sd;
          wave_fold10(g, m);
          if (slot_gid >= 0) flush_slot(s_slot, slot_gid, lane, flush_comp, p.grad_gauss);
          slot_gid = __builtin_amdgcn_readlane(batch_id, jj);
          // The wave's LDS operations complete in order: these stores follow
          // the flush's read of the previous Gaussian's sums.
          s_slot[lane] = m[0];
          s_slot[64 + lane] = m[1];
          s_slot[128 + lane] = m[2];
        }
      }
    };
    if (partial)
      walk(std::true_type{});
    else
      walk(std::false_type{});
  }
  if (slot_gid >= 0) {
    if constexpr (kCols == 1)
      flush_col_slot(reinterpret_cast<const float4*>(s_slot)[col_fidx], slot_gid, col_fcomp, p.grad_gauss);
    else
      flush_slot(s_slot, slot_gid, lane, flush_comp, p.grad_gauss);
  }
}

// How a tile is split over waves.  With small Gaussians (a few tiles each)
// two waves walk an ordinary tile, one 8x16 half each (two blocks, two
// pixels per lane): many waves per SIMD (few registers) hide the latency of
// the walk.  When the Gaussians are large (kWholeTiles: more than
// kWholeTilePairsPerPoint tiles each on average) one wave walks the whole
// tile (four blocks, four pixels per lane), so the moments of a Gaussian that
// covers most of the tile are folded and sent once per tile instead of
// twice.  Measured on one MI355X: halves 20% faster at 1M Gaussians, 1080p
// (about 3 pairs per Gaussian), whole tiles 36% faster at 5M with the large
// splats (about 30).  A tile whose list is longer than p.long_tile is walked
// by four one-wave workgroups, one 8x8 quadrant each: its serial walk, which
// bounds the kernel when a few tiles hold most of the pairs, is then
// shorter.  The grid is a segment of kFirst workgroups per tile (the halves
// or the whole tile of an ordinary tile, the first quadrants of a long one)
// followed by one of 4 - kFirst per tile for the other quadrants, which exit
// at once for ordinary tiles: workgroups go round-robin to the XCDs' CUs,
// and exiting workgroups interleaved with working ones at a fixed period
// would leave some CUs with none of the work, while at the end of the grid
// they only fill slots that the draining work leaves free.
constexpr int64_t kWholeTilePairsPerPoint = 4;

template <bool kDepth, bool kWholeTiles>
__device__ __forceinline__ void render_bwd_tiles(const RenderBwdParams& p) {
  constexpr int kFirst = kWholeTiles ? 1 : 2;
  __shared__ float4 s_rec[3 * 64];  // record j at s_rec[3 j .. 3 j + 2]
  __shared__ __align__(16) float s_slot[kSlotLdsFloats];
  const int first_units = kFirst * p.num_tiles;
  const int extra_units = (4 - kFirst) * p.num_tiles;
  const int seg = xcd_grid(first_units);
  const bool extra = (int)blockIdx.x >= seg;
  const int unit = extra ? xcd_unit(blockIdx.x - seg, extra_units) : xcd_unit(blockIdx.x, first_units);
  if (unit >= (extra ? extra_units : first_units)) return;  // segment padding
  const int slot = extra ? unit / (4 - kFirst) : unit / kFirst;
  // (clamped: a buffer the forward did not write cannot send a workgroup
  // outside the ranges)
  const int tile = p.tile_order ? imax(0, imin(p.tile_order[slot], p.num_tiles - 1)) : slot;
  const int quadrant = extra ? kFirst + unit % (4 - kFirst) : unit % kFirst;
  int2 rg = p.ranges[tile];
  rg.x = imax(0, imin(rg.x, p.num_rendered));
  rg.y = imax(rg.x, imin(rg.y, p.num_rendered));
  if (rg.y - rg.x > p.long_tile)
    render_bwd_slice<kDepth, 1, 1, false>(p, tile, quadrant, s_rec, s_slot);
  else if (!extra && kWholeTiles)
    render_bwd_slice<kDepth, 4, 2, true>(p, tile, 0, s_rec, s_slot);
  else if (!extra)
    render_bwd_slice<kDepth, 2, 1, false>(p, tile, quadrant, s_rec, s_slot);
}

// The halves and quadrants need 72 VGPRs, seven waves per SIMD (the bound
// keeps them at six or more); the whole-tile walk needs more.
template <bool kDepth>
__global__ __launch_bounds__(64, 6) void render_bwd_kernel(RenderBwdParams p) {
  render_bwd_tiles<kDepth, false>(p);
}

template <bool kDepth>
__global__ __launch_bounds__(64) void render_bwd_whole_kernel(RenderBwdParams p) {
  render_bwd_tiles<kDepth, true>(p);
}

struct PreprocessBwdParams {
  int P, K, degree;
  const float* means3d;
  const float* scales;
  const float* rotations;
  const float* cov3d;  // precomputed (N, 6) 3D covariances, or null
  float scale_modifier;
  const float* shs;
  const float* campos;
  const float* view;
  const float* proj;
  float tanfovx, tanfovy, focal_x, focal_y;
  const int* radii;
  const uint8_t* clamped;
  const float* grad_gauss;    // render_bwd's pixel moments (N,10)
  const float4* records;     // the forward's render records: conic and opacity
  float half_w, half_h;      // W/2, H/2: NDC scaling of the xy gradients
  const float* grad_proj_2d;
  const float* grad_conic_2d;
  const float* grad_conic_2d_inv;
  int flow_double;
  float filter_variance;  // Mip-Splatting screen-space variance added to cov2D; 0 = none
  float* grad_means3d;
  float* grad_means2d;
  float* grad_scales;
  float* grad_rotations;
  float* grad_cov3d;
  float* grad_sh;
  float* grad_opacity;
  float* grad_colors;
  int sh_vec16;  // K == 16 and shs / grad_sh 16-byte aligned: float4 SH access
};

struct V3 {
  float x, y, z;
};

__device__ __forceinline__ float dot3(V3 a, float b0, float b1, float b2) { return a.x * b0 + a.y * b1 + a.z * b2; }

// SH colour backward for one Gaussian: writes its K x 3 block of grad_sh and
// returns dL/dmean through the direction normalisation.  With kVec16 the
// block is K = 16 coefficients (48 floats) and sh_mem / gsh_mem are the
// caller's 48-float register arrays (the kernel moves them between HBM and
// registers through LDS); otherwise they point at the Gaussian's blocks in
// global memory.
template <bool kVec16>
__device__ __forceinline__ V3 sh_backward(const float* __restrict__ sh_mem, float* __restrict__ gsh_mem, int K,
                                          int degree, float dirx, float diry, float dirz, float g0, float g1,
                                          float g2) {
  if (kVec16) {
#pragma unroll
    for (int i = 0; i < 48; ++i) gsh_mem[i] = 0.0f;
  }
  const float* sh = sh_mem;
  float* gsh = gsh_mem;
  const float len_sq = dirx * dirx + diry * diry + dirz * dirz;
  const float inv_len = 1.0f / sqrtf(fmaxr(len_sq, 1.0e-20f));
  const float x = dirx * inv_len, y = diry * inv_len, z = dirz * inv_len;
  V3 dx = {0.0f, 0.0f, 0.0f}, dy = {0.0f, 0.0f, 0.0f}, dz = {0.0f, 0.0f, 0.0f};
  int written = 0;
  if (K > 0) {
    gsh[0] = kShC0 * g0;
    gsh[1] = kShC0 * g1;
    gsh[2] = kShC0 * g2;
    written = 1;
  }
  if (degree > 0 && K > 3) {
    const float w1 = -kShC1 * y, w2 = kShC1 * z, w3 = -kShC1 * x;
    gsh[3] = w1 * g0; gsh[4] = w1 * g1; gsh[5] = w1 * g2;
    gsh[6] = w2 * g0; gsh[7] = w2 * g1; gsh[8] = w2 * g2;
    gsh[9] = w3 * g0; gsh[10] = w3 * g1; gsh[11] = w3 * g2;
    written = 4;
    dx = {-kShC1 * sh[9], -kShC1 * sh[10], -kShC1 * sh[11]};
    dy = {-kShC1 * sh[3], -kShC1 * sh[4], -kShC1 * sh[5]};
    dz = {kShC1 * sh[6], kShC1 * sh[7], kShC1 * sh[8]};
    if (degree > 1 && K > 8) {
      const float xx = x * x, yy = y * y, zz = z * z;
      const float xy = x * y, yz = y * z, xz = x * z;
      const float w4 = kShC2_0 * xy, w5 = kShC2_1 * yz, w6 = kShC2_2 * (2.0f * zz - xx - yy);
      const float w7 = kShC2_3 * xz, w8 = kShC2_4 * (xx - yy);
      gsh[12] = w4 * g0; gsh[13] = w4 * g1; gsh[14] = w4 * g2;
      gsh[15] = w5 * g0; gsh[16] = w5 * g1; gsh[17] = w5 * g2;
      gsh[18] = w6 * g0; gsh[19] = w6 * g1; gsh[20] = w6 * g2;
      gsh[21] = w7 * g0; gsh[22] = w7 * g1; gsh[23] = w7 * g2;
      gsh[24] = w8 * g0; gsh[25] = w8 * g1; gsh[26] = w8 * g2;
      written = 9;
      const float ex4 = kShC2_0 * y, ex6 = kShC2_2 * (-2.0f * x), ex7 = kShC2_3 * z, ex8 = kShC2_4 * (2.0f * x);
      const float ey4 = kShC2_0 * x, ey5 = kShC2_1 * z, ey6 = kShC2_2 * (-2.0f * y), ey8 = kShC2_4 * (-2.0f * y);
      const float ez5 = kShC2_1 * y, ez6 = kShC2_2 * (4.0f * z), ez7 = kShC2_3 * x;
#define GS_C(k, c) sh[3 * (k) + (c)]
      dx.x = dx.x + ex4 * GS_C(4, 0) + ex6 * GS_C(6, 0) + ex7 * GS_C(7, 0) + ex8 * GS_C(8, 0);
      dx.y = dx.y + ex4 * GS_C(4, 1) + ex6 * GS_C(6, 1) + ex7 * GS_C(7, 1) + ex8 * GS_C(8, 1);
      dx.z = dx.z + ex4 * GS_C(4, 2) + ex6 * GS_C(6, 2) + ex7 * GS_C(7, 2) + ex8 * GS_C(8, 2);
      dy.x = dy.x + ey4 * GS_C(4, 0) + ey5 * GS_C(5, 0) + ey6 * GS_C(6, 0) + ey8 * GS_C(8, 0);
      dy.y = dy.y + ey4 * GS_C(4, 1) + ey5 * GS_C(5, 1) + ey6 * GS_C(6, 1) + ey8 * GS_C(8, 1);
      dy.z = dy.z + ey4 * GS_C(4, 2) + ey5 * GS_C(5, 2) + ey6 * GS_C(6, 2) + ey8 * GS_C(8, 2);
      dz.x = dz.x + ez5 * GS_C(5, 0) + ez6 * GS_C(6, 0) + ez7 * GS_C(7, 0);
      dz.y = dz.y + ez5 * GS_C(5, 1) + ez6 * GS_C(6, 1) + ez7 * GS_C(7, 1);
      dz.z = dz.z + ez5 * GS_C(5, 2) + ez6 * GS_C(6, 2) + ez7 * GS_C(7, 2);
      if (degree > 2 && K > 15) {
        const float w9 = kShC3_0 * y * (3.0f * xx - yy);
        const float w10 = kShC3_1 * xy * z;
        const float w11 = kShC3_2 * y * (4.0f * zz - xx - yy);
        const float w12 = kShC3_3 * z * (2.0f * zz - 3.0f * xx - 3.0f * yy);
        const float w13 = kShC3_4 * x * (4.0f * zz - xx - yy);
        const float w14 = kShC3_5 * z * (xx - yy);
        const float w15 = kShC3_6 * x * (xx - 3.0f * yy);
        gsh[27] = w9 * g0; gsh[28] = w9 * g1; gsh[29] = w9 * g2;
        gsh[30] = w10 * g0; gsh[31] = w10 * g1; gsh[32] = w10 * g2;
        gsh[33] = w11 * g0; gsh[34] = w11 * g1; gsh[35] = w11 * g2;
        gsh[36] = w12 * g0; gsh[37] = w12 * g1; gsh[38] = w12 * g2;
        gsh[39] = w13 * g0; gsh[40] = w13 * g1; gsh[41] = w13 * g2;
        gsh[42] = w14 * g0; gsh[43] = w14 * g1; gsh[44] = w14 * g2;
        gsh[45] = w15 * g0; gsh[46] = w15 * g1; gsh[47] = w15 * g2;
        written = 16;
        const float ex9 = kShC3_0 * (6.0f * xy), ex10 = kShC3_1 * yz, ex11 = kShC3_2 * (-2.0f * xy);
        const float ex12 = kShC3_3 * (-6.0f * xz), ex13 = kShC3_4 * (-3.0f * xx + 4.0f * zz - yy);
        const float ex14 = kShC3_5 * (2.0f * xz), ex15 = kShC3_6 * (3.0f * (xx - yy));
        const float ey9 = kShC3_0 * (3.0f * (xx - yy)), ey10 = kShC3_1 * xz;
        const float ey11 = kShC3_2 * (-3.0f * yy + 4.0f * zz - xx), ey12 = kShC3_3 * (-6.0f * yz);
        const float ey13 = kShC3_4 * (-2.0f * xy), ey14 = kShC3_5 * (-2.0f * yz), ey15 = kShC3_6 * (-6.0f * xy);
        const float ez10 = kShC3_1 * xy, ez11 = kShC3_2 * (8.0f * yz);
        const float ez12 = kShC3_3 * (3.0f * (2.0f * zz - xx - yy)), ez13 = kShC3_4 * (8.0f * xz);
        const float ez14 = kShC3_5 * (xx - yy);
#define GS_DX(acc, c)                                                                                      \
  acc = acc + ex9 * GS_C(9, c) + ex10 * GS_C(10, c) + ex11 * GS_C(11, c) + ex12 * GS_C(12, c) +           \
        ex13 * GS_C(13, c) + ex14 * GS_C(14, c) + ex15 * GS_C(15, c)
#define GS_DY(acc, c)                                                                                      \
  acc = acc + ey9 * GS_C(9, c) + ey10 * GS_C(10, c) + ey11 * GS_C(11, c) + ey12 * GS_C(12, c) +           \
        ey13 * GS_C(13, c) + ey14 * GS_C(14, c) + ey15 * GS_C(15, c)
#define GS_DZ(acc, c)                                                                                      \
  acc = acc + ez10 * GS_C(10, c) + ez11 * GS_C(11, c) + ez12 * GS_C(12, c) + ez13 * GS_C(13, c) +         \
        ez14 * GS_C(14, c)
        GS_DX(dx.x, 0); GS_DX(dx.y, 1); GS_DX(dx.z, 2);
        GS_DY(dy.x, 0); GS_DY(dy.y, 1); GS_DY(dy.z, 2);
        GS_DZ(dz.x, 0); GS_DZ(dz.y, 1); GS_DZ(dz.z, 2);
#undef GS_DX
#undef GS_DY
#undef GS_DZ
#undef GS_C
      }
    }
  }
  if (!kVec16) {
    for (int k = written; k < K; ++k) {
      gsh[3 * k + 0] = 0.0f;
      gsh[3 * k + 1] = 0.0f;
      gsh[3 * k + 2] = 0.0f;
    }
  }
  const float ddir0 = dot3(dx, g0, g1, g2);
  const float ddir1 = dot3(dy, g0, g1, g2);
  const float ddir2 = dot3(dz, g0, g1, g2);
  // d normalize(v) / dv applied to dL/ddir (math_kernels.py:90-97).
  const float sum2 = dirx * dirx + diry * diry + dirz * dirz;
  const float invsum32 = 1.0f / sqrtf(fmaxr(sum2 * sum2 * sum2, 1.0e-20f));
  V3 r;
  r.x = ((sum2 - dirx * dirx) * ddir0 - diry * dirx * ddir1 - dirz * dirx * ddir2) * invsum32;
  r.y = (-dirx * diry * ddir0 + (sum2 - diry * diry) * ddir1 - dirz * diry * ddir2) * invsum32;
  r.z = (-dirx * dirz * ddir0 - diry * dirz * ddir1 + (sum2 - dirz * dirz) * ddir2) * invsum32;
  return r;
}

// The float4 SH path (K = 16) moves each wave's coefficient and gradient
// blocks (64 Gaussians x 192 bytes, contiguous) between HBM and LDS with
// whole-wave accesses (64 consecutive float4, 1 KB, per instruction), and each
// lane works on its Gaussian's row in LDS: a lane's own 12 float4 at a
// 192-byte stride make every memory instruction touch 64 cache lines (the
// address unit was then busy for 80% of the kernel).  The coefficients are
// requested at the kernel's start, so their loads overlap the rest of the
// Gaussian backward; rows are 13 float4 apart, so that the lanes' row
// accesses fall in distinct LDS banks.  The staging is wave-wide, so every
// lane of the grid runs the Gaussian backward (lanes past P on Gaussian
// P - 1, storing nothing).  The 13 KB per wave hold the kernel to three
// waves per SIMD; staging 96 bytes per Gaussian at a time (four waves per
// SIMD) measured slower, its second half's loads waiting on the first's use.
constexpr int kShRow = 13;

struct ShStage {
  float4* rows;  // the wave's 64 rows of kShRow float4 in LDS
  int lane, w0, nvalid;  // w0: the wave's first Gaussian; nvalid: its Gaussians below P
};

// The wave's coefficient blocks into its LDS rows.  Each block's load is
// followed by its guarded LDS store, so the wave waits for the loads one at a
// time; issuing all twelve before the first store (clamped addresses,
// unguarded stores) measured slower at configs 2 and 3, the kernel's other
// loads then queueing behind 12 KB per wave.
__device__ __forceinline__ void sh_stage_in(const ShStage& st, const float* shs) {
  const float4* src = reinterpret_cast<const float4*>(shs) + (size_t)st.w0 * 12;
#pragma unroll
  for (int j = 0; j < 12; ++j) {
    const int f = j * 64 + st.lane, g = f / 12;
    if (g < st.nvalid) st.rows[g * kShRow + (f - g * 12)] = src[f];
  }
  __builtin_amdgcn_wave_barrier();  // the lanes' row reads follow these writes (LDS order)
}

// The wave's gradient blocks from its LDS rows to grad_sh (after every
// lane's rows are written: the wave's LDS accesses complete in order).
__device__ __forceinline__ void sh_stage_out(const ShStage& st, float* grad_sh) {
  __builtin_amdgcn_wave_barrier();
  float4* dst = reinterpret_cast<float4*>(grad_sh) + (size_t)st.w0 * 12;
#pragma unroll
  for (int j = 0; j < 12; ++j) {
    const int f = j * 64 + st.lane, g = f / 12;
    if (g < st.nvalid) dst[f] = st.rows[g * kShRow + (f - g * 12)];
  }
}

// Half h of a row (floats 24 h .. 24 h + 23 of the Gaussian's block).
__device__ __forceinline__ void row_half_in(const float4* row, int h, float (&v)[24]) {
#pragma unroll
  for (int k = 0; k < 6; ++k) {
    const float4 q = row[6 * h + k];
    v[4 * k + 0] = q.x;
    v[4 * k + 1] = q.y;
    v[4 * k + 2] = q.z;
    v[4 * k + 3] = q.w;
  }
}

__device__ __forceinline__ void row_half_out(float4* row, int h, const float (&v)[24]) {
#pragma unroll
  for (int k = 0; k < 6; ++k) row[6 * h + k] = make_float4(v[4 * k + 0], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
}

// sh_backward for K = 16 on the Gaussian's LDS row: its coefficients are
// read and replaced by their gradients half by half (24 live at a time).
// The direction gradient sums are accumulated coefficient by coefficient in
// ascending order, which is the association order of sh_backward's
// expressions, so the results are the same bit for bit.  `active` (a kept
// Gaussian below P) selects the lanes whose gradients are computed (the
// others write zeros).
__device__ __forceinline__ V3 sh_backward_row(float4* row, int degree, bool active, float dirx, float diry,
                                              float dirz, float g0, float g1, float g2) {
  const float len_sq = dirx * dirx + diry * diry + dirz * dirz;
  const float inv_len = 1.0f / sqrtf(fmaxr(len_sq, 1.0e-20f));
  const float x = dirx * inv_len, y = diry * inv_len, z = dirz * inv_len;
  const float xx = x * x, yy = y * y, zz = z * z;
  const float xy = x * y, yz = y * z, xz = x * z;
  const bool d1 = active && degree > 0, d2 = d1 && degree > 1, d3 = d2 && degree > 2;
  V3 dx = {0.0f, 0.0f, 0.0f}, dy = {0.0f, 0.0f, 0.0f}, dz = {0.0f, 0.0f, 0.0f};
  float v[24];
  // coefficients 0-7
  row_half_in(row, 0, v);
#define GS_C(k, c) v[3 * (k) + (c)]
  if (d1) {
    dx = {-kShC1 * GS_C(3, 0), -kShC1 * GS_C(3, 1), -kShC1 * GS_C(3, 2)};
    dy = {-kShC1 * GS_C(1, 0), -kShC1 * GS_C(1, 1), -kShC1 * GS_C(1, 2)};
    dz = {kShC1 * GS_C(2, 0), kShC1 * GS_C(2, 1), kShC1 * GS_C(2, 2)};
  }
  const float ex4 = kShC2_0 * y, ex6 = kShC2_2 * (-2.0f * x), ex7 = kShC2_3 * z, ex8 = kShC2_4 * (2.0f * x);
  const float ey4 = kShC2_0 * x, ey5 = kShC2_1 * z, ey6 = kShC2_2 * (-2.0f * y), ey8 = kShC2_4 * (-2.0f * y);
  const float ez5 = kShC2_1 * y, ez6 = kShC2_2 * (4.0f * z), ez7 = kShC2_3 * x;
  if (d2) {
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      float ax = dx.x, ay = dy.x, az = dz.x;
      if (c == 1) { ax = dx.y; ay = dy.y; az = dz.y; }
      if (c == 2) { ax = dx.z; ay = dy.z; az = dz.z; }
      ax = ax + ex4 * GS_C(4, c);
      ax = ax + ex6 * GS_C(6, c);
      ax = ax + ex7 * GS_C(7, c);
      ay = ay + ey4 * GS_C(4, c);
      ay = ay + ey5 * GS_C(5, c);
      ay = ay + ey6 * GS_C(6, c);
      az = az + ez5 * GS_C(5, c);
      az = az + ez6 * GS_C(6, c);
      az = az + ez7 * GS_C(7, c);
      if (c == 0) { dx.x = ax; dy.x = ay; dz.x = az; }
      if (c == 1) { dx.y = ax; dy.y = ay; dz.y = az; }
      if (c == 2) { dx.z = ax; dy.z = ay; dz.z = az; }
    }
  }
  // coefficients 8-15
  row_half_in(row, 1, v);
#undef GS_C
#define GS_C(k, c) v[3 * ((k) - 8) + (c)]
  if (d2) {
    dx.x = dx.x + ex8 * GS_C(8, 0); dx.y = dx.y + ex8 * GS_C(8, 1); dx.z = dx.z + ex8 * GS_C(8, 2);
    dy.x = dy.x + ey8 * GS_C(8, 0); dy.y = dy.y + ey8 * GS_C(8, 1); dy.z = dy.z + ey8 * GS_C(8, 2);
  }
  const float ex9 = kShC3_0 * (6.0f * xy), ex10 = kShC3_1 * yz, ex11 = kShC3_2 * (-2.0f * xy);
  const float ex12 = kShC3_3 * (-6.0f * xz), ex13 = kShC3_4 * (-3.0f * xx + 4.0f * zz - yy);
  const float ex14 = kShC3_5 * (2.0f * xz), ex15 = kShC3_6 * (3.0f * (xx - yy));
  const float ey9 = kShC3_0 * (3.0f * (xx - yy)), ey10 = kShC3_1 * xz;
  const float ey11 = kShC3_2 * (-3.0f * yy + 4.0f * zz - xx), ey12 = kShC3_3 * (-6.0f * yz);
  const float ey13 = kShC3_4 * (-2.0f * xy), ey14 = kShC3_5 * (-2.0f * yz), ey15 = kShC3_6 * (-6.0f * xy);
  const float ez10 = kShC3_1 * xy, ez11 = kShC3_2 * (8.0f * yz);
  const float ez12 = kShC3_3 * (3.0f * (2.0f * zz - xx - yy)), ez13 = kShC3_4 * (8.0f * xz);
  const float ez14 = kShC3_5 * (xx - yy);
  if (d3) {
#define GS_DX(acc, c)                                                                                      \
  acc = acc + ex9 * GS_C(9, c) + ex10 * GS_C(10, c) + ex11 * GS_C(11, c) + ex12 * GS_C(12, c) +           \
        ex13 * GS_C(13, c) + ex14 * GS_C(14, c) + ex15 * GS_C(15, c)
#define GS_DY(acc, c)                                                                                      \
  acc = acc + ey9 * GS_C(9, c) + ey10 * GS_C(10, c) + ey11 * GS_C(11, c) + ey12 * GS_C(12, c) +           \
        ey13 * GS_C(13, c) + ey14 * GS_C(14, c) + ey15 * GS_C(15, c)
#define GS_DZ(acc, c)                                                                                      \
  acc = acc + ez10 * GS_C(10, c) + ez11 * GS_C(11, c) + ez12 * GS_C(12, c) + ez13 * GS_C(13, c) +         \
        ez14 * GS_C(14, c)
    GS_DX(dx.x, 0); GS_DX(dx.y, 1); GS_DX(dx.z, 2);
    GS_DY(dy.x, 0); GS_DY(dy.y, 1); GS_DY(dy.z, 2);
    GS_DZ(dz.x, 0); GS_DZ(dz.y, 1); GS_DZ(dz.z, 2);
#undef GS_DX
#undef GS_DY
#undef GS_DZ
  }
#undef GS_C
  // gradients of coefficients 0-7, then 8-15 (zero beyond the degree)
  {
    const float w1 = -kShC1 * y, w2 = kShC1 * z, w3 = -kShC1 * x;
    const float w4 = kShC2_0 * xy, w5 = kShC2_1 * yz, w6 = kShC2_2 * (2.0f * zz - xx - yy);
    const float w7 = kShC2_3 * xz;
    const float wk[8] = {kShC0, w1, w2, w3, w4, w5, w6, w7};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const bool on = k == 0 ? active : (k < 4 ? d1 : d2);
      v[3 * k + 0] = on ? wk[k] * g0 : 0.0f;
      v[3 * k + 1] = on ? wk[k] * g1 : 0.0f;
      v[3 * k + 2] = on ? wk[k] * g2 : 0.0f;
    }
    row_half_out(row, 0, v);
  }
  {
    const float w8 = kShC2_4 * (xx - yy);
    const float w9 = kShC3_0 * y * (3.0f * xx - yy);
    const float w10 = kShC3_1 * xy * z;
    const float w11 = kShC3_2 * y * (4.0f * zz - xx - yy);
    const float w12 = kShC3_3 * z * (2.0f * zz - 3.0f * xx - 3.0f * yy);
    const float w13 = kShC3_4 * x * (4.0f * zz - xx - yy);
    const float w14 = kShC3_5 * z * (xx - yy);
    const float w15 = kShC3_6 * x * (xx - 3.0f * yy);
    const float wk[8] = {w8, w9, w10, w11, w12, w13, w14, w15};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const bool on = k == 0 ? d2 : d3;
      v[3 * k + 0] = on ? wk[k] * g0 : 0.0f;
      v[3 * k + 1] = on ? wk[k] * g1 : 0.0f;
      v[3 * k + 2] = on ? wk[k] * g2 : 0.0f;
    }
    row_half_out(row, 1, v);
  }
  const float ddir0 = dot3(dx, g0, g1, g2);
  const float ddir1 = dot3(dy, g0, g1, g2);
  const float ddir2 = dot3(dz, g0, g1, g2);
  // d normalize(v) / dv applied to dL/ddir (math_kernels.py:90-97).
  const float sum2 = dirx * dirx + diry * diry + dirz * dirz;
  const float invsum32 = 1.0f / sqrtf(fmaxr(sum2 * sum2 * sum2, 1.0e-20f));
  V3 r;
  r.x = ((sum2 - dirx * dirx) * ddir0 - diry * dirx * ddir1 - dirz * dirx * ddir2) * invsum32;
  r.y = (-dirx * diry * ddir0 + (sum2 - diry * diry) * ddir1 - dirz * diry * ddir2) * invsum32;
  r.z = (-dirx * dirz * ddir0 - diry * dirz * ddir1 + (sum2 - dirz * dirz) * ddir2) * invsum32;
  return r;
}

// One Gaussian's backward; `valid`: tid < P (else tid = P - 1 and nothing
// is stored).
__device__ __forceinline__ void preprocess_bwd_one(const PreprocessBwdParams& p, int tid, bool valid,
                                                   const ShStage& stage) {
  const float* __restrict__ V = p.view;
  const float* __restrict__ Pm = p.proj;
  const float mx = p.means3d[3 * tid + 0];
  const float my = p.means3d[3 * tid + 1];
  const float mz = p.means3d[3 * tid + 2];
  const int rad = p.radii[tid];
  const float* gg = p.grad_gauss + (size_t)tid * kGradFloats;
  // The render gradients from the pixel moments (m0 .. m4 = sums of v dx,
  // v dy, v dx^2, v dx dy, v dy^2 over the Gaussian's blended pixels) and
  // the record's conic (a, b, c) and opacity o:
  //   dL/dxy    = -(W/2, H/2) o (a m0 + b m1, c m1 + b m0),
  //   dL/dconic = -o/2 (m2, m3, m4),
  // the reference's per-pixel terms (backward_kernels.py:678-685) summed.
  // A Gaussian that was never rendered has zero moments (its record is not
  // read).
  // Every per-Gaussian word that a rendered Gaussian needs is loaded here,
  // together, so that the wave waits for memory once rather than once per
  // use below.
  const bool precomp = p.cov3d != nullptr;
  float4 r0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), r1 = r0, q_in = r0;
  float ax_in = 0.0f, ay_in = 0.0f, uc_in0 = 0.0f, uc_in1 = 0.0f, uc_in2 = 0.0f;
  float ci_in0 = 0.0f, ci_in1 = 0.0f, ci_in2 = 0.0f;
  float cv_in[6] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  if (rad > 0) {
    r0 = p.records[3 * (size_t)tid];
    r1 = p.records[3 * (size_t)tid + 1];
    if (p.grad_proj_2d) {
      ax_in = p.grad_proj_2d[2 * tid + 0];
      ay_in = p.grad_proj_2d[2 * tid + 1];
    }
    if (precomp) {
#pragma unroll
      for (int k = 0; k < 6; ++k) cv_in[k] = p.cov3d[6 * (size_t)tid + k];
    } else {
      cv_in[0] = p.scales[3 * tid + 0];
      cv_in[1] = p.scales[3 * tid + 1];
      cv_in[2] = p.scales[3 * tid + 2];
      q_in = reinterpret_cast<const float4*>(p.rotations)[tid];
    }
    if (p.grad_conic_2d) {
      uc_in0 = p.grad_conic_2d[3 * tid + 0];
      uc_in1 = p.grad_conic_2d[3 * tid + 1];
      uc_in2 = p.grad_conic_2d[3 * tid + 2];
    }
    if (p.grad_conic_2d_inv) {
      ci_in0 = p.grad_conic_2d_inv[3 * tid + 0];
      ci_in1 = p.grad_conic_2d_inv[3 * tid + 1];
      ci_in2 = p.grad_conic_2d_inv[3 * tid + 2];
    }
  }
  float rpx = 0.0f, rpy = 0.0f, rc0 = 0.0f, rc1 = 0.0f, rc2 = 0.0f;
  if (rad > 0) {
    const float o = r1.y;
    rpx = -p.half_w * (o * (r0.z * gg[0] + r0.w * gg[1]));
    rpy = -p.half_h * (o * (r1.x * gg[1] + r0.w * gg[0]));
    const float ho = -0.5f * o;
    rc0 = ho * gg[2];
    rc1 = ho * gg[3];
    rc2 = ho * gg[4];
  }
  const float ropa = gg[5];
  const float rcol0 = gg[6], rcol1 = gg[7], rcol2 = gg[8];
  const float rdepth = gg[9];

  // Part A: projected mean and depth.
  const float hom_x = Pm[0] * mx + Pm[4] * my + Pm[8] * mz + Pm[12];
  const float hom_y = Pm[1] * mx + Pm[5] * my + Pm[9] * mz + Pm[13];
  const float hom_w = Pm[3] * mx + Pm[7] * my + Pm[11] * mz + Pm[15];
  const float inv_w = 1.0f / (hom_w + 0.0000001f);
  float gx = rpx, gy = rpy;
  const float inv_w2 = inv_w * inv_w;
  if (rad > 0) {
    // absent upstream gradients (null) are zero
    float ax = ax_in;
    float ay = ay_in;
    if (p.flow_double) {
      ax = ax + rpx;
      ay = ay + rpy;
    }
    gx = gx + ax;
    gy = gy + ay;
  }
  const float gh = hom_x * gx + hom_y * gy;
  float pm_x = inv_w * (Pm[0] * gx + Pm[1] * gy) - Pm[3] * inv_w2 * gh;
  float pm_y = inv_w * (Pm[4] * gx + Pm[5] * gy) - Pm[7] * inv_w2 * gh;
  float pm_z = inv_w * (Pm[8] * gx + Pm[9] * gy) - Pm[11] * inv_w2 * gh;
  const float zv = V[2] * mx + V[6] * my + V[10] * mz + V[14];
  pm_x = pm_x + (V[2] - V[3] * zv) * rdepth;
  pm_y = pm_y + (V[6] - V[7] * zv) * rdepth;
  pm_z = pm_z + (V[10] - V[11] * zv) * rdepth;

  // Part B: cov2D -> cov3D -> scale / rotation, and the mean through the
  // EWA Jacobian.
  float gcm_x = 0.0f, gcm_y = 0.0f, gcm_z = 0.0f;
  float gs0 = 0.0f, gs1 = 0.0f, gs2 = 0.0f;
  float gq0 = 0.0f, gq1 = 0.0f, gq2 = 0.0f, gq3 = 0.0f;
  if (rad > 0) {
    const float x = V[0] * mx + V[4] * my + V[8] * mz + V[12];
    const float y = V[1] * mx + V[5] * my + V[9] * mz + V[13];
    const float z = V[2] * mx + V[6] * my + V[10] * mz + V[14];
    const float tz_inv = 1.0f / (z + 1.0e-7f);
    const float limx = kFovClamp * p.tanfovx;
    const float limy = kFovClamp * p.tanfovy;
    const float txtz = x * tz_inv;
    const float tytz = y * tz_inv;
    const float x_grad_mul = (txtz < -limx || txtz > limx) ? 0.0f : 1.0f;
    const float y_grad_mul = (tytz < -limy || tytz > limy) ? 0.0f : 1.0f;
    const float tx = clampr(txtz, -limx, limx);
    const float ty = clampr(tytz, -limy, limy);
    const float j00 = p.focal_x * tz_inv;
    const float j02 = -j00 * tx;
    const float j11 = p.focal_y * tz_inv;
    const float j12 = -j11 * ty;
    const float w00 = V[0], w01 = V[1], w02 = V[2];
    const float w10 = V[4], w11 = V[5], w12 = V[6];
    const float w20 = V[8], w21 = V[9], w22 = V[10];
    const float t00 = w00 * j00 + w02 * j02;
    const float t10 = w10 * j00 + w12 * j02;
    const float t20 = w20 * j00 + w22 * j02;
    const float t01 = w01 * j11 + w02 * j12;
    const float t11 = w11 * j11 + w12 * j12;
    const float t21 = w21 * j11 + w22 * j12;

    float ss0 = 0.0f, ss1 = 0.0f, ss2 = 0.0f, rr = 0.0f, xq = 0.0f, yq = 0.0f, zq = 0.0f;
    float r00 = 0.0f, r01 = 0.0f, r02 = 0.0f, r10 = 0.0f, r11 = 0.0f, r12 = 0.0f, r20 = 0.0f, r21 = 0.0f,
          r22 = 0.0f;
    float mm00 = 0.0f, mm01 = 0.0f, mm02 = 0.0f, mm10 = 0.0f, mm11 = 0.0f, mm12 = 0.0f, mm20 = 0.0f, mm21 = 0.0f,
          mm22 = 0.0f;
    float v00, v01, v02, v11, v12, v22;
    if (precomp) {
      v00 = cv_in[0]; v01 = cv_in[1]; v02 = cv_in[2]; v11 = cv_in[3]; v12 = cv_in[4]; v22 = cv_in[5];
    } else {
      ss0 = cv_in[0] * p.scale_modifier;
      ss1 = cv_in[1] * p.scale_modifier;
      ss2 = cv_in[2] * p.scale_modifier;
      rr = q_in.x; xq = q_in.y; yq = q_in.z; zq = q_in.w;
      r00 = 1.0f - 2.0f * (yq * yq + zq * zq);
      r01 = 2.0f * (xq * yq + rr * zq);
      r02 = 2.0f * (xq * zq - rr * yq);
      r10 = 2.0f * (xq * yq - rr * zq);
      r11 = 1.0f - 2.0f * (xq * xq + zq * zq);
      r12 = 2.0f * (yq * zq + rr * xq);
      r20 = 2.0f * (xq * zq + rr * yq);
      r21 = 2.0f * (yq * zq - rr * xq);
      r22 = 1.0f - 2.0f * (xq * xq + yq * yq);
      mm00 = ss0 * r00; mm01 = ss0 * r01; mm02 = ss0 * r02;
      mm10 = ss1 * r10; mm11 = ss1 * r11; mm12 = ss1 * r12;
      mm20 = ss2 * r20; mm21 = ss2 * r21; mm22 = ss2 * r22;
      // cov3D = M^T M, the forward's expression (preprocess_kernels.py:177-182).
      v00 = mm00 * mm00 + mm10 * mm10 + mm20 * mm20;
      v01 = mm00 * mm01 + mm10 * mm11 + mm20 * mm21;
      v02 = mm00 * mm02 + mm10 * mm12 + mm20 * mm22;
      v11 = mm01 * mm01 + mm11 * mm11 + mm21 * mm21;
      v12 = mm01 * mm02 + mm11 * mm12 + mm21 * mm22;
      v22 = mm02 * mm02 + mm12 * mm12 + mm22 * mm22;
    }

    const float vt0x = v00 * t00 + v01 * t10 + v02 * t20;
    const float vt0y = v01 * t00 + v11 * t10 + v12 * t20;
    const float vt0z = v02 * t00 + v12 * t10 + v22 * t20;
    const float vt1x = v00 * t01 + v01 * t11 + v02 * t21;
    const float vt1y = v01 * t01 + v11 * t11 + v12 * t21;
    const float vt1z = v02 * t01 + v12 * t11 + v22 * t21;
    const float aa = t00 * vt0x + t10 * vt0y + t20 * vt0z + 0.3f + p.filter_variance;
    const float bb = t00 * vt1x + t10 * vt1y + t20 * vt1z;
    const float cc = t01 * vt1x + t11 * vt1y + t21 * vt1z + 0.3f + p.filter_variance;
    const float denom = aa * cc - bb * bb;
    const float denom2inv = 1.0f / (denom * denom + 1.0e-7f);

    float uc0 = uc_in0;
    float uc1 = uc_in1;
    float uc2 = uc_in2;
    if (p.flow_double) {
      uc0 = uc0 + rc0;
      uc1 = uc1 + rc1;
      uc2 = uc2 + rc2;
    }
    const float tc0 = rc0 + uc0;
    const float tc1 = rc1 + uc1;
    const float tc2 = rc2 + uc2;
    float dL_da = denom2inv * (-cc * cc * tc0 + 2.0f * bb * cc * tc1 - bb * bb * tc2);
    float dL_dc = denom2inv * (-aa * aa * tc2 + 2.0f * aa * bb * tc1 - bb * bb * tc0);
    float dL_db = denom2inv * 2.0f * (bb * cc * tc0 - (aa * cc + bb * bb) * tc1 + aa * bb * tc2);
    if (p.grad_conic_2d_inv) {
      dL_da = dL_da + ci_in0;
      dL_db = dL_db + ci_in1;
      dL_dc = dL_dc + ci_in2;
    }

    const float gc0 = t00 * t00 * dL_da + t00 * t01 * dL_db + t01 * t01 * dL_dc;
    const float gc3 = t10 * t10 * dL_da + t10 * t11 * dL_db + t11 * t11 * dL_dc;
    const float gc5 = t20 * t20 * dL_da + t20 * t21 * dL_db + t21 * t21 * dL_dc;
    const float gc1 = 2.0f * t00 * t10 * dL_da + (t00 * t11 + t01 * t10) * dL_db + 2.0f * t01 * t11 * dL_dc;
    const float gc2 = 2.0f * t00 * t20 * dL_da + (t00 * t21 + t01 * t20) * dL_db + 2.0f * t01 * t21 * dL_dc;
    const float gc4 = 2.0f * t10 * t20 * dL_da + (t10 * t21 + t11 * t20) * dL_db + 2.0f * t11 * t21 * dL_dc;

    const float dL_dT00 = 2.0f * vt0x * dL_da + vt1x * dL_db;
    const float dL_dT01 = 2.0f * vt0y * dL_da + vt1y * dL_db;
    const float dL_dT02 = 2.0f * vt0z * dL_da + vt1z * dL_db;
    const float dL_dT10 = vt0x * dL_db + 2.0f * vt1x * dL_dc;
    const float dL_dT11 = vt0y * dL_db + 2.0f * vt1y * dL_dc;
    const float dL_dT12 = vt0z * dL_db + 2.0f * vt1z * dL_dc;
    const float dL_dJ00 = w00 * dL_dT00 + w10 * dL_dT01 + w20 * dL_dT02;
    const float dL_dJ02 = w02 * dL_dT00 + w12 * dL_dT01 + w22 * dL_dT02;
    const float dL_dJ11 = w01 * dL_dT10 + w11 * dL_dT11 + w21 * dL_dT12;
    const float dL_dJ12 = w02 * dL_dT10 + w12 * dL_dT11 + w22 * dL_dT12;
    const float dL_dtx = x_grad_mul * -j00 * tz_inv * dL_dJ02;
    const float dL_dty = y_grad_mul * -j11 * tz_inv * dL_dJ12;
    const float dL_dtz = -(j00 * dL_dJ00 + j11 * dL_dJ11 + 2.0f * j02 * dL_dJ02 + 2.0f * j12 * dL_dJ12) * tz_inv;
    gcm_x = w00 * dL_dtx + w01 * dL_dty + w02 * dL_dtz;
    gcm_y = w10 * dL_dtx + w11 * dL_dty + w12 * dL_dtz;
    gcm_z = w20 * dL_dtx + w21 * dL_dty + w22 * dL_dtz;

    if (precomp) {
      // dL/dcov3D is the output (backward_ops.py:734-737); no scale / rotation chain.
      float* gcv = p.grad_cov3d + 6 * (size_t)tid;
      if (valid) {
        gcv[0] = gc0; gcv[1] = gc1; gcv[2] = gc2; gcv[3] = gc3; gcv[4] = gc4; gcv[5] = gc5;
      }
    } else {
      const float sg00 = gc0, sg01 = 0.5f * gc1, sg02 = 0.5f * gc2;
      const float sg11 = gc3, sg12 = 0.5f * gc4, sg22 = gc5;
      const float dM00 = 2.0f * (mm00 * sg00 + mm01 * sg01 + mm02 * sg02);
      const float dM01 = 2.0f * (mm00 * sg01 + mm01 * sg11 + mm02 * sg12);
      const float dM02 = 2.0f * (mm00 * sg02 + mm01 * sg12 + mm02 * sg22);
      const float dM10 = 2.0f * (mm10 * sg00 + mm11 * sg01 + mm12 * sg02);
      const float dM11 = 2.0f * (mm10 * sg01 + mm11 * sg11 + mm12 * sg12);
      const float dM12 = 2.0f * (mm10 * sg02 + mm11 * sg12 + mm12 * sg22);
      const float dM20 = 2.0f * (mm20 * sg00 + mm21 * sg01 + mm22 * sg02);
      const float dM21 = 2.0f * (mm20 * sg01 + mm21 * sg11 + mm22 * sg12);
      const float dM22 = 2.0f * (mm20 * sg02 + mm21 * sg12 + mm22 * sg22);
      gs0 = p.scale_modifier * (dM00 * r00 + dM01 * r01 + dM02 * r02);
      gs1 = p.scale_modifier * (dM10 * r10 + dM11 * r11 + dM12 * r12);
      gs2 = p.scale_modifier * (dM20 * r20 + dM21 * r21 + dM22 * r22);
      const float dR00 = dM00 * ss0, dR01 = dM01 * ss0, dR02 = dM02 * ss0;
      const float dR10 = dM10 * ss1, dR11 = dM11 * ss1, dR12 = dM12 * ss1;
      const float dR20 = dM20 * ss2, dR21 = dM21 * ss2, dR22 = dM22 * ss2;
      gq0 = 2.0f * zq * (dR01 - dR10) + 2.0f * yq * (dR20 - dR02) + 2.0f * xq * (dR12 - dR21);
      gq1 = 2.0f * yq * (dR10 + dR01) + 2.0f * zq * (dR20 + dR02) + 2.0f * rr * (dR12 - dR21) -
            4.0f * xq * (dR22 + dR11);
      gq2 = 2.0f * xq * (dR10 + dR01) + 2.0f * rr * (dR20 - dR02) + 2.0f * zq * (dR12 + dR21) -
            4.0f * yq * (dR22 + dR00);
      gq3 = 2.0f * rr * (dR01 - dR10) + 2.0f * xq * (dR20 + dR02) + 2.0f * yq * (dR12 + dR21) -
            4.0f * zq * (dR11 + dR00);
    }
  } else if (p.grad_cov3d != nullptr) {
    float* gcv = p.grad_cov3d + 6 * (size_t)tid;
    if (valid)
      for (int k = 0; k < 6; ++k) gcv[k] = 0.0f;
  }

  // SH colour backward (its colour gradient is identically zero for culled
  // Gaussians, so their coefficient gradients are plain zeros).
  float gsh_x = 0.0f, gsh_y = 0.0f, gsh_z = 0.0f;
  if (p.shs != nullptr) {
    float* gsh = p.grad_sh + (size_t)tid * (size_t)(3 * p.K);
    const uint8_t cl = rad > 0 && p.clamped != nullptr ? p.clamped[tid] : 0;
    const float g0 = rcol0 * (1.0f - (float)(cl & 1));
    const float g1 = rcol1 * (1.0f - (float)((cl >> 1) & 1));
    const float g2 = rcol2 * (1.0f - (float)((cl >> 2) & 1));
    const float dirx = mx - p.campos[0], diry = my - p.campos[1], dirz = mz - p.campos[2];
    if (p.sh_vec16) {  // uniform: the whole wave stages its blocks
      const V3 gm = sh_backward_row(stage.rows + stage.lane * kShRow, p.degree, valid && rad > 0, dirx, diry,
                                    dirz, g0, g1, g2);
      if (rad > 0) {
        gsh_x = gm.x;
        gsh_y = gm.y;
        gsh_z = gm.z;
      }
    } else if (valid && rad > 0) {
      const float* sh = p.shs + (size_t)tid * (size_t)(3 * p.K);
      const V3 gm = sh_backward<false>(sh, gsh, p.K, p.degree, dirx, diry, dirz, g0, g1, g2);
      gsh_x = gm.x;
      gsh_y = gm.y;
      gsh_z = gm.z;
    } else if (valid) {
      for (int k = 0; k < 3 * p.K; ++k) gsh[k] = 0.0f;
    }
  }
  if (!valid) return;

  // Part C: accumulate.
  p.grad_means3d[3 * tid + 0] = pm_x + gcm_x + gsh_x;
  p.grad_means3d[3 * tid + 1] = pm_y + gcm_y + gsh_y;
  p.grad_means3d[3 * tid + 2] = pm_z + gcm_z + gsh_z;
  p.grad_means2d[3 * tid + 0] = rpx;
  p.grad_means2d[3 * tid + 1] = rpy;
  p.grad_means2d[3 * tid + 2] = 0.0f;
  if (p.cov3d == nullptr) {
    p.grad_scales[3 * tid + 0] = gs0;
    p.grad_scales[3 * tid + 1] = gs1;
    p.grad_scales[3 * tid + 2] = gs2;
    reinterpret_cast<float4*>(p.grad_rotations)[tid] = make_float4(gq0, gq1, gq2, gq3);
  }
  if (p.grad_opacity != nullptr) p.grad_opacity[tid] = ropa;
  if (p.grad_colors != nullptr) {
    p.grad_colors[3 * tid + 0] = rcol0;
    p.grad_colors[3 * tid + 1] = rcol1;
    p.grad_colors[3 * tid + 2] = rcol2;
  }
}

__global__ __launch_bounds__(256) void preprocess_bwd_kernel(PreprocessBwdParams p) {
  __shared__ float4 s_sh[256 / 64][64 * kShRow];
  if (p.P <= 0) return;
  const int tid = blockIdx.x * blockDim.x + threadIdx.x;
  ShStage stage;
  stage.lane = threadIdx.x & 63;
  stage.rows = s_sh[threadIdx.x >> 6];
  stage.w0 = tid - stage.lane;
  stage.nvalid = p.P - stage.w0 < 64 ? p.P - stage.w0 : 64;
  const bool staged = p.shs != nullptr && p.sh_vec16 != 0;  // uniform
  if (staged) sh_stage_in(stage, p.shs);
  preprocess_bwd_one(p, tid < p.P ? tid : p.P - 1, tid < p.P, stage);
  if (staged) sh_stage_out(stage, p.grad_sh);
}

}  // namespace gs

extern "C" int gs_render_bwd(int32_t image_width, int32_t image_height, int32_t num_points,
                             int64_t num_rendered, const int32_t* ranges,
                             const int32_t* point_list, const float* records, const float* background,
                             const float* out_alpha, const int32_t* n_contrib, const float* grad_color,
                             const float* grad_depth, const float* grad_alpha, int32_t compute_depth,
                             float* grad_gauss, const int32_t* tile_order, void* stream) {
  if (image_width <= 0 || image_height <= 0 || (long long)image_width * image_height > 0x7fffffffLL)
    return GS_ERR_INVALID_ARGUMENT;
  if (num_points <= 0 || num_rendered < 0) return GS_ERR_INVALID_ARGUMENT;
  if (num_rendered > 0x7fffffffLL) return GS_ERR_OVERFLOW;
  if (!ranges || !point_list || !records || !background || !out_alpha || !n_contrib || !grad_gauss)
    return GS_ERR_INVALID_ARGUMENT;
  if (reinterpret_cast<uintptr_t>(records) & 15) return GS_ERR_MISALIGNED;
  gs::RenderBwdParams p;
  p.W = image_width;
  p.H = image_height;
  p.grid_x = (image_width + gs::kBlockX - 1) / gs::kBlockX;
  p.num_tiles = p.grid_x * ((image_height + gs::kBlockY - 1) / gs::kBlockY);
  p.num_points = num_points;
  p.num_rendered = (int)num_rendered;
  p.ranges = reinterpret_cast<const int2*>(ranges);
  p.point_list = point_list;
  p.records = reinterpret_cast<const float4*>(records);
  p.bg = background;
  p.out_alpha = out_alpha;
  p.n_contrib = n_contrib;
  p.grad_color = grad_color;
  p.grad_depth = grad_depth;
  p.grad_alpha = grad_alpha;
  p.compute_depth = compute_depth;
  p.grad_gauss = grad_gauss;
  // four times the mean list length: only tiles that dominate the walk
  const int64_t long_tile = gs::kLongTileFactor * num_rendered / p.num_tiles;
  p.long_tile = long_tile > 0x7fffffffLL ? 0x7fffffff : (int)long_tile;
  const bool whole = num_rendered > gs::kWholeTilePairsPerPoint * (int64_t)num_points;
  const int first = whole ? 1 : 2;
  const hipStream_t s = (hipStream_t)stream;
  // Longest lists first, in the order the forward wrote (tile_order_pays).
  p.tile_order = tile_order && gs::tile_order_pays(num_rendered, num_points, p.num_tiles) ? tile_order : nullptr;
  const dim3 grid(gs::xcd_grid(first * p.num_tiles) + gs::xcd_grid((4 - first) * p.num_tiles));
  if (compute_depth) {
    if (whole)
      hipLaunchKernelGGL((gs::render_bwd_whole_kernel<true>), grid, dim3(64), 0, s, p);
    else
      hipLaunchKernelGGL((gs::render_bwd_kernel<true>), grid, dim3(64), 0, s, p);
  } else {
    if (whole)
      hipLaunchKernelGGL((gs::render_bwd_whole_kernel<false>), grid, dim3(64), 0, s, p);
    else
      hipLaunchKernelGGL((gs::render_bwd_kernel<false>), grid, dim3(64), 0, s, p);
  }
  return gs_status_from_hip(hipGetLastError());
}

extern "C" int gs_preprocess_bwd(int32_t P, int32_t sh_coeffs, int32_t degree, const float* means3d,
                                 const float* scales, const float* rotations, const float* cov3d_precomp,
                                 float scale_modifier,
                                 const float* shs, const float* campos, const float* viewmatrix,
                                 const float* projmatrix, float tanfovx, float tanfovy, float focal_x,
                                 float focal_y, const int32_t* radii, const uint8_t* clamped,
                                 const float* grad_gauss, const float* records, int32_t image_width,
                                 int32_t image_height, const float* grad_proj_2d, const float* grad_conic_2d,
                                 const float* grad_conic_2d_inv, int32_t flow_double, float filter_variance,
                                 float* grad_means3d, float* grad_means2d, float* grad_scales,
                                 float* grad_rotations,
                                 float* grad_cov3d, float* grad_sh, float* grad_opacity, float* grad_colors,
                                 void* stream) {
  if (P < 0) return GS_ERR_INVALID_ARGUMENT;
  if (!(filter_variance >= 0.0f) || !__builtin_isfinite(filter_variance)) return GS_ERR_INVALID_ARGUMENT;
  if (P == 0) return GS_OK;
  if (!means3d || !viewmatrix || !projmatrix || !radii || !grad_gauss || !records || !grad_means3d ||
      !grad_means2d)
    return GS_ERR_INVALID_ARGUMENT;
  if (image_width <= 0 || image_height <= 0) return GS_ERR_INVALID_ARGUMENT;
  if (reinterpret_cast<uintptr_t>(records) & 15) return GS_ERR_MISALIGNED;
  if (cov3d_precomp == nullptr && (!scales || !rotations || !grad_scales || !grad_rotations))
    return GS_ERR_INVALID_ARGUMENT;
  if (cov3d_precomp != nullptr && !grad_cov3d) return GS_ERR_INVALID_ARGUMENT;
  if (shs != nullptr && (grad_sh == nullptr || campos == nullptr || sh_coeffs <= 0)) return GS_ERR_INVALID_ARGUMENT;
  if (cov3d_precomp == nullptr &&
      ((reinterpret_cast<uintptr_t>(rotations) & 15) || (reinterpret_cast<uintptr_t>(grad_rotations) & 15)))
    return GS_ERR_MISALIGNED;
  gs::PreprocessBwdParams p;
  p.P = P;
  p.K = sh_coeffs;
  p.degree = degree;
  p.means3d = means3d;
  p.scales = scales;
  p.rotations = rotations;
  p.cov3d = cov3d_precomp;
  p.scale_modifier = scale_modifier;
  p.shs = shs;
  p.campos = campos;
  p.view = viewmatrix;
  p.proj = projmatrix;
  p.tanfovx = tanfovx;
  p.tanfovy = tanfovy;
  p.focal_x = focal_x;
  p.focal_y = focal_y;
  p.radii = radii;
  p.clamped = clamped;
  p.grad_gauss = grad_gauss;
  p.records = reinterpret_cast<const float4*>(records);
  p.half_w = 0.5f * (float)image_width;
  p.half_h = 0.5f * (float)image_height;
  p.grad_proj_2d = grad_proj_2d;
  p.grad_conic_2d = grad_conic_2d;
  p.grad_conic_2d_inv = grad_conic_2d_inv;
  p.flow_double = flow_double;
  p.filter_variance = filter_variance;
  p.grad_means3d = grad_means3d;
  p.grad_means2d = grad_means2d;
  p.grad_scales = grad_scales;
  p.grad_rotations = grad_rotations;
  p.grad_cov3d = grad_cov3d;
  p.grad_sh = grad_sh;
  p.grad_opacity = grad_opacity;
  p.grad_colors = grad_colors;
  const uintptr_t sh_addr_bits = reinterpret_cast<uintptr_t>(shs) | reinterpret_cast<uintptr_t>(grad_sh);
  p.sh_vec16 = (shs != nullptr && sh_coeffs == 16 && (sh_addr_bits & 15) == 0) ? 1 : 0;
  hipLaunchKernelGGL(gs::preprocess_bwd_kernel, dim3((P + 255) / 256), dim3(256), 0, (hipStream_t)stream, p);
  return gs_status_from_hip(hipGetLastError());
}
