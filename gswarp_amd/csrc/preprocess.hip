// Preprocess stage: one thread per Gaussian, fused
//   projection + near-plane cull          preprocess_kernels.py:131-146
//   cov3D = M^T M, M = diag(s) R(q)        preprocess_kernels.py:148-182
//   EWA cov2D = (M T)^T (M T) + 0.3 I      preprocess_kernels.py:184-219
//   or, for precomputed cov3D V, cov2D = T^T (V T) + 0.3 I with |det| < 1e-7
//   culled                                 preprocess_kernels.py:345-477
//   conic, radius, tile-rect cull          preprocess_kernels.py:221-244
//   outputs + tile coverage count          preprocess_kernels.py:246-269
//   SH degree 0..3 colour, +0.5, clamp     preprocess_kernels.py:272-342
//   optional Mip-Splatting filter: cov2D + f I, its conic, radius and tile
//   count for Gaussians the base cull keeps     backend_mip_3dgs.py:63-102
// The colour is written into a packed 48-byte render record together with
// the screen position, conic, opacity and depth, so the render kernels fetch
// one Gaussian with three 16-byte loads.  SH colour is evaluated for visible
// Gaussians only: for culled ones it is never read (no tile references them
// and their colour gradient is identically zero).
#include "gs_common.h"
#include "gs_capi.h"

namespace gs {

struct PreprocessParams {
  int P;
  int sh_coeffs;
  int sh_vec16;  // sh_coeffs == 16 and shs 16-byte aligned: float4 SH loads
  int degree;
  const float* means3d;
  const float* scales;
  const float* rotations;
  const float* cov3d;  // precomputed (N, 6) 3D covariances, or null
  float scale_modifier;
  const float* opacities;
  const float* shs;
  const float* colors;
  const float* view;
  const float* proj;
  const float* campos;
  float tanfovx, tanfovy, focal_x, focal_y;
  int W, H, grid_x, grid_y, coverage_mode;
  float filter_variance;  // Mip-Splatting screen-space variance; 0 = none
  int* radii;
  float* depths;
  float* proj_2d;
  float* conic_2d;
  float* conic_2d_inv;
  int* tiles_touched;
  int4* coverage;  // per-Gaussian packed cover masks (pack_cover), or null
  float4* records;
  uint8_t* clamped;
  unsigned* band_store;  // kBandSlots words per wave for the banded Gaussians' bands, or null
  // the binning's one-pass scan state: this kernel writes its per-256-Gaussian
  // aggregates and clears its status words (or null)
  unsigned long long* scan_agg;
  unsigned long long* scan_status;
  int scan_status_words;
};

// SH colour of one Gaussian; sh_mem points at its coefficient block (K x 3).
// With kVec16 the block is K = 16 coefficients, 16-byte aligned, read as 12
// float4 (4x fewer memory instructions than per-float loads, whose lanes
// each touch a different cache line); the arithmetic is the same.
template <bool kVec16>
__device__ __forceinline__ float3 sh_color(const float* __restrict__ sh_mem, int K, int degree, float x, float y,
                                           float z) {
  float sh_reg[kVec16 ? 48 : 1];
  if (kVec16) {
#pragma unroll
    for (int i = 0; i < 12; ++i) {
      const float4 v = reinterpret_cast<const float4*>(sh_mem)[i];
      sh_reg[4 * i + 0] = v.x;
      sh_reg[4 * i + 1] = v.y;
      sh_reg[4 * i + 2] = v.z;
      sh_reg[4 * i + 3] = v.w;
    }
  }
  const float* sh = kVec16 ? sh_reg : sh_mem;
  float3 c;
  c.x = kShC0 * sh[0];
  c.y = kShC0 * sh[1];
  c.z = kShC0 * sh[2];
  if (degree > 0 && K > 3) {
    const float b0 = -kShC1 * y, b1 = kShC1 * z, b2 = -kShC1 * x;
    c.x = c.x + b0 * sh[3];  c.y = c.y + b0 * sh[4];  c.z = c.z + b0 * sh[5];
    c.x = c.x + b1 * sh[6];  c.y = c.y + b1 * sh[7];  c.z = c.z + b1 * sh[8];
    c.x = c.x + b2 * sh[9];  c.y = c.y + b2 * sh[10]; c.z = c.z + b2 * sh[11];
    if (degree > 1 && K > 8) {
      const float xx = x * x, yy = y * y, zz = z * z;
      const float xy = x * y, yz = y * z, xz = x * z;
      const float w4 = kShC2_0 * xy;
      const float w5 = kShC2_1 * yz;
      const float w6 = kShC2_2 * (2.0f * zz - xx - yy);
      const float w7 = kShC2_3 * xz;
      const float w8 = kShC2_4 * (xx - yy);
      c.x = c.x + w4 * sh[12]; c.y = c.y + w4 * sh[13]; c.z = c.z + w4 * sh[14];
      c.x = c.x + w5 * sh[15]; c.y = c.y + w5 * sh[16]; c.z = c.z + w5 * sh[17];
      c.x = c.x + w6 * sh[18]; c.y = c.y + w6 * sh[19]; c.z = c.z + w6 * sh[20];
      c.x = c.x + w7 * sh[21]; c.y = c.y + w7 * sh[22]; c.z = c.z + w7 * sh[23];
      c.x = c.x + w8 * sh[24]; c.y = c.y + w8 * sh[25]; c.z = c.z + w8 * sh[26];
      if (degree > 2 && K > 15) {
        const float w9 = kShC3_0 * y * (3.0f * xx - yy);
        const float w10 = kShC3_1 * xy * z;
        const float w11 = kShC3_2 * y * (4.0f * zz - xx - yy);
        const float w12 = kShC3_3 * z * (2.0f * zz - 3.0f * xx - 3.0f * yy);
        const float w13 = kShC3_4 * x * (4.0f * zz - xx - yy);
        const float w14 = kShC3_5 * z * (xx - yy);
        const float w15 = kShC3_6 * x * (xx - 3.0f * yy);
        c.x = c.x + w9 * sh[27];  c.y = c.y + w9 * sh[28];  c.z = c.z + w9 * sh[29];
        c.x = c.x + w10 * sh[30]; c.y = c.y + w10 * sh[31]; c.z = c.z + w10 * sh[32];
        c.x = c.x + w11 * sh[33]; c.y = c.y + w11 * sh[34]; c.z = c.z + w11 * sh[35];
        c.x = c.x + w12 * sh[36]; c.y = c.y + w12 * sh[37]; c.z = c.z + w12 * sh[38];
        c.x = c.x + w13 * sh[39]; c.y = c.y + w13 * sh[40]; c.z = c.z + w13 * sh[41];
        c.x = c.x + w14 * sh[42]; c.y = c.y + w14 * sh[43]; c.z = c.z + w14 * sh[44];
        c.x = c.x + w15 * sh[45]; c.y = c.y + w15 * sh[46]; c.z = c.z + w15 * sh[47];
      }
    }
  }
  return c;
}

// Every lane of the grid stays to the end (lanes past P as culled
// Gaussians): the tile count is a wave-wide walk.
__global__ __launch_bounds__(256) void preprocess_fwd_kernel(PreprocessParams p) {
  static_assert(kScanAggGaussians == 256, "one workgroup's Gaussians per scan aggregate");
  __shared__ CoverCountLds s_cover[256 / 64];
  __shared__ ScanAggLds s_agg;
  __shared__ float4 s_rec[256 / 64][3 * 64];  // each wave's records, written out whole-wave
  const int idx0 = blockIdx.x * blockDim.x + threadIdx.x;
  const bool in_range = idx0 < p.P;
  bool rec_written = false;
  const int idx = in_range ? idx0 : p.P - 1;  // loads stay in bounds; nothing is stored for it
  // the next stage's one-pass scan starts from cleared status words (fewer
  // than this grid's threads)
  if (p.scan_status != nullptr && idx0 < p.scan_status_words) p.scan_status[idx0] = 0ull;
  const float* __restrict__ V = p.view;
  const float* __restrict__ Pm = p.proj;
  const float mx = p.means3d[3 * idx + 0];
  const float my = p.means3d[3 * idx + 1];
  const float mz = p.means3d[3 * idx + 2];

  int radius = 0;
  float depth = 0.0f, pxo = 0.0f, pyo = 0.0f;
  float con0 = 0.0f, con1 = 0.0f, con2 = 0.0f;
  float cov_a = 0.0f, cov_b = 0.0f, cov_c = 0.0f;
  int touched = 0;
  // inputs of the tile count, set for visible Gaussians
  bool count_it = false;
  float c_px = 0.0f, c_py = 0.0f, c_aa = 0.0f, c_cc = 0.0f, c_q0 = 0.0f, c_q1 = 0.0f, c_q2 = 0.0f, c_op = 0.0f;
  int c_rad = 0;

  const float p_view_z = V[2] * mx + V[6] * my + V[10] * mz + V[14];
  bool visible = in_range && p_view_z > kNearPlane;
  if (visible) {
    const float hom_x = Pm[0] * mx + Pm[4] * my + Pm[8] * mz + Pm[12];
    const float hom_y = Pm[1] * mx + Pm[5] * my + Pm[9] * mz + Pm[13];
    const float hom_w = Pm[3] * mx + Pm[7] * my + Pm[11] * mz + Pm[15];
    const float inv_w = 1.0f / (hom_w + 0.0000001f);
    const float p_proj_x = hom_x * inv_w;
    const float p_proj_y = hom_y * inv_w;

    float vx = V[0] * mx + V[4] * my + V[8] * mz + V[12];
    float vy = V[1] * mx + V[5] * my + V[9] * mz + V[13];
    const float vz = p_view_z;
    const float limx = kFovClamp * p.tanfovx;
    const float limy = kFovClamp * p.tanfovy;
    const float txtz = vx / vz;
    const float tytz = vy / vz;
    vx = clampr(txtz, -limx, limx) * vz;
    vy = clampr(tytz, -limy, limy) * vz;
    const float a_j = p.focal_x / vz;
    const float b_j = p.focal_y / vz;
    const float c_j = -(p.focal_x * vx) / (vz * vz);
    const float d_j = -(p.focal_y * vy) / (vz * vz);
    const float t00 = V[0] * a_j + V[2] * c_j;
    const float t10 = V[4] * a_j + V[6] * c_j;
    const float t20 = V[8] * a_j + V[10] * c_j;
    const float t01 = V[1] * b_j + V[2] * d_j;
    const float t11 = V[5] * b_j + V[6] * d_j;
    const float t21 = V[9] * b_j + V[10] * d_j;
    float ca, cb, cc;
    if (p.cov3d == nullptr) {
      // M = diag(s) R(q) with the reference's (transposed) rotation layout.
      const float s0 = p.scales[3 * idx + 0] * p.scale_modifier;
      const float s1 = p.scales[3 * idx + 1] * p.scale_modifier;
      const float s2 = p.scales[3 * idx + 2] * p.scale_modifier;
      const float4 q = reinterpret_cast<const float4*>(p.rotations)[idx];
      const float rr = q.x, xq = q.y, yq = q.z, zq = q.w;
      const float r00 = 1.0f - 2.0f * (yq * yq + zq * zq);
      const float r01 = 2.0f * (xq * yq + rr * zq);
      const float r02 = 2.0f * (xq * zq - rr * yq);
      const float r10 = 2.0f * (xq * yq - rr * zq);
      const float r11 = 1.0f - 2.0f * (xq * xq + zq * zq);
      const float r12 = 2.0f * (yq * zq + rr * xq);
      const float r20 = 2.0f * (xq * zq + rr * yq);
      const float r21 = 2.0f * (yq * zq - rr * xq);
      const float r22 = 1.0f - 2.0f * (xq * xq + yq * yq);
      const float m00 = s0 * r00, m01 = s0 * r01, m02 = s0 * r02;
      const float m10 = s1 * r10, m11 = s1 * r11, m12 = s1 * r12;
      const float m20 = s2 * r20, m21 = s2 * r21, m22 = s2 * r22;
      const float a00 = m00 * t00 + m01 * t10 + m02 * t20;
      const float a10 = m10 * t00 + m11 * t10 + m12 * t20;
      const float a20 = m20 * t00 + m21 * t10 + m22 * t20;
      const float a01 = m00 * t01 + m01 * t11 + m02 * t21;
      const float a11 = m10 * t01 + m11 * t11 + m12 * t21;
      const float a21 = m20 * t01 + m21 * t11 + m22 * t21;
      ca = a00 * a00 + a10 * a10 + a20 * a20 + 0.3f;
      cb = a00 * a01 + a10 * a11 + a20 * a21;
      cc = a01 * a01 + a11 * a11 + a21 * a21 + 0.3f;
    } else {
      const float* cv = p.cov3d + 6 * (size_t)idx;
      const float v00 = cv[0], v01 = cv[1], v02 = cv[2], v11 = cv[3], v12 = cv[4], v22 = cv[5];
      const float vt0x = v00 * t00 + v01 * t10 + v02 * t20;
      const float vt0y = v01 * t00 + v11 * t10 + v12 * t20;
      const float vt0z = v02 * t00 + v12 * t10 + v22 * t20;
      const float vt1x = v00 * t01 + v01 * t11 + v02 * t21;
      const float vt1y = v01 * t01 + v11 * t11 + v12 * t21;
      const float vt1z = v02 * t01 + v12 * t11 + v22 * t21;
      ca = t00 * vt0x + t10 * vt0y + t20 * vt0z + 0.3f;
      cb = t00 * vt1x + t10 * vt1y + t20 * vt1z;
      cc = t01 * vt1x + t11 * vt1y + t21 * vt1z + 0.3f;
    }
    const float det = ca * cc - cb * cb;
    // the fused kernel culls |det| <= 1e-7, the precomputed-covariance kernel |det| < 1e-7
    visible = p.cov3d == nullptr ? fabsf(det) > kDetEps : !(fabsf(det) < kDetEps);
    if (visible) {
      const float det_inv = 1.0f / det;
      const float k0 = cc * det_inv, k1 = -cb * det_inv, k2 = ca * det_inv;
      const float mid = 0.5f * (ca + cc);
      const float root = sqrtf(fmaxr(0.1f, mid * mid - det));
      const float lambda1 = mid + root;
      const float lambda2 = mid - root;
      const int rad = f2i(ceilf(3.0f * sqrtf(fmaxr(lambda1, lambda2))));
      const float ptx = ndc_to_pix(p_proj_x, p.W);
      const float pty = ndc_to_pix(p_proj_y, p.H);
      const int4 rect = tile_rect(ptx, pty, rad, rad, p.grid_x, p.grid_y);
      visible = (rect.z - rect.x) * (rect.w - rect.y) != 0;
      float fa = ca, fc = cc, q0 = k0, q1 = k1, q2 = k2;
      int frad = rad;
      if (visible && p.filter_variance != 0.0f) {
        // Mip filter on a kept Gaussian: culled unless the filtered
        // determinant exceeds 1e-12; depth and position stay.
        fa = ca + p.filter_variance;
        fc = cc + p.filter_variance;
        const float fdet = fa * fc - cb * cb;
        depth = p_view_z;
        pxo = ptx;
        pyo = pty;
        visible = fdet > 1.0e-12f;
        const float inv = 1.0f / fdet;
        q0 = fc * inv; q1 = -cb * inv; q2 = fa * inv;
        const float d = fa - fc;
        float disc = 0.25f * (d * d) + cb * cb;
        disc = disc < 0.0f ? 0.0f : disc;
        float lam = 0.5f * (fa + fc) + sqrtf(disc);
        lam = lam < 0.1f ? 0.1f : lam;
        frad = f2i(ceilf(3.0f * sqrtf(lam)));
      }
      if (visible) {
        const float op = p.opacities[idx];
        radius = frad;
        depth = p_view_z;
        pxo = ptx;
        pyo = pty;
        con0 = q0; con1 = q1; con2 = q2;
        cov_a = fa; cov_b = cb; cov_c = fc;
        count_it = true;
        c_px = ptx; c_py = pty; c_aa = fa; c_cc = fc; c_q0 = q0; c_q1 = q1; c_q2 = q2; c_op = op; c_rad = frad;

        float3 col;
        uint8_t clamp_bits = 0;
        if (p.colors != nullptr) {
          col.x = p.colors[3 * idx + 0];
          col.y = p.colors[3 * idx + 1];
          col.z = p.colors[3 * idx + 2];
        } else {
          const float dx = mx - p.campos[0];
          const float dy = my - p.campos[1];
          const float dz = mz - p.campos[2];
          const float len_sq = dx * dx + dy * dy + dz * dz;
          const float inv_len = 1.0f / sqrtf(fmaxr(len_sq, 1.0e-20f));
          const float* sh = p.shs + (size_t)idx * (size_t)(p.sh_coeffs * 3);
          col = p.sh_vec16 ? sh_color<true>(sh, p.sh_coeffs, p.degree, dx * inv_len, dy * inv_len, dz * inv_len)
                           : sh_color<false>(sh, p.sh_coeffs, p.degree, dx * inv_len, dy * inv_len, dz * inv_len);
          col.x = col.x + 0.5f;
          col.y = col.y + 0.5f;
          col.z = col.z + 0.5f;
          if (col.x < 0.0f) { col.x = 0.0f; clamp_bits |= 1; }
          if (col.y < 0.0f) { col.y = 0.0f; clamp_bits |= 2; }
          if (col.z < 0.0f) { col.z = 0.0f; clamp_bits |= 4; }
        }
        float4* rec = s_rec[threadIdx.x >> 6] + 3 * (threadIdx.x & 63);
        const float4 w0 = make_float4(ptx, pty, q0, q1);
        const float4 w1 = make_float4(q2, op, p_view_z, quad_cutoff(op));
        rec[0] = w0;
        rec[1] = w1;
        rec[2] = make_float4(col.x, col.y, col.z, __uint_as_float(record_extents(w0, w1)));
        rec_written = in_range;
        if (p.clamped != nullptr) p.clamped[idx] = clamp_bits;
      }
    }
  }
  {
    // The wave's records go out as three whole-wave stores of consecutive
    // float4 (lane l stores float4 64 q + l of the wave's 3 x 64, if its
    // Gaussian wrote a record), not as three 48-byte-strided stores per lane:
    // a third of the address-unit work.  The wave's LDS accesses complete in
    // order.
    const uint64_t written = __ballot(rec_written);
    __builtin_amdgcn_wave_barrier();
    const float4* rw = s_rec[threadIdx.x >> 6];
    float4* out = p.records + 3 * (size_t)(idx0 - (threadIdx.x & 63));
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const int f = 64 * q + (threadIdx.x & 63);
      if ((written >> (f / 3)) & 1) out[f] = rw[f];
    }
  }
  TileCover cover;
  touched = wave_count_covered_tiles(count_it, c_px, c_py, c_aa, c_cc, c_q0, c_q1, c_q2, c_op, c_rad, p.grid_x,
                                     p.grid_y, p.coverage_mode, cover, s_cover[threadIdx.x >> 6], p.band_store,
                                     (idx0 >> 6) * kBandSlots);
  if (p.scan_agg != nullptr) {
    // this workgroup's 256 Gaussians for the one-pass scan: depth range,
    // super-tile units and valid cover words
    int units = 0, valid = 0, bad = 0;
    if (p.coverage != nullptr && in_range) {
      const CoverWord w = unpack_cover(pack_cover(cover));
      units = super_units(w);
      valid = w.valid;
      bad = (touched > 0 && !w.valid) ? 1 : 0;
    }
    store_scan_aggregates(in_range && radius > 0, depth, units, valid, bad, s_agg, p.scan_agg);
  }
  if (!in_range) return;
  if (!visible && p.clamped != nullptr) p.clamped[idx] = 0;
  p.radii[idx] = radius;
  p.depths[idx] = depth;
  p.proj_2d[2 * idx + 0] = pxo;
  p.proj_2d[2 * idx + 1] = pyo;
  p.conic_2d[3 * idx + 0] = con0;
  p.conic_2d[3 * idx + 1] = con1;
  p.conic_2d[3 * idx + 2] = con2;
  p.conic_2d_inv[3 * idx + 0] = cov_a;
  p.conic_2d_inv[3 * idx + 1] = cov_b;
  p.conic_2d_inv[3 * idx + 2] = cov_c;
  p.tiles_touched[idx] = touched;
  if (p.coverage != nullptr) p.coverage[idx] = pack_cover(cover);
}

// Tile count and cover word of already projected Gaussians (the preprocess's
// count on given 2D inputs, as binning_kernels.py:56-123 recounts them):
// record (x, y, conic a, b | conic c, opacity), cov2D (a, b, c) and radius.
// Every lane of the grid stays to the end, as in the preprocess.
__global__ __launch_bounds__(256) void count_tiles_kernel(int P, const int* __restrict__ radii,
                                                          const float4* __restrict__ records,
                                                          const float* __restrict__ cov2d, int grid_x, int grid_y,
                                                          int coverage_mode, int* tiles_touched, int4* coverage) {
  __shared__ CoverCountLds s_cover[256 / 64];
  const int idx0 = blockIdx.x * blockDim.x + threadIdx.x;
  const bool in_range = idx0 < P;
  const int idx = in_range ? idx0 : P - 1;
  const int rad = radii[idx];
  const bool active = in_range && rad > 0;
  float4 r0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), r1 = r0;
  float aa = 0.0f, cc = 0.0f;
  if (active) {
    r0 = records[3 * (size_t)idx];
    r1 = records[3 * (size_t)idx + 1];
    aa = cov2d[3 * (size_t)idx];
    cc = cov2d[3 * (size_t)idx + 2];
  }
  TileCover cover;
  const int touched = wave_count_covered_tiles(active, r0.x, r0.y, aa, cc, r0.z, r0.w, r1.x, r1.y, rad, grid_x,
                                               grid_y, coverage_mode, cover, s_cover[threadIdx.x >> 6]);
  if (!in_range) return;
  tiles_touched[idx] = touched;
  if (coverage != nullptr) coverage[idx] = pack_cover(cover);
}

// markVisible: view-space z beyond the near plane (preprocess_kernels.py:604-617).
__global__ __launch_bounds__(256) void mark_visible_kernel(int P, const float* __restrict__ means3d,
                                                           const float* __restrict__ V, uint8_t* visible) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= P) return;
  const float mx = means3d[3 * idx + 0];
  const float my = means3d[3 * idx + 1];
  const float mz = means3d[3 * idx + 2];
  const float z = V[2] * mx + V[6] * my + V[10] * mz + V[14];
  visible[idx] = z > kNearPlane ? 1 : 0;
}

}  // namespace gs

extern "C" int gs_preprocess_fwd(int32_t P, int32_t sh_coeffs, int32_t degree, const float* means3d,
                                 const float* scales, const float* rotations, const float* cov3d_precomp,
                                 float scale_modifier,
                                 const float* opacities, const float* shs, const float* colors_precomp,
                                 const float* viewmatrix, const float* projmatrix, const float* campos,
                                 float tanfovx, float tanfovy, float focal_x, float focal_y,
                                 int32_t image_width, int32_t image_height, int32_t coverage_mode,
                                 float filter_variance, int32_t* radii, float* depths, float* proj_2d,
                                 float* conic_2d,
                                 float* conic_2d_inv, int32_t* tiles_touched, int32_t* coverage,
                                 float* records, uint8_t* clamped, int32_t* band_store,
                                 int64_t band_store_words, int64_t* scan_state, size_t scan_state_bytes,
                                 void* stream) {
  if (P < 0 || image_width <= 0 || image_height <= 0) return GS_ERR_INVALID_ARGUMENT;
  if (reinterpret_cast<uintptr_t>(scan_state) & 7) return GS_ERR_MISALIGNED;
  if (band_store != nullptr && (coverage == nullptr || gs_band_store_words(P) > 0x7fffffffLL)) {
    return coverage == nullptr ? GS_ERR_INVALID_ARGUMENT : GS_ERR_OVERFLOW;
  }
  if (band_store != nullptr && band_store_words < gs_band_store_words(P)) return GS_ERR_SCRATCH_TOO_SMALL;
  if (scan_state != nullptr && scan_state_bytes < gs_scan_state_bytes(P)) return GS_ERR_SCRATCH_TOO_SMALL;
  if (coverage_mode < 0 || coverage_mode > 2) return GS_ERR_INVALID_ARGUMENT;
  if (!(filter_variance >= 0.0f) || !__builtin_isfinite(filter_variance)) return GS_ERR_INVALID_ARGUMENT;
  if (P == 0) return GS_OK;
  if (!means3d || !opacities || !viewmatrix || !projmatrix || !radii || !depths || !proj_2d || !conic_2d ||
      !conic_2d_inv || !tiles_touched || !records)
    return GS_ERR_INVALID_ARGUMENT;
  if (cov3d_precomp == nullptr && (!scales || !rotations)) return GS_ERR_INVALID_ARGUMENT;
  if (colors_precomp == nullptr && (shs == nullptr || campos == nullptr || sh_coeffs <= 0))
    return GS_ERR_INVALID_ARGUMENT;
  if ((cov3d_precomp == nullptr && (reinterpret_cast<uintptr_t>(rotations) & 15)) ||
      (reinterpret_cast<uintptr_t>(records) & 15) || (reinterpret_cast<uintptr_t>(coverage) & 15))
    return GS_ERR_MISALIGNED;
  gs::PreprocessParams p;
  p.P = P;
  p.sh_coeffs = sh_coeffs;
  p.sh_vec16 = (shs != nullptr && sh_coeffs == 16 && (reinterpret_cast<uintptr_t>(shs) & 15) == 0) ? 1 : 0;
  p.degree = degree;
  p.means3d = means3d;
  p.scales = scales;
  p.rotations = rotations;
  p.cov3d = cov3d_precomp;
  p.scale_modifier = scale_modifier;
  p.opacities = opacities;
  p.shs = shs;
  p.colors = colors_precomp;
  p.view = viewmatrix;
  p.proj = projmatrix;
  p.campos = campos;
  p.tanfovx = tanfovx;
  p.tanfovy = tanfovy;
  p.focal_x = focal_x;
  p.focal_y = focal_y;
  p.W = image_width;
  p.H = image_height;
  p.grid_x = (image_width + gs::kBlockX - 1) / gs::kBlockX;
  p.grid_y = (image_height + gs::kBlockY - 1) / gs::kBlockY;
  p.coverage_mode = coverage_mode;
  p.filter_variance = filter_variance;
  p.radii = radii;
  p.depths = depths;
  p.proj_2d = proj_2d;
  p.conic_2d = conic_2d;
  p.conic_2d_inv = conic_2d_inv;
  p.tiles_touched = tiles_touched;
  p.coverage = reinterpret_cast<int4*>(coverage);
  p.records = reinterpret_cast<float4*>(records);
  p.clamped = clamped;
  p.band_store = reinterpret_cast<unsigned*>(band_store);
  p.scan_agg = reinterpret_cast<unsigned long long*>(scan_state);
  p.scan_status = p.scan_agg ? p.scan_agg + gs_scan_state_status_offset(P) : nullptr;
  p.scan_status_words = p.scan_agg ? (int)gs_scan_state_status_words(P) : 0;
  const int blocks = (P + 255) / 256;
  hipLaunchKernelGGL(gs::preprocess_fwd_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, p);
  return gs_status_from_hip(hipGetLastError());
}

extern "C" int64_t gs_band_store_words(int32_t P) {
  return P <= 0 ? 0 : (int64_t)((P + 63) / 64) * gs::kBandSlots;
}

extern "C" int gs_mark_visible(int32_t P, const float* means3d, const float* viewmatrix, uint8_t* visible,
                               void* stream) {
  if (P < 0) return GS_ERR_INVALID_ARGUMENT;
  if (P == 0) return GS_OK;
  if (!means3d || !viewmatrix || !visible) return GS_ERR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(gs::mark_visible_kernel, dim3((P + 255) / 256), dim3(256), 0, (hipStream_t)stream, P,
                     means3d, viewmatrix, visible);
  return gs_status_from_hip(hipGetLastError());
}

extern "C" int gs_count_tiles(int32_t P, const int32_t* radii, const float* records, const float* conic_2d_inv,
                              int32_t image_width, int32_t image_height, int32_t coverage_mode,
                              int32_t* tiles_touched, int32_t* coverage, void* stream) {
  if (P < 0 || image_width <= 0 || image_height <= 0) return GS_ERR_INVALID_ARGUMENT;
  if (coverage_mode < 0 || coverage_mode > 2) return GS_ERR_INVALID_ARGUMENT;
  if (P == 0) return GS_OK;
  if (!radii || !records || !conic_2d_inv || !tiles_touched) return GS_ERR_INVALID_ARGUMENT;
  if ((reinterpret_cast<uintptr_t>(records) & 15) || (reinterpret_cast<uintptr_t>(coverage) & 15))
    return GS_ERR_MISALIGNED;
  const int grid_x = (image_width + gs::kBlockX - 1) / gs::kBlockX;
  const int grid_y = (image_height + gs::kBlockY - 1) / gs::kBlockY;
  hipLaunchKernelGGL(gs::count_tiles_kernel, dim3((P + 255) / 256), dim3(256), 0, (hipStream_t)stream, P, radii,
                     reinterpret_cast<const float4*>(records), conic_2d_inv, grid_x, grid_y, coverage_mode,
                     tiles_touched, reinterpret_cast<int4*>(coverage));
  return gs_status_from_hip(hipGetLastError());
}
