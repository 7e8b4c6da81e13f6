/*
 * gs_oracle.c — CPU restatement of the fancifulland2718/gswarp 1.1.0
 * rasterizer path (Warp backend), used ONLY as test and benchmark
 * infrastructure: the parity checker in tests/, __graft_entry__.smoke() and
 * the cpu_baseline leg of bench.py.  Nothing in the product library links or
 * calls this file.
 *
 * Each function cites the reference file:line it restates (paths relative to
 * gswarp/_internal/backends/warp/).  Evaluation order of every fp32
 * expression follows the reference source left to right; the file is
 * compiled with -ffp-contract=off, so results are IEEE binary32 with one
 * rounding per operation.
 *
 * The reference's exp/log come from Warp builtins, which cannot be run here
 * (warp-lang is absent).  This oracle evaluates them with its own
 * published-method routines: exp by Cody–Waite reduction and a degree-6
 * minimax polynomial, ln by the atanh series in s = (m-1)/(m+1); both are
 * checked against libm in double precision by tests/test_oracle_pipeline.py
 * (test_exp_matches_libm, test_log_matches_libm).
 *
 * Differences from the reference that do not change results:
 *  - binning follows the reference's own dataflow: stable depth sort of all
 *    points, inclusive scan of tiles_touched in depth order, duplicate in
 *    depth order, stable tile sort (binning_ops.py:152-343);
 *  - render backward gradients are accumulated in double precision (the
 *    reference accumulates fp32 atomics in unspecified order); alongside
 *    them or_render_bwd can carry a first-order running error bound per
 *    gradient element (Wilkinson-style: each rounding contributes at most
 *    u = 2^-24 of its result's magnitude), which the tests use as the
 *    per-element tolerance for the GPU's different but equally valid fp32
 *    evaluation order.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define BLOCK_X 16
#define BLOCK_Y 16
#define NCH 3

/* constants.py:8-22 */
static const float SH_C0 = 0.28209479177387814f;
static const float SH_C1 = 0.4886025119029199f;
static const float SH_C2_0 = 1.0925484305920792f;
static const float SH_C2_1 = -1.0925484305920792f;
static const float SH_C2_2 = 0.31539156525252005f;
static const float SH_C2_3 = -1.0925484305920792f;
static const float SH_C2_4 = 0.5462742152960396f;
static const float SH_C3_0 = -0.5900435899266435f;
static const float SH_C3_1 = 2.890611442640554f;
static const float SH_C3_2 = -0.4570457994644658f;
static const float SH_C3_3 = 0.3731763325901154f;
static const float SH_C3_4 = -0.4570457994644658f;
static const float SH_C3_5 = 1.445305721320277f;
static const float SH_C3_6 = -0.5900435899266435f;
/* constants.py:35-45 */
static const float DET_EPSILON = 1.0e-7f;
static const float ONE_MINUS_ALPHA_MIN = 1.0e-5f;
static const float SNUGBOX_PIXEL_PADDING = 1.0f;
static const float COVERAGE_Q_EPSILON = 1.0e-4f;
#define TILE_COVERAGE_SNUGBOX 0
#define TILE_COVERAGE_ACCUTILE_SWEEP 1
#define TILE_COVERAGE_CONIC_RECT 2
#define TILE_COVERAGE_CONIC_MASK_MAX_TILES 64

static inline float fmin_(float a, float b) { return a < b ? a : b; }
static inline float fmax_(float a, float b) { return a > b ? a : b; }
static inline int imin_(int a, int b) { return a < b ? a : b; }
static inline int imax_(int a, int b) { return a > b ? a : b; }
static inline float clamp_(float x, float lo, float hi) { return x < lo ? lo : (x > hi ? hi : x); }

/* Truncating float->int32 with the saturating / NaN->0 semantics of the
 * GPU conversion instruction (int32(x) on the reference's device). */
static inline int f2i(float f) {
  if (!(f == f)) return 0;
  if (f >= 2147483648.0f) return 2147483647;
  if (f <= -2147483648.0f) return (-2147483647 - 1);
  return (int)f;
}

/* exp: Cody–Waite reduction x = n ln2 + r, |r| <= ln2/2, n the integer
 * nearest to x log2(e) taken from the low mantissa bits of
 * fmaf(x, log2e, 1.5*2^23), ln2 = 0.693359375 - 2.12194440e-4 (exact 9-bit
 * head); degree-6 minimax polynomial of e^r (relative error 3.6e-9 on
 * |r| <= ln2/2, coefficients from Lawson's iteration rounded to float) in
 * Horner form; exact 2^n scaling.  Every step one correctly rounded operation
 * (fmaf, exact subtraction), within 0.9 ulp of exp at every float of
 * [-87, 0]. */
float or_exp(float x) {
  if (x < -87.0f) return 0.0f;
  if (x > 88.0f) x = 88.0f;
  const float magic = 12582912.0f; /* 1.5 * 2^23 */
  const float n = fmaf(x, 1.44269504088896341f, magic) - magic;
  float r = fmaf(n, -0.693359375f, x);
  r = fmaf(n, 2.12194440e-4f, r);
  float p = fmaf(0x1.6a23dp-10f, r, 0x1.123a2p-7f);
  p = fmaf(p, r, 0x1.5558f2p-5f);
  p = fmaf(p, r, 0x1.555492p-3f);
  p = fmaf(p, r, 0x1.fffffcp-2f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)n);
}

/* ln: y = m 2^e, m in [sqrt(1/2), sqrt(2)); ln m = 2 atanh(s), s=(m-1)/(m+1). */
float or_log(float y) {
  int e;
  float m = frexpf(y, &e);
  if (m < 0.70710678118654752f) {
    m = m * 2.0f;
    e = e - 1;
  }
  const float s = (m - 1.0f) / (m + 1.0f);
  const float s2 = s * s;
  float p = 0.0909090909f;
  p = p * s2 + 0.111111111f;
  p = p * s2 + 0.142857143f;
  p = p * s2 + 0.2f;
  p = p * s2 + 0.333333333f;
  const float lnm = 2.0f * s + (2.0f * s) * (s2 * p);
  const float ef = (float)e;
  return ef * 0.693145751953125f + (lnm + ef * 1.42860677e-6f);
}

typedef struct {
  int x0, y0, x1, y1;
} rect4;

/* math_kernels.py:86-87 */
static inline float ndc_to_pix(float v, int size) { return ((v + 1.0f) * (float)size - 1.0f) * 0.5f; }

/* math_kernels.py:137-148 */
static inline rect4 compute_tile_rect(float px, float py, int rx, int ry, int grid_x, int grid_y) {
  rect4 r;
  r.x0 = imin_(grid_x, imax_(0, f2i((px - (float)rx) / (float)BLOCK_X)));
  r.y0 = imin_(grid_y, imax_(0, f2i((py - (float)ry) / (float)BLOCK_Y)));
  r.x1 = imin_(grid_x, imax_(0, f2i((px + (float)rx + (float)(BLOCK_X - 1)) / (float)BLOCK_X)));
  r.y1 = imin_(grid_y, imax_(0, f2i((py + (float)ry + (float)(BLOCK_Y - 1)) / (float)BLOCK_Y)));
  return r;
}

/* math_kernels.py:151-194 */
static inline rect4 snugbox_rect(float px, float py, float cov_aa, float cov_cc, float opacity, int cuda_radius,
                                 int grid_x, int grid_y) {
  const rect4 c = compute_tile_rect(px, py, cuda_radius, cuda_radius, grid_x, grid_y);
  const float t = 2.0f * or_log(fmax_(255.0f * opacity, 1.0f));
  rect4 z = {0, 0, 0, 0};
  if (t <= 0.0f) return z;
  const int rx = f2i(ceilf(sqrtf(fmax_(t * cov_aa, 0.0f)) + SNUGBOX_PIXEL_PADDING));
  const int ry = f2i(ceilf(sqrtf(fmax_(t * cov_cc, 0.0f)) + SNUGBOX_PIXEL_PADDING));
  const rect4 s = compute_tile_rect(px, py, rx, ry, grid_x, grid_y);
  rect4 r = {imax_(c.x0, s.x0), imax_(c.y0, s.y0), imin_(c.x1, s.x1), imin_(c.y1, s.y1)};
  return r;
}

/* math_kernels.py:197-204 */
static inline float conic_q(float x, float y, float a, float b, float c) {
  return a * x * x + 2.0f * b * x * y + c * y * y;
}

/* math_kernels.py:207-240 */
static int conic_rect_intersects_tile(float px, float py, float a, float b, float c, float threshold, int tile_x,
                                      int tile_y) {
  const float det = a * c - b * b;
  if (a <= 0.0f || c <= 0.0f || det <= DET_EPSILON) return 1;
  const float x0 = (float)(tile_x * BLOCK_X) - px;
  const float x1 = (float)(tile_x * BLOCK_X + BLOCK_X - 1) - px;
  const float y0 = (float)(tile_y * BLOCK_Y) - py;
  const float y1 = (float)(tile_y * BLOCK_Y + BLOCK_Y - 1) - py;
  if (x0 <= 0.0f && x1 >= 0.0f && y0 <= 0.0f && y1 >= 0.0f) return 1;
  float q_min = 3.402823466e38f;
  float y = clamp_(-b * x0 / c, y0, y1);
  q_min = fmin_(q_min, conic_q(x0, y, a, b, c));
  y = clamp_(-b * x1 / c, y0, y1);
  q_min = fmin_(q_min, conic_q(x1, y, a, b, c));
  float x = clamp_(-b * y0 / a, x0, x1);
  q_min = fmin_(q_min, conic_q(x, y0, a, b, c));
  x = clamp_(-b * y1 / a, x0, x1);
  q_min = fmin_(q_min, conic_q(x, y1, a, b, c));
  return q_min <= threshold + COVERAGE_Q_EPSILON;
}

/* math_kernels.py:243-303; returns [lo, hi) in out[0..1] */
static void accutile_band_interval(float pu, float pv, float cuu, float cuv, float cvv, float threshold, int tile_v,
                                   int block_u, int block_v, int rect_u_min, int rect_u_max, int out[2]) {
  const float det = cuu * cvv - cuv * cuv;
  if (cuu <= 0.0f || cvv <= 0.0f || det <= DET_EPSILON) {
    out[0] = rect_u_min;
    out[1] = rect_u_max;
    return;
  }
  const float threshold_safe = threshold + COVERAGE_Q_EPSILON;
  const float v0 = (float)(tile_v * block_v) - pv;
  const float v1 = (float)(tile_v * block_v + block_v - 1) - pv;
  float u_min = 3.402823466e38f;
  float u_max = -3.402823466e38f;
  int found = 0;
  float disc = cuu * threshold_safe - det * v0 * v0;
  if (disc >= -COVERAGE_Q_EPSILON) {
    const float half = sqrtf(fmax_(disc, 0.0f)) / cuu;
    const float center = -cuv * v0 / cuu;
    u_min = fmin_(u_min, center - half);
    u_max = fmax_(u_max, center + half);
    found = 1;
  }
  disc = cuu * threshold_safe - det * v1 * v1;
  if (disc >= -COVERAGE_Q_EPSILON) {
    const float half = sqrtf(fmax_(disc, 0.0f)) / cuu;
    const float center = -cuv * v1 / cuu;
    u_min = fmin_(u_min, center - half);
    u_max = fmax_(u_max, center + half);
    found = 1;
  }
  const float extent_u = sqrtf(fmax_(threshold_safe * cvv / det, 0.0f));
  const float v_at_min_u = cuv * extent_u / cvv;
  if (v_at_min_u >= v0 - COVERAGE_Q_EPSILON && v_at_min_u <= v1 + COVERAGE_Q_EPSILON) {
    u_min = fmin_(u_min, -extent_u);
    u_max = fmax_(u_max, -extent_u);
    found = 1;
  }
  const float v_at_max_u = -cuv * extent_u / cvv;
  if (v_at_max_u >= v0 - COVERAGE_Q_EPSILON && v_at_max_u <= v1 + COVERAGE_Q_EPSILON) {
    u_min = fmin_(u_min, extent_u);
    u_max = fmax_(u_max, extent_u);
    found = 1;
  }
  if (!found) {
    out[0] = rect_u_min;
    out[1] = rect_u_min;
    return;
  }
  const int tile_u_min = f2i(floorf((pu + u_min) / (float)block_u));
  const int tile_u_max = f2i(floorf((pu + u_max) / (float)block_u)) + 1;
  out[0] = imax_(rect_u_min, imin_(rect_u_max, tile_u_min));
  out[1] = imax_(rect_u_min, imin_(rect_u_max, tile_u_max));
}

/* Visitor over the tiles a Gaussian is binned to, in the reference's
 * emission order: binning_kernels.py:127-216 (mode ids coverage.py:128-132).
 * The conic-rect mode follows the recount of binning_kernels.py:56-124:
 * exact conic-rect test up to 64 candidate tiles, AccuTile beyond. */
typedef void (*tile_visitor)(void* ctx, int tile_x, int tile_y);

static int visit_covered_tiles(float px, float py, float cov_aa, float cov_cc, float ca, float cb, float cc,
                               float opacity, int radius, int grid_x, int grid_y, int mode, tile_visitor visit,
                               void* ctx) {
  const rect4 rect = snugbox_rect(px, py, cov_aa, cov_cc, opacity, radius, grid_x, grid_y);
  const int span_x = rect.x1 - rect.x0;
  const int span_y = rect.y1 - rect.y0;
  const int area = span_x * span_y;
  int count = 0;
  if (area <= 1 || mode == TILE_COVERAGE_SNUGBOX) {
    for (int ty = rect.y0; ty < rect.y1; ++ty)
      for (int tx = rect.x0; tx < rect.x1; ++tx) {
        if (visit) visit(ctx, tx, ty);
        ++count;
      }
    return count;
  }
  const float threshold = 2.0f * or_log(fmax_(255.0f * opacity, 1.0f));
  if (mode == TILE_COVERAGE_CONIC_RECT && area <= TILE_COVERAGE_CONIC_MASK_MAX_TILES) {
    for (int ty = rect.y0; ty < rect.y1; ++ty)
      for (int tx = rect.x0; tx < rect.x1; ++tx)
        if (conic_rect_intersects_tile(px, py, ca, cb, cc, threshold, tx, ty)) {
          if (visit) visit(ctx, tx, ty);
          ++count;
        }
    return count;
  }
  int iv[2];
  if (span_y <= span_x) {
    for (int ty = rect.y0; ty < rect.y1; ++ty) {
      accutile_band_interval(px, py, ca, cb, cc, threshold, ty, BLOCK_X, BLOCK_Y, rect.x0, rect.x1, iv);
      for (int tx = iv[0]; tx < iv[1]; ++tx) {
        if (visit) visit(ctx, tx, ty);
        ++count;
      }
    }
  } else {
    for (int tx = rect.x0; tx < rect.x1; ++tx) {
      accutile_band_interval(py, px, cc, cb, ca, threshold, tx, BLOCK_Y, BLOCK_X, rect.y0, rect.y1, iv);
      for (int ty = iv[0]; ty < iv[1]; ++ty) {
        if (visit) visit(ctx, tx, ty);
        ++count;
      }
    }
  }
  return count;
}

/* _count_covered_tiles_wp (math_kernels.py:306-390) for a batch of points;
 * mode as in visit_covered_tiles. */
void or_count_covered_tiles(int n, const float* points_xy, const float* cov2d, const float* conic_opacity,
                            const int* radii, int grid_x, int grid_y, int mode, int* counts) {
  for (int i = 0; i < n; ++i) {
    counts[i] = visit_covered_tiles(points_xy[2 * i], points_xy[2 * i + 1], cov2d[3 * i], cov2d[3 * i + 2],
                                    conic_opacity[4 * i], conic_opacity[4 * i + 1], conic_opacity[4 * i + 2],
                                    conic_opacity[4 * i + 3], radii[i], grid_x, grid_y, mode, NULL, NULL);
  }
}

typedef struct {
  int* tile_ids;
  int* points;
  long long off;
  long long limit; /* writes at or beyond limit are dropped */
  int point_id;
  int grid_x;
} emit_ctx;

static void emit_visit(void* vctx, int tx, int ty) {
  emit_ctx* c = (emit_ctx*)vctx;
  if (c->off >= 0 && c->off < c->limit) {
    c->tile_ids[c->off] = ty * c->grid_x + tx;
    c->points[c->off] = c->point_id;
  }
  c->off++;
}

/* Emission of (tile, point) pairs per point in the given order, as in
 * _duplicate_with_keys_warp_kernel (binning_kernels.py:325-363), with
 * explicit offsets; used by tests for count == emit checks. */
void or_emit_covered_tiles(int n, const float* points_xy, const float* cov2d, const float* conic_opacity,
                           const int* radii, int grid_x, int grid_y, int mode, const int* inclusive_offsets,
                           int* tile_ids, int* point_list) {
  for (int i = 0; i < n; ++i) {
    if (radii[i] <= 0) continue;
    emit_ctx c = {tile_ids, point_list, i > 0 ? inclusive_offsets[i - 1] : 0, n > 0 ? inclusive_offsets[n - 1] : 0,
                  i, grid_x};
    visit_covered_tiles(points_xy[2 * i], points_xy[2 * i + 1], cov2d[3 * i], cov2d[3 * i + 2],
                        conic_opacity[4 * i], conic_opacity[4 * i + 1], conic_opacity[4 * i + 2],
                        conic_opacity[4 * i + 3], radii[i], grid_x, grid_y, mode, emit_visit, &c);
  }
}

/* _forward_rgb_from_sh_v3_warp_kernel (preprocess_kernels.py:272-342) for one point. */
static void sh_forward_one(const float* mean, const float* campos, const float* sh, int degree, int K, float* rgb,
                           int* clamped) {
  const float d0 = mean[0] - campos[0], d1 = mean[1] - campos[1], d2 = mean[2] - campos[2];
  const float len_sq = d0 * d0 + d1 * d1 + d2 * d2;
  const float inv_len = 1.0f / sqrtf(fmax_(len_sq, 1.0e-20f));
  const float x = d0 * inv_len, y = d1 * inv_len, z = d2 * inv_len;
  float c[3];
  for (int ch = 0; ch < 3; ++ch) c[ch] = SH_C0 * sh[ch];
  if (degree > 0 && K > 3) {
    const float b0 = -SH_C1 * y, b1 = SH_C1 * z, b2 = -SH_C1 * x;
    for (int ch = 0; ch < 3; ++ch) c[ch] = c[ch] + b0 * sh[3 + ch];
    for (int ch = 0; ch < 3; ++ch) c[ch] = c[ch] + b1 * sh[6 + ch];
    for (int ch = 0; ch < 3; ++ch) c[ch] = c[ch] + b2 * sh[9 + ch];
    if (degree > 1 && K > 8) {
      const float xx = x * x, yy = y * y, zz = z * z, xy = x * y, yz = y * z, xz = x * z;
      const float w[5] = {SH_C2_0 * xy, SH_C2_1 * yz, SH_C2_2 * (2.0f * zz - xx - yy), SH_C2_3 * xz,
                          SH_C2_4 * (xx - yy)};
      for (int k = 0; k < 5; ++k)
        for (int ch = 0; ch < 3; ++ch) c[ch] = c[ch] + w[k] * sh[3 * (4 + k) + ch];
      if (degree > 2 && K > 15) {
        const float v[7] = {SH_C3_0 * y * (3.0f * xx - yy),
                            SH_C3_1 * xy * z,
                            SH_C3_2 * y * (4.0f * zz - xx - yy),
                            SH_C3_3 * z * (2.0f * zz - 3.0f * xx - 3.0f * yy),
                            SH_C3_4 * x * (4.0f * zz - xx - yy),
                            SH_C3_5 * z * (xx - yy),
                            SH_C3_6 * x * (xx - 3.0f * yy)};
        for (int k = 0; k < 7; ++k)
          for (int ch = 0; ch < 3; ++ch) c[ch] = c[ch] + v[k] * sh[3 * (9 + k) + ch];
      }
    }
  }
  for (int ch = 0; ch < 3; ++ch) {
    c[ch] = c[ch] + 0.5f;
    clamped[ch] = 0;
    if (c[ch] < 0.0f) {
      c[ch] = 0.0f;
      clamped[ch] = 1;
    }
    rgb[ch] = c[ch];
  }
}

/*
 * Preprocess, scales/rotations path: _fused_project_cov3d_cov2d_preprocess_sr_warp_kernel
 * (preprocess_kernels.py:83-269) then SH for all points (preprocess_kernels.py:272-342,
 * preprocess_ops.py:548-565); colors_precomp replaces the SH colour
 * (preprocess_ops.py:548-549).  focal_x/y are the host's W/(2 tanfovx) rounded to fp32.
 */
/* Mip-Splatting screen-space low-pass filter of one Gaussian, applied after the base preprocess
 * (backend_mip_3dgs.py:63-102): for radius > 0, cov2D += f I; culled (radius, conic, cov2D and tile
 * count zero) unless the filtered determinant exceeds 1e-12; otherwise conic = filtered inverse,
 * radius = ceil(3 sqrt(max(tr/2 + sqrt(max(((a-c)^2)/4 + b^2, 0)), 0.1))) and the tiles recounted
 * with the filtered values (binning_kernels.py:56-123, the same count as the base preprocess).
 * Depth and screen position keep their base values. */
static void mip_filter_one(int idx, float f, const float* opacities, int grid_x, int grid_y, int coverage_mode,
                           int* radii, const float* proj_2d, float* conic_2d, float* conic_2d_inv,
                           int* tiles_touched) {
  if (radii[idx] <= 0) return;
  const float a = conic_2d_inv[3 * idx] + f;
  const float b = conic_2d_inv[3 * idx + 1];
  const float c = conic_2d_inv[3 * idx + 2] + f;
  const float det = a * c - b * b;
  if (!(det > 1.0e-12f)) {
    radii[idx] = 0;
    tiles_touched[idx] = 0;
    for (int k = 0; k < 3; ++k) conic_2d[3 * idx + k] = conic_2d_inv[3 * idx + k] = 0.0f;
    return;
  }
  const float inv_det = 1.0f / det;
  const float con0 = c * inv_det, con1 = -b * inv_det, con2 = a * inv_det;
  const float trace = a + c;
  const float d = a - c;
  float disc = 0.25f * (d * d) + b * b;
  if (disc < 0.0f) disc = 0.0f;
  float lam = 0.5f * trace + sqrtf(disc);
  if (lam < 0.1f) lam = 0.1f;
  const int radius = f2i(ceilf(3.0f * sqrtf(lam)));
  radii[idx] = radius;
  conic_2d[3 * idx] = con0;
  conic_2d[3 * idx + 1] = con1;
  conic_2d[3 * idx + 2] = con2;
  conic_2d_inv[3 * idx] = a;
  conic_2d_inv[3 * idx + 1] = b;
  conic_2d_inv[3 * idx + 2] = c;
  tiles_touched[idx] = visit_covered_tiles(proj_2d[2 * idx], proj_2d[2 * idx + 1], a, c, con0, con1, con2,
                                           opacities[idx], radius, grid_x, grid_y, coverage_mode, NULL, NULL);
}

void or_preprocess(int P, int K, int degree, const float* means3d, const float* scales, const float* rotations,
                   const float* cov3d_precomp, float scale_modifier, const float* opacities, const float* shs,
                   const float* colors,
                   const float* V, const float* Pm, const float* campos, float tanfovx, float tanfovy,
                   float focal_x, float focal_y, int W, int H, int coverage_mode, float filter_variance,
                   int* radii, float* depths,
                   float* proj_2d, float* conic_2d, float* conic_2d_inv, int* tiles_touched, float* cov3d,
                   float* rgb, int* clamped, int* visible_mask) {
  const int grid_x = (W + BLOCK_X - 1) / BLOCK_X;
  const int grid_y = (H + BLOCK_Y - 1) / BLOCK_Y;
#pragma omp parallel for schedule(static)
  for (int idx = 0; idx < P; ++idx) {
    for (int k = 0; k < 6; ++k) cov3d[6 * idx + k] = 0.0f;
    depths[idx] = 0.0f;
    radii[idx] = 0;
    proj_2d[2 * idx] = proj_2d[2 * idx + 1] = 0.0f;
    for (int k = 0; k < 3; ++k) conic_2d[3 * idx + k] = conic_2d_inv[3 * idx + k] = 0.0f;
    tiles_touched[idx] = 0;
    const float* p = means3d + 3 * idx;
    const float p_view_z = V[2] * p[0] + V[6] * p[1] + V[10] * p[2] + V[14];
    if (p_view_z <= 0.2f) {
      visible_mask[idx] = 0;
      goto sh;
    }
    visible_mask[idx] = 1;
    {
      const float hom_x = Pm[0] * p[0] + Pm[4] * p[1] + Pm[8] * p[2] + Pm[12];
      const float hom_y = Pm[1] * p[0] + Pm[5] * p[1] + Pm[9] * p[2] + Pm[13];
      const float hom_w = Pm[3] * p[0] + Pm[7] * p[1] + Pm[11] * p[2] + Pm[15];
      const float inv_w = 1.0f / (hom_w + 0.0000001f);
      const float p_proj_x = hom_x * inv_w;
      const float p_proj_y = hom_y * inv_w;
      if (cov3d_precomp != NULL) {
        /* masked path for precomputed 3D covariances: preprocess_kernels.py:345-477 (cov2D as t^T (V t),
         * culled when |det| < 1e-7) after the projection of preprocess_kernels.py:604-624 */
        const float* cv = cov3d_precomp + 6 * idx;
        for (int k = 0; k < 6; ++k) cov3d[6 * idx + k] = cv[k];
        float x = V[0] * p[0] + V[4] * p[1] + V[8] * p[2] + V[12];
        float y = V[1] * p[0] + V[5] * p[1] + V[9] * p[2] + V[13];
        const float z = p_view_z;
        const float limx = 1.3f * tanfovx, limy = 1.3f * tanfovy;
        const float txtz = x / z, tytz = y / z;
        x = clamp_(txtz, -limx, limx) * z;
        y = clamp_(tytz, -limy, limy) * z;
        const float a = focal_x / z, b = focal_y / z;
        const float c = -(focal_x * x) / (z * z), d = -(focal_y * y) / (z * z);
        const float t00 = V[0] * a + V[2] * c, t10 = V[4] * a + V[6] * c, t20 = V[8] * a + V[10] * c;
        const float t01 = V[1] * b + V[2] * d, t11 = V[5] * b + V[6] * d, t21 = V[9] * b + V[10] * d;
        const float v00 = cv[0], v01 = cv[1], v02 = cv[2], v11 = cv[3], v12 = cv[4], v22 = cv[5];
        const float vt0x = v00 * t00 + v01 * t10 + v02 * t20;
        const float vt0y = v01 * t00 + v11 * t10 + v12 * t20;
        const float vt0z = v02 * t00 + v12 * t10 + v22 * t20;
        const float vt1x = v00 * t01 + v01 * t11 + v02 * t21;
        const float vt1y = v01 * t01 + v11 * t11 + v12 * t21;
        const float vt1z = v02 * t01 + v12 * t11 + v22 * t21;
        const float cov_a = t00 * vt0x + t10 * vt0y + t20 * vt0z + 0.3f;
        const float cov_b = t00 * vt1x + t10 * vt1y + t20 * vt1z;
        const float cov_c = t01 * vt1x + t11 * vt1y + t21 * vt1z + 0.3f;
        const float det = cov_a * cov_c - cov_b * cov_b;
        if (fabsf(det) < DET_EPSILON) goto sh;
        const float det_inv = 1.0f / det;
        const float con0 = cov_c * det_inv, con1 = -cov_b * det_inv, con2 = cov_a * det_inv;
        const float mid = 0.5f * (cov_a + cov_c);
        const float root = sqrtf(fmax_(0.1f, mid * mid - det));
        const int radius = f2i(ceilf(3.0f * sqrtf(fmax_(mid + root, mid - root))));
        const float point_x = ndc_to_pix(p_proj_x, W);
        const float point_y = ndc_to_pix(p_proj_y, H);
        const rect4 cr = compute_tile_rect(point_x, point_y, radius, radius, grid_x, grid_y);
        if ((cr.x1 - cr.x0) * (cr.y1 - cr.y0) == 0) goto sh;
        depths[idx] = p_view_z;
        radii[idx] = radius;
        proj_2d[2 * idx] = point_x;
        proj_2d[2 * idx + 1] = point_y;
        conic_2d[3 * idx] = con0;
        conic_2d[3 * idx + 1] = con1;
        conic_2d[3 * idx + 2] = con2;
        conic_2d_inv[3 * idx] = cov_a;
        conic_2d_inv[3 * idx + 1] = cov_b;
        conic_2d_inv[3 * idx + 2] = cov_c;
        tiles_touched[idx] = visit_covered_tiles(point_x, point_y, cov_a, cov_c, con0, con1, con2, opacities[idx],
                                                 radius, grid_x, grid_y, coverage_mode, NULL, NULL);
        goto sh;
      }
      const float s0 = scales[3 * idx] * scale_modifier;
      const float s1 = scales[3 * idx + 1] * scale_modifier;
      const float s2 = scales[3 * idx + 2] * scale_modifier;
      const float rr = rotations[4 * idx], xq = rotations[4 * idx + 1], yq = rotations[4 * idx + 2],
                  zq = rotations[4 * idx + 3];
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
      cov3d[6 * idx + 0] = m00 * m00 + m10 * m10 + m20 * m20;
      cov3d[6 * idx + 1] = m00 * m01 + m10 * m11 + m20 * m21;
      cov3d[6 * idx + 2] = m00 * m02 + m10 * m12 + m20 * m22;
      cov3d[6 * idx + 3] = m01 * m01 + m11 * m11 + m21 * m21;
      cov3d[6 * idx + 4] = m01 * m02 + m11 * m12 + m21 * m22;
      cov3d[6 * idx + 5] = m02 * m02 + m12 * m12 + m22 * m22;
      float vx = V[0] * p[0] + V[4] * p[1] + V[8] * p[2] + V[12];
      float vy = V[1] * p[0] + V[5] * p[1] + V[9] * p[2] + V[13];
      const float vz = p_view_z;
      const float limx = 1.3f * tanfovx;
      const float limy = 1.3f * tanfovy;
      const float txtz = vx / vz;
      const float tytz = vy / vz;
      vx = clamp_(txtz, -limx, limx) * vz;
      vy = clamp_(tytz, -limy, limy) * vz;
      const float a_j = focal_x / vz;
      const float b_j = focal_y / vz;
      const float c_j = -(focal_x * vx) / (vz * vz);
      const float d_j = -(focal_y * vy) / (vz * vz);
      const float t00 = V[0] * a_j + V[2] * c_j;
      const float t10 = V[4] * a_j + V[6] * c_j;
      const float t20 = V[8] * a_j + V[10] * c_j;
      const float t01 = V[1] * b_j + V[2] * d_j;
      const float t11 = V[5] * b_j + V[6] * d_j;
      const float t21 = V[9] * b_j + V[10] * d_j;
      const float a00 = m00 * t00 + m01 * t10 + m02 * t20;
      const float a10 = m10 * t00 + m11 * t10 + m12 * t20;
      const float a20 = m20 * t00 + m21 * t10 + m22 * t20;
      const float a01 = m00 * t01 + m01 * t11 + m02 * t21;
      const float a11 = m10 * t01 + m11 * t11 + m12 * t21;
      const float a21 = m20 * t01 + m21 * t11 + m22 * t21;
      const float cov_a = a00 * a00 + a10 * a10 + a20 * a20 + 0.3f;
      const float cov_b = a00 * a01 + a10 * a11 + a20 * a21;
      const float cov_c = a01 * a01 + a11 * a11 + a21 * a21 + 0.3f;
      const float det = cov_a * cov_c - cov_b * cov_b;
      if (fabsf(det) <= DET_EPSILON) goto sh;
      const float det_inv = 1.0f / det;
      const float con0 = cov_c * det_inv, con1 = -cov_b * det_inv, con2 = cov_a * det_inv;
      const float mid = 0.5f * (cov_a + cov_c);
      const float root = sqrtf(fmax_(0.1f, mid * mid - det));
      const float lambda1 = mid + root;
      const float lambda2 = mid - root;
      const int radius = f2i(ceilf(3.0f * sqrtf(fmax_(lambda1, lambda2))));
      const float point_x = ndc_to_pix(p_proj_x, W);
      const float point_y = ndc_to_pix(p_proj_y, H);
      const rect4 cr = compute_tile_rect(point_x, point_y, radius, radius, grid_x, grid_y);
      if ((cr.x1 - cr.x0) * (cr.y1 - cr.y0) == 0) goto sh;
      depths[idx] = p_view_z;
      radii[idx] = radius;
      proj_2d[2 * idx] = point_x;
      proj_2d[2 * idx + 1] = point_y;
      conic_2d[3 * idx] = con0;
      conic_2d[3 * idx + 1] = con1;
      conic_2d[3 * idx + 2] = con2;
      conic_2d_inv[3 * idx] = cov_a;
      conic_2d_inv[3 * idx + 1] = cov_b;
      conic_2d_inv[3 * idx + 2] = cov_c;
      tiles_touched[idx] = visit_covered_tiles(point_x, point_y, cov_a, cov_c, con0, con1, con2, opacities[idx],
                                               radius, grid_x, grid_y, coverage_mode, NULL, NULL);
    }
  sh:
    if (filter_variance != 0.0f)
      mip_filter_one(idx, filter_variance, opacities, grid_x, grid_y, coverage_mode, radii, proj_2d, conic_2d,
                     conic_2d_inv, tiles_touched);
    if (colors != NULL) {
      for (int ch = 0; ch < 3; ++ch) {
        rgb[3 * idx + ch] = colors[3 * idx + ch];
        clamped[3 * idx + ch] = 0;
      }
    } else {
      sh_forward_one(p, campos, shs + (size_t)idx * (size_t)(3 * K), degree, K, rgb + 3 * idx, clamped + 3 * idx);
    }
  }
}

/* _project_visible_points_warp_kernel (preprocess_kernels.py:604-617) */
void or_mark_visible(int P, const float* means3d, const float* V, int* visible) {
  for (int i = 0; i < P; ++i) {
    const float* p = means3d + 3 * i;
    const float z = V[2] * p[0] + V[6] * p[1] + V[10] * p[2] + V[14];
    visible[i] = z > 0.2f;
  }
}

/* Stable LSD radix sort of (uint32 key, int32 value) pairs, 8 bits per pass. */
static void stable_sort_u32(long long n, uint32_t* keys, int* vals) {
  if (n <= 1) return;
  uint32_t* k2 = (uint32_t*)malloc((size_t)n * sizeof(uint32_t));
  int* v2 = (int*)malloc((size_t)n * sizeof(int));
  for (int shift = 0; shift < 32; shift += 8) {
    long long count[257];
    memset(count, 0, sizeof(count));
    for (long long i = 0; i < n; ++i) count[((keys[i] >> shift) & 255) + 1]++;
    for (int d = 0; d < 256; ++d) count[d + 1] += count[d];
    for (long long i = 0; i < n; ++i) {
      const long long dst = count[(keys[i] >> shift) & 255]++;
      k2[dst] = keys[i];
      v2[dst] = vals[i];
    }
    memcpy(keys, k2, (size_t)n * sizeof(uint32_t));
    memcpy(vals, v2, (size_t)n * sizeof(int));
  }
  free(k2);
  free(v2);
}

/* Total pair count: sum of tiles_touched (binning_ops.py:222-252). */
long long or_num_rendered(int P, const int* tiles_touched) {
  long long s = 0;
  for (int i = 0; i < P; ++i) s += tiles_touched[i];
  return s;
}

/*
 * _build_binning_state, sort mode "warp_depth_stable_tile" (binning_ops.py:84-431):
 *   depth keys = fp32 depth bits as int32, payload = point index
 *     (binning_kernels.py:27-40), stable radix sort (binning_ops.py:187-189);
 *   tiles_touched gathered in depth order and inclusively scanned (binning_ops.py:218-222);
 *   duplicate in depth order (binning_kernels.py:411-451);
 *   stable radix sort of the R pairs by tile id (binning_ops.py:337-343);
 *   tile ranges (binning_kernels.py:468-487) over a zeroed (T,2) buffer.
 * R must equal or_num_rendered(); outputs: point_list (R), tile_ids (R), ranges (T,2).
 */
void or_binning(int P, const int* radii, const float* depths, const int* tiles_touched, const float* points_xy,
                const float* cov2d, const float* conic_opacity, int W, int H, int coverage_mode, long long R,
                int* point_list, int* tile_ids, int* ranges) {
  const int grid_x = (W + BLOCK_X - 1) / BLOCK_X;
  const int grid_y = (H + BLOCK_Y - 1) / BLOCK_Y;
  const int T = grid_x * grid_y;
  memset(ranges, 0, sizeof(int) * 2 * (size_t)T);
  if (P <= 0 || R <= 0) return;
  uint32_t* dkeys = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)P);
  int* order = (int*)malloc(sizeof(int) * (size_t)P);
  for (int i = 0; i < P; ++i) {
    int32_t bits;
    memcpy(&bits, &depths[i], 4);
    /* int32 keys are >= 0 here (depth > 0.2 or 0.0), so uint32 order == int32 order */
    dkeys[i] = (uint32_t)bits;
    order[i] = i;
  }
  stable_sort_u32(P, dkeys, order);
  long long off = 0;
  for (int j = 0; j < P; ++j) {
    const int i = order[j];
    if (radii[i] <= 0) {
      off += tiles_touched[i];
      continue;
    }
    emit_ctx c = {tile_ids, point_list, off, R, i, grid_x};
    visit_covered_tiles(points_xy[2 * i], points_xy[2 * i + 1], cov2d[3 * i], cov2d[3 * i + 2],
                        conic_opacity[4 * i], conic_opacity[4 * i + 1], conic_opacity[4 * i + 2],
                        conic_opacity[4 * i + 3], radii[i], grid_x, grid_y, coverage_mode, emit_visit, &c);
    off += tiles_touched[i];
  }
  free(dkeys);
  free(order);
  uint32_t* tk = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)R);
  for (long long i = 0; i < R; ++i) tk[i] = (uint32_t)tile_ids[i];
  stable_sort_u32(R, tk, point_list);
  for (long long i = 0; i < R; ++i) tile_ids[i] = (int)tk[i];
  free(tk);
  for (long long idx = 0; idx < R; ++idx) {
    const int curr = tile_ids[idx];
    if (idx == 0) {
      ranges[curr * 2] = 0;
    } else {
      const int prev = tile_ids[idx - 1];
      if (curr != prev) {
        ranges[prev * 2 + 1] = (int)idx;
        ranges[curr * 2] = (int)idx;
      }
    }
    if (idx == R - 1) ranges[curr * 2 + 1] = (int)R;
  }
}

/*
 * Gaussian exponent of a pixel offset (render_kernels.py:120 and
 * backward_kernels.py:643 via _compute_power, math_kernels.py:78-80):
 *   power = -0.5 (a dx^2 + c dy^2) - b dx dy,  conic co = (a, b, c).
 * Evaluated in this build's fixed fp32 form, the same in the gfx950 kernels:
 * the quadratic form q = fma(fma(c, dy, (b dx) 2), dy, (a dx) dx) with two
 * fused multiply-adds, and power = -0.5 q (exact).  The reference leaves the
 * contraction of this expression to its GPU compiler, so no rounding order
 * is fixed by it.
 */
static inline float blend_power(const float* co, float d_x, float d_y) {
  const float adxx = co[0] * d_x * d_x;
  const float b2dx = (co[1] * d_x) * 2.0f;
  const float q = fmaf(fmaf(co[2], d_y, b2dx), d_y, adxx);
  return -0.5f * q;
}

/*
 * _render_tiles_tiled256_warp_kernel (render_kernels.py:16-147), with the
 * flow auxiliaries of flow_kernels.py:159-166 when top_k > 0 (aux arrays
 * pre-filled with -1 / 0 / 0 as flow_ops.py:119-129 does).  The block-wide
 * early exit of the reference only skips work for pixels that are already
 * done, so each pixel is evaluated independently here.
 */
void or_render_fwd(int W, int H, const int* ranges, const int* point_list, const float* points_xy,
                   const float* features, const float* depths, const float* conic_opacity, const float* bg,
                   int compute_depth, int top_k, float* out_color, float* out_depth, float* out_alpha,
                   int* n_contrib, int* gs_per_pixel, float* weight_per_gs_pixel, float* x_mu) {
  const int grid_x = (W + BLOCK_X - 1) / BLOCK_X;
  const long long total = (long long)W * H;
  if (top_k > 0) {
    for (long long i = 0; i < (long long)top_k * total; ++i) {
      gs_per_pixel[i] = -1;
      weight_per_gs_pixel[i] = 0.0f;
      x_mu[i] = 0.0f;
      x_mu[(long long)top_k * total + i] = 0.0f;
    }
  }
#pragma omp parallel for schedule(dynamic, 64)
  for (long long pixel_id = 0; pixel_id < total; ++pixel_id) {
    const int pix_x = (int)(pixel_id % W), pix_y = (int)(pixel_id / W);
    const int tile_id = (pix_y / BLOCK_Y) * grid_x + pix_x / BLOCK_X;
    const int start = ranges[2 * tile_id], end = ranges[2 * tile_id + 1];
    float T = 1.0f;
    int contributor = 0, last_contributor = 0, n_success = 0;
    float color0 = 0.0f, color1 = 0.0f, color2 = 0.0f, weight = 0.0f, depth_acc = 0.0f;
    const float pixf_x = (float)pix_x, pixf_y = (float)pix_y;
    for (int k = start; k < end; ++k) {
      contributor = contributor + 1;
      const int id = point_list[k];
      const float* co = conic_opacity + 4 * id;
      const float d_x = points_xy[2 * id] - pixf_x;
      const float d_y = points_xy[2 * id + 1] - pixf_y;
      const float power = blend_power(co, d_x, d_y);
      if (power <= 0.0f) {
        const float alpha = fmin_(0.99f, co[3] * or_exp(power));
        if (alpha >= (1.0f / 255.0f)) {
          const float test_T = T * (1.0f - alpha);
          if (test_T < 0.0001f) break;
          const float contribution = alpha * T;
          /* colour and depth accumulate with one fused multiply-add each (this
           * build's fixed form; the reference leaves the contraction of
           * C += f * (alpha T) to its GPU compiler) */
          color0 = fmaf(features[3 * id], contribution, color0);
          color1 = fmaf(features[3 * id + 1], contribution, color1);
          color2 = fmaf(features[3 * id + 2], contribution, color2);
          weight = weight + contribution;
          if (compute_depth) depth_acc = fmaf(depths[id], contribution, depth_acc);
          if (top_k > 0 && n_success < top_k) {
            const long long aux = (long long)n_success * total + pixel_id;
            gs_per_pixel[aux] = id;
            weight_per_gs_pixel[aux] = contribution;
            x_mu[aux] = d_x;
            x_mu[(long long)top_k * total + aux] = d_y;
          }
          n_success = n_success + 1;
          T = test_T;
          last_contributor = contributor;
        }
      }
    }
    n_contrib[pixel_id] = last_contributor;
    out_color[pixel_id] = color0 + T * bg[0];
    out_color[total + pixel_id] = color1 + T * bg[1];
    out_color[2 * total + pixel_id] = color2 + T * bg[2];
    out_alpha[pixel_id] = weight;
    out_depth[pixel_id] = depth_acc;
  }
}

/*
 * _backward_render_tiles_warp32_kernel (backward_kernels.py:539-707) per pixel,
 * accumulating in double.  grad_out (P_gauss, 10): dx, dy, conic a, b, c,
 * opacity, r, g, b, depth (the reference's grad_points_xy, grad_conic_opacity,
 * grad_feature and grad_depths, backward_ops.py:200-208).
 *
 * Error bound (err_out, mag_out; both (P_gauss, 10) doubles, or NULL).  The
 * per-pixel terms above are fp32 expressions, and an fp32 implementation may
 * evaluate them in another algebraically equal order (a running dot product
 * S = U . acc in place of the per-channel recurrences; pixel moments summed
 * first and multiplied by the conic, opacity and W/2, H/2 once), with exp and
 * 1/x a few ulp off.  Alongside each term this routine carries a first-order
 * running bound (Wilkinson's running error analysis) on |computed - exact|
 * valid for any such evaluation, where "exact" is real arithmetic on the same
 * fp32 inputs (q, the conic, opacity, colours, depths, T_final = 1 - alpha and
 * the upstream gradients).  With u = 2^-24, per blended (pixel, Gaussian):
 *   G:      rel_G  = (0.75 q + 3) u   (exp(-q/2) by exp2 of a rounded product,
 *                                      <= 2 ulp of the exponential itself);
 *   alpha:  rel_a  = rel_G + u, 0 where both sides hit the 0.99 cap;
 *   1-alpha:rel_om = alpha rel_a / (1 - alpha) + u;
 *   T:      rel_T += rel_om + 2u per step back (a reciprocal and a product);
 *   S:      e_S  <- (1-alpha) e_S + alpha e_fu + alpha rel_a (M_fu + m_S) + 4u (M_fu + m_S),
 *           with M_fu = sum |F_ch U_ch| (colour, depth, alpha), e_fu = 5u M_fu,
 *           m_S <- (1-alpha) m_S + alpha M_fu its magnitude (m_S >= |S|),
 *           started at e_S = 3u m_S, m_S = sum |bg_ch U_ch|;
 *   v = G T (F.U - S):  e_v = G T (e_fu + e_S + u (M_fu + m_S)) + |v| (rel_G + rel_T + 2u).
 * Each column's term is a product of v (or alpha T) with exact per-Gaussian
 * and per-pixel factors; err_out sums  |factor| e_v + 4u |factor v|  (colour
 * and depth: |alpha T U| (rel_a + rel_T + 2u)), and mag_out sums the
 * term magnitudes with every sum written out in absolute values (column 0:
 * W/2 o |v| (|a dx| + |b dy|)), which bounds the rounding of any summation
 * order: a sum of m partial sums of these terms errs by at most
 * (depth of the summation tree) u mag_out.
 *
 * value_mode selects how the term values are computed (the blend decisions
 * are always the fp32 ones above): 0 the reference's fp32 expressions; 1 the
 * same expressions in double from the fp32 inputs ("exact" for the bound);
 * 2 a second fp32 order, the one a wave-parallel kernel uses (exp2 of a
 * rounded product, 1 - alpha inverted by a reciprocal, S = U . acc with fused
 * multiply-adds, pixel moments times per-Gaussian factors).  grad_out64, if
 * not NULL, receives the double sums.
 */
void or_render_bwd(int W, int H, int P_gauss, const int* ranges, const int* point_list, const float* points_xy,
                   const float* features, const float* depths, const float* conic_opacity, const float* bg,
                   const float* out_alpha, const int* n_contrib, const float* grad_color, const float* grad_depth,
                   const float* grad_alpha, int compute_depth, int value_mode, float* grad_out, double* grad_out64,
                   double* err_out, double* mag_out) {
  const int grid_x = (W + BLOCK_X - 1) / BLOCK_X;
  const long long total = (long long)W * H;
  const float ddelx_dx = 0.5f * (float)W;
  const float ddely_dy = 0.5f * (float)H;
  const int bound = err_out != NULL && mag_out != NULL;
  const double u = ldexp(1.0, -24);
  int nthreads = 1;
#ifdef _OPENMP
  nthreads = omp_get_max_threads();
#endif
  const size_t per_thread = (size_t)P_gauss * 10;
  const int nbuf = bound ? 3 : 1;
  double* acc = (double*)calloc((size_t)nthreads * per_thread * (size_t)nbuf, sizeof(double));
#pragma omp parallel
  {
    int tid = 0;
#ifdef _OPENMP
    tid = omp_get_thread_num();
#endif
    double* my = acc + (size_t)tid * per_thread * (size_t)nbuf;
    double* my_err = bound ? my + per_thread : NULL;
    double* my_mag = bound ? my + 2 * per_thread : NULL;
#pragma omp for schedule(dynamic, 64)
    for (long long pixel_id = 0; pixel_id < total; ++pixel_id) {
      const int pix_x = (int)(pixel_id % W), pix_y = (int)(pixel_id / W);
      const int tile_id = (pix_y / BLOCK_Y) * grid_x + pix_x / BLOCK_X;
      const int start = ranges[2 * tile_id], end = ranges[2 * tile_id + 1];
      if (end - start <= 0) continue;
      const int last_contributor = n_contrib[pixel_id];
      const float T_final = 1.0f - out_alpha[pixel_id];
      float T = T_final;
      const float pixf_x = (float)pix_x, pixf_y = (float)pix_y;
      const float g0 = grad_color[pixel_id], g1 = grad_color[total + pixel_id], g2 = grad_color[2 * total + pixel_id];
      const float gd = compute_depth ? grad_depth[pixel_id] : 0.0f;
      const float ga = grad_alpha[pixel_id];
      const float bg_dot = bg[0] * g0 + bg[1] * g1 + bg[2] * g2;
      float ar0 = 0.0f, ar1 = 0.0f, ar2 = 0.0f, adr = 0.0f, aar = 0.0f;
      float last_alpha = 0.0f, lc0 = 0.0f, lc1 = 0.0f, lc2 = 0.0f, last_depth = 0.0f;
      /* running bound state: relative error of T, error and magnitude of S */
      double rel_T = 0.0;
      double m_S = fabs((double)bg[0] * g0) + fabs((double)bg[1] * g1) + fabs((double)bg[2] * g2);
      double e_S = 3.0 * u * m_S;
      /* value_mode 1 / 2 state: T and S = U . acc (background included) */
      double xT = T_final, xS = (double)bg[0] * g0 + (double)bg[1] * g1 + (double)bg[2] * g2;
      float yT = T_final, yS = fmaf(bg[2], g2, fmaf(bg[1], g1, bg[0] * g0));
      for (int pos = last_contributor - 1; pos >= 0; --pos) {
        const int id = point_list[start + pos];
        const float* co = conic_opacity + 4 * id;
        const float d_x = points_xy[2 * id] - pixf_x;
        const float d_y = points_xy[2 * id + 1] - pixf_y;
        const float power = blend_power(co, d_x, d_y);
        if (!(power <= 0.0f)) continue;
        const float G = or_exp(power);
        const float alpha = fmin_(0.99f, co[3] * or_exp(power));
        if (!(alpha >= (1.0f / 255.0f))) continue;
        const float one_minus_alpha = fmax_(1.0f - alpha, ONE_MINUS_ALPHA_MIN);
        T = T / one_minus_alpha;
        const float dchannel_dcolor = alpha * T;
        const float* f = features + 3 * id;
        ar0 = last_alpha * lc0 + (1.0f - last_alpha) * ar0;
        ar1 = last_alpha * lc1 + (1.0f - last_alpha) * ar1;
        ar2 = last_alpha * lc2 + (1.0f - last_alpha) * ar2;
        lc0 = f[0];
        lc1 = f[1];
        lc2 = f[2];
        float dL_dopa = (f[0] - ar0) * g0 + (f[1] - ar1) * g1 + (f[2] - ar2) * g2;
        double* gg = my + (size_t)id * 10;
        if (compute_depth) {
          const float dv = depths[id];
          adr = last_alpha * last_depth + (1.0f - last_alpha) * adr;
          last_depth = dv;
          dL_dopa = dL_dopa + (dv - adr) * gd;
        }
        aar = last_alpha + (1.0f - last_alpha) * aar;
        dL_dopa = dL_dopa + (1.0f - aar) * ga;
        dL_dopa = dL_dopa * T;
        last_alpha = alpha;
        dL_dopa = dL_dopa + (-T_final / one_minus_alpha) * bg_dot;
        if (value_mode == 0) {
          gg[6] += (double)(dchannel_dcolor * g0);
          gg[7] += (double)(dchannel_dcolor * g1);
          gg[8] += (double)(dchannel_dcolor * g2);
          if (compute_depth) gg[9] += (double)(dchannel_dcolor * gd);
          const float dL_dG = co[3] * dL_dopa;
          const float gdx = G * d_x, gdy = G * d_y;
          const float dG_ddelx = -gdx * co[0] - gdy * co[1];
          const float dG_ddely = -gdy * co[2] - gdx * co[1];
          gg[0] += (double)(dL_dG * dG_ddelx * ddelx_dx);
          gg[1] += (double)(dL_dG * dG_ddely * ddely_dy);
          gg[2] += (double)(-0.5f * gdx * d_x * dL_dG);
          gg[3] += (double)(-0.5f * gdx * d_y * dL_dG);
          gg[4] += (double)(-0.5f * gdy * d_y * dL_dG);
          gg[5] += (double)(G * dL_dopa);
        } else if (value_mode == 1) {
          /* the same quantities in double: G, alpha, T and the reverse
           * recurrences from the fp32 inputs */
          const double Gd = exp((double)power);
          const double ad = fmin(0.99, (double)co[3] * Gd);
          const double omd = fmax(1.0 - ad, (double)ONE_MINUS_ALPHA_MIN);
          xT = xT / omd;
          const double U[5] = {g0, g1, g2, gd, ga};
          const double F[5] = {f[0], f[1], f[2], compute_depth ? depths[id] : 0.0, 1.0};
          double fu = 0.0;
          for (int c = 0; c < 5; ++c) fu += F[c] * U[c];
          const double dopa = xT * (fu - xS);
          const double v = Gd * dopa;
          const double dxd = d_x, dyd = d_y;
          gg[0] += -(double)ddelx_dx * co[3] * v * (co[0] * dxd + co[1] * dyd);
          gg[1] += -(double)ddely_dy * co[3] * v * (co[2] * dyd + co[1] * dxd);
          gg[2] += -0.5 * co[3] * v * dxd * dxd;
          gg[3] += -0.5 * co[3] * v * dxd * dyd;
          gg[4] += -0.5 * co[3] * v * dyd * dyd;
          gg[5] += v;
          for (int c = 0; c < (compute_depth ? 4 : 3); ++c) gg[6 + c] += ad * xT * U[c];
          xS = xS + ad * (fu - xS);
        } else {
          /* a second fp32 order */
          const float Gf = exp2f(-2.0f * power * (-0.5f * 1.44269504088896341f));
          const float af = fmin_(0.99f, co[3] * Gf);
          const float omf = 1.0f - af;
          yT = yT * (1.0f / omf);
          float fu = fmaf(f[2], g2, fmaf(f[1], g1, fmaf(f[0], g0, ga)));
          if (compute_depth) fu = fmaf(depths[id], gd, fu);
          const float dd = fu - yS;
          const float v = Gf * (yT * dd);
          const float vdx = v * d_x, vdy = v * d_y;
          const float o = co[3];
          gg[0] += (double)(-ddelx_dx * o * (co[0] * vdx + co[1] * vdy));
          gg[1] += (double)(-ddely_dy * o * (co[2] * vdy + co[1] * vdx));
          gg[2] += (double)(-0.5f * o * (vdx * d_x));
          gg[3] += (double)(-0.5f * o * (vdx * d_y));
          gg[4] += (double)(-0.5f * o * fmaf(vdy, d_y, 0.0f));
          gg[5] += (double)v;
          const float dch = af * yT;
          gg[6] += (double)(dch * g0);
          gg[7] += (double)(dch * g1);
          gg[8] += (double)(dch * g2);
          if (compute_depth) gg[9] += (double)(dch * gd);
          yS = fmaf(af, dd, yS);
        }
        if (bound) {
          const double q = -2.0 * (double)power;
          const double a = alpha, o = co[3];
          const double rel_G = (0.75 * q + 3.0) * u;
          /* both evaluations are capped when o G clears 0.99 by more than their error */
          const int capped = (double)co[3] * (double)G > 0.99 * (1.0 + 2.0 * rel_G + 2.0 * u);
          const double rel_a = capped ? 0.0 : rel_G + u;
          const double rel_om = a * rel_a / (1.0 - a) + u;
          rel_T += rel_om + 2.0 * u;
          const double Tn = T;
          double M_fu = fabs((double)f[0] * g0) + fabs((double)f[1] * g1) + fabs((double)f[2] * g2) + fabs((double)ga);
          if (compute_depth) M_fu += fabs((double)depths[id] * gd);
          const double e_fu = 5.0 * u * M_fu;
          const double v = (double)G * (double)dL_dopa;
          const double e_v = (double)G * Tn * (e_fu + e_S + u * (M_fu + m_S)) + fabs(v) * (rel_G + rel_T + 2.0 * u);
          const double av = fabs(v);
          const double adx = fabs((double)d_x), ady = fabs((double)d_y);
          const double fac[6] = {
              (double)ddelx_dx * o * (fabs((double)co[0]) * adx + fabs((double)co[1]) * ady),
              (double)ddely_dy * o * (fabs((double)co[2]) * ady + fabs((double)co[1]) * adx),
              0.5 * o * adx * adx,
              0.5 * o * adx * ady,
              0.5 * o * ady * ady,
              1.0,
          };
          double* ge = my_err + (size_t)id * 10;
          double* gm = my_mag + (size_t)id * 10;
          for (int k = 0; k < 6; ++k) {
            ge[k] += fac[k] * e_v + 4.0 * u * fac[k] * av;
            gm[k] += fac[k] * av;
          }
          const double rel_c = rel_a + rel_T + 2.0 * u;
          const double up[4] = {g0, g1, g2, gd};
          for (int k = 0; k < (compute_depth ? 4 : 3); ++k) {
            const double t = fabs(a * Tn * up[k]);
            ge[6 + k] += t * rel_c;
            gm[6 + k] += t;
          }
          /* this Gaussian joins what lies behind the next one */
          e_S = (1.0 - a) * e_S + a * e_fu + a * rel_a * (M_fu + m_S) + 4.0 * u * (M_fu + m_S);
          m_S = (1.0 - a) * m_S + a * M_fu;
        }
      }
    }
  }
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < (long long)per_thread; ++i) {
    double s = 0.0, se = 0.0, sm = 0.0;
    for (int t = 0; t < nthreads; ++t) {
      const double* base = acc + (size_t)t * per_thread * (size_t)nbuf;
      s += base[i];
      if (bound) {
        se += base[per_thread + (size_t)i];
        sm += base[2 * per_thread + (size_t)i];
      }
    }
    grad_out[i] = (float)s;
    if (grad_out64) grad_out64[i] = s;
    if (bound) {
      err_out[i] = se;
      mag_out[i] = sm;
    }
  }
  free(acc);
}

/*
 * SH backward (backward_kernels.py:298-398 for degree >= 2, 401-536 for
 * degree <= 1; identical mathematics) + fused preprocess backward
 * (backward_kernels.py:53-295) with the flow prep (flow_kernels.py:14-28,
 * flow_ops.py:337-360) when flow_double != 0.  cov3d is the forward's
 * stored cov3D (N,6).  grad_sh has the input's (N,K,3) shape, zero beyond
 * the evaluated bands (backward_ops.py:94, 123).
 */
void or_preprocess_bwd(int P, int K, int degree, const float* means3d, const float* scales, const float* rotations,
                       float scale_modifier, const float* cov3d, const float* shs, const float* campos,
                       const int* clamped, const float* V, const float* Pm, float tanfovx, float tanfovy,
                       float focal_x, float focal_y, const int* radii, const float* grad_gauss,
                       const float* grad_proj_2d, const float* grad_conic_2d, const float* grad_conic_2d_inv,
                       int flow_double, int cov3d_is_precomp, float filter_variance, float* grad_means3d,
                       float* grad_means2d,
                       float* grad_scales, float* grad_rotations, float* grad_cov3d, float* grad_sh) {
#pragma omp parallel for schedule(static)
  for (int tid = 0; tid < P; ++tid) {
    const float* mean = means3d + 3 * tid;
    const int rad = radii[tid];
    const float* gg = grad_gauss + 10 * (size_t)tid;
    /* SH backward */
    float gsm0 = 0.0f, gsm1 = 0.0f, gsm2 = 0.0f;
    int has_sh = shs != NULL;
    if (has_sh) {
      const float* sh = shs + (size_t)tid * (size_t)(3 * K);
      float* gsh = grad_sh + (size_t)tid * (size_t)(3 * K);
      for (int k = 0; k < 3 * K; ++k) gsh[k] = 0.0f;
      const float d0 = mean[0] - campos[0], d1 = mean[1] - campos[1], d2 = mean[2] - campos[2];
      const float len_sq = d0 * d0 + d1 * d1 + d2 * d2;
      const float inv_len = 1.0f / sqrtf(fmax_(len_sq, 1.0e-20f));
      const float x = d0 * inv_len, y = d1 * inv_len, z = d2 * inv_len;
      float g[3];
      for (int c = 0; c < 3; ++c) g[c] = gg[6 + c] * (1.0f - (float)clamped[3 * tid + c]);
      float ax[3] = {0, 0, 0}, ay[3] = {0, 0, 0}, az[3] = {0, 0, 0};
      if (K > 0)
        for (int c = 0; c < 3; ++c) gsh[c] = SH_C0 * g[c];
      if (degree > 0 && K > 3) {
        const float w1 = -SH_C1 * y, w2 = SH_C1 * z, w3 = -SH_C1 * x;
        for (int c = 0; c < 3; ++c) {
          gsh[3 + c] = w1 * g[c];
          gsh[6 + c] = w2 * g[c];
          gsh[9 + c] = w3 * g[c];
          ax[c] = (-SH_C1) * sh[9 + c];
          ay[c] = (-SH_C1) * sh[3 + c];
          az[c] = SH_C1 * sh[6 + c];
        }
        if (degree > 1 && K > 8) {
          const float xx = x * x, yy = y * y, zz = z * z, xy = x * y, yz = y * z, xz = x * z;
          const float w[5] = {SH_C2_0 * xy, SH_C2_1 * yz, SH_C2_2 * (2.0f * zz - xx - yy), SH_C2_3 * xz,
                              SH_C2_4 * (xx - yy)};
          for (int k = 0; k < 5; ++k)
            for (int c = 0; c < 3; ++c) gsh[3 * (4 + k) + c] = w[k] * g[c];
          for (int c = 0; c < 3; ++c) {
            const float* s = sh + c;
            ax[c] = ax[c] + (SH_C2_0 * y) * s[12] + (SH_C2_2 * (-2.0f * x)) * s[18] + (SH_C2_3 * z) * s[21] +
                    (SH_C2_4 * (2.0f * x)) * s[24];
            ay[c] = ay[c] + (SH_C2_0 * x) * s[12] + (SH_C2_1 * z) * s[15] + (SH_C2_2 * (-2.0f * y)) * s[18] +
                    (SH_C2_4 * (-2.0f * y)) * s[24];
            az[c] = az[c] + (SH_C2_1 * y) * s[15] + (SH_C2_2 * (4.0f * z)) * s[18] + (SH_C2_3 * x) * s[21];
          }
          if (degree > 2 && K > 15) {
            const float v[7] = {SH_C3_0 * y * (3.0f * xx - yy),
                                SH_C3_1 * xy * z,
                                SH_C3_2 * y * (4.0f * zz - xx - yy),
                                SH_C3_3 * z * (2.0f * zz - 3.0f * xx - 3.0f * yy),
                                SH_C3_4 * x * (4.0f * zz - xx - yy),
                                SH_C3_5 * z * (xx - yy),
                                SH_C3_6 * x * (xx - 3.0f * yy)};
            for (int k = 0; k < 7; ++k)
              for (int c = 0; c < 3; ++c) gsh[3 * (9 + k) + c] = v[k] * g[c];
            for (int c = 0; c < 3; ++c) {
              const float* s = sh + c;
              ax[c] = ax[c] + (SH_C3_0 * (6.0f * xy)) * s[27] + (SH_C3_1 * yz) * s[30] +
                      (SH_C3_2 * (-2.0f * xy)) * s[33] + (SH_C3_3 * (-6.0f * xz)) * s[36] +
                      (SH_C3_4 * (-3.0f * xx + 4.0f * zz - yy)) * s[39] + (SH_C3_5 * (2.0f * xz)) * s[42] +
                      (SH_C3_6 * (3.0f * (xx - yy))) * s[45];
              ay[c] = ay[c] + (SH_C3_0 * (3.0f * (xx - yy))) * s[27] + (SH_C3_1 * xz) * s[30] +
                      (SH_C3_2 * (-3.0f * yy + 4.0f * zz - xx)) * s[33] + (SH_C3_3 * (-6.0f * yz)) * s[36] +
                      (SH_C3_4 * (-2.0f * xy)) * s[39] + (SH_C3_5 * (-2.0f * yz)) * s[42] +
                      (SH_C3_6 * (-6.0f * xy)) * s[45];
              az[c] = az[c] + (SH_C3_1 * xy) * s[30] + (SH_C3_2 * (8.0f * yz)) * s[33] +
                      (SH_C3_3 * (3.0f * (2.0f * zz - xx - yy))) * s[36] + (SH_C3_4 * (8.0f * xz)) * s[39] +
                      (SH_C3_5 * (xx - yy)) * s[42];
            }
          }
        }
      }
      const float dd0 = ax[0] * g[0] + ax[1] * g[1] + ax[2] * g[2];
      const float dd1 = ay[0] * g[0] + ay[1] * g[1] + ay[2] * g[2];
      const float dd2 = az[0] * g[0] + az[1] * g[1] + az[2] * g[2];
      /* math_kernels.py:90-97 */
      const float sum2 = d0 * d0 + d1 * d1 + d2 * d2;
      const float invsum32 = 1.0f / sqrtf(fmax_(sum2 * sum2 * sum2, 1.0e-20f));
      gsm0 = ((sum2 - d0 * d0) * dd0 - d1 * d0 * dd1 - d2 * d0 * dd2) * invsum32;
      gsm1 = (-d0 * d1 * dd0 + (sum2 - d1 * d1) * dd1 - d2 * d1 * dd2) * invsum32;
      gsm2 = (-d0 * d2 * dd0 - d1 * d2 * dd1 + (sum2 - d2 * d2) * dd2) * invsum32;
    }
    if (cov3d_is_precomp) {
      /* non-fused chain for precomputed covariances (backward_ops.py:679-744):
       * projected means (backward_kernels.py:838-870), cov2D -> cov3D (backward_kernels.py:710-836) */
      const float hx = Pm[0] * mean[0] + Pm[4] * mean[1] + Pm[8] * mean[2] + Pm[12];
      const float hy = Pm[1] * mean[0] + Pm[5] * mean[1] + Pm[9] * mean[2] + Pm[13];
      const float hw = Pm[3] * mean[0] + Pm[7] * mean[1] + Pm[11] * mean[2] + Pm[15];
      const float iw = 1.0f / (hw + 0.0000001f);
      const float mul1 = hx * iw * iw, mul2 = hy * iw * iw;
      float gxy0 = gg[0], gxy1 = gg[1];
      if (rad > 0) {
        float ax = grad_proj_2d[2 * tid], ay = grad_proj_2d[2 * tid + 1];
        if (flow_double) {
          ax = ax + gg[0];
          ay = ay + gg[1];
        }
        gxy0 = gxy0 + ax;
        gxy1 = gxy1 + ay;
      }
      float ox = (Pm[0] * iw - Pm[3] * mul1) * gxy0 + (Pm[1] * iw - Pm[3] * mul2) * gxy1;
      float oy = (Pm[4] * iw - Pm[7] * mul1) * gxy0 + (Pm[5] * iw - Pm[7] * mul2) * gxy1;
      float oz = (Pm[8] * iw - Pm[11] * mul1) * gxy0 + (Pm[9] * iw - Pm[11] * mul2) * gxy1;
      const float mul3 = V[2] * mean[0] + V[6] * mean[1] + V[10] * mean[2] + V[14];
      ox = ox + (V[2] - V[3] * mul3) * gg[9];
      oy = oy + (V[6] - V[7] * mul3) * gg[9];
      oz = oz + (V[10] - V[11] * mul3) * gg[9];
      float cm0 = 0.0f, cm1 = 0.0f, cm2 = 0.0f;
      float* gcv = grad_cov3d + 6 * tid;
      for (int k = 0; k < 6; ++k) gcv[k] = 0.0f;
      if (rad > 0) {
        float x = V[0] * mean[0] + V[4] * mean[1] + V[8] * mean[2] + V[12];
        float y = V[1] * mean[0] + V[5] * mean[1] + V[9] * mean[2] + V[13];
        const float z = V[2] * mean[0] + V[6] * mean[1] + V[10] * mean[2] + V[14];
        const float limx = 1.3f * tanfovx, limy = 1.3f * tanfovy;
        const float txtz = x / z, tytz = y / z;
        const float tx = clamp_(txtz, -limx, limx) * z, ty = clamp_(tytz, -limy, limy) * z;
        const float xm = (txtz < -limx || txtz > limx) ? 0.0f : 1.0f;
        const float ym = (tytz < -limy || tytz > limy) ? 0.0f : 1.0f;
        const float j00 = focal_x / z, j02 = -(focal_x * tx) / (z * z);
        const float j11 = focal_y / z, j12 = -(focal_y * ty) / (z * z);
        const float w00 = V[0], w01 = V[1], w02 = V[2], w10 = V[4], w11 = V[5], w12 = V[6], w20 = V[8],
                    w21 = V[9], w22 = V[10];
        const float t00 = w00 * j00 + w02 * j02, t10 = w10 * j00 + w12 * j02, t20 = w20 * j00 + w22 * j02;
        const float t01 = w01 * j11 + w02 * j12, t11 = w11 * j11 + w12 * j12, t21 = w21 * j11 + w22 * j12;
        const float* cv = cov3d + 6 * tid;
        const float v00 = cv[0], v01 = cv[1], v02 = cv[2], v11 = cv[3], v12 = cv[4], v22 = cv[5];
        const float vt0x = v00 * t00 + v01 * t10 + v02 * t20;
        const float vt0y = v01 * t00 + v11 * t10 + v12 * t20;
        const float vt0z = v02 * t00 + v12 * t10 + v22 * t20;
        const float vt1x = v00 * t01 + v01 * t11 + v02 * t21;
        const float vt1y = v01 * t01 + v11 * t11 + v12 * t21;
        const float vt1z = v02 * t01 + v12 * t11 + v22 * t21;
        const float a = t00 * vt0x + t10 * vt0y + t20 * vt0z + 0.3f + filter_variance;
        const float b = t00 * vt1x + t10 * vt1y + t20 * vt1z;
        const float c = t01 * vt1x + t11 * vt1y + t21 * vt1z + 0.3f + filter_variance;
        const float denom = a * c - b * b;
        const float denom2inv = 1.0f / (denom * denom + 1.0e-7f);
        float u0 = grad_conic_2d[3 * tid], u1 = grad_conic_2d[3 * tid + 1], u2 = grad_conic_2d[3 * tid + 2];
        if (flow_double) {
          u0 = u0 + gg[2];
          u1 = u1 + gg[3];
          u2 = u2 + gg[4];
        }
        const float tc0 = gg[2] + u0, tc1 = gg[3] + u1, tc2 = gg[4] + u2;
        float dL_da = denom2inv * (-c * c * tc0 + 2.0f * b * c * tc1 + (denom - a * c) * tc2);
        float dL_dc = denom2inv * (-a * a * tc2 + 2.0f * a * b * tc1 + (denom - a * c) * tc0);
        float dL_db = denom2inv * 2.0f * (b * c * tc0 - (denom + 2.0f * b * b) * tc1 + a * b * tc2);
        dL_da = dL_da + grad_conic_2d_inv[3 * tid];
        dL_db = dL_db + grad_conic_2d_inv[3 * tid + 1];
        dL_dc = dL_dc + grad_conic_2d_inv[3 * tid + 2];
        gcv[0] = t00 * t00 * dL_da + t00 * t01 * dL_db + t01 * t01 * dL_dc;
        gcv[3] = t10 * t10 * dL_da + t10 * t11 * dL_db + t11 * t11 * dL_dc;
        gcv[5] = t20 * t20 * dL_da + t20 * t21 * dL_db + t21 * t21 * dL_dc;
        gcv[1] = 2.0f * t00 * t10 * dL_da + (t00 * t11 + t01 * t10) * dL_db + 2.0f * t01 * t11 * dL_dc;
        gcv[2] = 2.0f * t00 * t20 * dL_da + (t00 * t21 + t01 * t20) * dL_db + 2.0f * t01 * t21 * dL_dc;
        gcv[4] = 2.0f * t10 * t20 * dL_da + (t10 * t21 + t11 * t20) * dL_db + 2.0f * t11 * t21 * dL_dc;
        const float dT00 = 2.0f * (t00 * v00 + t10 * v01 + t20 * v02) * dL_da + (t01 * v00 + t11 * v01 + t21 * v02) * dL_db;
        const float dT01 = 2.0f * (t00 * v01 + t10 * v11 + t20 * v12) * dL_da + (t01 * v01 + t11 * v11 + t21 * v12) * dL_db;
        const float dT02 = 2.0f * (t00 * v02 + t10 * v12 + t20 * v22) * dL_da + (t01 * v02 + t11 * v12 + t21 * v22) * dL_db;
        const float dT10 = 2.0f * (t01 * v00 + t11 * v01 + t21 * v02) * dL_dc + (t00 * v00 + t10 * v01 + t20 * v02) * dL_db;
        const float dT11 = 2.0f * (t01 * v01 + t11 * v11 + t21 * v12) * dL_dc + (t00 * v01 + t10 * v11 + t20 * v12) * dL_db;
        const float dT12 = 2.0f * (t01 * v02 + t11 * v12 + t21 * v22) * dL_dc + (t00 * v02 + t10 * v12 + t20 * v22) * dL_db;
        const float dJ00 = w00 * dT00 + w10 * dT01 + w20 * dT02;
        const float dJ02 = w02 * dT00 + w12 * dT01 + w22 * dT02;
        const float dJ11 = w01 * dT10 + w11 * dT11 + w21 * dT12;
        const float dJ12 = w02 * dT10 + w12 * dT11 + w22 * dT12;
        const float tz_inv = 1.0f / z;
        const float tz2 = tz_inv * tz_inv, tz3 = tz2 * tz_inv;
        const float dtx = xm * -focal_x * tz2 * dJ02;
        const float dty = ym * -focal_y * tz2 * dJ12;
        const float dtz = -focal_x * tz2 * dJ00 - focal_y * tz2 * dJ11 + (2.0f * focal_x * tx) * tz3 * dJ02 +
                          (2.0f * focal_y * ty) * tz3 * dJ12;
        cm0 = V[0] * dtx + V[1] * dty + V[2] * dtz;
        cm1 = V[4] * dtx + V[5] * dty + V[6] * dtz;
        cm2 = V[8] * dtx + V[9] * dty + V[10] * dtz;
      }
      /* accumulation (backward_kernels.py:289-295 order: projected + cov + sh) */
      float a0 = ox + cm0, a1 = oy + cm1, a2 = oz + cm2;
      if (has_sh) {
        a0 = a0 + gsm0;
        a1 = a1 + gsm1;
        a2 = a2 + gsm2;
      }
      grad_means3d[3 * tid] = a0;
      grad_means3d[3 * tid + 1] = a1;
      grad_means3d[3 * tid + 2] = a2;
      grad_means2d[3 * tid] = gg[0];
      grad_means2d[3 * tid + 1] = gg[1];
      grad_means2d[3 * tid + 2] = 0.0f;
      continue;
    }
    /* Part A */
    const float hom_x = Pm[0] * mean[0] + Pm[4] * mean[1] + Pm[8] * mean[2] + Pm[12];
    const float hom_y = Pm[1] * mean[0] + Pm[5] * mean[1] + Pm[9] * mean[2] + Pm[13];
    const float hom_w = Pm[3] * mean[0] + Pm[7] * mean[1] + Pm[11] * mean[2] + Pm[15];
    const float inv_w = 1.0f / (hom_w + 0.0000001f);
    float gx = gg[0], gy = gg[1];
    const float inv_w2 = inv_w * inv_w;
    if (rad > 0) {
      float ax = grad_proj_2d[2 * tid], ay = grad_proj_2d[2 * tid + 1];
      if (flow_double) {
        ax = ax + gg[0];
        ay = ay + gg[1];
      }
      gx = gx + ax;
      gy = gy + ay;
    }
    const float gh = hom_x * gx + hom_y * gy;
    float pm_x = inv_w * (Pm[0] * gx + Pm[1] * gy) - Pm[3] * inv_w2 * gh;
    float pm_y = inv_w * (Pm[4] * gx + Pm[5] * gy) - Pm[7] * inv_w2 * gh;
    float pm_z = inv_w * (Pm[8] * gx + Pm[9] * gy) - Pm[11] * inv_w2 * gh;
    const float zz0 = V[2] * mean[0] + V[6] * mean[1] + V[10] * mean[2] + V[14];
    const float depth_grad = gg[9];
    pm_x = pm_x + (V[2] - V[3] * zz0) * depth_grad;
    pm_y = pm_y + (V[6] - V[7] * zz0) * depth_grad;
    pm_z = pm_z + (V[10] - V[11] * zz0) * depth_grad;
    /* Part B */
    float gc_x = 0.0f, gc_y = 0.0f, gc_z = 0.0f;
    float* gs = grad_scales + 3 * tid;
    float* gq = grad_rotations + 4 * tid;
    if (rad <= 0) {
      gs[0] = gs[1] = gs[2] = 0.0f;
      gq[0] = gq[1] = gq[2] = gq[3] = 0.0f;
    } else {
      const float x = V[0] * mean[0] + V[4] * mean[1] + V[8] * mean[2] + V[12];
      const float y = V[1] * mean[0] + V[5] * mean[1] + V[9] * mean[2] + V[13];
      const float z = V[2] * mean[0] + V[6] * mean[1] + V[10] * mean[2] + V[14];
      const float tz_inv = 1.0f / (z + 1.0e-7f);
      const float limx = 1.3f * tanfovx, limy = 1.3f * tanfovy;
      const float txtz = x * tz_inv, tytz = y * tz_inv;
      const float x_grad_mul = (txtz < -limx || txtz > limx) ? 0.0f : 1.0f;
      const float y_grad_mul = (tytz < -limy || tytz > limy) ? 0.0f : 1.0f;
      const float tx = clamp_(txtz, -limx, limx), ty = clamp_(tytz, -limy, limy);
      const float j00 = focal_x * tz_inv, j02 = -j00 * tx, j11 = focal_y * tz_inv, j12 = -j11 * ty;
      const float w00 = V[0], w01 = V[1], w02 = V[2], w10 = V[4], w11 = V[5], w12 = V[6], w20 = V[8], w21 = V[9],
                  w22 = V[10];
      const float t00 = w00 * j00 + w02 * j02, t10 = w10 * j00 + w12 * j02, t20 = w20 * j00 + w22 * j02;
      const float t01 = w01 * j11 + w02 * j12, t11 = w11 * j11 + w12 * j12, t21 = w21 * j11 + w22 * j12;
      const float* cv = cov3d + 6 * tid;
      const float v00 = cv[0], v01 = cv[1], v02 = cv[2], v11 = cv[3], v12 = cv[4], v22 = cv[5];
      const float vt0x = v00 * t00 + v01 * t10 + v02 * t20;
      const float vt0y = v01 * t00 + v11 * t10 + v12 * t20;
      const float vt0z = v02 * t00 + v12 * t10 + v22 * t20;
      const float vt1x = v00 * t01 + v01 * t11 + v02 * t21;
      const float vt1y = v01 * t01 + v11 * t11 + v12 * t21;
      const float vt1z = v02 * t01 + v12 * t11 + v22 * t21;
      const float aa = t00 * vt0x + t10 * vt0y + t20 * vt0z + 0.3f + filter_variance;
      const float bb = t00 * vt1x + t10 * vt1y + t20 * vt1z;
      const float cc = t01 * vt1x + t11 * vt1y + t21 * vt1z + 0.3f + filter_variance;
      const float denom = aa * cc - bb * bb;
      const float denom2inv = 1.0f / (denom * denom + 1.0e-7f);
      float u0 = grad_conic_2d[3 * tid], u1 = grad_conic_2d[3 * tid + 1], u2 = grad_conic_2d[3 * tid + 2];
      if (flow_double) {
        u0 = u0 + gg[2];
        u1 = u1 + gg[3];
        u2 = u2 + gg[4];
      }
      const float tc0 = gg[2] + u0, tc1 = gg[3] + u1, tc2 = gg[4] + u2;
      float dL_da = denom2inv * (-cc * cc * tc0 + 2.0f * bb * cc * tc1 - bb * bb * tc2);
      float dL_dc = denom2inv * (-aa * aa * tc2 + 2.0f * aa * bb * tc1 - bb * bb * tc0);
      float dL_db = denom2inv * 2.0f * (bb * cc * tc0 - (aa * cc + bb * bb) * tc1 + aa * bb * tc2);
      dL_da = dL_da + grad_conic_2d_inv[3 * tid];
      dL_db = dL_db + grad_conic_2d_inv[3 * tid + 1];
      dL_dc = dL_dc + grad_conic_2d_inv[3 * tid + 2];
      const float gc0 = t00 * t00 * dL_da + t00 * t01 * dL_db + t01 * t01 * dL_dc;
      const float gc3 = t10 * t10 * dL_da + t10 * t11 * dL_db + t11 * t11 * dL_dc;
      const float gc5 = t20 * t20 * dL_da + t20 * t21 * dL_db + t21 * t21 * dL_dc;
      const float gc1 = 2.0f * t00 * t10 * dL_da + (t00 * t11 + t01 * t10) * dL_db + 2.0f * t01 * t11 * dL_dc;
      const float gc2 = 2.0f * t00 * t20 * dL_da + (t00 * t21 + t01 * t20) * dL_db + 2.0f * t01 * t21 * dL_dc;
      const float gc4 = 2.0f * t10 * t20 * dL_da + (t10 * t21 + t11 * t20) * dL_db + 2.0f * t11 * t21 * dL_dc;
      const float dT00 = 2.0f * vt0x * dL_da + vt1x * dL_db, dT01 = 2.0f * vt0y * dL_da + vt1y * dL_db,
                  dT02 = 2.0f * vt0z * dL_da + vt1z * dL_db;
      const float dT10 = vt0x * dL_db + 2.0f * vt1x * dL_dc, dT11 = vt0y * dL_db + 2.0f * vt1y * dL_dc,
                  dT12 = vt0z * dL_db + 2.0f * vt1z * dL_dc;
      const float dJ00 = w00 * dT00 + w10 * dT01 + w20 * dT02;
      const float dJ02 = w02 * dT00 + w12 * dT01 + w22 * dT02;
      const float dJ11 = w01 * dT10 + w11 * dT11 + w21 * dT12;
      const float dJ12 = w02 * dT10 + w12 * dT11 + w22 * dT12;
      const float dtx = x_grad_mul * -j00 * tz_inv * dJ02;
      const float dty = y_grad_mul * -j11 * tz_inv * dJ12;
      const float dtz = -(j00 * dJ00 + j11 * dJ11 + 2.0f * j02 * dJ02 + 2.0f * j12 * dJ12) * tz_inv;
      gc_x = w00 * dtx + w01 * dty + w02 * dtz;
      gc_y = w10 * dtx + w11 * dty + w12 * dtz;
      gc_z = w20 * dtx + w21 * dty + w22 * dtz;
      const float ss0 = scales[3 * tid] * scale_modifier, ss1 = scales[3 * tid + 1] * scale_modifier,
                  ss2 = scales[3 * tid + 2] * scale_modifier;
      const float rr = rotations[4 * tid], xq = rotations[4 * tid + 1], yq = rotations[4 * tid + 2],
                  zq = rotations[4 * tid + 3];
      const float r00 = 1.0f - 2.0f * (yq * yq + zq * zq), r01 = 2.0f * (xq * yq + rr * zq),
                  r02 = 2.0f * (xq * zq - rr * yq);
      const float r10 = 2.0f * (xq * yq - rr * zq), r11 = 1.0f - 2.0f * (xq * xq + zq * zq),
                  r12 = 2.0f * (yq * zq + rr * xq);
      const float r20 = 2.0f * (xq * zq + rr * yq), r21 = 2.0f * (yq * zq - rr * xq),
                  r22 = 1.0f - 2.0f * (xq * xq + yq * yq);
      const float m00 = ss0 * r00, m01 = ss0 * r01, m02 = ss0 * r02, m10 = ss1 * r10, m11 = ss1 * r11,
                  m12 = ss1 * r12, m20 = ss2 * r20, m21 = ss2 * r21, m22 = ss2 * r22;
      const float s00 = gc0, s01 = 0.5f * gc1, s02 = 0.5f * gc2, s11 = gc3, s12 = 0.5f * gc4, s22 = gc5;
      const float dM00 = 2.0f * (m00 * s00 + m01 * s01 + m02 * s02);
      const float dM01 = 2.0f * (m00 * s01 + m01 * s11 + m02 * s12);
      const float dM02 = 2.0f * (m00 * s02 + m01 * s12 + m02 * s22);
      const float dM10 = 2.0f * (m10 * s00 + m11 * s01 + m12 * s02);
      const float dM11 = 2.0f * (m10 * s01 + m11 * s11 + m12 * s12);
      const float dM12 = 2.0f * (m10 * s02 + m11 * s12 + m12 * s22);
      const float dM20 = 2.0f * (m20 * s00 + m21 * s01 + m22 * s02);
      const float dM21 = 2.0f * (m20 * s01 + m21 * s11 + m22 * s12);
      const float dM22 = 2.0f * (m20 * s02 + m21 * s12 + m22 * s22);
      gs[0] = scale_modifier * (dM00 * r00 + dM01 * r01 + dM02 * r02);
      gs[1] = scale_modifier * (dM10 * r10 + dM11 * r11 + dM12 * r12);
      gs[2] = scale_modifier * (dM20 * r20 + dM21 * r21 + dM22 * r22);
      const float dR00 = dM00 * ss0, dR01 = dM01 * ss0, dR02 = dM02 * ss0;
      const float dR10 = dM10 * ss1, dR11 = dM11 * ss1, dR12 = dM12 * ss1;
      const float dR20 = dM20 * ss2, dR21 = dM21 * ss2, dR22 = dM22 * ss2;
      gq[0] = 2.0f * zq * (dR01 - dR10) + 2.0f * yq * (dR20 - dR02) + 2.0f * xq * (dR12 - dR21);
      gq[1] = 2.0f * yq * (dR10 + dR01) + 2.0f * zq * (dR20 + dR02) + 2.0f * rr * (dR12 - dR21) -
              4.0f * xq * (dR22 + dR11);
      gq[2] = 2.0f * xq * (dR10 + dR01) + 2.0f * rr * (dR20 - dR02) + 2.0f * zq * (dR12 + dR21) -
              4.0f * yq * (dR22 + dR00);
      gq[3] = 2.0f * rr * (dR01 - dR10) + 2.0f * xq * (dR20 + dR02) + 2.0f * yq * (dR12 + dR21) -
              4.0f * zq * (dR11 + dR00);
    }
    /* Part C */
    float a0 = pm_x + gc_x, a1 = pm_y + gc_y, a2 = pm_z + gc_z;
    if (has_sh) {
      a0 = a0 + gsm0;
      a1 = a1 + gsm1;
      a2 = a2 + gsm2;
    }
    grad_means3d[3 * tid] = a0;
    grad_means3d[3 * tid + 1] = a1;
    grad_means3d[3 * tid + 2] = a2;
    grad_means2d[3 * tid] = gg[0];
    grad_means2d[3 * tid + 1] = gg[1];
    grad_means2d[3 * tid + 2] = 0.0f;
  }
}

int or_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void or_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}
