// Forward render: one 256-thread workgroup (4 wave64) per 16x16 tile, one
// pixel per lane.  Gaussians of the tile's sorted list are staged 256 at a
// time in LDS (three float4 per Gaussian from the packed render record); a
// workgroup-wide vote ends the tile once every pixel's transmittance is done.
// Semantics follow render_kernels.py:16-147 (and flow_kernels.py:31-176 for
// the flow variant):
//   power > 0 skipped; alpha = min(0.99, o*exp(power)); alpha < 1/255 skipped;
//   T*(1-alpha) < 1e-4 ends the pixel without blending that Gaussian;
//   colour += f*alpha*T, alpha_out = sum alpha*T, depth = sum z*alpha*T;
//   n_contrib = 1-based list index of the last blended Gaussian.
// Exponents below the record's power_cutoff are skipped without evaluating
// exp: their alpha is provably below 1/255, so no decision changes.
#include "gs_common.h"
#include "gs_capi.h"

namespace gs {

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
};

template <bool kFlow>
__global__ __launch_bounds__(kTilePixels) void render_fwd_kernel(RenderFwdParams p) {
  __shared__ float4 s_r0[kTilePixels];
  __shared__ float4 s_r1[kTilePixels];
  __shared__ float4 s_r2[kTilePixels];
  __shared__ int s_id[kFlow ? kTilePixels : 1];

  const int tile = blockIdx.x;
  const int tx = tile % p.grid_x;
  const int ty = tile / p.grid_x;
  const int px = tx * kBlockX + (threadIdx.x % kBlockX);
  const int py = ty * kBlockY + (threadIdx.x / kBlockX);
  const bool inside = px < p.W && py < p.H;
  const int P = p.W * p.H;
  const int pix = py * p.W + px;
  int2 rg = p.ranges[tile];
  // Ranges come from gs_tile_ranges over num_rendered sorted pairs; the clamp
  // only guards against inconsistent caller input.
  rg.x = imax(0, imin(rg.x, p.num_rendered));
  rg.y = imax(rg.x, imin(rg.y, p.num_rendered));
  const int n = rg.y - rg.x;
  const float pfx = (float)px;
  const float pfy = (float)py;

  float T = 1.0f;
  int last = 0;
  float c0 = 0.0f, c1 = 0.0f, c2 = 0.0f, wsum = 0.0f, dacc = 0.0f;
  int done = inside ? 0 : 1;
  int n_success = 0;
  const bool aux = kFlow && p.write_aux != 0;

  const int rounds = (n + kTilePixels - 1) / kTilePixels;
  for (int r = 0; r < rounds; ++r) {
    if (__syncthreads_count(done) == kTilePixels) break;
    const int progress = r * kTilePixels + threadIdx.x;
    if (progress < n) {
      int id = p.point_list[rg.x + progress];
      if ((unsigned)id >= (unsigned)p.num_points) id = 0;
      const float4* rec = p.records + 3 * (size_t)id;
      s_r0[threadIdx.x] = rec[0];
      s_r1[threadIdx.x] = rec[1];
      s_r2[threadIdx.x] = rec[2];
      if (kFlow) s_id[threadIdx.x] = id;
    }
    __syncthreads();
    const int batch = imin(kTilePixels, n - r * kTilePixels);
    if (!done) {
      for (int j = 0; j < batch; ++j) {
        const float4 a = s_r0[j];
        const float4 b = s_r1[j];
        const float dx = a.x - pfx;
        const float dy = a.y - pfy;
        const float power = -0.5f * (a.z * dx * dx + b.x * dy * dy) - a.w * dx * dy;
        if (!(power <= 0.0f) || power < b.w) continue;
        const float alpha = fminr(kAlphaMax, b.y * exp_sw(power));
        if (alpha < kAlphaMin) continue;
        const float test_T = T * (1.0f - alpha);
        if (test_T < kTransmittanceMin) {
          done = 1;
          break;
        }
        const float contribution = alpha * T;
        const float4 f = s_r2[j];
        c0 = c0 + f.x * contribution;
        c1 = c1 + f.y * contribution;
        c2 = c2 + f.z * contribution;
        wsum = wsum + contribution;
        if (p.compute_depth) dacc = dacc + b.z * contribution;
        if (aux && n_success < p.top_k) {
          const size_t aux_idx = (size_t)n_success * P + pix;
          p.gs_per_pixel[aux_idx] = s_id[j];
          p.weight[aux_idx] = contribution;
          p.x_mu[aux_idx] = dx;
          p.x_mu[(size_t)p.top_k * P + aux_idx] = dy;
        }
        if (kFlow) ++n_success;
        T = test_T;
        last = r * kTilePixels + j + 1;
      }
    }
  }

  if (inside) {
    p.n_contrib[pix] = last;
    p.out_color[pix] = c0 + T * p.bg[0];
    p.out_color[P + pix] = c1 + T * p.bg[1];
    p.out_color[2 * P + pix] = c2 + T * p.bg[2];
    p.out_alpha[pix] = wsum;
    p.out_depth[pix] = dacc;
    if (aux) {
      for (int k = n_success; k < p.top_k; ++k) {
        const size_t aux_idx = (size_t)k * P + pix;
        p.gs_per_pixel[aux_idx] = -1;
        p.weight[aux_idx] = 0.0f;
        p.x_mu[aux_idx] = 0.0f;
        p.x_mu[(size_t)p.top_k * P + aux_idx] = 0.0f;
      }
    }
  }
}

static int launch_render_fwd(const RenderFwdParams& p, bool flow, hipStream_t s) {
  if (flow)
    hipLaunchKernelGGL(render_fwd_kernel<true>, dim3(p.num_tiles), dim3(kTilePixels), 0, s, p);
  else
    hipLaunchKernelGGL(render_fwd_kernel<false>, dim3(p.num_tiles), dim3(kTilePixels), 0, s, p);
  return gs_status_from_hip(hipGetLastError());
}

}  // namespace gs

static int gs_render_fwd_common(int32_t W, int32_t H, int32_t num_points, int64_t num_rendered,
                                const int32_t* ranges, const int32_t* point_list,
                                const float* records, const float* background, int32_t compute_depth,
                                int32_t write_aux, int32_t top_k, float* out_color, float* out_depth,
                                float* out_alpha, int32_t* n_contrib, int32_t* gs_per_pixel, float* weight,
                                float* x_mu, bool flow, void* stream) {
  if (W <= 0 || H <= 0 || (long long)W * H > 0x7fffffffLL) return GS_ERR_INVALID_ARGUMENT;
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
  return gs::launch_render_fwd(p, flow, (hipStream_t)stream);
}

extern "C" int gs_render_fwd(int32_t image_width, int32_t image_height, int32_t num_points,
                             int64_t num_rendered, const int32_t* ranges,
                             const int32_t* point_list, const float* records, const float* background,
                             int32_t compute_depth, float* out_color, float* out_depth, float* out_alpha,
                             int32_t* n_contrib, void* stream) {
  return gs_render_fwd_common(image_width, image_height, num_points, num_rendered, ranges, point_list, records,
                              background, compute_depth, 0,
                              0, out_color, out_depth, out_alpha, n_contrib, nullptr, nullptr, nullptr, false,
                              stream);
}

extern "C" int gs_render_fwd_flow(int32_t image_width, int32_t image_height, int32_t num_points,
                                  int64_t num_rendered, const int32_t* ranges,
                                  const int32_t* point_list, const float* records, const float* background,
                                  int32_t compute_depth, int32_t write_aux, int32_t top_k, float* out_color,
                                  float* out_depth, float* out_alpha, int32_t* n_contrib, int32_t* gs_per_pixel,
                                  float* weight_per_gs_pixel, float* x_mu, void* stream) {
  return gs_render_fwd_common(image_width, image_height, num_points, num_rendered, ranges, point_list, records,
                              background, compute_depth, write_aux, top_k, out_color, out_depth, out_alpha, n_contrib, gs_per_pixel,
                              weight_per_gs_pixel, x_mu, true, stream);
}
