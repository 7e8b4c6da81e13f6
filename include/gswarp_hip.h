/*
 * gswarp_hip.h — C ABI of the gfx950 3D Gaussian Splatting rasterizer.
 *
 * Every entry point is extern "C", takes device pointers, explicit sizes and
 * a HIP stream (passed as void*, i.e. hipStream_t), enqueues its kernels on
 * that stream and returns an int status: GS_OK (0), a GS_ERR_* code, or a
 * positive hipError_t value.  No entry point allocates memory (device or
 * host) or keeps mutable state between calls: scratch is caller-provided and
 * sized by the matching *_scratch_bytes / *_workspace_bytes query, and the
 * read-back's host slot is the caller's (gs_readback_slot_bytes).  Calls on
 * different streams with disjoint buffers may run concurrently.  One entry
 * point is the exception, by design: gs_scan_tiles_static keeps its scratch
 * in a fixed device array of the library (one per GPU), so calls that
 * overlap on one GPU race on it.  ABI version (gs_version): 10200.
 *
 * Each function replaces one stage of the reference host pipeline
 * (fancifulland2718/gswarp 1.1.0, Warp backend); the stage it replaces is
 * cited above its declaration as file:line under
 * gswarp/_internal/backends/warp/.
 *
 * Layouts (N = Gaussians, K = SH coefficients per Gaussian, P = W*H pixels,
 * T = ceil(W/16)*ceil(H/16) tiles, R = Gaussian/tile pairs):
 *   means3d (N,3), scales (N,3), rotations (N,4) [w,x,y,z], opacities (N),
 *   shs (N,K,3), colors (N,3), view/proj (4,4) row-vector convention,
 *   campos (3), background (3): all fp32, C-contiguous.
 *   records (N,12) fp32, 16-byte aligned: per-Gaussian render record
 *     (x, y, conic_a, conic_b | conic_c, opacity, depth, power_cutoff |
 *      r, g, b, extents): extents packs the half-widths of the pixel
 *      region the record can blend as two binary16 (rounded up) for the
 *      blend kernels' culling; gs_render_* expect it as gs_preprocess_fwd
 *      writes it.
 *   images: color (3,H,W), depth (1,H,W), alpha (1,H,W), n_contrib (H,W) int32.
 *   ranges (T,2) int32 [start, end) into the sorted pair list.
 *   grad_gauss (N,10) fp32, zero-initialised by the caller, accumulated by
 *     gs_render_bwd: per Gaussian, sums over the pixels that blend it of
 *     v = G * dL/dalpha_hat times (dx, dy, dx^2, dx dy, dy^2, 1), with
 *     (dx, dy) = mean - pixel, then the colour (r, g, b) and depth gradients.
 *     Column 5 (sum v) is dL/dopacity; gs_preprocess_bwd turns columns 0-4
 *     into the xy and conic gradients with the record's conic and opacity.
 */
#ifndef GSWARP_HIP_H
#define GSWARP_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GS_OK 0
#define GS_ERR_INVALID_ARGUMENT (-1)
#define GS_ERR_MISALIGNED (-2)
#define GS_ERR_SCRATCH_TOO_SMALL (-3)
#define GS_ERR_OVERFLOW (-4)
#define GS_ERR_TOO_LARGE (-5)

#define GS_COVERAGE_SNUGBOX 0
#define GS_COVERAGE_ACCUTILE_SWEEP 1
#define GS_COVERAGE_CONIC_RECT 2

#define GS_RECORD_FLOATS 12
#define GS_GRAD_FLOATS 10

/* Library version as 10000*major + 100*minor + patch. */
int gs_version(void);

/* Human-readable text for a status returned by any gs_* call. */
const char* gs_status_string(int status);

/*
 * Fused preprocess: projection, near-plane cull, EWA 2D covariance, conic,
 * radius, tile-rect cull, tile-coverage count and (when colors_precomp is
 * NULL) SH colour of degree `degree` from K = sh_coeffs coefficients.  The 3D
 * covariance comes from scales and rotations, or, when cov3d_precomp (N, 6:
 * xx, xy, xz, yy, yz, zz) is non-NULL, is taken as given (scales / rotations
 * may then be NULL), with the reference's masked-kernel arithmetic.
 * Culled Gaussians get radius 0 and zero outputs; records are written only
 * for visible Gaussians.  clamped (N bytes, optional) receives the per-channel
 * clamp flags of the SH colour as bits 0..2.  A non-zero filter_variance
 * (finite, >= 0) applies the Mip-Splatting screen-space filter to the kept
 * Gaussians: cov2D + f I, its conic, the radius ceil(3 sqrt(max(lambda_max,
 * 0.1))) and the tile count are recomputed; a filtered determinant <= 1e-12
 * culls (depth and position are kept).  coverage ((N,4) int32, 16-byte
 * aligned, optional) receives each Gaussian's cover word: for a non-empty
 * tile rectangle with origin below 2^16 and spans below 2^8 (zero word
 * otherwise) the rectangle, whether every tile of it is covered, and, when
 * it has at most 64 cells, a 64-bit mask of the covered cells in the order of
 * the coverage walk, which the emission entry points read instead of
 * re-deriving the tiles.  band_store (optional, with coverage;
 * band_store_words >= gs_band_store_words(P) int32) receives the coverage
 * bands (one word per tile row or column: lo | hi << 16) of the Gaussians
 * whose word has neither a mask nor a full rectangle, 512 words per wave of
 * 64 Gaussians; such a word then holds the index of its bands (or -1 when
 * they did not fit), and gs_bin_buckets reads them instead of recomputing
 * them.  scan_state (optional, scan_state_bytes >= gs_scan_state_bytes(P)
 * bytes, 8-byte aligned) is prepared for
 * gs_scan_tiles_onepass as gs_scan_state_prepare would prepare it from these
 * outputs, from the values in registers (no launch or read of its own).
 * Replaces: preprocess_ops.py:289-581 (preprocess_gaussians) with
 * preprocess_kernels.py:83-269 (scales/rotations), preprocess_kernels.py:345-477
 * and 604-624 (precomputed covariances), the SH kernel
 * preprocess_kernels.py:272-342, and the Mip filter of backend_mip_3dgs.py:63-102
 * (whose tile recount is binning_kernels.py:56-123).
 */
int gs_preprocess_fwd(int32_t P, int32_t sh_coeffs, int32_t degree, const float* means3d,
                      const float* scales, const float* rotations, const float* cov3d_precomp, float scale_modifier,
                      const float* opacities, const float* shs, const float* colors_precomp,
                      const float* viewmatrix, const float* projmatrix, const float* campos,
                      float tanfovx, float tanfovy, float focal_x, float focal_y,
                      int32_t image_width, int32_t image_height, int32_t coverage_mode,
                      float filter_variance, int32_t* radii, float* depths, float* proj_2d, float* conic_2d,
                      float* conic_2d_inv, int32_t* tiles_touched, int32_t* coverage, float* records,
                      uint8_t* clamped, int32_t* band_store, int64_t band_store_words, int64_t* scan_state,
                      size_t scan_state_bytes, void* stream);
int64_t gs_band_store_words(int32_t P);

/*
 * Tile coverage of already projected Gaussians: for each i with radii[i] > 0,
 * tiles_touched[i] = the number of tiles it is binned to under coverage_mode
 * and, when coverage (optional, (N,4) int32, 16-byte aligned) is given, its
 * cover word, both exactly as gs_preprocess_fwd computes them; radius 0
 * gives 0.  records (N,12) supplies the screen position, conic and opacity
 * (floats 0-5 of the record), conic_2d_inv (N,3) the 2D covariance.
 * Replaces: binning_kernels.py:56-123 (_recount_covered_tiles_warp_kernel)
 * with math_kernels.py:306-390 (_count_covered_tiles_wp).
 */
int gs_count_tiles(int32_t P, const int32_t* radii, const float* records, const float* conic_2d_inv,
                   int32_t image_width, int32_t image_height, int32_t coverage_mode, int32_t* tiles_touched,
                   int32_t* coverage, void* stream);

/*
 * visible[i] = view-space z of means3d[i] > 0.2.
 * Replaces: preprocess_ops.py:584-595 (mark_visible) with
 * preprocess_kernels.py:604-624.
 */
int gs_mark_visible(int32_t P, const float* means3d, const float* viewmatrix, uint8_t* visible,
                    void* stream);

/*
 * Depth-sort input of the depth-then-tile binning: keys_out[i] = float bits
 * of depths[i] when radii[i] > 0, else 0; values_out[i] = i.  Sorted stably
 * (gs_sort_pairs_u32 on 32 bits) they give the reference's depth order with
 * culled Gaussians first.
 * Replaces: binning_kernels.py:27-40 (_prepare_depth_sort_payload, unpacked
 * layout) before the depth sort at binning_ops.py:152-222.
 */
int gs_depth_keys(int32_t P, const int32_t* radii, const float* depths, uint32_t* keys_out, int32_t* values_out,
                  void* stream);

/*
 * Inclusive prefix sum of tiles_touched[order[j]] (order == NULL: point
 * order) into offsets, plus, in the two int64 at info_dev (device memory):
 * info[0] = the exact total pair count, info[1] = (max << 32 | min) of the
 * float bits of depths[i] over the Gaussians with radii[i] > 0 (0 when there
 * are none, or when radii and depths are both NULL, which skips the range).
 * offsets are only meaningful when the total fits in int32.
 * Replaces: memory.py:539-551 (_inclusive_scan_i32) and
 * binning_ops.py:62-81 (_wide_pair_count_if_needed).
 */
size_t gs_scan_scratch_bytes(int32_t P);
int gs_scan_tiles(int32_t P, const int32_t* tiles_touched, const int32_t* order, const int32_t* radii,
                  const float* depths, int32_t* offsets, int64_t* info_dev, void* scratch, size_t scratch_bytes,
                  void* stream);

/*
 * gs_scan_tiles without a scratch argument: the scratch is a fixed device
 * array inside the library (256 KiB per GPU, held until the process ends),
 * so the call allocates nothing.  P may not exceed
 * gs_scan_tiles_static_max_points() (2^26); larger P returns
 * GS_ERR_TOO_LARGE.  Outputs and arguments are those of gs_scan_tiles.  All
 * calls on one GPU share the array: calls that overlap in time on one GPU
 * (two streams, two threads) race and give wrong results; serialise them.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops, harnesses
 * that forbid hipMalloc).
 */
int32_t gs_scan_tiles_static_max_points(void);
int gs_scan_tiles_static(int32_t P, const int32_t* tiles_touched, const int32_t* order, const int32_t* radii,
                         const float* depths, int32_t* offsets, int64_t* info_dev, void* stream);

/*
 * gs_scan_tiles in point order (order == NULL) that also sizes the bucketed
 * binning: with coverage = gs_preprocess_fwd's cover words it stores, after
 * info[0] and info[1] as gs_scan_tiles does, info[2] = the number of
 * (Gaussian, super-tile) entries, i.e. the sum over the valid cover words of
 * the 8 x 8-tile squares their tile rectangle meets (-1 when a Gaussian with
 * tiles has no valid word: its rectangle does not fit the word), and
 * info[3] = the number of valid words.  info_dev holds four int64; the
 * scratch is gs_scan_scratch_bytes(P) bytes.
 * Replaces: memory.py:539-551 and binning_ops.py:62-81, as gs_scan_tiles.
 */
int gs_scan_tiles_entries(int32_t P, const int32_t* tiles_touched, const int32_t* radii, const float* depths,
                          const int32_t* coverage, int32_t* offsets, int64_t* info_dev, void* scratch,
                          size_t scratch_bytes, void* stream);

/*
 * The point-order scan of gs_scan_tiles, and with sized != 0 the bucketed
 * binning's sizes of gs_scan_tiles_entries (info[0..3]), in one kernel that
 * reads only tiles_touched: a decoupled look-back over blocks of 4096
 * Gaussians.  The depth range and the sizes come from the state, which
 * gs_scan_state_prepare (from radii, depths and, for the sizes, the cover
 * words) or gs_preprocess_fwd (scan_state) prepares: per 256 Gaussians their
 * depth range, super-tile units and valid cover words, and five zero words
 * per 4096 (gs_scan_state_status_words(P) int64 from word
 * gs_scan_state_status_offset(P)).  A state serves one scan.  Every wait of
 * a block on its predecessors is bounded by spin_limit sleeps (about 64
 * cycles each; 2^20 is far beyond any normal wait): a block whose look-back
 * times out adds up the counts before it itself (slower, same offsets), and
 * a final wait that times out stores info[1] = the widest depth range (every
 * positive float) and info[2] = -1, info[3] = 0, as for a Gaussian without a
 * valid cover word.  Otherwise outputs equal gs_scan_tiles'
 * (gs_scan_tiles_entries').
 * Concurrent calls must use distinct states.
 * Replaces: memory.py:539-551 and binning_ops.py:62-81, as gs_scan_tiles.
 */
size_t gs_scan_state_bytes(int32_t P);
int64_t gs_scan_state_status_offset(int32_t P);
int64_t gs_scan_state_status_words(int32_t P);
int gs_scan_state_prepare(int32_t P, const int32_t* tiles_touched, const int32_t* radii, const float* depths,
                          const int32_t* coverage, void* state, size_t state_bytes, void* stream);
int gs_scan_tiles_onepass(int32_t P, const int32_t* tiles_touched, int32_t* offsets, int64_t* info_dev,
                          void* state, size_t state_bytes, int32_t sized, int32_t spin_limit, void* stream);

/*
 * Copies count (1 to 16) int64 at info_dev into slot[0, count), returning
 * once the work enqueued on the stream before the call has completed.  The
 * slot is the caller's host memory of gs_readback_slot_bytes() bytes (256:
 * the info words first, a flag word last), 8-byte aligned.  When the device
 * can address it (hipHostMalloc with hipHostMallocPortable |
 * hipHostMallocMapped | hipHostMallocCoherent), a one-wave kernel publishes
 * the words into it and raises its flag to seq, and the host spins on the
 * flag, polling the stream, instead of a copy and a blocking synchronisation
 * (the copy and synchronisation remain the fallback, and serve slots in
 * pageable memory).  seq must be positive and differ from the value the
 * flag holds (the caller counts its uses of the slot: seq = previous + 1;
 * GS_ERR_INVALID_ARGUMENT otherwise).  A slot serves one call at a time:
 * calls that overlap (two threads, two streams) need distinct slots.  The
 * wait is a spin on the host core that yields it to other runnable threads
 * after about 10^4 polls.
 * Replaces: binning_ops.py:243-252 (the num_rendered .item()).
 */
size_t gs_readback_slot_bytes(void);
int gs_info_readback(const int64_t* info_dev, int64_t* slot, int64_t seq, int32_t count, void* stream);

/*
 * gs_info_readback of the two int64 at info_dev (pair count and depth range):
 * the single device-to-host synchronisation of a forward pass.
 * Replaces: binning_ops.py:243-252 (the num_rendered .item()).
 */
int gs_num_rendered_readback(const int64_t* info_dev, int64_t* slot, int64_t seq, void* stream);

/*
 * For every Gaussian i with radius > 0, emits one key per covered tile at
 * offsets[i-1] (0 for i == 0):
 *   key = ((tile_id << depth_bits) | (float_bits(depth_i) - depth_min)) << value_bits | v
 * with v = i when value_bits > 0 (values_out unused, may be NULL), else
 * v = 0 and values_out[pair] = i.  depth_min / depth_bits come from the
 * range gs_scan_tiles reports (depth_bits = bit length of max - min); the
 * tile, depth and value fields must fit in 64 bits and i in value_bits.
 * Pairs are produced in point-index order; a stable sort on the tile and
 * depth fields then yields the reference's (tile, depth, index) order.
 * coverage (optional) is gs_preprocess_fwd's cover words for the same
 * inputs; Gaussians with a mask are emitted from it.  depths (optional) is
 * gs_preprocess_fwd's depths, read instead of the records' copy.
 * Replaces: binning_kernels.py:411-451 with binning_kernels.py:127-216 and
 * the depth sort that precedes it (binning_ops.py:152-222).
 */
int gs_duplicate_keys(int32_t P, const int32_t* radii, const float* records, const float* conic_2d_inv,
                      const int32_t* coverage, const float* depths, const int32_t* offsets, int32_t image_width,
                      int32_t image_height,
                      int32_t coverage_mode, int64_t num_rendered, uint32_t depth_min, int32_t depth_bits,
                      int32_t value_bits, uint64_t* keys_out, int32_t* values_out, void* stream);

/*
 * Depth-then-tile binning emission: thread j emits the covered tiles of
 * Gaussian order[j] (radius > 0) at offsets[j-1] (0 for j == 0) as
 * (tile id, point index) pairs.  With order the depth-sorted point list, a
 * stable sort of the tile ids then yields the reference's per-tile lists.
 * coverage (optional) as for gs_duplicate_keys.
 * Replaces: binning_kernels.py:411-451 (_duplicate_with_keys_from_order)
 * with binning_kernels.py:127-216.
 */
int gs_duplicate_tiles(int32_t P, const int32_t* order, const int32_t* radii, const float* records,
                       const float* conic_2d_inv, const int32_t* coverage, const int32_t* offsets,
                       int32_t image_width,
                       int32_t image_height, int32_t coverage_mode, int64_t num_rendered, uint32_t* tiles_out,
                       int32_t* values_out, void* stream);

/*
 * Stable LSD radix sorts in gs_sort_num_passes(key_bits) = ceil(key_bits / 8)
 * passes of at most 8 bits (the field split evenly), ping-ponging between the primary
 * and the _alt buffers: the result ends in the primary buffers when
 * gs_sort_num_passes(key_bits) is even, else in the _alt ones.
 * gs_sort_pairs_u64 sorts (uint64 key, int32 value) pairs on the low
 * key_bits bits; gs_sort_keys_u64 sorts keys alone and gs_sort_pairs_u32
 * (uint32 key, int32 value) pairs, both on bits [lo_bit, lo_bit + key_bits)
 * (bits below lo_bit ride along).
 * Replaces: binning_ops.py:337-343 and memory.py:586-600
 * (wp.utils.radix_sort_pairs on tile ids).
 */
int gs_sort_num_passes(int32_t key_bits);
size_t gs_sort_scratch_bytes(int64_t n);
int gs_sort_pairs_u64(int64_t n, int32_t key_bits, uint64_t* keys, int32_t* values, uint64_t* keys_alt,
                      int32_t* values_alt, void* scratch, size_t scratch_bytes, void* stream);
int gs_sort_keys_u64(int64_t n, int32_t lo_bit, int32_t key_bits, uint64_t* keys, uint64_t* keys_alt,
                     void* scratch, size_t scratch_bytes, void* stream);
int gs_sort_pairs_u32(int64_t n, int32_t lo_bit, int32_t key_bits, uint32_t* keys, int32_t* values,
                      uint32_t* keys_alt, int32_t* values_alt, void* scratch, size_t scratch_bytes, void* stream);

/*
 * ranges[t] = [start, end) of tile t = key >> tile_shift in the sorted keys;
 * empty tiles [0, 0].  With value_bits > 0 also writes
 * point_list[i] = key_i & (2^value_bits - 1).
 * Replaces: binning_kernels.py:468-487 (_identify_tile_ranges) and the zero
 * fill at binning_ops.py:233.
 */
int gs_tile_ranges(int64_t n, const uint64_t* sorted_keys, int32_t tile_shift, int32_t value_bits,
                   int32_t num_tiles, int32_t* ranges, int32_t* point_list, void* stream);
/* The same for sorted uint32 tile ids (depth-then-tile binning). */
int gs_tile_ranges_u32(int64_t n, const uint32_t* sorted_tiles, int32_t num_tiles, int32_t* ranges, void* stream);

/*
 * Second half of the packed-key binning sort.  keys holds the packed
 * (tile, depth field, point) keys already sorted stably by their tile field,
 * so each tile's keys are contiguous and in point order, and ranges holds
 * their [start, end) (gs_tile_ranges).  Each tile's segment is sorted stably
 * by bits [lo_bit, lo_bit + key_bits) (the depth field), which gives the
 * order of a full (tile, depth, point) key sort, and
 * point_list[i] = key_i & (2^value_bits - 1) is written.  With write_keys the
 * sorted keys are also written back to keys; without it the keys of tiles
 * longer than 2048 are left permuted within their segment.  keys_alt
 * (n keys) is scratch for those tiles.  Allocates nothing.
 * Replaces: binning_ops.py:337-343 (the stable tile sort of the
 * depth-ordered pairs) together with the depth order of
 * binning_ops.py:152-222, i.e. the final per-tile (depth, point) order.
 */
int gs_sort_tile_segments(int64_t n, uint64_t* keys, uint64_t* keys_alt, int32_t num_tiles, const int32_t* ranges,
                          int32_t lo_bit, int32_t key_bits, int32_t value_bits, int32_t* point_list,
                          int32_t write_keys, void* stream);

/*
 * The packed-key binning after the pair count is known, in one call:
 * gs_duplicate_keys into workspace, gs_sort_keys_u64 on the tile field,
 * gs_tile_ranges into ranges ((T, 2) int32, T = tiles of the image) and
 * gs_sort_tile_segments into point_list (num_rendered int32).  workspace
 * holds two key buffers and the sort scratch:
 * gs_bin_packed_workspace_bytes(num_rendered) bytes.  With sorted_keys_out
 * (num_rendered uint64) the fully sorted keys are copied there too.
 * value_bits must be >= 1 (the point index is packed in the key).
 * stage_events, if not NULL, holds five hipEvent_t recorded on the stream
 * before emission and after emission, the tile sort, the ranges and the
 * segment sort (for per-stage timing).
 * Replaces: binning_ops.py:84-431 (_build_binning_state) after the
 * num_rendered read-back at binning_ops.py:243-252.
 */
size_t gs_bin_packed_workspace_bytes(int64_t num_rendered);
int gs_bin_packed(int32_t P, const int32_t* radii, const float* records, const float* conic_2d_inv,
                  const int32_t* coverage, const float* depths, const int32_t* offsets, int32_t image_width,
                  int32_t image_height,
                  int32_t coverage_mode,
                  int64_t num_rendered, uint32_t depth_min, int32_t depth_bits, int32_t value_bits, void* workspace,
                  size_t workspace_bytes, int32_t* ranges, int32_t* point_list, uint64_t* sorted_keys_out,
                  void* const* stage_events, void* stream);

/*
 * gs_num_rendered_readback (into slot, with seq, as there) followed, in the
 * same call, by gs_bin_packed into
 * buffers allocated before the pair count was known (point_list for up to
 * `capacity` pairs, workspace of gs_bin_packed_workspace_bytes(capacity)
 * bytes), so the binning launches without a return to the caller.  The key
 * layout is tile | depth field (bit length of the visible depth-bit range)
 * | point index (max(1, bit length of P - 1) bits); the packed dataflow is
 * used when the fields fit in 64 bits and, with max_pairs_per_point > 0,
 * num_rendered <= max_pairs_per_point * P.  result (5 int64):
 * num_rendered, depth_min, depth_bits, value_bits, and 1 if the binning was
 * launched or 0 if the caller must bin itself (count outside
 * [1, 2^31 - 1], above capacity, or another dataflow).  With out_color
 * non-NULL the binning is followed by gs_render_fwd into out_color,
 * out_depth, out_alpha and n_contrib (background, compute_depth as there)
 * and result (6 int64) ends with 1 if it was launched; that render zeroes
 * grad_clear as gs_render_fwd_clear does (grad_clear_floats 0: nothing),
 * and only when it is launched; tile_order is gs_render_fwd's.  stage_events, if not
 * NULL, holds the five events of gs_bin_packed and a sixth recorded after
 * the render.  The keys are emitted into the start of workspace before the
 * count is read back (the kernel reads the layout and the count from
 * info_dev, at most capacity keys), so workspace is written even when the
 * call then launches no binning (result[4] == 0); info_dev must hold the
 * scan's words (and offsets its offsets).
 * Replaces: binning_ops.py:243-252 (the .item() read-back) together with
 * the binning that follows it and render_ops.py:16-93.
 */
int gs_readback_bin_packed(const int64_t* info_dev, int64_t* slot, int64_t seq, int32_t P, const int32_t* radii,
                           const float* records, const float* conic_2d_inv, const int32_t* coverage,
                           const float* depths, const int32_t* offsets, int32_t image_width, int32_t image_height,
                           int32_t coverage_mode,
                           int32_t max_pairs_per_point, int64_t capacity, void* workspace, size_t workspace_bytes,
                           int32_t* ranges, int32_t* point_list, const float* background, int32_t compute_depth,
                           float* out_color, float* out_depth, float* out_alpha, int32_t* n_contrib,
                           float* grad_clear, int64_t grad_clear_floats, void* const* stage_events,
                           int64_t* result, int32_t* tile_order, void* stream);

/*
 * Bucketed binning, for many tiles per Gaussian: the per-tile lists in
 * (depth, point index) order, written straight into point_list
 * (num_rendered int32) with their ranges ((T, 2) int32; [0, 0] for empty
 * tiles), without a key per pair.  The Gaussians with a valid cover word
 * (coverage from gs_preprocess_fwd; num_valid of them) are sorted stably by
 * the bits of depths[i] above depth_min; each yields, per 8 x 8-tile square
 * its tile rectangle meets, an entry (point index, mask of the covered tiles
 * there; num_entries of them in all), which a stable partition lists per
 * square in depth order; each square's entries are then written into the
 * lists of the tiles they cover.  num_entries and num_valid are
 * gs_scan_tiles_entries's info[2] and info[3], depth_min / depth_max its
 * visible depth-bit range (info[1]); band_store (optional) and records are
 * gs_preprocess_fwd's: the stored coverage bands, and the conic of Gaussians
 * whose bands were not stored, which are recomputed.  The image may
 * be at most 255 x 255 tiles (GS_ERR_TOO_LARGE otherwise).  workspace is
 * gs_bin_buckets_workspace_bytes(P, num_valid, num_entries, W, H) bytes,
 * 16-byte aligned.  stage_events, if not NULL, holds four hipEvent_t
 * recorded before the depth sort and after it, after the super-square
 * entries and after the tile lists.
 * Replaces: binning_ops.py:152-222 (depth sort) and binning_ops.py:297-431
 * (duplicate-with-keys from the depth order, tile sort and tile ranges):
 * the same lists and ranges.
 */
size_t gs_bin_buckets_workspace_bytes(int32_t P, int32_t num_valid, int64_t num_entries, int32_t image_width,
                                      int32_t image_height);
int gs_bin_buckets(int32_t P, int32_t num_valid, int64_t num_entries, int64_t num_rendered, const float* depths,
                   uint32_t depth_min, uint32_t depth_max, const int32_t* coverage, const int32_t* band_store,
                   const float* records, int32_t image_width, int32_t image_height, void* workspace,
                   size_t workspace_bytes, int32_t* ranges, int32_t* point_list, void* const* stage_events,
                   void* stream);

/*
 * The tiles ordered by their list length (ranges (T, 2)), longest first,
 * into order (num_tiles int32): the order in which the blend kernels take
 * the tiles when given an order buffer, so that the longest walks start
 * first and the end of the grid is made of short ones.  One workgroup.
 * No counterpart in the reference (its kernels take the tiles in tile
 * order); it changes no result, only the schedule.
 */
int gs_tile_order(int32_t num_tiles, const int32_t* ranges, int32_t* order, void* stream);

/*
 * Per-tile front-to-back alpha blending of 16x16 tiles, each covered by
 * independent wave64 workgroups that own a slice of its rows.
 * num_points (N) and num_rendered (R) bound every index read from ranges and
 * point_list.
 * Writes color + T*bg, alpha = sum of weights, depth (zero unless
 * compute_depth) and n_contrib (1-based index of the last blended Gaussian).
 * tile_order (optional, T int32 of caller memory): when given, R <= 4 N
 * and R >= 192 T, the call first orders the tiles into it (gs_tile_order)
 * and its workgroups take them longest list first; otherwise they take them
 * in tile order and the buffer is not written.  Keep it for gs_render_bwd.
 * The results do not depend on it.
 * Replaces: render_ops.py:16-93 with render_kernels.py:16-147.
 */
int gs_render_fwd(int32_t image_width, int32_t image_height, int32_t num_points, int64_t num_rendered,
                  const int32_t* ranges,
                  const int32_t* point_list, const float* records, const float* background,
                  int32_t compute_depth, float* out_color, float* out_depth, float* out_alpha,
                  int32_t* n_contrib, int32_t* tile_order, void* stream);

/*
 * gs_render_fwd that also sets clear_floats floats at clear (16-byte
 * aligned; clear_floats 0: nothing) to zero, spread over the blend's
 * workgroups: the backward's grad_gauss accumulator, zeroed by the forward
 * without a launch of its own.  The buffer must not overlap any other
 * argument.
 * Replaces: render_ops.py:16-93 together with the zero fill of the
 * backward's render accumulators (backward_ops.py:203, the torch.zeros of
 * the combined per-Gaussian gradient buffer).
 */
int gs_render_fwd_clear(int32_t image_width, int32_t image_height, int32_t num_points, int64_t num_rendered,
                        const int32_t* ranges, const int32_t* point_list, const float* records,
                        const float* background, int32_t compute_depth, float* out_color, float* out_depth,
                        float* out_alpha, int32_t* n_contrib, float* clear, int64_t clear_floats,
                        int32_t* tile_order, void* stream);

/*
 * gs_render_fwd plus the flow auxiliaries of the first top_k blended
 * Gaussians per pixel, front to back: ids (top_k,H,W) int32 (-1 when fewer),
 * weights alpha*T (top_k,H,W), and x_mu (2,top_k,H,W) = mean - pixel.
 * Every slot of every pixel is written.  With write_aux == 0 the aux
 * pointers may be NULL.
 * Replaces: flow_ops.py:109-193 with flow_kernels.py:31-176.
 */
int gs_render_fwd_flow(int32_t image_width, int32_t image_height, int32_t num_points, int64_t num_rendered,
                       const int32_t* ranges,
                       const int32_t* point_list, const float* records, const float* background,
                       int32_t compute_depth, int32_t write_aux, int32_t top_k, float* out_color,
                       float* out_depth, float* out_alpha, int32_t* n_contrib, int32_t* gs_per_pixel,
                       float* weight_per_gs_pixel, float* x_mu, int32_t* tile_order, void* stream);

/*
 * Reverse blend: accumulates per-Gaussian pixel moments of the loss
 * gradient (the grad_gauss layout above) into grad_gauss (N,10), which the
 * caller zero-initialises.  grad_color, grad_depth and grad_alpha may each
 * be NULL: an absent upstream gradient is zero.  tile_order: the buffer
 * that the forward call over the same ranges (gs_render_fwd, _clear, _flow
 * or gs_readback_bin_packed) was given, or NULL; under the forward's
 * condition (R <= 4 N, R >= 192 T) the workgroups take the tiles in the
 * order the forward wrote into it, otherwise in tile order.
 * Replaces: backward_ops.py:183-290 with backward_kernels.py:539-707.
 */
int gs_render_bwd(int32_t image_width, int32_t image_height, int32_t num_points, int64_t num_rendered,
                  const int32_t* ranges,
                  const int32_t* point_list, const float* records, const float* background,
                  const float* out_alpha, const int32_t* n_contrib, const float* grad_color,
                  const float* grad_depth, const float* grad_alpha, int32_t compute_depth,
                  float* grad_gauss, const int32_t* tile_order, void* stream);

/*
 * Fused per-Gaussian backward: SH colour backward (when shs != NULL), the
 * projected-mean and depth gradients, cov2D -> cov3D -> scale/rotation
 * gradients, and the accumulation into grad_means3d / grad_means2d (z = 0).
 * flow_double != 0 adds the render xy/conic gradients a second time into the
 * projected-mean and conic chains, as the reference flow backward does with
 * enable_flow_grad.  grad_sh (N,K,3) is fully written (zeros beyond the
 * evaluated bands); grad_opacity (N) and grad_colors (N,3, when non-NULL)
 * are copied out of grad_gauss.  The xy and conic render gradients are
 * formed from grad_gauss's moments with the conic and opacity of records
 * (the forward's, 16-byte aligned) and image_width / 2, image_height / 2.  With cov3d_precomp non-NULL the cov2D
 * gradient is returned as grad_cov3d (N, 6) instead of being chained into
 * grad_scales / grad_rotations (which may then be NULL).  filter_variance is
 * the forward's Mip-Splatting variance (0 without the filter), added to the
 * recomputed cov2D as in backward_kernels.py:176-178.  The upstream
 * gradients grad_proj_2d, grad_conic_2d and grad_conic_2d_inv may be NULL
 * (zero).
 * Replaces: backward_ops.py:376-746 with backward_kernels.py:53-295 (fused),
 * backward_kernels.py:710-870 (precomputed covariances),
 * backward_kernels.py:298-536 and flow_kernels.py:14-28.
 */
int gs_preprocess_bwd(int32_t P, int32_t sh_coeffs, int32_t degree, const float* means3d,
                      const float* scales, const float* rotations, const float* cov3d_precomp, float scale_modifier,
                      const float* shs, const float* campos, const float* viewmatrix,
                      const float* projmatrix, float tanfovx, float tanfovy, float focal_x, float focal_y,
                      const int32_t* radii, const uint8_t* clamped, const float* grad_gauss,
                      const float* records, int32_t image_width, int32_t image_height, const float* grad_proj_2d,
                      const float* grad_conic_2d, const float* grad_conic_2d_inv,
                      int32_t flow_double, float filter_variance, float* grad_means3d, float* grad_means2d,
                      float* grad_scales, float* grad_rotations, float* grad_cov3d, float* grad_sh,
                      float* grad_opacity, float* grad_colors, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GSWARP_HIP_H */
