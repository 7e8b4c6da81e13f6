// Internal helpers shared by the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/gswarp_hip.h"

static inline int gs_status_from_hip(hipError_t e) { return e == hipSuccess ? GS_OK : (int)e; }

// Number of 8-bit LSD radix passes needed for key_bits significant bits.
static inline int gs_passes_for_bits(int key_bits) { return key_bits <= 0 ? 0 : (key_bits + 7) / 8; }

// Number of bits needed to represent v >= 0 (0 for v == 0).
static inline int gs_bit_length(long long v) {
  int b = 0;
  while (v > 0) {
    ++b;
    v >>= 1;
  }
  return b;
}

// Entry points shared between the library's sources (not in the public
// header).  gs_render_fwd_clear_ordered is gs_render_fwd_clear whose tile
// order the caller may already have written into tile_order (order_ready,
// gs_tile_order over the same ranges); gs_sort_tile_segments_ordered is
// gs_sort_tile_segments whose workgroups take the tiles in the given order
// (a permutation of the tiles, longest list first; null: tile order).
int gs_render_fwd_clear_ordered(int32_t image_width, int32_t image_height, int32_t num_points, int64_t num_rendered,
                                const int32_t* ranges, const int32_t* point_list, const float* records,
                                const float* background, int32_t compute_depth, float* out_color, float* out_depth,
                                float* out_alpha, int32_t* n_contrib, float* clear, int64_t clear_floats,
                                int32_t* tile_order, bool order_ready, void* stream);
int gs_sort_tile_segments_ordered(int64_t n, uint64_t* keys, uint64_t* keys_alt, int32_t num_tiles,
                                  const int32_t* ranges, int32_t lo_bit, int32_t key_bits, int32_t value_bits,
                                  int32_t* point_list, int32_t write_keys, const int32_t* order, void* stream);
