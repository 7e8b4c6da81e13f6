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
