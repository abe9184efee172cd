// Wavefront-wide integer helpers for gfx950 (wave64), device code only.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace st {

// Total over the wave of per-lane values below 64, by bit slices: one
// ballot per bit and a scalar popcount of it.
__device__ __forceinline__ uint32_t wave_total_small(uint32_t v) {
  uint32_t t = 0;
#pragma unroll
  for (int k = 0; k < 6; ++k) t += static_cast<uint32_t>(__popcll(__ballot((v >> k) & 1u))) << k;
  return t;
}

// Inclusive sum along each row of 16 lanes by DPP row shifts (a lane whose
// source lies before its row's start adds 0): lane 15 of a row holds the
// row's total.
__device__ __forceinline__ uint32_t row16_inclusive_sum(uint32_t v) {
  v += __builtin_amdgcn_update_dpp(0u, v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0u, v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0u, v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0u, v, 0x118, 0xF, 0xF, false);  // row_shr:8
  return v;
}

// Inclusive prefix sum over the wave (the row sums, then row_bcast:15 adds
// lane 15 into rows 1 and 3 and row_bcast:31 lane 31 into rows 2 and 3);
// *total receives the wave's sum.
__device__ __forceinline__ uint32_t wave_inclusive_sum(uint32_t v, uint32_t* total) {
  uint32_t x = row16_inclusive_sum(v);
  x += __builtin_amdgcn_update_dpp(0u, x, 0x142, 0xA, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0u, x, 0x143, 0xC, 0xF, false);
  *total = __builtin_amdgcn_readlane(x, 63);
  return x;
}

// Bits of a lane's 32-doc half-word that fall below num_docs; the half-word's
// first doc (its bit 31) is first_doc.
__device__ __forceinline__ uint32_t valid_doc_mask(int64_t first_doc, int64_t num_docs) {
  const int64_t valid = num_docs - first_doc;
  if (valid >= 32) return ~0u;
  if (valid <= 0) return 0u;
  return ~0u << (32 - static_cast<int>(valid));
}

}  // namespace st
