// Wavefront-wide integer helpers for gfx950 (wave64), device code only.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace st {

// Exclusive prefix and total over the wave of per-lane values below 64, by
// bit slices: one ballot per bit, mbcnt for the lanes below, a scalar
// popcount for the total.  No cross-lane data movement through LDS.
struct WaveScan {
  uint32_t excl, total;
};

__device__ __forceinline__ WaveScan wave_scan_small(uint32_t v) {
  WaveScan r{0u, 0u};
#pragma unroll
  for (int k = 0; k < 6; ++k) {
    const uint64_t m = __ballot((v >> k) & 1u);
    r.excl += __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                        __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u))
              << k;
    r.total += static_cast<uint32_t>(__popcll(m)) << k;
  }
  return r;
}

__device__ __forceinline__ uint32_t wave_total_small(uint32_t v) {
  uint32_t t = 0;
#pragma unroll
  for (int k = 0; k < 6; ++k) t += static_cast<uint32_t>(__popcll(__ballot((v >> k) & 1u))) << k;
  return t;
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
