// One K of the search kernel per translation unit (the build sets
// ST_SEARCH_K = 1..10), so that the instantiations compile in parallel.
#include "bloom_search_kernel.hpp"

#ifndef ST_SEARCH_K
#error "ST_SEARCH_K must be defined"
#endif

namespace st {

template <>
KernelFn search_kernel_for<ST_SEARCH_K>(int mode, bool quad) {
  if constexpr (QuadShape<ST_SEARCH_K>::NB >= 4) {
    if (quad) {
      switch (mode) {
        case kOutBool: return bloom_search_kernel<ST_SEARCH_K, kOutBool, true>;
        case kOutCounts: return bloom_search_kernel<ST_SEARCH_K, kOutCounts, true>;
        default: return bloom_search_kernel<ST_SEARCH_K, kOutPacked, true>;
      }
    }
  }
  switch (mode) {
    case kOutBool: return bloom_search_kernel<ST_SEARCH_K, kOutBool, false>;
    case kOutCounts: return bloom_search_kernel<ST_SEARCH_K, kOutCounts, false>;
    default: return bloom_search_kernel<ST_SEARCH_K, kOutPacked, false>;
  }
}

}  // namespace st

namespace st {

template <>
WideFn wide_kernel_for<ST_SEARCH_K>() {
  if constexpr (ST_SEARCH_K <= 7) {
    return bloom_wide_kernel<ST_SEARCH_K>;
  } else {
    return nullptr;
  }
}

}  // namespace st
