// One K of the search kernel per translation unit (the build sets
// ST_SEARCH_K = 1..10), so that the instantiations compile in parallel.
#include "bloom_search_kernel.hpp"

#ifndef ST_SEARCH_K
#error "ST_SEARCH_K must be defined"
#endif

namespace st {

template <>
KernelFn search_kernel_for<ST_SEARCH_K>(int mode) {
  switch (mode) {
    case kOutBool: return bloom_search_kernel<ST_SEARCH_K, kOutBool>;
    case kOutCounts: return bloom_search_kernel<ST_SEARCH_K, kOutCounts>;
    default: return bloom_search_kernel<ST_SEARCH_K, kOutPacked>;
  }
}

}  // namespace st
