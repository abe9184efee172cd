// Library-wide entry points: error reporting, version, the host hash and the
// cluster column-geometry kernel.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <string>

#include "st_common.hpp"
#include "st_errors.hpp"

namespace st {

namespace {
thread_local std::string g_last_error;
}

void set_last_error(const std::string& msg) { g_last_error = msg; }

namespace {

// generate_column_info_for_clusters (bloom_index_search.cpp:520-534).
__global__ void column_info_kernel(const int64_t* __restrict__ offsets,
                                   const int64_t* __restrict__ lengths, int64_t n,
                                   int32_t* __restrict__ counts,
                                   int32_t* __restrict__ starts,
                                   int8_t* __restrict__ firsts) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t start = offsets[i];
  const int64_t len = lengths[i];
  const int8_t first = static_cast<int8_t>(start % kBitsPerColumn);
  starts[i] = static_cast<int32_t>(start / kBitsPerColumn);
  firsts[i] = first;
  counts[i] = len > 0 ? static_cast<int32_t>((len + first + kBitsPerColumn - 1) /
                                             kBitsPerColumn)
                      : 0;
}

}  // namespace
}  // namespace st

extern "C" const char* st_last_error(void) { return st::g_last_error.c_str(); }

extern "C" const char* st_version(void) { return "silvertorch_amd 0.1.0 (gfx950)"; }

extern "C" uint64_t st_murmur_hash3_2x64(uint64_t x, uint64_t y, uint64_t seed) {
  return st::murmur_pair(x, y, seed);
}

extern "C" int st_generate_column_info_for_clusters(
    const int64_t* offsets, const int64_t* lengths, int64_t n,
    int32_t* column_counts, int32_t* start_columns, int8_t* first_offsets,
    void* stream) {
  using namespace st;
  return guarded([&] {
    ST_CHECK(n >= 0, "negative cluster count");
    if (n == 0) return;
    ST_CHECK(offsets && lengths && column_counts && start_columns && first_offsets,
             "null device pointer");
    const int threads = 256;
    const int64_t blocks = (n + threads - 1) / threads;
    hipLaunchKernelGGL(column_info_kernel, dim3(static_cast<unsigned>(blocks)),
                       dim3(threads), 0, static_cast<hipStream_t>(stream), offsets,
                       lengths, n, column_counts, start_columns, first_offsets);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
      throw Error(ST_ERR_HIP, cat("column_info_kernel launch failed: ",
                                  hipGetErrorString(e)));
  });
}
