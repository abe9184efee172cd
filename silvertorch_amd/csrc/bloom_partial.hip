// Cluster-restricted search for gfx950: the plan of each (row, cluster) work
// item evaluated on the columns that cover the cluster's docs.
//
// Replaces bloom_index_search_batch_return_partial_response
// (bloom_index_search.cpp:246-395 on CPU, bloom_index_search_cuda.cu:617-1648
// on CUDA).  The host (st_search_plan_partial_items) lays out the response;
// here one wave takes one item at a time and each lane one 64-bit column
// word: the program is wave-uniform (scalar loads), the bundle width and so
// the row positions are the lane's own, resolved from the term hashes as
// signature_match does (bloom_index_search.cpp:40-61).
#include <hip/hip_runtime.h>

#include "plan_eval.hpp"
#include "search_plan.hpp"
#include "st_common.hpp"
#include "st_errors.hpp"

namespace st {
namespace {

constexpr int kPartialThreads = 256;

#define ST_CONST __attribute__((address_space(4)))

template <int K, int kStack>
__global__ __launch_bounds__(kPartialThreads) void partial_search_kernel(
    const int64_t* __restrict__ index, int64_t index_numel, const int64_t* __restrict__ bbo,
    const uint32_t* __restrict__ blob, const st_partial_item* __restrict__ items,
    int64_t num_items, int32_t hash_k, uint32_t pos_bytes, int64_t* __restrict__ out) {
  EvalArgs a;
  a.index = index;
  a.index_numel = index_numel;
  a.hash_k = hash_k;
  a.pos_bytes = pos_bytes;
  const ST_CONST uint32_t* blob32 = (const ST_CONST uint32_t*)(blob);
  const ST_CONST uint64_t* blob64 = (const ST_CONST uint64_t*)(blob);
  const int lane = threadIdx.x & 63;
  const int64_t waves = static_cast<int64_t>(gridDim.x) * (kPartialThreads / 64);
  const int64_t first_wave = static_cast<int64_t>(blockIdx.x) * (kPartialThreads / 64) +
                             __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // st_partial_item as 8 words: first_column, out_offset (2 each),
  // num_columns, program, hashes, reserved
  static_assert(sizeof(st_partial_item) == 32, "st_partial_item layout");
  const ST_CONST uint32_t* words = (const ST_CONST uint32_t*)(items);
  auto i64_at = [](const ST_CONST uint32_t* w) {
    return static_cast<int64_t>((static_cast<uint64_t>(w[1]) << 32) | w[0]);
  };
  for (int64_t i = first_wave; i < num_items; i += waves) {
    const ST_CONST uint32_t* w = words + i * 8;
    const int64_t first_column = i64_at(w), out_offset = i64_at(w + 2);
    const int32_t num_columns = static_cast<int32_t>(w[4]);
    const ST_CONST uint32_t* prog = blob32 + w[5];
    const ST_CONST uint64_t* hashes = blob64 + w[6];
    for (int32_t j0 = 0; j0 < num_columns; j0 += 64) {
      const int32_t j = j0 + lane;
      if (j >= num_columns) break;
      const Column c = column_of(bbo, first_column + j);
      out[out_offset + j] = static_cast<int64_t>(eval_program<K, kStack>(a, c, prog, hashes));
    }
  }
}

using PartialFn = void (*)(const int64_t*, int64_t, const int64_t*, const uint32_t*,
                           const st_partial_item*, int64_t, int32_t, uint32_t, int64_t*);

// Programs of up to kSearchMaxStack slots use the short stack; deeper ones
// (generic batches) the long one.
template <int kStack>
PartialFn select_partial_stack(int k) {
  switch (k) {
    case 0: return partial_search_kernel<0, kStack>;
    case 1: return partial_search_kernel<1, kStack>;
    case 2: return partial_search_kernel<2, kStack>;
    case 3: return partial_search_kernel<3, kStack>;
    case 4: return partial_search_kernel<4, kStack>;
    case 5: return partial_search_kernel<5, kStack>;
    case 6: return partial_search_kernel<6, kStack>;
    case 7: return partial_search_kernel<7, kStack>;
    case 8: return partial_search_kernel<8, kStack>;
    case 9: return partial_search_kernel<9, kStack>;
    case 10: return partial_search_kernel<10, kStack>;
    default: fail("unsupported k_eff ", k);
  }
}

PartialFn select_partial(int k, int max_stack) {
  return max_stack > kSearchMaxStack ? select_partial_stack<kGenericMaxStack>(k)
                                     : select_partial_stack<kSearchMaxStack>(k);
}

int cu_count_here() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    n = 256;
  return n;
}

}  // namespace
}  // namespace st

extern "C" int st_bloom_index_search_partial(const int64_t* bloom_index,
                                             int64_t bloom_index_numel,
                                             const int64_t* bundle_b_offsets,
                                             int64_t num_bundles, const st_search_plan* plan,
                                             const void* plan_blob_device,
                                             const st_partial_item* items_device,
                                             int64_t num_items, int64_t* out, void* stream) {
  using namespace st;
  return guarded([&] {
    ST_CHECK(plan != nullptr, "plan is null");
    ST_CHECK(num_items >= 0 && num_bundles >= 0 && bloom_index_numel >= 0, "negative sizes");
    if (num_items == 0) return;
    ST_CHECK(items_device != nullptr && out != nullptr && bundle_b_offsets != nullptr &&
                 plan_blob_device != nullptr,
             "null device pointer");
    ST_CHECK(bloom_index != nullptr || bloom_index_numel == 0, "bloom_index is null");
    const int64_t per_block = kPartialThreads / 64;
    const int64_t blocks =
        std::min<int64_t>((num_items + per_block - 1) / per_block, 8ll * cu_count_here());
    hipLaunchKernelGGL(select_partial(plan->k_eff, plan->max_stack), dim3(static_cast<unsigned>(blocks)),
                       dim3(kPartialThreads), 0, static_cast<hipStream_t>(stream), bloom_index,
                       bloom_index_numel, bundle_b_offsets,
                       static_cast<const uint32_t*>(plan_blob_device), items_device, num_items,
                       static_cast<int32_t>(plan->hash_k), static_cast<uint32_t>(plan->kp) * 4u,
                       out);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
      throw Error(ST_ERR_HIP, cat("partial search kernel launch failed: ", hipGetErrorString(e)));
  });
}
