// Host side of the batched search: kernel selection, launch and the C ABI
// entry points (the device code is in bloom_search_kernel.hpp).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "bloom_search_kernel.hpp"

namespace st {
namespace {

KernelFn select_kernel(int k, int mode) {
  switch (k) {
    case 0:
    case 1: return search_kernel_for<1>(mode);
    case 2: return search_kernel_for<2>(mode);
    case 3: return search_kernel_for<3>(mode);
    case 4: return search_kernel_for<4>(mode);
    case 5: return search_kernel_for<5>(mode);
    case 6: return search_kernel_for<6>(mode);
    case 7: return search_kernel_for<7>(mode);
    case 8: return search_kernel_for<8>(mode);
    case 9: return search_kernel_for<9>(mode);
    case 10: return search_kernel_for<10>(mode);
    default: fail("unsupported k_eff ", k);
  }
}

int device_cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  static std::mutex mu;
  static std::vector<int> cache;
  std::lock_guard<std::mutex> lock(mu);
  if (dev >= static_cast<int>(cache.size())) cache.resize(dev + 1, 0);
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
            hipSuccess ||
        n <= 0)
      n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

}  // namespace

int cu_count() { return device_cu_count(); }

}  // namespace st

namespace st {
namespace {

// Validates the arguments and launches the search kernel once per batch.
void launch_search(const int64_t* bloom_index, int64_t bloom_index_numel,
                   const int64_t* bundle_b_offsets, int64_t num_bundles,
                   const st_search_plan* plan, const void* plan_blob_device, int mode,
                   void* out, int64_t* counts, int64_t num_docs, hipStream_t stream) {
  ST_CHECK(bundle_b_offsets != nullptr && out != nullptr && plan_blob_device != nullptr,
           "null device pointer");
  ST_CHECK(bloom_index != nullptr || bloom_index_numel == 0, "bloom_index is null");
  ST_CHECK(plan->bound_bundles < 0 || plan->bound_bundles == num_bundles,
           "plan was bound to ", plan->bound_bundles, " bundles, the index has ",
           num_bundles);
  KernelFn fn = select_kernel(plan->k_eff, mode);
  const int grid = static_cast<int>(
      std::min<int64_t>(num_bundles, static_cast<int64_t>(device_cu_count())));
  const char* blob = static_cast<const char*>(plan_blob_device);
  const bool bound = plan->bound_bundles >= 0;
  auto at = [&](uint64_t off) { return reinterpret_cast<const uint32_t*>(blob + off); };
  for (const SearchBatch& bt : plan->batches) {
    hipLaunchKernelGGL(
        fn, dim3(grid), dim3(kSearchThreads), 0, stream, bloom_index, bloom_index_numel,
        bundle_b_offsets, num_bundles, at(bt.off_wave), at(bt.off_insn_start),
        at(bt.off_insns), reinterpret_cast<const uint64_t*>(blob + bt.off_hashes),
        bound ? at(plan->off_bundle_slot) : nullptr,
        bound ? at(plan->off_bundle_order) : nullptr,
        bound ? at(bt.off_bound_start) : nullptr, bound ? at(bt.off_bound) : nullptr,
        bound ? bt.bound_words : 0u, bt.num_terms, static_cast<int32_t>(plan->hash_k),
        num_bundles * 32, out, counts, num_docs);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
      throw Error(ST_ERR_HIP, cat("search kernel launch failed: ", hipGetErrorString(e)));
  }
}

}  // namespace

void compact_scan_counts(int64_t* counts, int64_t num_queries, int64_t nch,
                         int64_t* row_offsets, hipStream_t s);
void compact_zero_offsets(int64_t* row_offsets, int64_t n, hipStream_t s);

}  // namespace st

extern "C" int st_bloom_index_search_batch(
    const int64_t* bloom_index, int64_t bloom_index_numel,
    const int64_t* bundle_b_offsets, int64_t num_bundles,
    const st_search_plan* plan, const void* plan_blob_device,
    int return_bool_mask, void* out, void* stream) {
  using namespace st;
  return guarded([&] {
    ST_CHECK(plan != nullptr, "plan is null");
    ST_CHECK(num_bundles >= 0 && bloom_index_numel >= 0, "negative sizes");
    if (plan->num_queries == 0 || num_bundles == 0) return;
    launch_search(bloom_index, bloom_index_numel, bundle_b_offsets, num_bundles, plan,
                  plan_blob_device, return_bool_mask ? kOutBool : kOutPacked, out, nullptr, 0,
                  static_cast<hipStream_t>(stream));
  });
}

extern "C" int st_bloom_index_search_batch_counts(
    const int64_t* bloom_index, int64_t bloom_index_numel,
    const int64_t* bundle_b_offsets, int64_t num_bundles,
    const st_search_plan* plan, const void* plan_blob_device, int64_t num_docs,
    int64_t* packed_out, void* workspace, int64_t* row_offsets, void* stream) {
  using namespace st;
  return guarded([&] {
    ST_CHECK(plan != nullptr, "plan is null");
    ST_CHECK(num_bundles >= 0 && bloom_index_numel >= 0, "negative sizes");
    ST_CHECK(num_docs >= 0, "num_docs must be non-negative, got ", num_docs);
    ST_CHECK(row_offsets != nullptr, "row_offsets is null");
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (plan->num_queries == 0 || num_bundles == 0) {
      compact_zero_offsets(row_offsets, plan->num_queries + 1, s);
      return;
    }
    ST_CHECK(workspace != nullptr, "workspace is null");
    int64_t* counts = static_cast<int64_t*>(workspace);
    launch_search(bloom_index, bloom_index_numel, bundle_b_offsets, num_bundles, plan,
                  plan_blob_device, kOutCounts, packed_out, counts, num_docs, s);
    // one chunk of the compaction is one bundle: counts are already per item
    compact_scan_counts(counts, plan->num_queries, num_bundles, row_offsets, s);
  });
}
