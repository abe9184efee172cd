// Launch of the generic search kernel (bloom_generic.hip) for one generic
// batch of a plan.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

#include "search_plan.hpp"

namespace st {

// Output modes, as the batch kernels': int64 words, one byte per doc, int64
// words plus per-(row, bundle) match counts of docs below num_docs.
constexpr int kGenericPacked = 0;
constexpr int kGenericBool = 1;
constexpr int kGenericCounts = 2;

void launch_generic_batch(const int64_t* index, int64_t index_numel, const int64_t* bbo,
                          int64_t num_bundles, const void* plan_blob_device,
                          const SearchBatch& bt, const std::vector<uint32_t>& starts,
                          const std::vector<uint32_t>& insns, int k_eff, int hash_k, int kp,
                          int out_mode, void* out, int64_t* counts, int64_t num_docs,
                          hipStream_t stream);

}  // namespace st
