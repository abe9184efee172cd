// Host side of the batched search: kernel selection, launch and the C ABI
// entry points (the device code is in bloom_search_kernel.hpp).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "bloom_search_kernel.hpp"

namespace st {
namespace {

WideFn select_wide_kernel(int k) {
  switch (k) {
    case 1: return wide_kernel_for<1>();
    case 2: return wide_kernel_for<2>();
    case 3: return wide_kernel_for<3>();
    case 4: return wide_kernel_for<4>();
    case 5: return wide_kernel_for<5>();
    case 6: return wide_kernel_for<6>();
    case 7: return wide_kernel_for<7>();
    default: return nullptr;
  }
}

KernelFn select_kernel(int k, int mode, bool quad) {
  switch (k) {
    case 0:
    case 1: return search_kernel_for<1>(mode, quad);
    case 2: return search_kernel_for<2>(mode, quad);
    case 3: return search_kernel_for<3>(mode, quad);
    case 4: return search_kernel_for<4>(mode, quad);
    case 5: return search_kernel_for<5>(mode, quad);
    case 6: return search_kernel_for<6>(mode, quad);
    case 7: return search_kernel_for<7>(mode, quad);
    case 8: return search_kernel_for<8>(mode, quad);
    case 9: return search_kernel_for<9>(mode, quad);
    case 10: return search_kernel_for<10>(mode, quad);
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

// ------------------------------------------------- width binding on the device
// The host-side equivalent is st_search_plan_bind_widths (search_plan.cpp).

constexpr int kCensusThreads = 1024;
constexpr int kCensusCap = 4096;  // distinct widths tracked; more stay unslotted
constexpr int kCensusCache = 16384;  // bundle widths kept in LDS between passes
constexpr long long kCensusEmpty = -1;

__device__ __forceinline__ uint32_t census_hash(long long w) {
  return static_cast<uint32_t>((static_cast<unsigned long long>(w) * 0x9E3779B97F4A7C15ull) >> 52) &
         (kCensusCap - 1);
}

// Entry of width w in the table, inserting it when `insert`; -1 when absent
// (or the table is full).
__device__ int census_find(long long* keys, long long w, bool insert) {
  uint32_t h = census_hash(w);
  for (int probe = 0; probe < kCensusCap; ++probe, h = (h + 1) & (kCensusCap - 1)) {
    long long k = keys[h];
    if (k == w) return static_cast<int>(h);
    if (k == kCensusEmpty) {
      if (!insert) return -1;
      k = static_cast<long long>(atomicCAS(reinterpret_cast<unsigned long long*>(keys + h),
                                           static_cast<unsigned long long>(kCensusEmpty),
                                           static_cast<unsigned long long>(w)));
      if (k == kCensusEmpty || k == w) return static_cast<int>(h);
    }
  }
  return -1;
}

__device__ __forceinline__ long long bundle_width(const int64_t* bbo, int64_t i) {
  const int64_t w = bbo[i + 1] - bbo[i];
  return w > 0 ? w : 0;
}

// One workgroup: the kMaxWidthSlots most frequent widths get slots (ties to
// the smaller width), every bundle its slot, and the visiting order groups
// bundles by slot (a counting sort; order within a slot is arbitrary).
__global__ __launch_bounds__(kCensusThreads) void width_census_kernel(
    const int64_t* __restrict__ bbo, int64_t nb, uint32_t* __restrict__ num_slots,
    int64_t* __restrict__ slot_width, uint32_t* __restrict__ bundle_slot,
    uint32_t* __restrict__ bundle_order) {
  __shared__ long long keys[kCensusCap];
  __shared__ uint32_t count[kCensusCap];
  __shared__ uint32_t slot_of[kCensusCap];
  __shared__ uint32_t dense[kCensusCap];
  __shared__ uint32_t n_dense;
  __shared__ uint32_t cursor[kMaxWidthSlots + 1];
  __shared__ uint32_t wcache[kCensusCache];  // widths of the first bundles
  // Width of bundle i: from the LDS cache after the first pass (widths of
  // 2^32 rows and more are read again).
  auto width_of = [&](int64_t i) -> long long {
    const uint32_t c = i < kCensusCache ? wcache[i] : 0xFFFFFFFFu;
    return c != 0xFFFFFFFFu ? static_cast<long long>(c) : bundle_width(bbo, i);
  };
  for (int e = threadIdx.x; e < kCensusCap; e += kCensusThreads) {
    keys[e] = kCensusEmpty;
    count[e] = 0u;
    slot_of[e] = kNoWidthSlot;
  }
  if (threadIdx.x == 0) n_dense = 0u;
  if (threadIdx.x <= kMaxWidthSlots) cursor[threadIdx.x] = 0u;
  __syncthreads();
  for (int64_t i = threadIdx.x; i < nb; i += kCensusThreads) {
    const long long w = bundle_width(bbo, i);
    if (i < kCensusCache) wcache[i] = w < 0xFFFFFFFFll ? static_cast<uint32_t>(w) : 0xFFFFFFFFu;
    const int e = census_find(keys, w, true);
    if (e >= 0) atomicAdd(count + e, 1u);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < kCensusCap; e += kCensusThreads)
    if (keys[e] != kCensusEmpty) dense[atomicAdd(&n_dense, 1u)] = static_cast<uint32_t>(e);
  __syncthreads();
  const uint32_t n = n_dense;
  for (uint32_t a = threadIdx.x; a < n; a += kCensusThreads) {
    const uint32_t e = dense[a];
    const uint32_t c = count[e];
    const long long w = keys[e];
    uint32_t rank = 0;
    for (uint32_t b = 0; b < n; ++b) {
      const uint32_t f = dense[b];
      rank += (count[f] > c || (count[f] == c && keys[f] < w)) ? 1u : 0u;
    }
    if (rank < static_cast<uint32_t>(kMaxWidthSlots)) {
      slot_of[e] = rank;
      slot_width[rank] = w;
    }
  }
  if (threadIdx.x == 0) *num_slots = n < static_cast<uint32_t>(kMaxWidthSlots) ? n : kMaxWidthSlots;
  __syncthreads();
  for (int64_t i = threadIdx.x; i < nb; i += kCensusThreads) {
    const int e = census_find(keys, width_of(i), false);
    const uint32_t sl = e >= 0 ? slot_of[e] : kNoWidthSlot;
    bundle_slot[i] = sl;
    atomicAdd(cursor + (sl == kNoWidthSlot ? kMaxWidthSlots : sl), 1u);
  }
  __syncthreads();
  if (threadIdx.x == 0) {  // bucket sizes -> bucket starts
    // num_slots[1]: every bundle has a slot, and every slot width is wide
    bool all_wide = cursor[kMaxWidthSlots] == 0;
    const uint32_t ns = n < static_cast<uint32_t>(kMaxWidthSlots) ? n : kMaxWidthSlots;
    for (uint32_t s = 0; s < ns; ++s) all_wide &= wide_width(slot_width[s]);
    num_slots[1] = all_wide ? 1u : 0u;
    uint32_t run = 0;
    for (int b = 0; b <= kMaxWidthSlots; ++b) {
      const uint32_t c = cursor[b];
      cursor[b] = run;
      run += c;
    }
  }
  __syncthreads();
  for (int64_t i = threadIdx.x; i < nb; i += kCensusThreads) {
    const int e = census_find(keys, width_of(i), false);
    const uint32_t sl = e >= 0 ? slot_of[e] : kNoWidthSlot;
    const uint32_t pos = atomicAdd(cursor + (sl == kNoWidthSlot ? kMaxWidthSlots : sl), 1u);
    bundle_order[pos] = static_cast<uint32_t>(i);
  }
}

// Position r of a term at width b, as term_positions (search_plan.cpp) and
// signature_match (bloom_index_search.cpp:40-61) resolve it: over hashes
// p < hash_k, b_p = (int16)(h[p] % b), repeats skipped, at most k_eff kept,
// unused slots repeat the first; LDS byte offsets for staged widths, rows
// relative to the bundle start otherwise.
__device__ uint32_t device_term_position(const uint64_t* h, int hash_k, int k_eff, int64_t b,
                                         int r) {
  int16_t found[kMaxSearchK];
  int cnt = 0;
  if (b > 0) {
    for (int p = 0; p < hash_k && cnt < k_eff; ++p) {
      const int16_t bp = static_cast<int16_t>(h[p] % static_cast<uint64_t>(b));
      bool dup = false;
      for (int j = 0; j < cnt; ++j) dup |= found[j] == bp;
      if (!dup) found[cnt++] = bp;
    }
  }
  const int16_t row = cnt == 0 ? 0 : (r < cnt ? found[r] : found[0]);
  if (b <= kSearchTileRows)
    return static_cast<uint32_t>(cnt == 0 ? kSearchZerosRow : row) * 256u;
  if (wide_width(b))
    return static_cast<uint32_t>(cnt == 0 ? kWideZerosRow : row) * kWideSliceBytes;
  return cnt == 0 ? static_cast<uint32_t>(kPosZeros)
                  : static_cast<uint32_t>(static_cast<int32_t>(row));
}

// Expands a batch's width-block template for every slot.
__global__ void bind_fill_kernel(const uint32_t* __restrict__ tmpl,
                                 const uint32_t* __restrict__ code, uint32_t words,
                                 const uint64_t* __restrict__ hashes, int hash_k, int k_eff,
                                 const uint32_t* __restrict__ num_slots,
                                 const int64_t* __restrict__ slot_width,
                                 uint32_t* __restrict__ bound) {
  const uint32_t sl = blockIdx.y;
  if (sl >= *num_slots) return;
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= words) return;
  const int64_t b = slot_width[sl];
  const uint32_t c = code[i];
  uint32_t v;
  if (c == kTmplCopy) {
    v = tmpl[i];
  } else if (c == kTmplOnes) {
    v = b <= kSearchTileRows ? static_cast<uint32_t>(kSearchOnesRow) * 256u
        : wide_width(b)      ? static_cast<uint32_t>(kWideOnesRow) * kWideSliceBytes
                             : static_cast<uint32_t>(kPosOnes);
  } else if (c == kTmplZeros) {
    v = b <= kSearchTileRows ? static_cast<uint32_t>(kSearchZerosRow) * 256u
        : wide_width(b)      ? static_cast<uint32_t>(kWideZerosRow) * kWideSliceBytes
                             : static_cast<uint32_t>(kPosZeros);
  } else {
    const uint32_t t = (c >> 4) - 1u;
    v = device_term_position(hashes + static_cast<uint64_t>(t) * hash_k, hash_k, k_eff, b,
                             static_cast<int>(c & 15u));
  }
  bound[static_cast<uint64_t>(sl) * words + i] = v;
}

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
  const int grid = static_cast<int>(
      std::min<int64_t>(num_bundles, static_cast<int64_t>(device_cu_count())));
  const char* blob = static_cast<const char*>(plan_blob_device);
  const bool bound = plan->bound_bundles >= 0;
  auto at = [&](uint64_t off) { return reinterpret_cast<const uint32_t*>(blob + off); };
  if (plan->device_bind) {
    // Width binding on the device, ahead of the search on the same stream.
    char* dev = const_cast<char*>(blob);
    auto* nsl = reinterpret_cast<uint32_t*>(dev + plan->off_num_slots);
    auto* sw = reinterpret_cast<int64_t*>(dev + plan->off_slot_width);
    hipLaunchKernelGGL(width_census_kernel, dim3(1), dim3(kCensusThreads), 0, stream,
                       bundle_b_offsets, num_bundles, nsl, sw,
                       reinterpret_cast<uint32_t*>(dev + plan->off_bundle_slot),
                       reinterpret_cast<uint32_t*>(dev + plan->off_bundle_order));
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
      throw Error(ST_ERR_HIP, cat("width census launch failed: ", hipGetErrorString(e)));
    for (const SearchBatch& bt : plan->batches) {
      if (bt.bound_words == 0) continue;
      hipLaunchKernelGGL(bind_fill_kernel, dim3((bt.bound_words + 255) / 256, kMaxWidthSlots),
                         dim3(256), 0, stream, at(bt.off_tmpl), at(bt.off_tmpl_code),
                         bt.bound_words, reinterpret_cast<const uint64_t*>(blob + bt.off_hashes),
                         static_cast<int>(plan->hash_k), plan->k_eff, nsl, sw,
                         reinterpret_cast<uint32_t*>(dev + bt.off_bound));
      e = hipGetLastError();
      if (e != hipSuccess)
        throw Error(ST_ERR_HIP, cat("bind fill launch failed: ", hipGetErrorString(e)));
    }
  }
  // Wide bundles (kSearchTileRows < b <= kWideRows, width-bound) have their
  // literal streams evaluated by the column-slice kernel, in packed mode;
  // the per-batch kernels then skip those streams there.  With host-bound
  // widths the launch is decided here; with device binding the kernel
  // returns at once when no slot width is wide.
  WideFn wide_fn = nullptr;
  if (bound && mode == kOutPacked && plan->off_wide != 0) {
    wide_fn = select_wide_kernel(plan->k_eff);
    if (wide_fn != nullptr && !plan->device_bind) {
      bool any = false;
      for (int64_t w : plan->slot_width) any |= wide_width(w);
      if (!any) wide_fn = nullptr;
    }
  }
  for (const SearchBatch& bt : plan->batches) {
    // 2 tells the kernel that every program of the batch is in the stream,
    // so that wide bundles need nothing from it
    uint32_t wide_flag = 0;
    if (wide_fn != nullptr) {
      const auto* wo = reinterpret_cast<const uint32_t*>(plan->blob.data() + bt.off_wave);
      const auto* sk = reinterpret_cast<const uint32_t*>(plan->blob.data() + bt.off_stream_skip);
      bool all = true;
      for (int w = 0; w < kSearchWaves; ++w) all &= wo[w + 1] - wo[w] == sk[w];
      wide_flag = all ? 2u : 1u;
    }
    // Nothing for the per-batch kernel when the wide-bundle kernel covers
    // every bundle (known here with host-bound widths).
    if (wide_flag == 2 && !plan->device_bind && plan->all_wide) continue;
    // Quad-lane stream evaluation when the batch's literal stream fits the
    // LDS area after the tile and a stream step holds whole quads (k <= 7).
    const int kk = std::max(plan->k_eff, 1);
    const bool quad = bound && bt.stream_words != 0 &&
                      bt.stream_words <= kQuadStreamMaxWords &&
                      stream_block_records(kk) >= 4;
    KernelFn fn = select_kernel(plan->k_eff, mode, quad);
    hipLaunchKernelGGL(
        fn, dim3(grid), dim3(kSearchThreads), 0, stream, bloom_index, bloom_index_numel,
        bundle_b_offsets, num_bundles, at(bt.off_wave), at(bt.off_insn_start),
        at(bt.off_insns), reinterpret_cast<const uint64_t*>(blob + bt.off_hashes),
        bound ? at(plan->off_bundle_slot) : nullptr,
        // The quad instance reads its programs from LDS, so it visits bundles
        // in index order: neighbouring workgroups then write neighbouring
        // output columns at the same time.
        bound && !quad ? at(plan->off_bundle_order) : nullptr,
        bound ? at(bt.off_bound_start) : nullptr, bound ? at(bt.off_bound) : nullptr,
        bound ? bt.bound_words : 0u, bound ? at(bt.off_stream_wave) : nullptr,
        bound ? at(bt.off_stream_skip) : nullptr, bound ? bt.stream_off : 0u,
        bound ? bt.stream_words : 0u, bound ? bt.stream_masks : 0u, bt.num_terms,
        static_cast<int32_t>(plan->hash_k),
        num_bundles * 32, out, counts, num_docs, wide_flag,
        plan->device_bind ? at(plan->off_num_slots) : nullptr);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
      throw Error(ST_ERR_HIP, cat("search kernel launch failed: ", hipGetErrorString(e)));
  }
  if (wide_fn != nullptr) {
    hipLaunchKernelGGL(wide_fn, dim3(grid), dim3(kSearchThreads), 0, stream, bloom_index,
                       bloom_index_numel, bundle_b_offsets, num_bundles,
                       at(plan->off_bundle_slot),
                       plan->device_bind ? at(plan->off_num_slots) : nullptr,
                       plan->device_bind
                           ? reinterpret_cast<const int64_t*>(blob + plan->off_slot_width)
                           : nullptr,
                       reinterpret_cast<const uint32_t*>(blob), at(plan->off_wide),
                       num_bundles * 32, static_cast<int64_t*>(out));
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
      throw Error(ST_ERR_HIP, cat("wide search kernel launch failed: ", hipGetErrorString(e)));
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
