// Host side of the batched search: kernel selection, launch and the C ABI
// entry points (the device code is in bloom_search_kernel.hpp).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "bloom_generic.hpp"
#include "bloom_search_kernel.hpp"
#include "wide_balance.hpp"

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

constexpr int kBindThreads = 1024;
constexpr int kBindGrid = 256;     // workgroups of the binding kernel
// Distinct widths the census tracks.  An index with more gets no slots at
// all (every bundle resolves its positions itself): whether the table
// overflows does not depend on the order of insertions, so every workgroup
// of the binding kernel reaches the same decision.
constexpr int kCensusCap = 2048;
constexpr int kBindChunk = 16;     // bundle widths loaded per thread at a time
constexpr int kBindHashBatch = 8;  // term hashes loaded per thread at a time
constexpr int kBindFillBatch = 4;  // template words loaded per thread at a time
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

// Runs f(i, width of bundle i) over all bundles, this thread's share,
// kBindChunk widths loaded before any is used (the loads overlap).
template <typename F>
__device__ __forceinline__ void for_each_width(const int64_t* bbo, int64_t nb, F&& f) {
  for (int64_t base = 0; base < nb; base += static_cast<int64_t>(kBindThreads) * kBindChunk) {
    long long w[kBindChunk];
#pragma unroll
    for (int j = 0; j < kBindChunk; ++j) {
      const int64_t i = base + threadIdx.x + static_cast<int64_t>(j) * kBindThreads;
      w[j] = i < nb ? bundle_width(bbo, i) : 0;
    }
#pragma unroll
    for (int j = 0; j < kBindChunk; ++j) {
      const int64_t i = base + threadIdx.x + static_cast<int64_t>(j) * kBindThreads;
      if (i < nb) f(i, w[j]);
    }
  }
}

// The bundle widths a thread visits, loaded once and kept in registers for
// the census passes when they fit (nb <= kBindThreads * kBindChunk); the
// passes over a larger index reload them.
struct WidthRegs {
  long long w[kBindChunk];
  bool held;
};

__device__ __forceinline__ void load_widths(const int64_t* bbo, int64_t nb, WidthRegs& r) {
  r.held = nb <= static_cast<int64_t>(kBindThreads) * kBindChunk;
  if (!r.held) return;
#pragma unroll
  for (int j = 0; j < kBindChunk; ++j) {
    const int64_t i = threadIdx.x + static_cast<int64_t>(j) * kBindThreads;
    r.w[j] = i < nb ? bundle_width(bbo, i) : 0;
  }
}

// for_each_width from the registers when they hold the widths.
template <typename F>
__device__ __forceinline__ void each_width(const int64_t* bbo, int64_t nb, const WidthRegs& r, F&& f) {
  if (!r.held) {
    for_each_width(bbo, nb, f);
    return;
  }
#pragma unroll
  for (int j = 0; j < kBindChunk; ++j) {
    const int64_t i = threadIdx.x + static_cast<int64_t>(j) * kBindThreads;
    if (i < nb) f(i, r.w[j]);
  }
}

// Width binding of a device-bound plan (the host-side equivalent is
// st_search_plan_bind_widths, search_plan.cpp), in two launches.
//
// bind_prologue_kernel: workgroups [0, upload_groups) copy the plan's bytes
// from pinned host memory into the device blob (when the caller left that
// to the search call); workgroup `upload_groups` takes the census of the
// bundle widths -- every width gets a slot, in increasing width, when there
// are at most kMaxWidthSlots of them, else the kMaxWidthSlots most frequent
// do (ties to the smaller width) -- and writes the slot table, every bundle's slot
// and, when `bundle_order` is given, a visiting order grouped by slot (a
// counting sort; order within a slot is arbitrary) -- with `order_if_wide`
// only when some slot width is wide (the wide-bundle kernel's order).  The
// census reads only the bundle offsets, so it runs while the copy waits on
// PCIe.  With `upload_done` set, each upload workgroup then stores
// `upload_value` to upload_done[its index]: the host can reuse the pinned
// source once every group's word holds the value (no event on the stream).
constexpr int kUploadPerThread = 4;   // 16-byte pieces per thread of an upload group
constexpr uint64_t kUploadGroupBytes = 16ull * kBindThreads * kUploadPerThread;

__global__ __launch_bounds__(kBindThreads) void bind_prologue_kernel(
    const uint8_t* __restrict__ host_src, uint8_t* __restrict__ blob, int64_t upload_bytes,
    uint32_t upload_groups, unsigned long long* upload_done, unsigned long long upload_value,
    const int64_t* __restrict__ bbo, int64_t nb,
    uint32_t* __restrict__ num_slots, int64_t* __restrict__ slot_width,
    uint32_t* __restrict__ bundle_slot, uint32_t* __restrict__ bundle_order,
    uint32_t order_if_wide) {
  const int tid = threadIdx.x;
  if (blockIdx.x < upload_groups) {
    typedef uint32_t v4 __attribute__((ext_vector_type(4)));
    const int64_t vec = upload_bytes / 16;
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kBindThreads * kUploadPerThread;
    v4 v[kUploadPerThread];
#pragma unroll
    for (int j = 0; j < kUploadPerThread; ++j) {
      const int64_t i = base + tid + static_cast<int64_t>(j) * kBindThreads;
      if (i < vec) v[j] = reinterpret_cast<const v4*>(host_src)[i];
    }
#pragma unroll
    for (int j = 0; j < kUploadPerThread; ++j) {
      const int64_t i = base + tid + static_cast<int64_t>(j) * kBindThreads;
      if (i < vec) reinterpret_cast<v4*>(blob)[i] = v[j];
    }
    if (blockIdx.x == 0 && tid < 16 && vec * 16 + tid < upload_bytes) blob[vec * 16 + tid] = host_src[vec * 16 + tid];
    if (upload_done != nullptr) {
      // every thread's loads of the source have returned (their data went
      // into the stores above) before any thread passes the barrier
      __syncthreads();
      if (tid == 0)
        __hip_atomic_store(upload_done + blockIdx.x, upload_value, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
    }
    return;
  }
  if (num_slots == nullptr) return;  // host-bound plan: nothing to bind
  __shared__ long long keys[kCensusCap];
  __shared__ uint32_t count[kCensusCap];
  __shared__ uint32_t slot_of[kCensusCap];
  __shared__ uint32_t dense[kCensusCap];     // table entry of each distinct width
  __shared__ long long dense_w[kCensusCap];  // its width and count, stored flat so
  __shared__ uint32_t dense_c[kCensusCap];   // that the rank loop reads no pointer chain
  __shared__ uint32_t n_dense;
  __shared__ uint32_t overflow;
  __shared__ long long s_width[kMaxWidthSlots];
  __shared__ uint32_t cursor[kMaxWidthSlots + 1];
  __shared__ uint32_t any_wide, unslotted;
  WidthRegs wr;
  load_widths(bbo, nb, wr);  // in flight while the table is cleared
  for (int e = tid; e < kCensusCap; e += kBindThreads) {
    keys[e] = kCensusEmpty;
    count[e] = 0u;
    slot_of[e] = kNoWidthSlot;
  }
  if (tid == 0) {
    n_dense = 0u;
    overflow = 0u;
    any_wide = 0u;
    unslotted = 0u;
  }
  if (tid <= kMaxWidthSlots) cursor[tid] = 0u;
  __syncthreads();
  // the distinct widths (no counts yet: with at most kMaxWidthSlots of them
  // every width gets a slot and how often each occurs does not matter)
  each_width(bbo, nb, wr, [&](int64_t, long long w) {
    if (overflow) return;  // the outcome is decided
    if (census_find(keys, w, true) < 0) overflow = 1u;
  });
  __syncthreads();
  if (overflow) {  // no slots: clear the table (census_find then finds nothing)
    for (int e = tid; e < kCensusCap; e += kBindThreads) keys[e] = kCensusEmpty;
    __syncthreads();
  }
  for (int e = tid; e < kCensusCap; e += kBindThreads) {
    const long long w = keys[e];
    if (w != kCensusEmpty) {
      const uint32_t a = atomicAdd(&n_dense, 1u);
      dense[a] = static_cast<uint32_t>(e);
      dense_w[a] = w;
    }
  }
  __syncthreads();
  const uint32_t n = n_dense;
  // slot of each width: with more widths than slots, the kMaxWidthSlots
  // most frequent (ties to the smaller width) after counting them;
  // otherwise all of them in increasing width
  const bool counted = n > static_cast<uint32_t>(kMaxWidthSlots);  // uniform
  if (counted) {
    each_width(bbo, nb, wr, [&](int64_t, long long w) {
      atomicAdd(count + census_find(keys, w, false), 1u);  // every width is in the table
    });
    __syncthreads();
    for (uint32_t a = tid; a < n; a += kBindThreads) dense_c[a] = count[dense[a]];
    __syncthreads();
  }
  for (uint32_t a = tid; a < n; a += kBindThreads) {
    const long long w = dense_w[a];
    uint32_t rank = 0;
    if (counted) {
      const uint32_t c = dense_c[a];
#pragma unroll 8
      for (uint32_t b = 0; b < n; ++b) {
        const uint32_t cb = dense_c[b];
        rank += (cb > c || (cb == c && dense_w[b] < w)) ? 1u : 0u;
      }
    } else {
#pragma unroll 8
      for (uint32_t b = 0; b < n; ++b) rank += dense_w[b] < w ? 1u : 0u;
    }
    if (rank < static_cast<uint32_t>(kMaxWidthSlots)) {
      slot_of[dense[a]] = rank;
      s_width[rank] = w;
      if (wide_width(w)) any_wide = 1u;
    }
  }
  __syncthreads();
  const uint32_t ns = n < static_cast<uint32_t>(kMaxWidthSlots) ? n : kMaxWidthSlots;
  if (tid < static_cast<int>(ns)) slot_width[tid] = s_width[tid];
  // the visiting order grouped by slot, when asked for (bucket counts only
  // then)
  const bool order = bundle_order != nullptr && (order_if_wide == 0u || any_wide != 0u);  // uniform
  each_width(bbo, nb, wr, [&](int64_t i, long long w) {
    const int e = census_find(keys, w, false);
    const uint32_t sl = e >= 0 ? slot_of[e] : kNoWidthSlot;
    bundle_slot[i] = sl;
    if (sl == kNoWidthSlot) unslotted = 1u;
    if (order) atomicAdd(cursor + (sl == kNoWidthSlot ? kMaxWidthSlots : sl), 1u);
  });
  __syncthreads();
  static_assert(kMaxWidthSlots == 64, "one wave scans the slot buckets");
  if (tid < 64) {
    // num_slots[1]: every bundle has a slot, and every slot width is wide
    const bool narrow = tid < static_cast<int>(ns) && !wide_width(s_width[tid]);
    const bool all_wide = __ballot(narrow) == 0ull && unslotted == 0u;
    if (order) {
      // bucket sizes -> bucket starts (exclusive scan over the wave; the
      // unslotted bucket goes last)
      const uint32_t c = cursor[tid];
      uint32_t incl = c;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const uint32_t y = __shfl_up(incl, d, 64);
        if (tid >= d) incl += y;
      }
      cursor[tid] = incl - c;
      if (tid == 63) cursor[kMaxWidthSlots] = incl;
    }
    if (tid == 0) {
      num_slots[0] = ns;
      num_slots[1] = all_wide ? 1u : 0u;
      num_slots[2] = any_wide;
    }
  }
  if (order) {
    __syncthreads();
    each_width(bbo, nb, wr, [&](int64_t i, long long w) {
      const int e = census_find(keys, w, false);
      const uint32_t sl = e >= 0 ? slot_of[e] : kNoWidthSlot;
      const uint32_t at = atomicAdd(cursor + (sl == kNoWidthSlot ? kMaxWidthSlots : sl), 1u);
      bundle_order[at] = static_cast<uint32_t>(i);
    });
  }
}

// bind_fill_kernel: workgroup g serves slot g % ns and part g / ns of the
// slot's width blocks: it resolves the row positions of every batch term at
// the slot's width once (as signature_match does, bloom_index_search.cpp:
// 40-61: b_p = (int16)(h[p] % b) over p < hash_k, repeats skipped, at most
// k_eff kept, unused positions repeat the first) and expands its part of
// every batch's width-block template.  On a wide slot the literal stream's
// positions are written unit by unit instead (its part of the units), in
// the read order balance_wide_choice gives them; the words of the two passes
// are disjoint, so no workgroup reads what another writes.
__global__ __launch_bounds__(kBindThreads) void bind_fill_kernel(
    char* __restrict__ blob, uint64_t off_table, uint32_t n_batches, int hash_k, int k_eff, int kp,
    const uint32_t* __restrict__ num_slots, const int64_t* __restrict__ slot_width) {
  __shared__ uint32_t pos[kSearchPosSlots];
  const int tid = threadIdx.x;
  const uint32_t ns = num_slots[0];
  if (ns == 0) return;
  const uint32_t parts = gridDim.x / ns;
  if (parts == 0 || blockIdx.x >= parts * ns) return;
  const uint32_t sl = blockIdx.x % ns, part = blockIdx.x / ns;
  const long long b = slot_width[sl];
  const FastMod64 fm = make_fastmod_dev(static_cast<uint64_t>(b > 0 ? b : 1));
  const bool staged = b <= kSearchTileRows, wide = wide_width(b);
  const uint32_t ones = staged ? static_cast<uint32_t>(kSearchOnesRow) * 256u
                        : wide ? static_cast<uint32_t>(kWideOnesRow) * kWideSliceBytes
                               : static_cast<uint32_t>(kPosOnes);
  const uint32_t zeros = staged ? static_cast<uint32_t>(kSearchZerosRow) * 256u
                         : wide ? static_cast<uint32_t>(kWideZerosRow) * kWideSliceBytes
                                : static_cast<uint32_t>(kPosZeros);
  const uint64_t* table = reinterpret_cast<const uint64_t*>(blob + off_table);
  // a template word at this slot's width; pos holds the batch's positions
  const auto resolve = [&](uint32_t c, uint32_t t) -> uint32_t {
    if (c == kTmplCopy) return t;
    if (c == kTmplOnes) return ones;
    if (c == kTmplZeros) return zeros;
    return pos[((c >> 4) - 1u) * kp + (c & 15u)];
  };
  // positions per stream record (the unit pass runs when balance_applies)
  const int ks = k_eff > 1 ? k_eff : 1;
  for (uint32_t t = 0; t < n_batches; ++t) {
    const uint64_t* e = table + static_cast<uint64_t>(t) * kBindTableWords;
    const uint32_t* tmpl = reinterpret_cast<const uint32_t*>(blob + e[0]);
    const uint32_t* code = reinterpret_cast<const uint32_t*>(blob + e[1]);
    const uint64_t* hashes = reinterpret_cast<const uint64_t*>(blob + e[2]);
    uint32_t* bound = reinterpret_cast<uint32_t*>(blob + e[3]);
    const uint32_t words = static_cast<uint32_t>(e[4]);
    const uint32_t n_terms = static_cast<uint32_t>(e[5]);
    const uint32_t* units = reinterpret_cast<const uint32_t*>(blob + e[6]);
    const uint32_t n_units = wide ? static_cast<uint32_t>(e[7]) : 0u;
    // stream words left to the unit pass (none unless it runs)
    const uint32_t s_lo = static_cast<uint32_t>(e[8]);
    const uint32_t s_hi = n_units != 0 ? s_lo + static_cast<uint32_t>(e[8] >> 32) : s_lo;
    if (words == 0) continue;
    const uint32_t w0 = static_cast<uint32_t>(static_cast<uint64_t>(words) * part / parts);
    const uint32_t w1 = static_cast<uint32_t>(static_cast<uint64_t>(words) * (part + 1) / parts);
    // the part's first template words, loaded before the positions are
    // resolved (they do not depend on them)
    uint32_t c[kBindFillBatch], tw[kBindFillBatch];
#pragma unroll
    for (int j = 0; j < kBindFillBatch; ++j) {
      const uint32_t i = w0 + tid + j * kBindThreads;
      c[j] = i < w1 ? code[i] : kTmplCopy;
      tw[j] = i < w1 ? tmpl[i] : 0u;
    }
    // the previous batch's positions are no longer read (for the first batch
    // no barrier: its wait for all loads would hold the hashes' loads behind
    // the template words')
    if (t != 0) __syncthreads();
    for (uint32_t u = tid; u < n_terms; u += kBindThreads) {
      int16_t found[kMaxSearchK];
      int cnt = 0;
      if (b > 0) {
        const uint64_t* h = hashes + static_cast<uint64_t>(u) * hash_k;
        for (int p0 = 0; p0 < hash_k && cnt < k_eff; p0 += kBindHashBatch) {
          // the batch's hashes are loaded before any is used (one wait)
          uint64_t hv[kBindHashBatch];
#pragma unroll
          for (int j = 0; j < kBindHashBatch; ++j) hv[j] = p0 + j < hash_k ? h[p0 + j] : 0;
#pragma unroll
          for (int j = 0; j < kBindHashBatch; ++j) {
            if (p0 + j >= hash_k || cnt >= k_eff) break;
            const int16_t bp = static_cast<int16_t>(fast_mod(hv[j], fm));
            bool dup = false;
            for (int q = 0; q < cnt; ++q) dup |= found[q] == bp;
            if (!dup) found[cnt++] = bp;
          }
        }
      }
      for (int r = 0; r < kp; ++r) {
        const int16_t row = cnt == 0 ? 0 : (r < cnt ? found[r] : found[0]);
        uint32_t v;
        if (cnt == 0) v = zeros;
        else if (staged) v = static_cast<uint32_t>(row) * 256u;
        else if (wide) v = static_cast<uint32_t>(row) * kWideSliceBytes;
        else v = static_cast<uint32_t>(static_cast<int32_t>(row));
        pos[u * kp + r] = v;
      }
    }
    __syncthreads();
    uint32_t* dst = bound + static_cast<uint64_t>(sl) * words;
    for (uint32_t i0 = w0; i0 < w1; i0 += kBindThreads * kBindFillBatch) {
      // every load of the batch is issued before any value is used (the
      // first batch's before the positions)
      if (i0 != w0) {
#pragma unroll
        for (int j = 0; j < kBindFillBatch; ++j) {
          const uint32_t i = i0 + tid + j * kBindThreads;
          c[j] = i < w1 ? code[i] : kTmplCopy;
          tw[j] = i < w1 ? tmpl[i] : 0u;
        }
      }
#pragma unroll
      for (int j = 0; j < kBindFillBatch; ++j) {
        const uint32_t i = i0 + tid + j * kBindThreads;
        if (i >= w1) break;
        if (c[j] != kTmplCopy && i >= s_lo && i < s_hi) continue;  // the unit pass's
        dst[i] = resolve(c[j], tw[j]);
      }
    }
    if (n_units == 0) continue;
    const int srw = bound_record_words(ks);
    const uint32_t u0 = static_cast<uint32_t>(static_cast<uint64_t>(n_units) * part / parts);
    const uint32_t u1 = static_cast<uint32_t>(static_cast<uint64_t>(n_units) * (part + 1) / parts);
    for (uint32_t u = u0 + tid; u < u1; u += kBindThreads) {
      const uint32_t* c = code + units[u];
      uint32_t res[kBalanceRecords], choice[kBalanceRecords];
#pragma unroll
      for (int i = 0; i < kBalanceRecords; ++i) {
        res[i] = 0;
        for (int j = 0; j < ks; ++j) res[i] |= wide_bank_group(resolve(c[i * srw + j], 0u)) << (2 * j);
      }
      balance_wide_choice(res, ks, choice);
      uint32_t* d = dst + units[u];
#pragma unroll
      for (int i = 0; i < kBalanceRecords; ++i)
        for (int k = 0; k < ks; ++k)
          d[i * srw + k] = resolve(c[i * srw + balance_source(res[i], choice[i], k, ks)], 0u);
    }
  }
}

static_assert(kOutPacked == kGenericPacked && kOutBool == kGenericBool &&
                  kOutCounts == kGenericCounts,
              "one output-mode numbering for the batch and generic kernels");

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
  // The plan's bytes, when the caller left the copy to this call
  // (st_search_plan_upload_source), and the width census of a device-bound
  // plan: one launch, ahead of the search on the same stream.
  const uint64_t upload_bytes = plan->upload_source != nullptr ? plan->blob.size() : 0;
  const uint32_t upload_groups =
      static_cast<uint32_t>((upload_bytes + kUploadGroupBytes - 1) / kUploadGroupBytes);
  if (upload_bytes != 0 || plan->device_bind) {
    char* dev = const_cast<char*>(blob);
    // The visiting order is needed by batches outside the quad-lane path
    // (the quad instance visits bundles in index order) and by the
    // wide-bundle kernel when some slot width is wide.
    bool need_order = false;
    for (const SearchBatch& bt : plan->batches)
      need_order |= !bt.generic &&
                    !(bt.stream_words != 0 && bt.stream_words <= kQuadStreamMaxWords &&
                      stream_block_records(std::max(plan->k_eff, 1)) >= 4);
    const bool db = plan->device_bind;
    hipLaunchKernelGGL(bind_prologue_kernel, dim3(upload_groups + (db ? 1 : 0)), dim3(kBindThreads), 0,
                       stream, static_cast<const uint8_t*>(plan->upload_device_src),
                       reinterpret_cast<uint8_t*>(dev), static_cast<int64_t>(upload_bytes), upload_groups,
                       upload_bytes != 0 ? static_cast<unsigned long long*>(plan->upload_signal_device)
                                         : nullptr,
                       static_cast<unsigned long long>(plan->upload_signal_value),
                       bundle_b_offsets, num_bundles,
                       db ? reinterpret_cast<uint32_t*>(dev + plan->off_num_slots) : nullptr,
                       db ? reinterpret_cast<int64_t*>(dev + plan->off_slot_width) : nullptr,
                       db ? reinterpret_cast<uint32_t*>(dev + plan->off_bundle_slot) : nullptr,
                       db && (need_order || plan->off_wide != 0)
                           ? reinterpret_cast<uint32_t*>(dev + plan->off_bundle_order)
                           : nullptr,
                       need_order ? 0u : 1u);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
      throw Error(ST_ERR_HIP, cat("plan upload / width census launch failed: ", hipGetErrorString(e)));
    if (db) {
      hipLaunchKernelGGL(bind_fill_kernel, dim3(kBindGrid), dim3(kBindThreads), 0, stream, dev,
                         plan->off_bind_table, static_cast<uint32_t>(plan->batches.size()),
                         static_cast<int>(plan->hash_k), plan->k_eff, plan->kp,
                         reinterpret_cast<const uint32_t*>(dev + plan->off_num_slots),
                         reinterpret_cast<const int64_t*>(dev + plan->off_slot_width));
      e = hipGetLastError();
      if (e != hipSuccess)
        throw Error(ST_ERR_HIP, cat("width binding launch failed: ", hipGetErrorString(e)));
    }
  }
  // Wide bundles (kSearchTileRows < b <= kWideRows, width-bound) have their
  // literal streams evaluated by the column-slice phase, in packed mode; the
  // per-batch kernels then skip those streams there.  With host-bound widths
  // the phase is decided here; with device binding it ends at once when no
  // slot width is wide.
  WideFn wide_fn = nullptr;
  if (bound && mode == kOutPacked && plan->off_wide != 0) {
    wide_fn = select_wide_kernel(plan->k_eff);
    if (wide_fn != nullptr && !plan->device_bind) {
      bool any = false;
      for (int64_t w : plan->slot_width) any |= wide_width(w);
      if (!any) wide_fn = nullptr;
    }
  }
  // Which batches launch the per-batch kernel; the last of them also runs
  // the wide-bundle phase (no launch of its own then).
  std::vector<uint32_t> wide_flags(plan->batches.size(), 0u);
  std::vector<char> launched(plan->batches.size(), 0);
  size_t last_launch = plan->batches.size();
  for (size_t bi = 0; bi < plan->batches.size(); ++bi) {
    const SearchBatch& bt = plan->batches[bi];
    if (bt.generic) continue;
    // 2 tells the kernel that every program of the batch is in the stream,
    // so that wide bundles need nothing from it
    if (wide_fn != nullptr) {
      const auto* wo = reinterpret_cast<const uint32_t*>(plan->blob.data() + bt.off_wave);
      const auto* sk = reinterpret_cast<const uint32_t*>(plan->blob.data() + bt.off_stream_skip);
      bool all = true;
      for (int w = 0; w < kSearchWaves; ++w) all &= wo[w + 1] - wo[w] == sk[w];
      wide_flags[bi] = all ? 2u : 1u;
    }
    // Nothing for the per-batch kernel when the wide-bundle phase covers
    // every bundle (known here with host-bound widths), unless it carries
    // that phase.
    launched[bi] = !(wide_flags[bi] == 2 && !plan->device_bind && plan->all_wide);
    if (launched[bi]) last_launch = bi;
  }
  if (wide_fn != nullptr && last_launch == plan->batches.size()) {
    // the last streamed batch launches only to carry the wide phase
    for (size_t bi = 0; bi < plan->batches.size(); ++bi)
      if (!plan->batches[bi].generic) last_launch = bi;
    if (last_launch < plan->batches.size()) launched[last_launch] = 1;
  }
  const bool wide_in_search = wide_fn != nullptr && last_launch < plan->batches.size();
  for (size_t bi = 0; bi < plan->batches.size(); ++bi) {
    const SearchBatch& bt = plan->batches[bi];
    if (bt.generic) {
      launch_generic_batch(bloom_index, bloom_index_numel, bundle_b_offsets, num_bundles,
                           plan_blob_device, bt, plan->batch_starts[bi], plan->batch_insns[bi],
                           plan->k_eff, static_cast<int>(plan->hash_k), plan->kp, mode, out,
                           counts, num_docs, stream);
      continue;
    }
    if (!launched[bi]) continue;
    const bool carry_wide = wide_in_search && bi == last_launch;
    // 3: a launch that only carries the wide phase (host-bound, all wide)
    const uint32_t wide_flag =
        carry_wide && wide_flags[bi] == 2 && !plan->device_bind && plan->all_wide ? 3u : wide_flags[bi];
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
        plan->device_bind ? at(plan->off_num_slots) : nullptr,
        carry_wide ? at(plan->off_wide) : nullptr,
        carry_wide ? at(plan->off_bundle_order) : nullptr,
        carry_wide ? reinterpret_cast<const uint32_t*>(blob) : nullptr);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
      throw Error(ST_ERR_HIP, cat("search kernel launch failed: ", hipGetErrorString(e)));
  }
  if (wide_fn != nullptr && !wide_in_search) {
    hipLaunchKernelGGL(wide_fn, dim3(grid), dim3(kSearchThreads), 0, stream, bloom_index,
                       bloom_index_numel, bundle_b_offsets, num_bundles,
                       at(plan->off_bundle_slot), at(plan->off_bundle_order),
                       plan->device_bind ? at(plan->off_num_slots) : nullptr,
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

extern "C" int st_search_plan_upload_source(st_search_plan* plan, const void* pinned_host) {
  using namespace st;
  return guarded([&] {
    ST_CHECK(plan != nullptr, "plan is null");
    if (pinned_host == nullptr) {
      plan->upload_source = plan->upload_device_src = nullptr;
      return;
    }
    ST_CHECK(reinterpret_cast<uintptr_t>(pinned_host) % 16 == 0,
             "the pinned plan buffer must be 16-byte aligned");
    void* dev = nullptr;
    const hipError_t e = hipHostGetDevicePointer(&dev, const_cast<void*>(pinned_host), 0);
    ST_CHECK(e == hipSuccess, "the plan buffer is not pinned, device-accessible host memory (",
             hipGetErrorString(e), ")");
    ST_CHECK(reinterpret_cast<uintptr_t>(dev) % 16 == 0, "the pinned plan buffer must be 16-byte aligned");
    plan->upload_source = pinned_host;
    plan->upload_device_src = dev;
  });
}

extern "C" int64_t st_search_plan_upload_groups(const st_search_plan* plan) {
  if (plan == nullptr || plan->upload_source == nullptr) return 0;
  return static_cast<int64_t>((plan->blob.size() + st::kUploadGroupBytes - 1) / st::kUploadGroupBytes);
}

extern "C" int st_search_plan_upload_signal(st_search_plan* plan, void* pinned_words,
                                            uint64_t value) {
  using namespace st;
  return guarded([&] {
    ST_CHECK(plan != nullptr, "plan is null");
    if (pinned_words == nullptr) {
      plan->upload_signal_device = nullptr;
      return;
    }
    ST_CHECK(reinterpret_cast<uintptr_t>(pinned_words) % 8 == 0,
             "the pinned signal words must be 8-byte aligned");
    void* dev = nullptr;
    const hipError_t e = hipHostGetDevicePointer(&dev, pinned_words, 0);
    ST_CHECK(e == hipSuccess, "the signal words are not pinned, device-accessible host memory (",
             hipGetErrorString(e), ")");
    plan->upload_signal_device = dev;
    plan->upload_signal_value = value;
  });
}

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
