// Batched boolean search over the bundled bloom index, for gfx950.
//
// Replaces process_documents / bloom_index_search_common
// (bloom_index_search_cuda.cu:575-615, :940-1029) and the CPU loop
// bloom_index_search_common_cpu (bloom_index_search.cpp:173-243).
//
// Layout (unchanged from the reference, bloom_indexer.cpp:72-110): bundle i
// owns rows [off[i], off[i+1]) of 32 int64 words; word (row, c) holds the
// bloom bit `row` of the 64 docs of column c, doc 64c+j at bit 63-j.
//
// Work decomposition: one 1024-thread workgroup per CU walks bundles
// blockIdx.x, blockIdx.x + gridDim.x, ...  For each bundle it
//   1. moves the bundle's rows (prefetched into registers while the previous
//      bundle was evaluated) into LDS, so the index is read from HBM once per
//      query batch;
//   2. resolves every distinct batch term to its k row positions for this
//      bundle's width b -- once per bundle instead of once per (query,
//      column) -- skipping the step when b equals the previous bundle's;
//   3. has each wave run its queries' accumulator programs: lane l owns the
//      32-bit half (l & 1) of column l >> 1, so one wave covers the 32
//      columns of the bundle for one query and all control flow is
//      wave-uniform.
// Bundles wider than the LDS tile are evaluated from global memory with the
// same programs.
#include <hip/hip_runtime.h>

#include <mutex>
#include <vector>

#include "search_plan.hpp"
#include "st_common.hpp"
#include "st_errors.hpp"

namespace st {
namespace {

// Native 4 x u32 vector (usable with the nontemporal builtins).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kPrefetch = kSearchTileRows * 16 / kSearchThreads;  // uint4/thread
static_assert(kPrefetch * kSearchThreads == kSearchTileRows * 16, "tile split");

struct SearchArgs {
  const int64_t* index;
  int64_t index_numel;
  const int64_t* bundle_offsets;
  int64_t num_bundles;
  const uint32_t* wave_off;
  const uint32_t* rows;
  const uint32_t* insn_start;
  const uint32_t* insns;
  const uint64_t* hashes;
  uint32_t num_terms;
  int32_t hash_k;
  int64_t out_cols;  // columns per output row = num_bundles * 32
  void* out;
};

__device__ __forceinline__ uint32_t uniform(uint32_t v) {
  return __builtin_amdgcn_readfirstlane(v);
}

// Width and first row of bundle `bnd`; a negative width (malformed offsets)
// reads as an empty bundle.
__device__ __forceinline__ void bundle_extent(const SearchArgs& a, int64_t bnd,
                                              int64_t& start, int64_t& b) {
  start = a.bundle_offsets[bnd];
  b = a.bundle_offsets[bnd + 1] - start;
  if (b < 0) b = 0;
}

__device__ __forceinline__ void prefetch_tile(const SearchArgs& a, int64_t bnd,
                                              u32x4 (&pre)[kPrefetch]) {
  int64_t start, b;
  bundle_extent(a, bnd, start, b);
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < kPrefetch; ++i) pre[i] = u32x4{0, 0, 0, 0};
  if (b > kSearchTileRows) return;
  const int64_t chunks = b * 16;
  const u32x4* src = reinterpret_cast<const u32x4*>(a.index + start * 32);
#pragma unroll
  for (int i = 0; i < kPrefetch; ++i) {
    const int c = tid + i * kSearchThreads;
    // chunk c holds words start*32 + 2c and + 2c + 1
    if (c < chunks && start * 32 + 2 * c + 1 < a.index_numel) {
      pre[i] = __builtin_nontemporal_load(src + c);
    }
  }
}

// Resolves term u's positions for width b, as signature_match does
// (bloom_index_search.cpp:40-61): over hashes p < hash_k, while fewer than K
// are resolved, b_p = (int16)(h[p] % b); repeats of an earlier b_p are
// skipped.  Unused slots repeat slot 0 (AND is idempotent).
template <int K>
__device__ __forceinline__ int resolve_positions(const uint64_t* h, int hash_k,
                                                 const FastMod64& fm,
                                                 int16_t (&found)[K]) {
  int cnt = 0;
  for (int p = 0; p < hash_k && cnt < K; ++p) {
    const int16_t bp = static_cast<int16_t>(fast_mod(h[p], fm));
    bool dup = false;
#pragma unroll
    for (int j = 0; j < K; ++j) dup |= (j < cnt) && (found[j] == bp);
    if (!dup) {
#pragma unroll
      for (int j = 0; j < K; ++j)
        if (j == cnt) found[j] = bp;
      ++cnt;
    }
  }
  return cnt;
}

// Expands a 32-bit match half into 32 bool bytes, most significant bit
// first (the doc order of bloom_index_search.cpp:231-236).
__device__ __forceinline__ void store_bool32(uint8_t* dst, uint32_t bits) {
  const uint32_t y = __builtin_bitreverse32(bits);
  uint32_t w[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) w[j] = (((y >> (4 * j)) & 0xFu) * 0x00204081u) & 0x01010101u;
  u32x4* d = reinterpret_cast<u32x4*>(dst);
  __builtin_nontemporal_store(u32x4{w[0], w[1], w[2], w[3]}, d);
  __builtin_nontemporal_store(u32x4{w[4], w[5], w[6], w[7]}, d + 1);
}

template <int K, bool kBoolOut>
__global__ __launch_bounds__(kSearchThreads) void bloom_search_kernel(
    SearchArgs a) {
  constexpr int KP = K <= 4 ? 4 : (K <= 8 ? 8 : 12);
  __shared__ u32x4 tile[(kSearchTileRows + 2) * 16];
  __shared__ uint32_t pos[kSearchPosSlots];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const uint32_t wave = uniform(tid >> 6);

  if (tid < 32) {
    const uint32_t fill = tid < 16 ? ~0u : 0u;
    tile[kSearchOnesRow * 16 + (tid & 15) + (tid & 16)] = u32x4{fill, fill, fill, fill};
  }

  u32x4 pre[kPrefetch];
  int64_t bundle = blockIdx.x;
  if (bundle < a.num_bundles) prefetch_tile(a, bundle, pre);

  int64_t prev_b = -1;
  const uint32_t s_begin = uniform(a.wave_off[wave]);
  const uint32_t s_end = uniform(a.wave_off[wave + 1]);
  const char* tile_lane = reinterpret_cast<const char*>(tile) + lane * 4;
  const uint32_t* index32 = reinterpret_cast<const uint32_t*>(a.index);

  for (; bundle < a.num_bundles; bundle += gridDim.x) {
    int64_t start, b;
    bundle_extent(a, bundle, start, b);
    const bool staged = b <= kSearchTileRows;

    __syncthreads();  // previous bundle's readers are done with tile and pos
    if (staged) {
      const int64_t chunks = b * 16;
#pragma unroll
      for (int i = 0; i < kPrefetch; ++i) {
        const int c = tid + i * kSearchThreads;
        if (c < chunks) tile[c] = pre[i];
      }
    }
    if (b != prev_b) {
      const FastMod64 fm = make_fastmod(static_cast<uint64_t>(b));
      for (uint32_t u = tid; u < a.num_terms; u += kSearchThreads) {
        int16_t found[K];
#pragma unroll
        for (int j = 0; j < K; ++j) found[j] = 0;
        int cnt = 0;
        if (b > 0) cnt = resolve_positions<K>(a.hashes + static_cast<uint64_t>(u) * a.hash_k,
                                              a.hash_k, fm, found);
        uint32_t* dst = pos + u * KP;
#pragma unroll
        for (int j = 0; j < KP; ++j) {
          const int16_t r = (j < K && j < cnt) ? found[j < K ? j : 0] : found[0];
          uint32_t v;
          if (staged) {
            v = (cnt == 0 ? kSearchZerosRow : static_cast<int>(r)) * 256u;
          } else {
            v = cnt == 0 ? static_cast<uint32_t>(kPosZeros)
                         : static_cast<uint32_t>(static_cast<int32_t>(r));
          }
          dst[j] = v;
        }
      }
      prev_b = b;
    }
    __syncthreads();

    const int64_t next = bundle + gridDim.x;
    if (next < a.num_bundles) prefetch_tile(a, next, pre);

    // Evaluate this wave's queries on the bundle.
    for (uint32_t s = s_begin; s < s_end; ++s) {
      const uint32_t i0 = a.insn_start[s];
      const uint32_t i1 = a.insn_start[s + 1];
      uint32_t acc = 0;
      uint32_t stk[kSearchMaxStack];
      uint32_t sp = 0;
      for (uint32_t i = i0; i < i1; ++i) {
        const uint32_t w = a.insns[i];
        const uint32_t op = w & 7u;
        const uint32_t mode = (w >> 3) & 3u;
        uint32_t v;
        if (op == kInsTerm) {
          const uint32_t* pp = pos + (w >> 6) * KP;
          uint32_t p[KP];
#pragma unroll
          for (int j = 0; j < KP; j += 4) {
            const u32x4 q4 = *reinterpret_cast<const u32x4*>(pp + j);
            p[j] = q4.x;
            p[j + 1] = q4.y;
            p[j + 2] = q4.z;
            p[j + 3] = q4.w;
          }
          v = ~0u;
          if (staged) {
#pragma unroll
            for (int j = 0; j < K; ++j)
              v &= *reinterpret_cast<const uint32_t*>(tile_lane + p[j]);
          } else {
#pragma unroll
            for (int j = 0; j < K; ++j) {
              const int32_t r = static_cast<int32_t>(p[j]);
              uint32_t word = 0;
              if (r != kPosZeros) {
                const int64_t row = start + r;
                if (row >= 0 && (row * 32 + (lane >> 1)) < a.index_numel)
                  word = index32[row * 64 + lane];
              }
              v &= word;
            }
          }
        } else if (op == kInsConst) {
          v = ~0u;
        } else if (op == kInsPush) {
          stk[sp++] = acc;
          continue;
        } else if (op == kInsPop) {
          v = acc;
          acc = stk[--sp];
        } else {  // kInsNot
          acc = ~acc;
          continue;
        }
        if (w & 32u) v = ~v;
        acc = mode == kModeSet ? v : (mode == kModeAnd ? (acc & v) : (acc | v));
      }

      const int64_t col0 = static_cast<int64_t>(a.rows[s]) * a.out_cols + bundle * 32;
      if constexpr (kBoolOut) {
        uint8_t* dst = static_cast<uint8_t*>(a.out) + (col0 + (lane >> 1)) * 64 +
                       ((lane & 1) ? 0 : 32);
        store_bool32(dst, acc);
      } else {
        uint32_t* dst = static_cast<uint32_t*>(a.out) + col0 * 2 + lane;
        __builtin_nontemporal_store(acc, dst);
      }
    }
  }
}

using KernelFn = void (*)(SearchArgs);

template <int K>
KernelFn pick(bool bool_out) {
  return bool_out ? bloom_search_kernel<K, true> : bloom_search_kernel<K, false>;
}

KernelFn select_kernel(int k, bool bool_out) {
  switch (k) {
    case 0:
    case 1: return pick<1>(bool_out);
    case 2: return pick<2>(bool_out);
    case 3: return pick<3>(bool_out);
    case 4: return pick<4>(bool_out);
    case 5: return pick<5>(bool_out);
    case 6: return pick<6>(bool_out);
    case 7: return pick<7>(bool_out);
    case 8: return pick<8>(bool_out);
    case 9: return pick<9>(bool_out);
    case 10: return pick<10>(bool_out);
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
    ST_CHECK(bundle_b_offsets != nullptr && out != nullptr &&
                 plan_blob_device != nullptr,
             "null device pointer");
    ST_CHECK(bloom_index != nullptr || bloom_index_numel == 0,
             "bloom_index is null");
    KernelFn fn = select_kernel(plan->k_eff, return_bool_mask != 0);
    const int grid = static_cast<int>(
        std::min<int64_t>(num_bundles, static_cast<int64_t>(device_cu_count())));
    const char* blob = static_cast<const char*>(plan_blob_device);
    for (const SearchBatch& bt : plan->batches) {
      SearchArgs a;
      a.index = bloom_index;
      a.index_numel = bloom_index_numel;
      a.bundle_offsets = bundle_b_offsets;
      a.num_bundles = num_bundles;
      a.wave_off = reinterpret_cast<const uint32_t*>(blob + bt.off_wave);
      a.rows = reinterpret_cast<const uint32_t*>(blob + bt.off_row);
      a.insn_start = reinterpret_cast<const uint32_t*>(blob + bt.off_insn_start);
      a.insns = reinterpret_cast<const uint32_t*>(blob + bt.off_insns);
      a.hashes = reinterpret_cast<const uint64_t*>(blob + bt.off_hashes);
      a.num_terms = bt.num_terms;
      a.hash_k = static_cast<int32_t>(plan->hash_k);
      a.out_cols = num_bundles * 32;
      a.out = out;
      hipLaunchKernelGGL(fn, dim3(grid), dim3(kSearchThreads), 0,
                         static_cast<hipStream_t>(stream), a);
      hipError_t e = hipGetLastError();
      if (e != hipSuccess)
        throw Error(ST_ERR_HIP, cat("search kernel launch failed: ",
                                    hipGetErrorString(e)));
    }
  });
}
