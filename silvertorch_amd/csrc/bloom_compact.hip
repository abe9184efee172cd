// Compaction of matching doc ids for gfx950.
//
// The reference has no operator for this; its users call
// mask[:, :num_docs].nonzero() on the search output (README.md:191-193,
// :265-266).  Here the packed search output int64[Q, C] (C = 32 columns per
// bundle, doc 64c+i of a row at bit 63-i of word c) becomes, per query, the
// ascending ids d < num_docs whose bit is set, as CSR:
//   ids[row_offsets[q] .. row_offsets[q+1]).
//
// A chunk is the 32 words (2048 docs) of one bundle; an item is one
// (query, chunk) pair, and items are numbered query-major.  Three steps:
//   count    one wave per item: lane l holds the 32-bit half (l & 1) of word
//            l >> 1 (one coalesced 256-byte row per wave), masks docs at or
//            past num_docs, popcounts; the wave sum is the item's count.
//   scan     one flat exclusive scan over the counts in item order: since the
//            ids are laid out query by query and, within a query, chunk by
//            chunk, the scanned value of an item is its first output slot.
//            row_offsets[q] is the value of item (q, 0); row_offsets[Q] is
//            the total.
//   write    one wave per item again: an exclusive wave prefix of the lane
//            popcounts places each lane's ids (lane order is doc order), and
//            every lane writes its set bits from the most significant down.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "st_common.hpp"
#include "st_errors.hpp"

namespace st {
int cu_count();

namespace {

constexpr int kCompactThreads = 256;            // 4 waves per workgroup
constexpr int kCompactWaves = kCompactThreads / 64;
constexpr int kItemsPerWave = 8;                // row loads in flight per wave
constexpr int kChunkWords = kColumnsPerBundle;  // 32 words = 2048 docs

constexpr int kScanThreads = 1024;
constexpr int kScanPerThread = 8;
constexpr int kScanTile = kScanThreads * kScanPerThread;

// The lane's 32 doc bits of item `item`, masked to docs < num_docs; bit 31 is
// the lane's first doc.  *first_doc receives the doc id of bit 31.
__device__ __forceinline__ uint32_t lane_bits(const uint32_t* __restrict__ packed32,
                                              int64_t num_columns, int64_t nch,
                                              int64_t num_docs, int64_t item, int lane,
                                              int64_t* first_doc) {
  const int64_t q = item / nch;
  const int64_t ch = item - q * nch;
  const int64_t w = ch * kChunkWords + (lane >> 1);  // column within the row
  const int half = lane & 1;                          // 0: docs 0-31 of the word
  const int64_t base = w * kBitsPerColumn + half * 32;
  *first_doc = base;
  if (w >= num_columns || base >= num_docs) return 0u;
  // Little-endian words: the high half (docs 0-31) is the second u32.
  uint32_t bits = __builtin_nontemporal_load(packed32 + 2 * (q * num_columns + w) + 1 - half);
  const int64_t valid = num_docs - base;
  if (valid < 32) bits &= ~0u << (32 - static_cast<int>(valid));
  return bits;
}

__device__ __forceinline__ int64_t wave_sum(int64_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ uint32_t wave_exclusive_prefix(uint32_t v, int lane) {
  uint32_t x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  return x - v;
}

__global__ __launch_bounds__(kCompactThreads) void compact_count_kernel(
    const uint32_t* __restrict__ packed32, int64_t num_columns, int64_t nch,
    int64_t num_docs, int64_t n_items, int64_t* __restrict__ counts) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * kCompactWaves + (threadIdx.x >> 6);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kCompactWaves * kItemsPerWave;
  for (int64_t first = wave * kItemsPerWave; first < n_items; first += stride) {
    uint32_t bits[kItemsPerWave];
#pragma unroll
    for (int u = 0; u < kItemsPerWave; ++u) {
      int64_t doc;
      bits[u] = first + u < n_items
                    ? lane_bits(packed32, num_columns, nch, num_docs, first + u, lane, &doc)
                    : 0u;
    }
#pragma unroll
    for (int u = 0; u < kItemsPerWave; ++u) {
      const int64_t c = wave_sum(__builtin_popcount(bits[u]));
      if (lane == 0 && first + u < n_items) counts[first + u] = c;
    }
  }
}

// Exclusive scan of 1024 per-thread values across the workgroup; returns the
// thread's exclusive prefix and leaves the total in *total.
__device__ __forceinline__ int64_t block_exclusive_scan(int64_t v, int64_t* total) {
  __shared__ int64_t wave_tot[kScanThreads / 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int64_t x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int64_t y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) wave_tot[wave] = x;
  __syncthreads();
  int64_t before = 0, sum = 0;
  for (int j = 0; j < kScanThreads / 64; ++j) {
    const int64_t t = wave_tot[j];
    before += j < wave ? t : 0;
    sum += t;
  }
  __syncthreads();  // wave_tot may be reused by the caller's next scan
  *total = sum;
  return before + x - v;
}

// Phase 1: sum of each tile of kScanTile counts.
__global__ __launch_bounds__(kScanThreads) void scan_reduce_kernel(
    const int64_t* __restrict__ data, int64_t n, int64_t* __restrict__ tile_sums) {
  const int64_t start = static_cast<int64_t>(blockIdx.x) * kScanTile;
  int64_t s = 0;
#pragma unroll
  for (int j = 0; j < kScanPerThread; ++j) {
    const int64_t i = start + static_cast<int64_t>(j) * kScanThreads + threadIdx.x;
    if (i < n) s += data[i];
  }
  int64_t total;
  block_exclusive_scan(s, &total);
  if (threadIdx.x == 0) tile_sums[blockIdx.x] = total;
}

// Phase 2: exclusive scan of the tile sums in place (one workgroup); the
// grand total goes to row_offsets[num_queries].
__global__ __launch_bounds__(kScanThreads) void scan_tiles_kernel(
    int64_t* __restrict__ tile_sums, int64_t n_tiles, int64_t* __restrict__ row_offsets,
    int64_t num_queries) {
  int64_t carry = 0;
  for (int64_t base = 0; base < n_tiles; base += kScanTile) {
    int64_t v[kScanPerThread];
    int64_t s = 0;
#pragma unroll
    for (int j = 0; j < kScanPerThread; ++j) {
      const int64_t i = base + static_cast<int64_t>(threadIdx.x) * kScanPerThread + j;
      v[j] = i < n_tiles ? tile_sums[i] : 0;
      s += v[j];
    }
    int64_t total;
    int64_t run = carry + block_exclusive_scan(s, &total);
#pragma unroll
    for (int j = 0; j < kScanPerThread; ++j) {
      const int64_t i = base + static_cast<int64_t>(threadIdx.x) * kScanPerThread + j;
      if (i < n_tiles) tile_sums[i] = run;
      run += v[j];
    }
    carry += total;
  }
  if (threadIdx.x == 0) row_offsets[num_queries] = carry;
}

// Phase 3: exclusive scan within each tile plus the tile's offset, in place;
// items (q, 0) give row_offsets[q].
__global__ __launch_bounds__(kScanThreads) void scan_apply_kernel(
    int64_t* __restrict__ data, int64_t n, const int64_t* __restrict__ tile_offsets,
    int64_t nch, int64_t* __restrict__ row_offsets) {
  const int64_t start = static_cast<int64_t>(blockIdx.x) * kScanTile +
                        static_cast<int64_t>(threadIdx.x) * kScanPerThread;
  int64_t v[kScanPerThread];
  int64_t s = 0;
#pragma unroll
  for (int j = 0; j < kScanPerThread; ++j) {
    v[j] = start + j < n ? data[start + j] : 0;
    s += v[j];
  }
  int64_t total;
  int64_t run = tile_offsets[blockIdx.x] + block_exclusive_scan(s, &total);
#pragma unroll
  for (int j = 0; j < kScanPerThread; ++j) {
    const int64_t i = start + j;
    if (i < n) {
      data[i] = run;
      if (i % nch == 0) row_offsets[i / nch] = run;
    }
    run += v[j];
  }
}

__global__ void zero_offsets_kernel(int64_t* __restrict__ row_offsets, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) row_offsets[i] = 0;
}

template <typename Id>
__global__ __launch_bounds__(kCompactThreads) void compact_write_kernel(
    const uint32_t* __restrict__ packed32, int64_t num_columns, int64_t nch,
    int64_t num_docs, int64_t n_items, const int64_t* __restrict__ item_base,
    Id* __restrict__ ids) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * kCompactWaves + (threadIdx.x >> 6);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kCompactWaves * kItemsPerWave;
  for (int64_t first = wave * kItemsPerWave; first < n_items; first += stride) {
    uint32_t bits[kItemsPerWave];
    int64_t doc0[kItemsPerWave];
#pragma unroll
    for (int u = 0; u < kItemsPerWave; ++u) {
      bits[u] = first + u < n_items
                    ? lane_bits(packed32, num_columns, nch, num_docs, first + u, lane, &doc0[u])
                    : 0u;
    }
#pragma unroll
    for (int u = 0; u < kItemsPerWave; ++u) {
      if (first + u >= n_items) break;  // wave-uniform
      uint32_t b = bits[u];
      int64_t pos = item_base[first + u] +
                    wave_exclusive_prefix(static_cast<uint32_t>(__builtin_popcount(b)), lane);
      while (b != 0u) {
        const int lz = __builtin_clz(b);
        ids[pos++] = static_cast<Id>(doc0[u] + lz);
        b &= ~(0x80000000u >> lz);
      }
    }
  }
}

int compact_grid(int64_t n_items) {
  const int64_t per_block = static_cast<int64_t>(kCompactWaves) * kItemsPerWave;
  const int64_t want = (n_items + per_block - 1) / per_block;
  return static_cast<int>(std::max<int64_t>(
      1, std::min<int64_t>(want, static_cast<int64_t>(cu_count()) * 8)));
}

int64_t num_chunks(int64_t num_columns) {
  return (num_columns + kChunkWords - 1) / kChunkWords;
}

void check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) throw Error(ST_ERR_HIP, cat(what, " launch failed: ", hipGetErrorString(e)));
}

void check_shape(int64_t num_queries, int64_t num_columns, int64_t num_docs) {
  ST_CHECK(num_queries >= 0 && num_columns >= 0, "negative mask shape [", num_queries,
           ", ", num_columns, "]");
  ST_CHECK(num_docs >= 0, "num_docs must be non-negative, got ", num_docs);
  ST_CHECK(num_columns <= (INT64_MAX / 64) && num_queries <= INT64_MAX / (num_columns + 1),
           "mask shape too large");
}

}  // namespace
}  // namespace st

extern "C" int64_t st_bloom_compact_workspace_bytes(int64_t num_queries, int64_t num_columns) {
  if (num_queries <= 0 || num_columns <= 0) return 0;
  const int64_t items = num_queries * st::num_chunks(num_columns);
  const int64_t tiles = (items + st::kScanTile - 1) / st::kScanTile;
  return 8 * (items + tiles);
}

extern "C" int st_bloom_compact_offsets(const int64_t* packed, int64_t num_queries,
                                        int64_t num_columns, int64_t num_docs,
                                        void* workspace, int64_t* row_offsets, void* stream) {
  using namespace st;
  return guarded([&] {
    check_shape(num_queries, num_columns, num_docs);
    ST_CHECK(row_offsets != nullptr, "row_offsets is null");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t nch = num_chunks(num_columns);
    const int64_t items = num_queries * nch;
    if (items == 0) {
      const int64_t n = num_queries + 1;
      hipLaunchKernelGGL(zero_offsets_kernel, dim3(static_cast<unsigned>((n + 255) / 256)),
                         dim3(256), 0, s, row_offsets, n);
      check_launch("zero_offsets_kernel");
      return;
    }
    ST_CHECK(packed != nullptr && workspace != nullptr, "null device pointer");
    int64_t* counts = static_cast<int64_t*>(workspace);
    const int64_t tiles = (items + kScanTile - 1) / kScanTile;
    int64_t* tile_sums = counts + items;
    const uint32_t* p32 = reinterpret_cast<const uint32_t*>(packed);
    hipLaunchKernelGGL(compact_count_kernel, dim3(compact_grid(items)), dim3(kCompactThreads),
                       0, s, p32, num_columns, nch, num_docs, items, counts);
    check_launch("compact_count_kernel");
    hipLaunchKernelGGL(scan_reduce_kernel, dim3(static_cast<unsigned>(tiles)),
                       dim3(kScanThreads), 0, s, counts, items, tile_sums);
    check_launch("scan_reduce_kernel");
    hipLaunchKernelGGL(scan_tiles_kernel, dim3(1), dim3(kScanThreads), 0, s, tile_sums, tiles,
                       row_offsets, num_queries);
    check_launch("scan_tiles_kernel");
    hipLaunchKernelGGL(scan_apply_kernel, dim3(static_cast<unsigned>(tiles)),
                       dim3(kScanThreads), 0, s, counts, items, tile_sums, nch, row_offsets);
    check_launch("scan_apply_kernel");
  });
}

extern "C" int st_bloom_compact_ids(const int64_t* packed, int64_t num_queries,
                                    int64_t num_columns, int64_t num_docs,
                                    const void* workspace, void* ids, int ids_int64,
                                    void* stream) {
  using namespace st;
  return guarded([&] {
    check_shape(num_queries, num_columns, num_docs);
    const int64_t nch = num_chunks(num_columns);
    const int64_t items = num_queries * nch;
    if (items == 0) return;
    ST_CHECK(packed != nullptr && workspace != nullptr, "null device pointer");
    ST_CHECK(ids_int64 || std::min(num_docs, num_columns * kBitsPerColumn) <= INT32_MAX,
             "int32 ids cannot hold doc ids up to ", num_docs);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint32_t* p32 = reinterpret_cast<const uint32_t*>(packed);
    const int64_t* base = static_cast<const int64_t*>(workspace);
    if (ids_int64) {
      hipLaunchKernelGGL(compact_write_kernel<int64_t>, dim3(compact_grid(items)),
                         dim3(kCompactThreads), 0, s, p32, num_columns, nch, num_docs, items,
                         base, static_cast<int64_t*>(ids));
    } else {
      hipLaunchKernelGGL(compact_write_kernel<int32_t>, dim3(compact_grid(items)),
                         dim3(kCompactThreads), 0, s, p32, num_columns, nch, num_docs, items,
                         base, static_cast<int32_t*>(ids));
    }
    check_launch("compact_write_kernel");
  });
}
