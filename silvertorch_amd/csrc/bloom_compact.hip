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
//   count    when num_columns is a multiple of 32, item i is bytes
//            [256 i, 256 i + 256) of the mask: each lane loads 16 bytes, a
//            row of 16 lanes holds one item and DPP row shifts sum its
//            popcounts (one load instruction covers four items); otherwise
//            one wave per item, lane l holding the 32-bit half (l & 1) of
//            word l >> 1.  Docs at or past num_docs are masked out.
//   scan     one flat exclusive scan over the counts in item order: since the
//            ids are laid out query by query and, within a query, chunk by
//            chunk, the scanned value of an item is its first output slot.
//            row_offsets[q] is the value of item (q, 0); row_offsets[Q] is
//            the total.
//   write    one wave per item, lane l again holding half (l & 1) of word
//            l >> 1 (lane order is doc order): a DPP prefix of the lane
//            popcounts places each lane's ids, which the lane stages in LDS as
//            16-bit offsets within the chunk (lowest bit of the bit-reversed
//            half first); the wave then writes the item's run with 16-byte
//            stores.  A wave takes kWriteItems consecutive items at a time
//            and loads the next such group before it stages the current one.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "st_common.hpp"
#include "st_errors.hpp"
#include "wave_ops.hpp"

namespace st {
int cu_count();

namespace {

constexpr int kCompactThreads = 256;            // 4 waves per workgroup
constexpr int kCompactWaves = kCompactThreads / 64;
constexpr int kCountItems = 8;   // row loads in flight per wave, count pass by rows
constexpr int kCountLines = 4;   // 1 KB loads (4 items each) in flight, count pass by lines
constexpr int kWriteItems = 4;   // items per group of the write pass
constexpr int kChunkWords = kColumnsPerBundle;  // 32 words = 2048 docs

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4_u __attribute__((ext_vector_type(4), aligned(4)));
typedef int64_t i64x2_u __attribute__((ext_vector_type(2), aligned(8)));

constexpr int kScanThreads = 1024;
constexpr int kScanPerThread = 8;
constexpr int kScanTile = kScanThreads * kScanPerThread;
// the per-tile passes (reduce, apply) take tiles of kPartTile counts, 256
// threads each, so that a call's tiles cover the CUs (cfg2: 610 tiles)
constexpr int kPartThreads = 256;
constexpr int kPartTile = kPartThreads * kScanPerThread;
// up to this many tiles the apply pass sums the tile sums before its own
// tile itself (no separate scan of the tile sums; at most ~4 MB of L2 reads)
constexpr int64_t kPartPrefixTiles = 1024;

// The lane's 32 doc bits of item (q, ch), masked to docs < num_docs; bit 31
// is the lane's first doc, whose offset within the chunk is 32 * lane.
__device__ __forceinline__ uint32_t lane_bits(const uint32_t* __restrict__ packed32,
                                              int64_t num_columns, int64_t num_docs,
                                              int64_t q, int64_t ch, int lane) {
  const int64_t w = ch * kChunkWords + (lane >> 1);  // column within the row
  const int half = lane & 1;                          // 0: docs 0-31 of the word
  const int64_t base = w * kBitsPerColumn + half * 32;
  if (w >= num_columns || base >= num_docs) return 0u;
  // Little-endian words: the high half (docs 0-31) is the second u32.
  const uint32_t bits = __builtin_nontemporal_load(packed32 + 2 * (q * num_columns + w) + 1 - half);
  return bits & valid_doc_mask(base, num_docs);
}

// Items first .. first+kItemsPerWave-1 as (query, chunk) pairs: one division
// per group, then increments.
struct ItemCursor {
  int64_t q, ch;
  __device__ ItemCursor(int64_t first, int64_t nch) : q(first / nch), ch(first - (first / nch) * nch) {}
  __device__ void next(int64_t nch) {
    if (++ch == nch) {
      ch = 0;
      ++q;
    }
  }
};

__global__ __launch_bounds__(kCompactThreads) void compact_count_kernel(
    const uint32_t* __restrict__ packed32, int64_t num_columns, int64_t nch,
    int64_t num_docs, int64_t n_items, int64_t* __restrict__ counts) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * kCompactWaves + (threadIdx.x >> 6);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kCompactWaves * kCountItems;
  for (int64_t first = wave * kCountItems; first < n_items; first += stride) {
    uint32_t bits[kCountItems];
    ItemCursor it(first, nch);
#pragma unroll
    for (int u = 0; u < kCountItems; ++u) {
      bits[u] = first + u < n_items ? lane_bits(packed32, num_columns, num_docs, it.q, it.ch, lane)
                                    : 0u;
      it.next(nch);
    }
#pragma unroll
    for (int u = 0; u < kCountItems; ++u) {
      const uint32_t c = wave_total_small(static_cast<uint32_t>(__builtin_popcount(bits[u])));
      if (lane == 0 && first + u < n_items) counts[first + u] = c;
    }
  }
}

// Count pass over contiguous items (num_columns a multiple of 32).  Lane l
// of a wave loads bytes [16 l, 16 l + 16) of a 1 KB line of four items: row
// r = l >> 4 of the wave holds item 4 g + r, lane l & 15 its docs
// 128 (l & 15) .. + 127 (u32 y: docs 0-31, x: 32-63, w: 64-95, z: 96-127).
__global__ __launch_bounds__(kCompactThreads) void compact_count_lines_kernel(
    const u32x4* __restrict__ packed16, int64_t nch, int64_t num_docs, int64_t n_items,
    int64_t* __restrict__ counts) {
  const int lane = threadIdx.x & 63;
  const int row = lane >> 4, rl = lane & 15;
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * kCompactWaves + (threadIdx.x >> 6);
  const int64_t lines = (n_items + 3) / 4;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kCompactWaves * kCountLines;
  for (int64_t g0 = wave * kCountLines; g0 < lines; g0 += stride) {
    u32x4 v[kCountLines];
#pragma unroll
    for (int u = 0; u < kCountLines; ++u) {
      const int64_t item = 4 * (g0 + u) + row;
      v[u] = item < n_items ? __builtin_nontemporal_load(packed16 + 64 * (g0 + u) + lane)
                            : u32x4{0u, 0u, 0u, 0u};
    }
    int64_t item = 4 * g0 + row;
    int64_t ch = item % nch;
#pragma unroll
    for (int u = 0; u < kCountLines; ++u) {
      u32x4 w = v[u];
      const int64_t first_doc = ch * kDocsPerBundle + 128 * rl;
      if (first_doc + 128 > num_docs) {
        w.y &= valid_doc_mask(first_doc, num_docs);
        w.x &= valid_doc_mask(first_doc + 32, num_docs);
        w.w &= valid_doc_mask(first_doc + 64, num_docs);
        w.z &= valid_doc_mask(first_doc + 96, num_docs);
      }
      const uint32_t c = row16_inclusive_sum(
          static_cast<uint32_t>(__builtin_popcount(w.x) + __builtin_popcount(w.y) +
                                __builtin_popcount(w.z) + __builtin_popcount(w.w)));
      if (rl == 15 && item < n_items) counts[item] = c;
      item += 4;
      ch += 4;
      while (ch >= nch) ch -= nch;
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

// Phase 1: sum of each tile of kPartTile counts (coalesced loads).
__global__ __launch_bounds__(kPartThreads) void scan_reduce_kernel(
    const int64_t* __restrict__ data, int64_t n, int64_t* __restrict__ tile_sums) {
  __shared__ int64_t wave_sum[kPartThreads / 64];
  const int64_t start = static_cast<int64_t>(blockIdx.x) * kPartTile;
  int64_t s = 0;
#pragma unroll
  for (int j = 0; j < kScanPerThread; ++j) {
    const int64_t i = start + static_cast<int64_t>(j) * kPartThreads + threadIdx.x;
    if (i < n) s += data[i];
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
  if ((threadIdx.x & 63) == 0) wave_sum[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t t = 0;
#pragma unroll
    for (int w = 0; w < kPartThreads / 64; ++w) t += wave_sum[w];
    tile_sums[blockIdx.x] = t;
  }
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
// items (q, 0) give row_offsets[q].  The tile goes through LDS so that the
// global loads and stores are coalesced while each thread scans 8
// consecutive counts; the LDS copy has one pad entry per 8 so that those
// reads (72 bytes apart across lanes) spread over the banks.
__device__ __forceinline__ int part_slot(int e) { return e + (e >> 3); }

// With kPrefix the tile sums are not scanned beforehand: each workgroup
// sums those of the tiles before its own (calls of at most kPartPrefixTiles
// tiles), and the last one writes the total to row_offsets[num_queries].
template <bool kPrefix>
__global__ __launch_bounds__(kPartThreads) void scan_apply_kernel(
    int64_t* __restrict__ data, int64_t n, const int64_t* __restrict__ tile_offsets,
    int64_t nch, int64_t* __restrict__ row_offsets, int64_t num_queries) {
  __shared__ int64_t tile[kPartTile + kPartTile / 8];
  __shared__ int64_t wave_tot[kPartThreads / 64];
  __shared__ int64_t wave_pre[kPartThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t start = static_cast<int64_t>(blockIdx.x) * kPartTile;
  if constexpr (kPrefix) {
    int64_t pre = 0;
    for (uint32_t t = tid; t < blockIdx.x; t += kPartThreads) pre += tile_offsets[t];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) pre += __shfl_xor(pre, off, 64);
    if (lane == 0) wave_pre[wave] = pre;
  }
#pragma unroll
  for (int j = 0; j < kScanPerThread; ++j) {
    const int e = j * kPartThreads + tid;
    tile[part_slot(e)] = start + e < n ? data[start + e] : 0;
  }
  __syncthreads();
  int64_t v[kScanPerThread];
  int64_t s = 0;
#pragma unroll
  for (int j = 0; j < kScanPerThread; ++j) {
    v[j] = tile[part_slot(tid * kScanPerThread + j)];
    s += v[j];
  }
  int64_t x = s;  // inclusive scan of the thread sums over the wave
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int64_t y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) wave_tot[wave] = x;
  __syncthreads();
  int64_t base;
  if constexpr (kPrefix) {
    base = 0;
#pragma unroll
    for (int w = 0; w < kPartThreads / 64; ++w) base += wave_pre[w];
    if (blockIdx.x == gridDim.x - 1 && tid == kPartThreads - 1) {
      int64_t tot = base;
#pragma unroll
      for (int w = 0; w < kPartThreads / 64; ++w) tot += wave_tot[w];
      row_offsets[num_queries] = tot;
    }
  } else {
    base = tile_offsets[blockIdx.x];
  }
  int64_t run = base + x - s;
#pragma unroll
  for (int w = 0; w < kPartThreads / 64; ++w) run += w < wave ? wave_tot[w] : 0;
  const int64_t first = start + static_cast<int64_t>(tid) * kScanPerThread;
  int64_t q = first / nch, r = first - q * nch;
#pragma unroll
  for (int j = 0; j < kScanPerThread; ++j) {
    if (first + j < n && r == 0) row_offsets[q] = run;
    tile[part_slot(tid * kScanPerThread + j)] = run;
    run += v[j];
    if (++r == nch) {
      r = 0;
      ++q;
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kScanPerThread; ++j) {
    const int e = j * kPartThreads + tid;
    if (start + e < n) data[start + e] = tile[part_slot(e)];
  }
}

__global__ void zero_offsets_kernel(int64_t* __restrict__ row_offsets, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) row_offsets[i] = 0;
}

// The lane's 32 doc bits of item (q, ch) as loaded (not yet masked at
// num_docs); 0 for columns past the row's end, which only the last chunk
// of a row has when num_columns is not a multiple of 32.
__device__ __forceinline__ uint32_t load_lane_half(const uint32_t* __restrict__ packed32,
                                                   int64_t num_columns, int64_t q, int64_t ch,
                                                   int lane) {
  const int64_t w0 = ch * kChunkWords;
  if ((lane >> 1) >= num_columns - w0) return 0u;
  return __builtin_nontemporal_load(packed32 + 2 * (q * num_columns + w0) + (lane ^ 1));
}

// Writes the item's staged run my[0 .. total) as ids doc0 + my[i] to
// dst[0 .. total), 16 bytes per lane and store; the run's last partial unit
// is written id by id (the ids after it belong to the next item).
__device__ __forceinline__ void write_run(const uint16_t* my, uint32_t total, int lane,
                                          int64_t doc0, int32_t* dst) {
  const int32_t d0 = static_cast<int32_t>(doc0);  // ids fit int32 (checked by the host)
  for (uint32_t i = 4u * lane; i < total; i += 256u) {
    const uint2 pr = *reinterpret_cast<const uint2*>(my + i);
    const int32_t a = d0 + static_cast<int32_t>(pr.x & 0xFFFFu);
    const int32_t b = d0 + static_cast<int32_t>(pr.x >> 16);
    const int32_t c = d0 + static_cast<int32_t>(pr.y & 0xFFFFu);
    const int32_t d = d0 + static_cast<int32_t>(pr.y >> 16);
    if (i + 4u <= total) {
      *reinterpret_cast<i32x4_u*>(dst + i) = i32x4_u{a, b, c, d};
    } else {
      dst[i] = a;
      if (i + 1u < total) dst[i + 1] = b;
      if (i + 2u < total) dst[i + 2] = c;
    }
  }
}

__device__ __forceinline__ void write_run(const uint16_t* my, uint32_t total, int lane,
                                          int64_t doc0, int64_t* dst) {
  for (uint32_t i = 2u * lane; i < total; i += 128u) {
    const uint32_t pr = *reinterpret_cast<const uint32_t*>(my + i);
    const int64_t a = doc0 + static_cast<int64_t>(pr & 0xFFFFu);
    const int64_t b = doc0 + static_cast<int64_t>(pr >> 16);
    if (i + 2u <= total) {
      *reinterpret_cast<i64x2_u*>(dst + i) = i64x2_u{a, b};
    } else {
      dst[i] = a;
    }
  }
}

template <typename Id>
__global__ __launch_bounds__(kCompactThreads) void compact_write_kernel(
    const uint32_t* __restrict__ packed32, int64_t num_columns, int64_t nch,
    int64_t num_docs, int64_t n_items, const int64_t* __restrict__ item_base,
    Id* __restrict__ ids) {
  __shared__ __align__(16) uint16_t stage[kCompactWaves][kDocsPerBundle];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  uint16_t* my = stage[wv];
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * kCompactWaves + wv;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kCompactWaves * kWriteItems;
  const int64_t step_q = stride / nch, step_ch = stride - step_q * nch;
  const uint32_t lane_doc = static_cast<uint32_t>(lane) * 32u;
  int64_t first = wave * kWriteItems;
  if (first >= n_items) return;
  ItemCursor at(first, nch);  // first item of the current group
  uint32_t next_bits[kWriteItems];
  int64_t next_pos[kWriteItems];
  const auto load_group = [&](int64_t f, ItemCursor it) {
#pragma unroll
    for (int u = 0; u < kWriteItems; ++u) {
      const bool valid = f + u < n_items;
      next_bits[u] = valid ? load_lane_half(packed32, num_columns, it.q, it.ch, lane) : 0u;
      next_pos[u] = valid ? item_base[f + u] : 0;
      it.next(nch);
    }
  };
  load_group(first, at);
  for (; first < n_items; first += stride) {
    uint32_t bits[kWriteItems];
    int64_t pos[kWriteItems];
#pragma unroll
    for (int u = 0; u < kWriteItems; ++u) {
      bits[u] = next_bits[u];
      pos[u] = next_pos[u];
    }
    ItemCursor it = at;
    at.q += step_q;
    at.ch += step_ch;
    if (at.ch >= nch) {
      at.ch -= nch;
      ++at.q;
    }
    if (first + stride < n_items) load_group(first + stride, at);
#pragma unroll
    for (int u = 0; u < kWriteItems; ++u) {
      if (first + u >= n_items) break;  // wave-uniform
      const int64_t doc0 = it.ch * kDocsPerBundle;
      uint32_t b = bits[u];
      if (doc0 + kDocsPerBundle > num_docs) b &= valid_doc_mask(doc0 + lane_doc, num_docs);
      const uint32_t pc = static_cast<uint32_t>(__builtin_popcount(b));
      uint32_t total;
      const uint32_t incl = wave_inclusive_sum(pc, &total);
      uint16_t* sp = my + (incl - pc);
      for (uint32_t r = __builtin_bitreverse32(b); r != 0u; r &= r - 1u)
        *sp++ = static_cast<uint16_t>(lane_doc + static_cast<uint32_t>(__builtin_ctz(r)));
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      write_run(my, total, lane, doc0, ids + pos[u]);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      it.next(nch);
    }
  }
}

// As many workgroups as are resident at once (no tail of late workgroups),
// fewer when there are not enough items.
template <typename Kernel>
int compact_grid(Kernel kernel, int64_t n_items, int items_per_wave) {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kCompactThreads, 0) !=
          hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  const int64_t per_block = static_cast<int64_t>(kCompactWaves) * items_per_wave;
  const int64_t want = (n_items + per_block - 1) / per_block;
  return static_cast<int>(std::max<int64_t>(
      1, std::min<int64_t>(want, static_cast<int64_t>(cu_count()) * per_cu)));
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

// Turns the per-(query, chunk) match counts at the start of a compaction
// workspace into output positions, in place, and fills row_offsets.
void compact_scan_counts(int64_t* counts, int64_t num_queries, int64_t nch,
                         int64_t* row_offsets, hipStream_t s) {
  const int64_t items = num_queries * nch;
  const int64_t tiles = (items + kPartTile - 1) / kPartTile;
  int64_t* tile_sums = counts + items;
  hipLaunchKernelGGL(scan_reduce_kernel, dim3(static_cast<unsigned>(tiles)),
                     dim3(kPartThreads), 0, s, counts, items, tile_sums);
  check_launch("scan_reduce_kernel");
  if (tiles <= kPartPrefixTiles) {
    hipLaunchKernelGGL(scan_apply_kernel<true>, dim3(static_cast<unsigned>(tiles)),
                       dim3(kPartThreads), 0, s, counts, items, tile_sums, nch, row_offsets,
                       num_queries);
    check_launch("scan_apply_kernel");
    return;
  }
  hipLaunchKernelGGL(scan_tiles_kernel, dim3(1), dim3(kScanThreads), 0, s, tile_sums, tiles,
                     row_offsets, num_queries);
  check_launch("scan_tiles_kernel");
  hipLaunchKernelGGL(scan_apply_kernel<false>, dim3(static_cast<unsigned>(tiles)),
                     dim3(kPartThreads), 0, s, counts, items, tile_sums, nch, row_offsets,
                     num_queries);
  check_launch("scan_apply_kernel");
}

void compact_zero_offsets(int64_t* row_offsets, int64_t n, hipStream_t s) {
  hipLaunchKernelGGL(zero_offsets_kernel, dim3(static_cast<unsigned>((n + 255) / 256)),
                     dim3(256), 0, s, row_offsets, n);
  check_launch("zero_offsets_kernel");
}

}  // namespace st

extern "C" int64_t st_bloom_compact_workspace_bytes(int64_t num_queries, int64_t num_columns) {
  if (num_queries <= 0 || num_columns <= 0) return 0;
  const int64_t items = num_queries * st::num_chunks(num_columns);
  const int64_t tiles = (items + st::kPartTile - 1) / st::kPartTile;
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
      compact_zero_offsets(row_offsets, num_queries + 1, s);
      return;
    }
    ST_CHECK(packed != nullptr && workspace != nullptr, "null device pointer");
    int64_t* counts = static_cast<int64_t*>(workspace);
    const uint32_t* p32 = reinterpret_cast<const uint32_t*>(packed);
    if (num_columns % kChunkWords == 0 && reinterpret_cast<uintptr_t>(packed) % 16 == 0) {
      hipLaunchKernelGGL(compact_count_lines_kernel,
                         dim3(compact_grid(compact_count_lines_kernel, (items + 3) / 4, kCountLines)),
                         dim3(kCompactThreads), 0, s, reinterpret_cast<const u32x4*>(packed), nch,
                         num_docs, items, counts);
      check_launch("compact_count_lines_kernel");
    } else {
      hipLaunchKernelGGL(compact_count_kernel,
                         dim3(compact_grid(compact_count_kernel, items, kCountItems)),
                         dim3(kCompactThreads), 0, s, p32, num_columns, nch, num_docs, items,
                         counts);
      check_launch("compact_count_kernel");
    }
    compact_scan_counts(counts, num_queries, nch, row_offsets, s);
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
      hipLaunchKernelGGL(compact_write_kernel<int64_t>,
                         dim3(compact_grid(compact_write_kernel<int64_t>, items, kWriteItems)),
                         dim3(kCompactThreads), 0, s, p32, num_columns, nch, num_docs, items,
                         base, static_cast<int64_t*>(ids));
    } else {
      hipLaunchKernelGGL(compact_write_kernel<int32_t>,
                         dim3(compact_grid(compact_write_kernel<int32_t>, items, kWriteItems)),
                         dim3(kCompactThreads), 0, s, p32, num_columns, nch, num_docs, items,
                         base, static_cast<int32_t*>(ids));
    }
    check_launch("compact_write_kernel");
  });
}
