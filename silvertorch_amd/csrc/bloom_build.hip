// Bloom index build for gfx950.
//
// Replaces bloom_index_build (bloom_indexer.cpp:26-113 on CPU,
// bloom_indexer_cuda.cu:253-389 and :137-251 / :506-711 on CUDA) with three
// kernels:
//   widths_kernel   one workgroup per bundle of 2048 docs: per-doc term count
//                   (feature_offsets[(d+1)F] - feature_offsets[dF]), bundle
//                   max, b = (int64)((double)(max * k) * b_multiplier); also
//                   checks that feature_offsets never decreases.
//   scan_kernel     one workgroup: exclusive prefix sum of the widths into
//                   bundle_b_offsets, plus the totals the host needs.
//   scatter_kernel  one workgroup per bundle: zeroes a b x 32-word tile in
//                   LDS, hashes every (doc, feature, value) term of the bundle
//                   (one thread per value, its doc and feature from an LDS
//                   map of the slot group), ORs its k bits into the tile with
//                   LDS atomics and writes the tile out with coalesced stores.
//                   Bundles of up to kBuildSliceRows rows go in four passes of
//                   512 docs, each over a b x 8-word tile (the docs' columns);
//                   wider ones OR straight into global memory.
// The reference's per-doc byte signatures and 64-way transpose
// (bloom_indexer_cuda.cu:137-251, ~N*b/8 bytes of scratch) are not needed.
#include <hip/hip_runtime.h>

#include "st_common.hpp"
#include "st_errors.hpp"

namespace st {
int cu_count();

namespace {

constexpr int kWidthThreads = 256;
constexpr int kScanThreads = 1024;
constexpr int kBuildThreads = 1024;
constexpr int kBuildTileRows = 512;
constexpr int kBuildTileWords = kBuildTileRows * 32;
constexpr int kBuildSliceRows = kBuildTileWords / 8;  // rows of a 8-column slice tile
constexpr int kBuildSlices = 4;                       // 512-doc passes of a sliced bundle
constexpr int kBuildFeatureCache = 256;  // murmur_mix_x of the first feature ids, in LDS
constexpr int kBuildValueMap = 7168;     // values of a slot group mapped to their slot in LDS

// stats layout (device int64[6]):
//   [0] total rows  [1] max bundle width  [2] non-decreasing violation flag
//   [3] feature_offsets[0]  [4] feature_offsets[N*F]  [5] reserved
constexpr int kStatsLen = 6;

__global__ void init_stats_kernel(int64_t* __restrict__ stats) {
  if (threadIdx.x < kStatsLen) stats[threadIdx.x] = 0;
}

__device__ __forceinline__ int64_t wave_max(int64_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const int64_t o = __shfl_xor(v, off, 64);
    v = o > v ? o : v;
  }
  return v;
}

// Feature counts up to this stage a chunk's offsets in LDS (below).
constexpr int kWidthStageFeatures = 16;

__global__ __launch_bounds__(kWidthThreads) void widths_kernel(
    const int64_t* __restrict__ offsets, int64_t num_docs, int64_t num_features,
    int64_t k, double b_multiplier, int64_t* __restrict__ bundle_b_offsets,
    int64_t* __restrict__ stats) {
  __shared__ int64_t red[kWidthThreads / 64];
  __shared__ int64_t stage[kWidthThreads * kWidthStageFeatures + 1];
  const int64_t bundle = blockIdx.x;
  const int64_t doc0 = bundle * kDocsPerBundle;
  const int64_t doc1 = min(doc0 + kDocsPerBundle, num_docs);
  const int64_t F = num_features;
  int bad = 0;
  int64_t best = 0;
  if (F <= kWidthStageFeatures) {
    // Chunks of kWidthThreads docs: the chunk's offsets (F per doc and the
    // next doc's first) are loaded once with coalesced loads into registers,
    // the next chunk's loads are issued before this chunk is evaluated, and
    // the values pass through LDS so that thread t can check that its doc's
    // offsets never decrease and take its count from the first and the last.
    constexpr int kPer = kWidthStageFeatures + 1;  // ns <= kPer * kWidthThreads
    int64_t r[kPer];
    const auto load = [&](int64_t c0) {
      const int64_t ns = min<int64_t>(kWidthThreads, doc1 - c0) * F + 1;
      const int64_t* src = offsets + c0 * F;
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int64_t i = threadIdx.x + u * kWidthThreads;
        r[u] = i < ns ? src[i] : 0;
      }
    };
    if (doc0 < doc1) load(doc0);
    for (int64_t c0 = doc0; c0 < doc1; c0 += kWidthThreads) {
      const int64_t nd = min<int64_t>(kWidthThreads, doc1 - c0);
      const int64_t ns = nd * F + 1;
      __syncthreads();  // the previous chunk's readers are done with stage
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int64_t i = threadIdx.x + u * kWidthThreads;
        if (i < ns) stage[i] = r[u];
      }
      __syncthreads();
      if (c0 + kWidthThreads < doc1) load(c0 + kWidthThreads);
      if (threadIdx.x < nd) {
        const int64_t* o = stage + threadIdx.x * F;
        for (int64_t f = 0; f < F; ++f) bad |= o[f + 1] < o[f];
        const int64_t cnt = o[F] - o[0];
        best = cnt > best ? cnt : best;
      }
    }
  } else {
    // Wide docs: every offset is read once for the monotonicity check, the
    // doc boundaries again for the counts (L2 hits).
    for (int64_t s = doc0 * F + threadIdx.x; s < doc1 * F; s += kWidthThreads)
      bad |= offsets[s + 1] < offsets[s];
    for (int64_t d = doc0 + threadIdx.x; d < doc1; d += kWidthThreads) {
      const int64_t cnt = offsets[(d + 1) * F] - offsets[d * F];
      best = cnt > best ? cnt : best;
    }
  }
  best = wave_max(best);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
  if (__any(bad) && (threadIdx.x & 63) == 0) atomicOr(reinterpret_cast<unsigned long long*>(stats + 2), 1ull);
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t m = red[0];
    for (int i = 1; i < kWidthThreads / 64; ++i) m = red[i] > m ? red[i] : m;
    const int64_t b = static_cast<int64_t>(static_cast<double>(m * k) * b_multiplier);
    bundle_b_offsets[bundle + 1] = b;
    atomicMax(reinterpret_cast<unsigned long long*>(stats + 1),
              static_cast<unsigned long long>(b < 0 ? 0 : b));
  }
}

// In-place exclusive scan: on entry bundle_b_offsets[i+1] holds width i.
__global__ __launch_bounds__(kScanThreads) void scan_kernel(
    const int64_t* __restrict__ offsets, int64_t num_slots, int64_t nb,
    int64_t* __restrict__ bundle_b_offsets, int64_t* __restrict__ stats) {
  __shared__ int64_t part[kScanThreads];
  const int t = threadIdx.x;
  const int64_t per = (nb + kScanThreads - 1) / kScanThreads;
  const int64_t lo = min<int64_t>(t * per, nb);
  const int64_t hi = min<int64_t>(lo + per, nb);
  int64_t sum = 0;
  for (int64_t i = lo; i < hi; ++i) sum += bundle_b_offsets[i + 1];
  part[t] = sum;
  __syncthreads();
  for (int off = 1; off < kScanThreads; off <<= 1) {
    const int64_t v = t >= off ? part[t - off] : 0;
    __syncthreads();
    part[t] += v;
    __syncthreads();
  }
  int64_t run = t == 0 ? 0 : part[t - 1];
  for (int64_t i = lo; i < hi; ++i) {
    run += bundle_b_offsets[i + 1];
    bundle_b_offsets[i + 1] = run;
  }
  if (t == 0) {
    bundle_b_offsets[0] = 0;
    stats[0] = part[kScanThreads - 1];
    stats[3] = offsets[0];
    stats[4] = offsets[num_slots];
  }
}

// First K distinct positions murmur(fid, value, seed) % b over seeds
// 0, 1, 2, ... (assign_one_bits_position, bloom_index_util.cuh:183-207).
// b >= K always holds for bundles that have terms (b >= floor(K *
// b_multiplier) >= K), so the loop ends.
// The first K seeds are hashed unrolled with constant seeds and compared
// pairwise; only when two of them collide (about K^2 / 2b of the keys) does
// the key keep the first occurrence of each position, in seed order, and go
// on with seeds K, K + 1, ... as the sequential search would.
template <int K>
__device__ __forceinline__ void build_positions(uint64_t mx, uint64_t my,
                                                const FastMod64& fm,
                                                uint32_t (&found)[K]) {
  // The seed-independent rotations once per key; seeds stay far below
  // 2^27 (k distinct positions out of b >= k need few more than k seeds).
  const uint64_t rx = rotl64(mx, 27), ry = rotl64(my, 31);
  const bool small = fm.d < (1ull << 30);
  bool distinct = true;
#pragma unroll
  for (int j = 0; j < K; ++j) {
    const uint64_t h = murmur_finish_rot(rx, ry, static_cast<uint64_t>(j));
    found[j] = small ? fast_mod_small(h, fm) : static_cast<uint32_t>(fast_mod(h, fm));
#pragma unroll
    for (int i = 0; i < j; ++i) distinct &= found[i] != found[j];
  }
  if (distinct) return;
  uint32_t first[K];
#pragma unroll
  for (int j = 0; j < K; ++j) first[j] = found[j];
  int cnt = 0;
#pragma unroll
  for (int j = 0; j < K; ++j) {
    bool dup = false;
#pragma unroll
    for (int i = 0; i < j; ++i) dup |= first[i] == first[j];
    if (!dup) {
#pragma unroll
      for (int s = 0; s < K; ++s)
        if (s == cnt) found[s] = first[j];
      ++cnt;
    }
  }
  uint64_t seed = K;
  while (cnt < K) {
    const uint64_t h = seed < (1ull << 27) ? murmur_finish_rot(rx, ry, seed) : murmur_finish(mx, my, seed);
    ++seed;
    const uint32_t p = small ? fast_mod_small(h, fm) : static_cast<uint32_t>(fast_mod(h, fm));
    bool dup = false;
#pragma unroll
    for (int j = 0; j < K; ++j) dup |= (j < cnt) && (found[j] == p);
    if (!dup) {
#pragma unroll
      for (int j = 0; j < K; ++j)
        if (j == cnt) found[j] = p;
      ++cnt;
    }
  }
}

struct ScatterArgs {
  const int32_t* feature_ids;
  const int64_t* offsets;
  const int64_t* values;
  int64_t num_values;
  int64_t num_features;
  int64_t num_docs;
  int64_t k;
  const int64_t* bundle_b_offsets;
  unsigned long long* index;
};

// Swizzled LDS word of a tile of 2^lc columns (row p, column c): spreads the
// 64 lanes of a wave, which mostly share a column, over the LDS banks.
__device__ __forceinline__ int tile_word(uint32_t p, uint32_t c, int lc) {
  return static_cast<int>((p << lc) + (c ^ (p & ((1u << lc) - 1u))));
}

// Sets the term's bits either in the LDS tile or in global memory.
template <int K>
__device__ __forceinline__ void scatter_term(const ScatterArgs& a, int lc,
                                             unsigned long long* tile,
                                             unsigned long long* gbase,
                                             const FastMod64& fm, uint64_t mx,
                                             uint64_t my, uint32_t col,
                                             unsigned long long bit) {
  uint32_t found[K];
#pragma unroll
  for (int j = 0; j < K; ++j) found[j] = 0;
  build_positions<K>(mx, my, fm, found);
#pragma unroll
  for (int j = 0; j < K; ++j) {
    if (lc >= 0) {
      atomicOr(tile + tile_word(found[j], col, lc), bit);
    } else {
      atomicOr(gbase + static_cast<uint64_t>(found[j]) * 32 + col, bit);
    }
  }
}

// Runtime-k variant for k above the templated range (k <= 64).
__device__ void scatter_term_generic(const ScatterArgs& a, int lc,
                                     unsigned long long* tile,
                                     unsigned long long* gbase,
                                     const FastMod64& fm, uint64_t mx,
                                     uint64_t my, uint32_t col,
                                     unsigned long long bit) {
  uint32_t found[kMaxBuildK];
  const int k = static_cast<int>(a.k);
  int cnt = 0;
  uint64_t seed = 0;
  while (cnt < k) {
    const uint32_t p = static_cast<uint32_t>(fast_mod(murmur_finish(mx, my, seed++), fm));
    bool dup = false;
    for (int j = 0; j < cnt; ++j) dup |= found[j] == p;
    if (!dup) found[cnt++] = p;
  }
  for (int j = 0; j < k; ++j) {
    if (lc >= 0) {
      atomicOr(tile + tile_word(found[j], col, lc), bit);
    } else {
      atomicOr(gbase + static_cast<uint64_t>(found[j]) * 32 + col, bit);
    }
  }
}

template <int K>
__device__ __forceinline__ void scatter_value(const ScatterArgs& a, int lc,
                                              unsigned long long* tile,
                                              unsigned long long* gbase, const FastMod64& fm,
                                              uint64_t mx, int64_t value, uint32_t col,
                                              unsigned long long bit) {
  const uint64_t my = murmur_mix_y(static_cast<uint64_t>(value));
  if constexpr (K > 0) {
    scatter_term<K>(a, lc, tile, gbase, fm, mx, my, col, bit);
  } else {
    scatter_term_generic(a, lc, tile, gbase, fm, mx, my, col, bit);
  }
}

// One workgroup per bundle.  The bundle's (doc, feature) slots go in groups
// of kBuildThreads: each slot thread records its doc and feature for each of
// its values in an LDS map, then the threads take the group's values one
// each (all lanes hash, value loads coalesce).  A group with more values than
// the map holds walks them per slot instead.  The seed-independent half of
// the feature id's hash comes from LDS.  With one workgroup per CU nothing
// else covers the workgroup's global-load waits, so the loads are issued a
// step ahead: the next group's offsets during this group, the next value
// of a thread before the current one is hashed.
template <int K>
__global__ __launch_bounds__(kBuildThreads) void scatter_kernel(ScatterArgs a) {
  __shared__ unsigned long long tile[kBuildTileWords];
  __shared__ uint64_t mxc[kBuildFeatureCache];
  __shared__ uint32_t vmap[kBuildValueMap];  // doc | feature << 11 of each value

  const int tid = threadIdx.x;
  const int64_t bundle = blockIdx.x;
  const int64_t start = a.bundle_b_offsets[bundle];
  const int64_t b = a.bundle_b_offsets[bundle + 1] - start;
  // tile columns 2^lc: the whole bundle (32), a 512-doc slice (8), or no
  // tile (-1: bits go straight to global memory)
  const int lc = b <= kBuildTileRows ? 5 : (b <= kBuildSliceRows ? 3 : -1);
  const int passes = lc == 3 ? kBuildSlices : 1;
  unsigned long long* gbase = a.index + start * 32;
  const int64_t F = a.num_features;
  const int64_t cached = min<int64_t>(F, kBuildFeatureCache);

  for (int i = tid; i < cached; i += kBuildThreads)
    mxc[i] = murmur_mix_x(static_cast<uint64_t>(static_cast<int64_t>(a.feature_ids[i])));
  if (lc < 0) {
    for (int64_t w = tid; w < b * 32; w += kBuildThreads) gbase[w] = 0;
    __threadfence();
  }
  const FastMod64 fm = make_fastmod(static_cast<uint64_t>(b > 0 ? b : 1));
  const int64_t doc0 = bundle * kDocsPerBundle;
  const int64_t doc1 = min(doc0 + kDocsPerBundle, a.num_docs);
  const int64_t* offs = a.offsets + doc0 * F;
  const bool mappable = F < (1 << 21);  // doc (11 bits) and feature share a u32
  auto mx_of = [&](int64_t f) -> uint64_t {
    return f < cached
               ? mxc[f]
               : murmur_mix_x(static_cast<uint64_t>(static_cast<int64_t>(a.feature_ids[f])));
  };
  // Values outside [0, num_values) are never read (the host rejects offsets
  // that would point there before launching).
  auto clampv = [&](int64_t v) { return min<int64_t>(max<int64_t>(v, 0), a.num_values); };

  for (int pass = 0; pass < passes; ++pass) {
    // this pass's docs [dlo, dhi) (bundle-relative) and first tile column
    const int64_t dlo = lc == 3 ? pass * (kDocsPerBundle / kBuildSlices) : 0;
    const int64_t dhi = lc == 3 ? min<int64_t>(dlo + kDocsPerBundle / kBuildSlices, doc1 - doc0)
                                : doc1 - doc0;
    const uint32_t c0 = static_cast<uint32_t>(dlo >> 6);
    const int64_t tw = lc < 0 ? 0 : (b << lc);
    const int64_t slot_lo = dlo * F, slot_hi = max<int64_t>(dhi, dlo) * F;
    // the offsets a group reads: its slot's two and the group's two bounds
    struct GroupOffsets {
      int64_t o0, o1, g0, g1;
    };
    auto load_group = [&](int64_t g) {
      GroupOffsets o{0, 0, 0, 0};
      if (g >= slot_hi) return o;
      const int64_t rel = g + tid;
      if (rel < slot_hi) {
        o.o0 = offs[rel];
        o.o1 = offs[rel + 1];
      }
      o.g0 = offs[g];
      o.g1 = offs[min<int64_t>(g + kBuildThreads, slot_hi)];
      return o;
    };
    // the first group's offsets are in flight while the tile is cleared
    GroupOffsets next = load_group(b > 0 ? slot_lo : slot_hi);
    for (int64_t w = tid; w < tw; w += kBuildThreads) tile[w] = 0;
    __syncthreads();
    for (int64_t g = slot_lo; b > 0 && g < slot_hi; g += kBuildThreads) {
      const GroupOffsets cur = next;
      next = load_group(g + kBuildThreads);
      const int64_t rel = g + tid;
      const bool has_slot = rel < slot_hi;
      const int64_t v0 = has_slot ? clampv(cur.o0) : 0;
      const int64_t v1 = has_slot ? clampv(cur.o1) : 0;
      const int64_t d = has_slot ? rel / F : 0;
      const int64_t f = has_slot ? rel - d * F : 0;
      const int64_t gv0 = clampv(cur.g0);
      const int64_t gv1 = clampv(cur.g1);
      if (mappable && gv1 - gv0 <= kBuildValueMap) {  // uniform across the workgroup
        // Value loads are clamped to the group's last value rather than
        // predicated: with the same loads on every path the next value stays
        // in flight while the current one is hashed.  The first is issued
        // before the map is built.
        const int64_t last = max<int64_t>(gv1 - 1, gv0);
        const bool any = gv1 > gv0;  // uniform
        int64_t j = gv0 + tid;
        int64_t value = any ? a.values[min(j, last)] : 0;
        __syncthreads();  // previous group's readers are done with vmap
        for (int64_t i = v0; i < v1; ++i)
          vmap[i - gv0] = static_cast<uint32_t>(d) | (static_cast<uint32_t>(f) << 11);
        __syncthreads();
        for (; j < gv1; j += kBuildThreads) {
          const int64_t value_next = a.values[min(j + kBuildThreads, last)];
          const uint32_t m = vmap[j - gv0];
          const uint32_t dd = m & 2047u;
          scatter_value<K>(a, lc, tile, gbase, fm, mx_of(m >> 11), value, (dd >> 6) - c0,
                           1ull << (63 - (dd & 63)));
          value = value_next;
        }
      } else if (v0 < v1) {
        const uint64_t mx = mx_of(f);
        for (int64_t j = v0; j < v1; ++j)
          scatter_value<K>(a, lc, tile, gbase, fm, mx, a.values[j],
                           static_cast<uint32_t>(d >> 6) - c0, 1ull << (63 - (d & 63)));
      }
    }
    __syncthreads();
    if (lc >= 0) {
      const uint32_t cmask = (1u << lc) - 1u;
      for (int64_t w = tid; w < tw; w += kBuildThreads) {
        const uint32_t p = static_cast<uint32_t>(w >> lc);
        const uint32_t c = static_cast<uint32_t>(w) & cmask;
        __builtin_nontemporal_store(tile[tile_word(p, c, lc)],
                                    gbase + static_cast<int64_t>(p) * 32 + c0 + c);
      }
      if (pass + 1 < passes) __syncthreads();  // the stores have read the tile
    }
  }
}

using ScatterFn = void (*)(ScatterArgs);

ScatterFn select_scatter(int64_t k) {
  switch (k) {
    case 1: return scatter_kernel<1>;
    case 2: return scatter_kernel<2>;
    case 3: return scatter_kernel<3>;
    case 4: return scatter_kernel<4>;
    case 5: return scatter_kernel<5>;
    case 6: return scatter_kernel<6>;
    case 7: return scatter_kernel<7>;
    case 8: return scatter_kernel<8>;
    case 9: return scatter_kernel<9>;
    case 10: return scatter_kernel<10>;
    default: return scatter_kernel<0>;
  }
}

void check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    throw Error(ST_ERR_HIP, cat(what, " launch failed: ", hipGetErrorString(e)));
}

}  // namespace
}  // namespace st

extern "C" int st_bloom_build_bundle_offsets(const int64_t* feature_offsets,
                                             int64_t num_docs,
                                             int64_t num_features, int64_t k,
                                             double b_multiplier,
                                             int64_t* bundle_b_offsets,
                                             int64_t* stats, void* stream) {
  using namespace st;
  return guarded([&] {
    ST_CHECK(num_features >= 1, "feature_ids must not be empty");
    ST_CHECK(num_docs >= 0, "negative document count");
    ST_CHECK(k >= 0 && k <= kMaxBuildK, "k must be in [0, ", kMaxBuildK,
             "], got ", k);
    ST_CHECK(b_multiplier > 1.0, "b_multiplier must be greater than 1.0");
    ST_CHECK(feature_offsets && bundle_b_offsets && stats, "null device pointer");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t nb = (num_docs + kDocsPerBundle - 1) / kDocsPerBundle;
    hipLaunchKernelGGL(init_stats_kernel, dim3(1), dim3(64), 0, s, stats);
    check_launch("init_stats_kernel");
    if (nb > 0) {
      hipLaunchKernelGGL(widths_kernel, dim3(static_cast<unsigned>(nb)),
                         dim3(kWidthThreads), 0, s, feature_offsets, num_docs,
                         num_features, k, b_multiplier, bundle_b_offsets, stats);
      check_launch("widths_kernel");
    }
    hipLaunchKernelGGL(scan_kernel, dim3(1), dim3(kScanThreads), 0, s,
                       feature_offsets, num_docs * num_features, nb,
                       bundle_b_offsets, stats);
    check_launch("scan_kernel");
  });
}

extern "C" int st_bloom_index_build(const int32_t* feature_ids,
                                    const int64_t* feature_offsets,
                                    const int64_t* feature_values,
                                    int64_t num_features, int64_t num_docs,
                                    int64_t num_values, int64_t k,
                                    const int64_t* bundle_b_offsets,
                                    int64_t max_b, int64_t* bloom_index,
                                    int64_t bloom_index_numel, void* stream) {
  using namespace st;
  return guarded([&] {
    ST_CHECK(num_features >= 1, "feature_ids must not be empty");
    ST_CHECK(num_docs >= 0 && num_values >= 0, "negative sizes");
    ST_CHECK(k >= 0 && k <= kMaxBuildK, "k must be in [0, ", kMaxBuildK,
             "], got ", k);
    const int64_t nb = (num_docs + kDocsPerBundle - 1) / kDocsPerBundle;
    if (nb == 0 || bloom_index_numel == 0) return;
    ST_CHECK(feature_ids && feature_offsets && bundle_b_offsets && bloom_index,
             "null device pointer");
    ST_CHECK(num_values == 0 || feature_values, "feature_values is null");
    (void)max_b;
    ScatterArgs a;
    a.feature_ids = feature_ids;
    a.offsets = feature_offsets;
    a.values = feature_values;
    a.num_values = num_values;
    a.num_features = num_features;
    a.num_docs = num_docs;
    a.k = k;
    a.bundle_b_offsets = bundle_b_offsets;
    a.index = reinterpret_cast<unsigned long long*>(bloom_index);
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(select_scatter(k), dim3(static_cast<unsigned>(nb)),
                       dim3(kBuildThreads), 0, s, a);
    check_launch("scatter_kernel");
  });
}
