// Fused bloom filter + top-k scoring for gfx950.
//
// No reference operator: the closest relatives are the bloom-filtered
// scoring of fused_kmean_ann (fused_kmean_ann_cuda.cu:545-551, :1797-1926)
// and at::topk in fresh_index_post_processing.cpp:245-250.  For every query
// q, among docs d < num_docs whose bit is set in the packed search output
// (doc 64c+i of row q at bit 63-i of word c), return the `topk` best by
//   score(q, d) = sum_j bf16(emb[d, j]) * bf16(x[q, j])   (fp32 accumulation)
// ordered by score descending, then doc id ascending; missing entries are
// id -1 and score -inf (the reference's padding, fused_kmean_ann.cpp:139-167).
//
// Scoring is a dense bf16 contraction on the matrix cores
// (v_mfma_f32_32x32x16_bf16): each wave holds the embeddings of 64 docs in
// registers (two 32-doc A operands) and sweeps the query chunk staged in LDS
// 32 queries at a time, so one LDS read of a query fragment feeds two MFMAs.
// A 32 x 32 tile whose filter bits are all zero is skipped.
//
// Selection is exact and runs in rounds over growing doc ranges: a scored
// pair enters query q's candidate list when it passes the filter and its
// score is at least thr[q]; after each round one workgroup per query sorts
// its candidates (bitonic, in LDS) down to the best `topk` and sets thr[q] to
// the score of the topk-th, so later rounds emit only pairs that can still
// enter.  A candidate list has a fixed capacity; if any round overflows one,
// the whole selection is redone with rounds too small to overflow.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <vector>

#include "st_common.hpp"
#include "st_errors.hpp"

namespace st {
int cu_count();

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kScoreThreads = 512;   // 8 waves; one workgroup per CU
constexpr int kScoreWaves = kScoreThreads / 64;
constexpr int kDocsPerWave = 64;     // two 32-doc MFMA A operands
constexpr int kDocsPerStep = kScoreWaves * kDocsPerWave;
constexpr int kQueryTile = 32;
constexpr int kLdsBytes = 160 * 1024;
constexpr int kSelectThreads = 256;
constexpr int kSelectSlots = 4096;   // bitonic buffer: best 2048 + a chunk of 2048
constexpr int kSelectChunk = kSelectSlots / 2;
constexpr int kMaxTopk = kSelectChunk;
constexpr uint32_t kCandidateCapacity = 32768;  // per query
constexpr int64_t kRoundAlign = 2048;

// Monotone map of floats to unsigned ints (larger float -> larger int).
__device__ __forceinline__ uint32_t ordered_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float from_ordered(uint32_t o) {
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}

// Sort key: score descending, then doc id ascending, as one descending
// 64-bit key.  Key 0 sorts below every real key.
__device__ __forceinline__ uint64_t make_key(float score, int64_t doc) {
  return (static_cast<uint64_t>(ordered_bits(score)) << 32) |
         (0xFFFFFFFFu - static_cast<uint32_t>(doc));
}

struct TopkState {
  uint32_t* counts;    // [Q] candidates held
  float* thr;          // [Q] entry threshold
  uint64_t* cand;      // [Q * capacity] keys
  uint32_t* overflow;  // [1]
  uint32_t capacity;
};

__global__ void topk_reset_kernel(TopkState st, int64_t num_queries) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < num_queries) {
    st.counts[i] = 0u;
    st.thr[i] = -INFINITY;
  }
  if (i == 0) st.overflow[0] = 0u;
}

// LDS bytes per query of a chunk: its row (D bf16) plus, per wave, the two
// u32 filter words of the wave's 64 docs.
template <int D>
constexpr int lds_bytes_per_query() {
  return D * 2 + kScoreWaves * 8;
}

template <int D>
constexpr int64_t query_chunk() {
  return (kLdsBytes / lds_bytes_per_query<D>()) / kQueryTile * kQueryTile;
}

// Scores docs [lo, hi) against queries [q_begin, q_begin + q_count).
// LDS: the query rows (16-byte pieces XOR-swizzled by row, so the 32 rows a
// wave reads at once hit distinct banks), then per wave the filter words of
// its 64 docs for every query of the chunk.
template <int D>
__global__ __launch_bounds__(kScoreThreads) void topk_score_kernel(
    const uint16_t* __restrict__ emb, const uint16_t* __restrict__ qv,
    const uint32_t* __restrict__ mask32, int64_t num_columns, int64_t q_begin,
    int64_t q_count, int64_t lo, int64_t hi, TopkState st) {
  constexpr int S = D / 16;        // MFMA k-steps
  constexpr int kPieces = D / 8;   // 16-byte pieces per row
  // 16 lanes read at once on gfx950 (64 banks): spread 16 rows.
  constexpr int kSwz = kPieces < 16 ? kPieces - 1 : 15;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int q_tiles = static_cast<int>((q_count + kQueryTile - 1) / kQueryTile);
  const int rows = q_tiles * kQueryTile;
  uint32_t* masks = reinterpret_cast<uint32_t*>(lds + static_cast<int64_t>(rows) * D * 2) +
                    wave * rows * 2;  // [tile][64]: lanes 0-31 docs 0-31, 32-63 docs 32-63

  for (int i = threadIdx.x; i < rows * kPieces; i += kScoreThreads) {
    const int r = i / kPieces, c = i - r * kPieces;
    bf16x8 v = {};
    if (r < q_count) v = *reinterpret_cast<const bf16x8*>(qv + (q_begin + r) * D + c * 8);
    *reinterpret_cast<bf16x8*>(lds + r * (D * 2) + ((c ^ (r & kSwz)) << 4)) = v;
  }
  __syncthreads();

  for (int64_t base = lo + static_cast<int64_t>(blockIdx.x) * kDocsPerStep; base < hi;
       base += static_cast<int64_t>(gridDim.x) * kDocsPerStep) {
    const int64_t d0 = base + wave * kDocsPerWave;  // first doc of this wave
    if (d0 >= hi) continue;                         // wave-uniform
    // Filter words of the wave's 64 docs for every query: docs 0-31 of a
    // word are its high half, the second u32 in memory (d0 is a multiple of
    // 64 within the round).
    {
      constexpr int kBatch = 16;  // loads in flight before the LDS stores
      const int64_t col = d0 >> 6;
      const int half = lane >> 5;
      const bool has = half == 0 || d0 + 32 < hi;
      // docs at or past hi never pass (bit 31 is the half-word's first doc)
      const int64_t left = hi - (d0 + 32 * half);
      const uint32_t valid = left >= 32 ? ~0u : (left <= 0 ? 0u : ~0u << (32 - static_cast<int>(left)));
      for (int t0 = 0; t0 < q_tiles; t0 += kBatch) {
        uint32_t mv[kBatch];
        // Unconditional loads from a valid address (selected afterwards), so
        // that all of them are in flight before the first is waited for.
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          const int64_t ql = static_cast<int64_t>(t0 + u) * kQueryTile + (lane & 31);
          const bool ok = t0 + u < q_tiles && ql < q_count && has;
          const int64_t idx = ok ? (q_begin + ql) * 2 * num_columns + 2 * col + 1 - half : 0;
          mv[u] = mask32[idx];
          mv[u] = ok ? mv[u] & valid : 0u;
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
          if (t0 + u < q_tiles) masks[(t0 + u) * 64 + lane] = mv[u];
      }
    }
    bf16x8 a0[S], a1[S];
    {
      const int kofs = (lane >> 5) * 8;
      // Rows past hi read row hi - 1 (valid) and are zeroed afterwards.
      const int64_t da = d0 + (lane & 31), db = da + 32;
      const int64_t ra = da < hi ? da : hi - 1, rb = db < hi ? db : hi - 1;
#pragma unroll
      for (int s = 0; s < S; ++s) {
        a0[s] = *reinterpret_cast<const bf16x8*>(emb + ra * D + s * 16 + kofs);
        a1[s] = *reinterpret_cast<const bf16x8*>(emb + rb * D + s * 16 + kofs);
      }
      if (da >= hi) {
#pragma unroll
        for (int s = 0; s < S; ++s) a0[s] = bf16x8{};
      }
      if (db >= hi) {
#pragma unroll
        for (int s = 0; s < S; ++s) a1[s] = bf16x8{};
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float th_next = st.thr[q_begin + ((lane & 31) < q_count ? (lane & 31) : 0)];
    for (int t = 0; t < q_tiles; ++t) {
      const int ql = t * kQueryTile + (lane & 31);  // query of this lane's column
      const bool qvalid = ql < q_count;
      const int64_t q = q_begin + ql;
      const float th = qvalid ? th_next : INFINITY;
      {  // threshold of the next tile, one tile ahead (clamped address)
        const int qn = ql + kQueryTile;
        th_next = st.thr[q_begin + (qn < q_count ? qn : 0)];
      }
      // lane's column: docs 0-31 in slot (lane & 31), docs 32-63 in slot 32 + (lane & 31)
      const uint32_t m0 = masks[t * 64 + (lane & 31)];
      const uint32_t m1 = masks[t * 64 + 32 + (lane & 31)];
      if (__ballot((m0 | m1) != 0u) == 0) continue;  // no filter bit in the tile
      // All query fragments first (one LDS latency per tile), then the two
      // MFMA chains; a half-tile without filter bits still runs (rare at
      // useful selectivities, and cheaper than a branch per MFMA).
      f32x16 acc0 = {}, acc1 = {};
      const uint8_t* qrow = lds + ql * (D * 2);
      const int sw = ql & kSwz;
      bf16x8 b[S];
#pragma unroll
      for (int s = 0; s < S; ++s)
        b[s] = *reinterpret_cast<const bf16x8*>(qrow + (((2 * s + (lane >> 5)) ^ sw) << 4));
#pragma unroll
      for (int s = 0; s < S; ++s) {
        acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0[s], b[s], acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1[s], b[s], acc1, 0, 0, 0);
      }
      // acc[j] holds doc row 8*(j/4) + 4*(lane/32) + j%4 of the tile, query
      // column lane % 32.
      {
        // Gate on the lane maxima (no score of the tile at the threshold),
        // then per-lane hit bits, one atomic per query per tile for a run of
        // slots, and the writes.
        float mx = fmaxf(acc0[0], acc1[0]);
#pragma unroll
        for (int j = 1; j < 16; ++j) mx = fmaxf(mx, fmaxf(acc0[j], acc1[j]));
        if (__ballot(mx >= th) == 0) continue;
        uint32_t hits = 0u;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int r = 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
          const bool h0 = ((m0 >> (31 - r)) & 1u) && acc0[j] >= th;
          const bool h1 = ((m1 >> (31 - r)) & 1u) && acc1[j] >= th;
          hits |= (h0 ? 1u << j : 0u) | (h1 ? 1u << (16 + j) : 0u);
        }
        if (__ballot(hits != 0u) == 0) continue;
        const uint32_t cnt = __builtin_popcount(hits);
        const uint32_t cnt_pair = __shfl_xor(cnt, 32, 64);  // lanes l, l ^ 32: same query
        uint32_t base = 0u;
        if (lane < 32 && cnt + cnt_pair > 0u) base = atomicAdd(st.counts + q, cnt + cnt_pair);
        const uint32_t base_pair = __shfl_xor(base, 32, 64);
        uint32_t slot = lane < 32 ? base : base_pair + cnt_pair;
        while (__ballot(hits != 0u) != 0) {
          if (hits != 0u) {
            const int j = __builtin_ctz(hits);
            hits &= hits - 1u;
            const int jj = j & 15;
            const bool second = j >= 16;
            float v = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) v = jj == i ? (second ? acc1[i] : acc0[i]) : v;
            const int64_t doc = d0 + (second ? 32 : 0) + 8 * (jj >> 2) + 4 * (lane >> 5) + (jj & 3);
            if (slot < st.capacity) st.cand[q * st.capacity + slot] = make_key(v, doc);
            else atomicOr(st.overflow, 1u);
            ++slot;
          }
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

// Descending bitonic sort of the first `size` keys in LDS (a power of two).
__device__ void bitonic_sort_desc(uint64_t* keys, int size) {
  for (int k = 2; k <= size; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < size / 2; i += kSelectThreads) {
        // i-th compare pair of this stage: lower index lo, partner lo + j
        const int lo = ((i & ~(j - 1)) << 1) | (i & (j - 1));
        const int hi = lo + j;
        const bool desc = (lo & k) == 0;  // direction of this k-block
        const uint64_t x = keys[lo], y = keys[hi];
        if ((x < y) == desc) {
          keys[lo] = y;
          keys[hi] = x;
        }
      }
      __syncthreads();
    }
  }
}

// One workgroup per query: keeps the best `topk` candidates (sorted), sets
// the entry threshold, and on the last round writes the outputs.
__global__ __launch_bounds__(kSelectThreads) void topk_select_kernel(
    TopkState st, int64_t topk, int final_round, int64_t* __restrict__ out_ids,
    float* __restrict__ out_scores) {
  __shared__ uint64_t keys[kSelectSlots];
  const int64_t q = blockIdx.x;
  uint64_t* cand = st.cand + q * st.capacity;
  const uint32_t n = min(st.counts[q], st.capacity);
  if (n <= static_cast<uint32_t>(kSelectSlots)) {
    // One sort of the smallest power of two holding every candidate.
    int size = 64;
    while (size < static_cast<int>(n)) size <<= 1;
    for (int i = threadIdx.x; i < size; i += kSelectThreads) keys[i] = i < static_cast<int>(n) ? cand[i] : 0ull;
    __syncthreads();
    bitonic_sort_desc(keys, size);
  } else {
    // Keys 0 .. kSelectChunk-1 hold the best so far; each chunk of
    // candidates is sorted in behind them.
    for (int i = threadIdx.x; i < kSelectChunk; i += kSelectThreads) keys[i] = 0ull;
    for (uint32_t c0 = 0; c0 < n; c0 += kSelectChunk) {
      for (int i = threadIdx.x; i < kSelectChunk; i += kSelectThreads)
        keys[kSelectChunk + i] = c0 + i < n ? cand[c0 + i] : 0ull;
      __syncthreads();
      bitonic_sort_desc(keys, kSelectSlots);
    }
  }
  const uint32_t kept = min(n, static_cast<uint32_t>(topk));
  if (final_round) {
    for (int64_t i = threadIdx.x; i < topk; i += kSelectThreads) {
      const bool have = i < kept;
      out_ids[q * topk + i] = have ? static_cast<int64_t>(0xFFFFFFFFu - static_cast<uint32_t>(keys[i]))
                                   : -1;
      out_scores[q * topk + i] = have ? from_ordered(static_cast<uint32_t>(keys[i] >> 32)) : -INFINITY;
    }
    return;
  }
  for (uint32_t i = threadIdx.x; i < kept; i += kSelectThreads) cand[i] = keys[i];
  if (threadIdx.x == 0) {
    st.counts[q] = kept;
    st.thr[q] = kept == topk ? from_ordered(static_cast<uint32_t>(keys[topk - 1] >> 32)) : -INFINITY;
  }
}

void check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) throw Error(ST_ERR_HIP, cat(what, " launch failed: ", hipGetErrorString(e)));
}

template <int D>
void launch_score(const uint16_t* emb, const uint16_t* qv, const uint32_t* mask32,
                  int64_t num_columns, int64_t num_queries, int64_t lo, int64_t hi,
                  const TopkState& st, hipStream_t s) {
  const int64_t q_chunk = query_chunk<D>();
  const int64_t steps = (hi - lo + kDocsPerStep - 1) / kDocsPerStep;
  const int grid = static_cast<int>(std::max<int64_t>(
      1, std::min<int64_t>(steps, static_cast<int64_t>(cu_count()))));
  for (int64_t qb = 0; qb < num_queries; qb += q_chunk) {
    const int64_t qn = std::min(q_chunk, num_queries - qb);
    const size_t lds = static_cast<size_t>((qn + kQueryTile - 1) / kQueryTile * kQueryTile) *
                       lds_bytes_per_query<D>();
    hipLaunchKernelGGL(topk_score_kernel<D>, dim3(grid), dim3(kScoreThreads), lds, s, emb, qv,
                       mask32, num_columns, qb, qn, lo, hi, st);
    check_launch("topk_score_kernel");
  }
}

using ScoreFn = void (*)(const uint16_t*, const uint16_t*, const uint32_t*, int64_t, int64_t,
                         int64_t, int64_t, const TopkState&, hipStream_t);

ScoreFn score_fn(int64_t dim) {
  switch (dim) {
    case 64: return launch_score<64>;
    case 128: return launch_score<128>;
    case 256: return launch_score<256>;
    default: fail("embedding dimension ", dim, " is not supported (64, 128 or 256)");
  }
}

// The scoring kernel stages up to 160 KB of queries in LDS.
void set_lds_limits() {
  static std::once_flag once;
  static hipError_t status = hipSuccess;
  std::call_once(once, [] {
    for (const void* k : {reinterpret_cast<const void*>(topk_score_kernel<64>),
                          reinterpret_cast<const void*>(topk_score_kernel<128>),
                          reinterpret_cast<const void*>(topk_score_kernel<256>)}) {
      const hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
      if (e != hipSuccess && status == hipSuccess) status = e;
    }
  });
  if (status != hipSuccess)
    throw Error(ST_ERR_HIP, cat("hipFuncSetAttribute failed: ", hipGetErrorString(status)));
}

// Doc ranges of the rounds: a first round of 8192 docs, then each round
// eight times everything before it (rounds aligned to bundles), or, in the
// safe schedule, rounds no larger than a candidate list can always hold.
std::vector<int64_t> round_bounds(int64_t num_docs, int64_t topk, bool safe) {
  std::vector<int64_t> b{0};
  int64_t pos = 0;
  const int64_t safe_step =
      std::max<int64_t>(kRoundAlign, (static_cast<int64_t>(kCandidateCapacity) - topk) / kRoundAlign * kRoundAlign);
  while (pos < num_docs) {
    int64_t step = safe ? safe_step : (pos == 0 ? 8192 : 8 * pos);
    step = (step + kRoundAlign - 1) / kRoundAlign * kRoundAlign;
    pos = std::min(num_docs, pos + step);
    b.push_back(pos);
  }
  return b;
}

}  // namespace
}  // namespace st

extern "C" int64_t st_filtered_topk_workspace_bytes(int64_t num_queries) {
  if (num_queries <= 0) return 0;
  return num_queries * (4 + 4 + 8 * static_cast<int64_t>(st::kCandidateCapacity)) + 256;
}

extern "C" int st_filtered_topk(const int64_t* packed, int64_t num_queries,
                                int64_t num_columns, int64_t num_docs,
                                const void* doc_embeddings, const void* query_embeddings,
                                int64_t dim, int64_t topk, void* workspace,
                                int64_t* out_ids, float* out_scores, void* stream) {
  using namespace st;
  return guarded([&] {
    ST_CHECK(num_queries >= 0 && num_columns >= 0 && num_docs >= 0, "negative sizes");
    ST_CHECK(topk >= 1 && topk <= kMaxTopk, "topk must be in [1, ", kMaxTopk, "], got ", topk);
    ST_CHECK(num_docs <= num_columns * kBitsPerColumn,
             "num_docs ", num_docs, " exceeds the mask's ", num_columns * kBitsPerColumn, " docs");
    ST_CHECK(num_docs <= 0xFFFFFFFFll, "doc ids must fit 32 bits");
    if (num_queries == 0) return;
    ST_CHECK(out_ids && out_scores && workspace, "null device pointer");
    ST_CHECK(num_docs == 0 || (packed && doc_embeddings && query_embeddings), "null device pointer");
    ST_CHECK(reinterpret_cast<uintptr_t>(doc_embeddings) % 16 == 0 &&
                 reinterpret_cast<uintptr_t>(query_embeddings) % 16 == 0,
             "embeddings must be 16-byte aligned");
    const ScoreFn score = score_fn(dim);
    set_lds_limits();
    hipStream_t s = static_cast<hipStream_t>(stream);
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    TopkState state;
    state.counts = reinterpret_cast<uint32_t*>(ws);
    state.thr = reinterpret_cast<float*>(ws + 4 * num_queries);
    state.overflow = reinterpret_cast<uint32_t*>(ws + 8 * num_queries);
    state.cand = reinterpret_cast<uint64_t*>(ws + ((8 * num_queries + 4 + 255) / 256) * 256);
    state.capacity = kCandidateCapacity;
    const uint16_t* emb = static_cast<const uint16_t*>(doc_embeddings);
    const uint16_t* qv = static_cast<const uint16_t*>(query_embeddings);
    const uint32_t* m32 = reinterpret_cast<const uint32_t*>(packed);
    const unsigned qgrid = static_cast<unsigned>(num_queries);

    for (int attempt = 0; attempt < 2; ++attempt) {
      const bool safe = attempt == 1;
      hipLaunchKernelGGL(topk_reset_kernel, dim3(static_cast<unsigned>((num_queries + 255) / 256)),
                         dim3(256), 0, s, state, num_queries);
      check_launch("topk_reset_kernel");
      const std::vector<int64_t> bounds = round_bounds(num_docs, topk, safe);
      for (size_t r = 0; r + 1 < bounds.size(); ++r) {
        score(emb, qv, m32, num_columns, num_queries, bounds[r], bounds[r + 1], state, s);
        const bool last = r + 2 == bounds.size();
        hipLaunchKernelGGL(topk_select_kernel, dim3(qgrid), dim3(kSelectThreads), 0, s, state,
                           topk, last ? 1 : 0, out_ids, out_scores);
        check_launch("topk_select_kernel");
      }
      if (bounds.size() == 1) {  // no docs: every output is padding
        hipLaunchKernelGGL(topk_select_kernel, dim3(qgrid), dim3(kSelectThreads), 0, s, state,
                           topk, 1, out_ids, out_scores);
        check_launch("topk_select_kernel");
        return;
      }
      if (safe) return;  // rounds of this schedule cannot overflow
      uint32_t overflow = 0;
      hipError_t e = hipMemcpyAsync(&overflow, state.overflow, 4, hipMemcpyDeviceToHost, s);
      if (e == hipSuccess) e = hipStreamSynchronize(s);
      if (e != hipSuccess)
        throw Error(ST_ERR_HIP, cat("reading the overflow flag failed: ", hipGetErrorString(e)));
      if (!overflow) return;
    }
  });
}
