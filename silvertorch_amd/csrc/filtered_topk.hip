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
// (v_mfma_f32_32x32x16_bf16): each wave keeps the fragments of its 32 or 64
// queries in registers (B operands) for the whole launch, the workgroup
// streams 64 KB steps of doc rows and their filter words through LDS (the
// next step is loaded into registers while the current one is scored), and
// one LDS read of a doc fragment feeds the MFMAs of every query tile of the
// wave.  A doc tile whose filter bits are all zero for the wave is skipped.
//
// Selection is exact and runs in rounds over growing doc ranges: a scored
// pair enters query q's candidate list when it passes the filter and its
// score is at least thr[q]; after each round one workgroup per query keeps
// the best `topk` of its candidates (a radix select in LDS; the last round
// sorts them, bitonic) and sets thr[q] to the score of the topk-th, so later
// rounds emit only pairs that can still enter.  A candidate list has a fixed capacity; if any round overflows one,
// the whole selection is redone with rounds too small to overflow.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <utility>
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
constexpr int kQueryTile = 32;
constexpr int kLdsBytes = 160 * 1024;
constexpr int kSelectThreads = 256;
constexpr int kSelectSlots = 4096;   // candidates gathered into LDS for the selection
constexpr int kMaxTopk = 2048;
constexpr uint32_t kCandidateCapacity = 32768;  // per query
// A query's candidate list: the best kept so far in slots [0, kMaxTopk), then
// one segment per scoring workgroup (at most kMaxSegments of them), each
// filled by its workgroup alone.
constexpr int kMaxSegments = 256;
constexpr uint32_t kSegmentSlots = kCandidateCapacity - kMaxTopk;
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
  uint32_t* counts;    // [Q] best candidates kept (<= topk)
  float* thr;          // [Q] entry threshold
  uint64_t* cand;      // [Q * capacity] keys
  uint32_t* segn;      // [Q * kMaxSegments] entries in each segment
  uint32_t* overflow;  // [1]
  uint32_t capacity;
  uint32_t seg;        // slots per segment in the current round
};

__global__ void topk_reset_kernel(TopkState st, int64_t num_queries) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < num_queries) {
    st.counts[i] = 0u;
    st.thr[i] = -INFINITY;
  }
  if (i == 0) st.overflow[0] = 0u;
}

// Scoring geometry for embedding dimension D.  Each of the 8 waves keeps
// QT query tiles (32 queries each) as MFMA B operands in registers, so one
// launch pass covers 8 * 32 * QT queries; the workgroup streams its docs in
// steps of kDocs rows (32 KB of embeddings) through two LDS buffers, each with
// the queries' filter words for those docs.
template <int D>
struct ScoreShape {
  static constexpr int S = D / 16;                     // MFMA k-steps
  static constexpr int QT = D <= 128 ? 2 : 1;          // query tiles per wave
  static constexpr int kQueries = kScoreWaves * kQueryTile * QT;  // per pass
  static constexpr int kStepBytes = 32768;
  static constexpr int kDocs = kStepBytes / (2 * D);   // docs per step
  static constexpr int kDocTiles = kDocs / 32;
  static constexpr int kPieces = D / 8;                // 16-byte pieces per doc row
  // Rows padded by 16 bytes: the 16 rows an A-operand read serves at once
  // start 4 banks apart, and every piece sits at a fixed offset of its row.
  static constexpr int kRowBytes = 2 * D + 16;
  static constexpr int kCols = kDocs / 64;             // mask columns per step
  static constexpr int kMaskWords = kDocTiles + 1;     // u32 per query, padded
  static constexpr int kDocBuf = kDocs * kRowBytes;
  static constexpr int kMaskBuf = kQueries * kMaskWords * 4;
  static constexpr int kBuf = kDocBuf + kMaskBuf;
  static constexpr int kLds = 2 * kBuf + kQueries * 4;  // + segment slot counters
  static constexpr int kDocLoads = kStepBytes / 16 / kScoreThreads;  // u32x4 per thread
  static constexpr int kMaskLoads = (kQueries * kCols + kScoreThreads - 1) / kScoreThreads;
  static_assert(kLds <= kLdsBytes, "two steps must fit in LDS");
  static_assert(kDocs % 64 == 0 && kStepBytes % (16 * kScoreThreads) == 0, "step shape");
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Filter bits of the 32 docs from g0 that lie below hi (doc g0 at bit 31).
__device__ __forceinline__ uint32_t valid_doc_mask(int64_t g0, int64_t hi) {
  const int64_t left = hi - g0;
  return left >= 32 ? ~0u : (left <= 0 ? 0u : ~0u << (32 - static_cast<int>(left)));
}

// acc[j] of a 32 x 32 MFMA result holds doc row 8 (j / 4) + 4 h + j % 4 of
// the tile for lane half h = lane / 32 (query column lane % 32).  Returns the
// filter bits of those rows, row of acc[j] at bit j (doc row r of m at bit
// 31 - r).
__device__ __forceinline__ uint32_t lane_rows(uint32_t m, int h) {
  uint32_t x = (__builtin_bitreverse32(m) >> (4 * h)) & 0x0F0F0F0Fu;
  x = (x | (x >> 4)) & 0x00FF00FFu;
  return (x | (x >> 8)) & 0xFFFFu;
}

// Whether this lane's part of a 32 x 32 score tile (16 docs of its query)
// may hold a candidate: a filter bit, and a score at the threshold.
__device__ __forceinline__ bool tile_gate(const f32x16& acc, uint32_t m, float th) {
  float mx = acc[0];
#pragma unroll
  for (int j = 1; j < 16; ++j) mx = fmaxf(mx, acc[j]);
  return m != 0u && mx >= th;
}

// Candidates of one 32 x 32 score tile (docs x this lane's query): pairs that
// pass the filter with a score >= th go to the query's candidate list.
// Called by the whole wave.
__device__ __forceinline__ void tile_candidates(const TopkState& st, const f32x16& acc, uint32_t m,
                                                float th, int64_t q, uint32_t* slot_count,
                                                int64_t doc0, int lane) {
  uint32_t ge = 0u;
#pragma unroll
  for (int j = 15; j >= 0; --j) ge = (ge << 1) | (acc[j] >= th ? 1u : 0u);
  const int h = lane >> 5;
  uint32_t hits = ge & lane_rows(m, h);
  if (__ballot(hits != 0u) == 0) return;
  const uint32_t cnt = __builtin_popcount(hits);
  const uint32_t cnt_pair = __shfl_xor(cnt, 32, 64);  // lanes l, l ^ 32: same query
  // slots of this workgroup's segment, counted in LDS
  uint32_t base = 0u;
  if (lane < 32 && cnt + cnt_pair > 0u) base = atomicAdd(slot_count, cnt + cnt_pair);
  const uint32_t base_pair = __shfl_xor(base, 32, 64);
  uint32_t slot = lane < 32 ? base : base_pair + cnt_pair;
  uint64_t* seg = st.cand + q * st.capacity + kMaxTopk + static_cast<uint64_t>(blockIdx.x) * st.seg;
  while (__ballot(hits != 0u) != 0) {
    if (hits != 0u) {
      const int j = __builtin_ctz(hits);
      hits &= hits - 1u;
      float v = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) v = j == i ? acc[i] : v;
      const int64_t doc = doc0 + 8 * (j >> 2) + 4 * h + (j & 3);
      if (slot < st.seg) seg[slot] = make_key(v, doc);
      else atomicOr(st.overflow, 1u);
      ++slot;
    }
  }
}

// Scores docs [lo, hi) against queries [q_begin, q_begin + q_count)
// (q_count <= ScoreShape<D>::kQueries).  Wave w holds queries
// w * 32 * QT + 32 t + (lane & 31) of tile t as B operands (lanes 32-63
// carry the second half of each 16-wide k step); each workgroup takes one
// contiguous run of steps.  A step's rows and filter words are loaded into
// registers while the step before is scored and stored into the other LDS
// buffer after it, so each step needs one barrier.
template <int D>
__global__ __launch_bounds__(kScoreThreads) void topk_score_kernel(
    const uint16_t* __restrict__ emb, const uint16_t* __restrict__ qv,
    const uint64_t* __restrict__ mask64, int64_t num_columns, int64_t q_begin,
    int64_t q_count, int64_t lo, int64_t hi, int64_t steps_per_group, TopkState st) {
  using SS = ScoreShape<D>;
  constexpr int S = SS::S, QT = SS::QT;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int h = lane >> 5;

  const int64_t first = lo + static_cast<int64_t>(blockIdx.x) * steps_per_group * SS::kDocs;
  const int64_t last = min(hi, first + steps_per_group * SS::kDocs);
  uint32_t* segn = st.segn + q_begin * kMaxSegments + blockIdx.x;  // query stride kMaxSegments
  if (first >= last) {  // whole workgroup; its segments stay empty
    for (int i = tid; i < q_count; i += kScoreThreads) segn[i * kMaxSegments] = 0u;
    return;
  }
  // Entries this workgroup put in each query's segment.
  uint32_t* slot_count = reinterpret_cast<uint32_t*>(lds + 2 * SS::kBuf);
  for (int i = tid; i < SS::kQueries; i += kScoreThreads) slot_count[i] = 0u;

  // This wave's query fragments (zero past q_count) and entry thresholds
  // (fixed for the launch).
  bf16x8 b[QT][S];
  int ql[QT];
  float th[QT];
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    ql[t] = (wave * QT + t) * kQueryTile + (lane & 31);
    const bool valid = ql[t] < q_count;
    const uint16_t* row = qv + (q_begin + (valid ? ql[t] : 0)) * D + h * 8;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      b[t][s] = *reinterpret_cast<const bf16x8*>(row + s * 16);
      if (!valid) b[t][s] = bf16x8{};
    }
    th[t] = st.thr[q_begin + (valid ? ql[t] : 0)];
  }

  u32x4 dpre[SS::kDocLoads];
  uint64_t mpre[SS::kMaskLoads];
  // Step d0's rows and filter words into registers: rows at or past hi read
  // as zero, and so do columns past the last and queries past the chunk.
  // d0 is a multiple of 64; a mask row is only 8-byte aligned.
  auto prefetch = [&](int64_t d0) {
    const int64_t rows = hi - d0 < SS::kDocs ? hi - d0 : SS::kDocs;
    const u32x4* src = reinterpret_cast<const u32x4*>(emb + d0 * D);
#pragma unroll
    for (int i = 0; i < SS::kDocLoads; ++i) {
      const int c = tid + i * kScoreThreads;
      dpre[i] = (c / SS::kPieces < rows) ? __builtin_nontemporal_load(src + c) : u32x4{0, 0, 0, 0};
    }
    const int64_t col0 = d0 >> 6;
#pragma unroll
    for (int i = 0; i < SS::kMaskLoads; ++i) {
      const int w = tid + i * kScoreThreads;
      const int qq = w / SS::kCols, cc = w - qq * SS::kCols;
      const bool ok = qq < q_count && col0 + cc < num_columns;
      mpre[i] = ok ? mask64[(q_begin + qq) * num_columns + col0 + cc] : 0ull;
    }
  };
  // The registers into LDS buffer buf, with the filter bits of docs at or
  // past hi cleared.  A column word holds docs 0-31 in its high half.
  auto stage = [&](int buf, int64_t d0) {
    uint8_t* docs = lds + buf * SS::kBuf;
    uint32_t* masks = reinterpret_cast<uint32_t*>(docs + SS::kDocBuf);
#pragma unroll
    for (int i = 0; i < SS::kDocLoads; ++i) {
      const int c = tid + i * kScoreThreads;
      const int r = c / SS::kPieces, k = c - r * SS::kPieces;
      *reinterpret_cast<u32x4*>(docs + r * SS::kRowBytes + k * 16) = dpre[i];
    }
#pragma unroll
    for (int i = 0; i < SS::kMaskLoads; ++i) {
      const int w = tid + i * kScoreThreads;
      if (w >= SS::kQueries * SS::kCols) continue;
      const int qq = w / SS::kCols, cc = w - qq * SS::kCols;
      const int64_t g0 = d0 + 64 * cc;
      uint32_t* dst = masks + qq * SS::kMaskWords + 2 * cc;
      dst[0] = static_cast<uint32_t>(mpre[i] >> 32) & valid_doc_mask(g0, hi);
      dst[1] = static_cast<uint32_t>(mpre[i]) & valid_doc_mask(g0 + 32, hi);
    }
  };

  prefetch(first);
  stage(0, first);
  if (first + SS::kDocs < last) prefetch(first + SS::kDocs);
  __syncthreads();
  // Scored tiles whose epilogue is still to run (two accumulator sets).
  f32x16 acc[2][QT];
  uint32_t mb[2][QT];
  int64_t docb[2] = {0, 0};
  bool pend[2] = {false, false};
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      acc[x][t] = f32x16{};
      mb[x][t] = 0u;
    }
  int buf = 0;
  for (int64_t d0 = first; d0 < last; d0 += SS::kDocs, buf ^= 1) {
    const uint8_t* docs = lds + buf * SS::kBuf;
    const uint32_t* masks = reinterpret_cast<const uint32_t*>(docs + SS::kDocBuf);
    uint32_t m[QT][SS::kDocTiles];
#pragma unroll
    for (int t = 0; t < QT; ++t)
#pragma unroll
      for (int dt = 0; dt < SS::kDocTiles; ++dt)
        m[t][dt] = masks[ql[t] * SS::kMaskWords + dt];  // zero past q_count
    // A operands: doc row 32 dt + (lane & 31), k half h.  The step's
    // fragments are read from LDS in one stream, kAhead ahead of their MFMAs
    // and across tile boundaries (rows past hi are zero in LDS and carry no
    // filter bit).  The epilogue of a tile is deferred to the next tile,
    // whose MFMAs its gate is interleaved with, so each wave keeps the
    // matrix cores fed by itself.  Tiles alternate between the two
    // accumulator sets; pend[x] says set x holds a tile still to finish.  A
    // step with no filter bit for any of the wave's queries is skipped.
    bool any = false;
#pragma unroll
    for (int t = 0; t < QT; ++t)
#pragma unroll
      for (int dt = 0; dt < SS::kDocTiles; ++dt) any |= m[t][dt] != 0u;
    if (__ballot(any) != 0) {
      constexpr int kFrags = SS::kDocTiles * S;
      constexpr int kAhead = 3;
      const uint8_t* arow = docs + (lane & 31) * SS::kRowBytes + h * 16;
      bf16x8 fr[kAhead + 1];
      auto read = [&](int g) {
        fr[g % (kAhead + 1)] = *reinterpret_cast<const bf16x8*>(
            arow + (g / S) * 32 * SS::kRowBytes + (g % S) * 32);
      };
#pragma unroll
      for (int g = 0; g < kAhead; ++g) read(g);
#pragma unroll
      for (int dt = 0; dt < SS::kDocTiles; ++dt) {
        const int cb = dt & 1, pb = cb ^ 1;
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const int g = dt * S + s;
          if (g + kAhead < kFrags) read(g + kAhead);
#pragma unroll
          for (int t = 0; t < QT; ++t)
            acc[cb][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fr[g % (kAhead + 1)], b[t][s],
                                                                 s == 0 ? f32x16{} : acc[cb][t], 0, 0, 0);
        }
        bool gate[QT];
#pragma unroll
        for (int t = 0; t < QT; ++t) gate[t] = tile_gate(acc[pb][t], mb[pb][t], th[t]) & pend[pb];
        // MFMAs with a fragment read and the pending tile's gate VALU work
        // between them
#pragma unroll
        for (int i = 0; i < S; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
          for (int t = 0; t < QT; ++t) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
          }
        }
#pragma unroll
        for (int t = 0; t < QT; ++t)
          if (__ballot(gate[t]) != 0)
            tile_candidates(st, acc[pb][t], mb[pb][t], th[t], q_begin + ql[t], slot_count + ql[t],
                            docb[pb], lane);
        pend[cb] = true;
        pend[pb] = false;
#pragma unroll
        for (int t = 0; t < QT; ++t) mb[cb][t] = m[t][dt];
        docb[cb] = d0 + dt * 32;
      }
    }
    const int64_t next = d0 + SS::kDocs;
    if (next < last) {
      stage(buf ^ 1, next);
      if (next + SS::kDocs < last) prefetch(next + SS::kDocs);
    }
    __syncthreads();
  }
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    if (pend[x]) {
#pragma unroll
      for (int t = 0; t < QT; ++t)
        if (__ballot(tile_gate(acc[x][t], mb[x][t], th[t])) != 0)
          tile_candidates(st, acc[x][t], mb[x][t], th[t], q_begin + ql[t], slot_count + ql[t],
                          docb[x], lane);
    }
  }
  __syncthreads();
  for (int i = tid; i < q_count; i += kScoreThreads) segn[i * kMaxSegments] = min(slot_count[i], st.seg);
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

// Writes the best m = min(n, k) of the n distinct keys key_at(0 .. n-1) to
// keys[0, m) in no particular order and returns m; *min_key receives the
// smallest of them.  key_at may read keys[] itself (the keys are gathered
// before keys[] is written).  A radix select over the bits in which the keys differ
// (8 bits a pass, one LDS histogram per wave) finds the lower bound L of the
// best m (the m-th key itself, or the start of a digit bucket that holds
// exactly the keys still needed), then the keys >= L are gathered.  Called
// by the whole workgroup; the keys stay in LDS.
template <typename Key>
__device__ uint32_t select_best(Key key_at, uint64_t* keys, uint32_t n, uint32_t k, uint64_t* min_key) {
  constexpr int kWaves = kSelectThreads / 64;
  __shared__ uint32_t hist[kWaves][256];
  __shared__ uint64_t red_and[kWaves], red_or[kWaves];
  __shared__ uint64_t s_prefix, s_min;
  __shared__ uint32_t s_remaining, s_done, s_count;
  __shared__ uint64_t picked[kMaxTopk];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t m = min(n, k);
  uint64_t bound = 0ull;  // keys >= bound are the best m
  if (n > k) {
    uint64_t kand = ~0ull, kor = 0ull;
    for (uint32_t i = tid; i < n; i += kSelectThreads) {
      const uint64_t key = key_at(i);
      kand &= key;
      kor |= key;
    }
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) {
      kand &= __shfl_xor(kand, d, 64);
      kor |= __shfl_xor(kor, d, 64);
    }
    if (lane == 0) {
      red_and[wave] = kand;
      red_or[wave] = kor;
    }
    for (int i = tid; i < kWaves * 256; i += kSelectThreads) (&hist[0][0])[i] = 0u;
    __syncthreads();
    kand = ~0ull;
    kor = 0ull;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      kand &= red_and[w];
      kor |= red_or[w];
    }
    const uint64_t diff = kand ^ kor;  // nonzero: n > k >= 1 distinct keys
    uint64_t prefix = kand & ~(~0ull >> __builtin_clzll(diff));
    uint32_t remaining = k;
    for (int shift = ((63 - __builtin_clzll(diff)) / 8) * 8; shift >= 0; shift -= 8) {
      const uint64_t hi_mask = shift + 8 >= 64 ? 0ull : (~0ull << (shift + 8));
      for (uint32_t i = tid; i < n; i += kSelectThreads) {
        const uint64_t key = key_at(i);
        if ((key & hi_mask) == (prefix & hi_mask)) atomicAdd(&hist[wave][(key >> shift) & 0xFFu], 1u);
      }
      __syncthreads();
      if (wave == 0) {
        // bins from the top digit down: 4 per lane, lane 0 holding 255..252
        uint32_t c[4], sum = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          c[i] = 0;
#pragma unroll
          for (int w = 0; w < kWaves; ++w) c[i] += hist[w][255 - (lane * 4 + i)];
          sum += c[i];
        }
        uint32_t incl = sum;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
          const uint32_t y = __shfl_up(incl, d, 64);
          if (lane >= d) incl += y;
        }
        uint32_t run = incl - sum;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (run < remaining && run + c[i] >= remaining) {
            const int digit = 255 - (lane * 4 + i);
            s_prefix = (prefix & hi_mask) | (static_cast<uint64_t>(digit) << shift);
            s_remaining = remaining - run;
            s_done = run + c[i] == remaining ? 1u : 0u;  // the whole bucket is needed
          }
          run += c[i];
        }
      }
      __syncthreads();
      prefix = s_prefix;
      remaining = s_remaining;
      const bool done = s_done != 0u;
      for (int i = tid; i < kWaves * 256; i += kSelectThreads) (&hist[0][0])[i] = 0u;
      __syncthreads();
      if (done) break;
    }
    bound = prefix;  // the bucket's lowest key, or the m-th key after the last pass
  }
  if (tid == 0) {
    s_count = 0u;
    s_min = ~0ull;
  }
  __syncthreads();
  for (uint32_t i = tid; i < n; i += kSelectThreads) {
    const uint64_t key = key_at(i);
    if (key >= bound) {
      picked[atomicAdd(&s_count, 1u)] = key;
      atomicMin(&s_min, key);
    }
  }
  __syncthreads();
  for (uint32_t i = tid; i < m; i += kSelectThreads) keys[i] = picked[i];
  *min_key = s_min;
  __syncthreads();
  return m;
}

// One workgroup per query: keeps the best `topk` candidates (unordered
// between rounds), sets the entry threshold, and on the last round writes
// the outputs, sorted.  The
// candidates are the kept best (slots [0, counts[q])) followed by the entries
// of the round's nseg segments, gathered in that order.
__global__ __launch_bounds__(kSelectThreads) void topk_select_kernel(
    TopkState st, int64_t topk, int nseg, int final_round, int64_t* __restrict__ out_ids,
    float* __restrict__ out_scores) {
  static_assert(kSelectThreads == kMaxSegments, "one thread per segment");
  __shared__ uint64_t keys[kSelectSlots];
  __shared__ uint32_t start[kMaxSegments + 1];  // virtual index of each segment's first entry
  const int64_t q = blockIdx.x;
  uint64_t* cand = st.cand + q * st.capacity;
  const uint32_t kept = st.counts[q];
  // Exclusive scan of the segment counts, one thread per segment.
  const int g = threadIdx.x;
  const uint32_t mine = g < nseg ? min(st.segn[q * kMaxSegments + g], st.seg) : 0u;
  start[g + 1] = mine;
  if (g == 0) start[0] = 0u;
  __syncthreads();
  for (int off = 1; off < kMaxSegments; off <<= 1) {
    const uint32_t v = g + 1 - off >= 1 ? start[g + 1 - off] : 0u;
    __syncthreads();
    start[g + 1] += v;
    __syncthreads();
  }
  const uint32_t n = kept + start[kMaxSegments];
  // Candidate v of the virtual list: the kept best, then the segments.
  auto at = [&](uint32_t v) -> uint64_t {
    if (v < kept) return cand[v];
    const uint32_t w = v - kept;
    int lo = 0, hi = nseg;  // last segment with start <= w
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (start[mid] <= w) lo = mid;
      else hi = mid;
    }
    return cand[kMaxTopk + static_cast<uint64_t>(lo) * st.seg + (w - start[lo])];
  };
  // the best min(n, topk) to the front of keys[], unordered: candidates
  // gathered into LDS when they fit (several radix passes read them), else
  // read from their segments on each pass
  uint64_t sel_min = 0ull;
  uint32_t best;
  if (n <= static_cast<uint32_t>(kSelectSlots)) {
    for (int i = threadIdx.x; i < static_cast<int>(n); i += kSelectThreads) keys[i] = at(i);
    __syncthreads();
    best = select_best([&](uint32_t i) { return keys[i]; }, keys, n, static_cast<uint32_t>(topk), &sel_min);
  } else {
    best = select_best(at, keys, n, static_cast<uint32_t>(topk), &sel_min);
  }
  if (final_round) {
    int size = 64;
    while (size < static_cast<int>(best)) size <<= 1;
    for (int i = static_cast<int>(best) + threadIdx.x; i < size; i += kSelectThreads) keys[i] = 0ull;
    __syncthreads();
    bitonic_sort_desc(keys, size);
    for (int64_t i = threadIdx.x; i < topk; i += kSelectThreads) {
      const bool have = i < best;
      out_ids[q * topk + i] = have ? static_cast<int64_t>(0xFFFFFFFFu - static_cast<uint32_t>(keys[i])) : -1;
      out_scores[q * topk + i] = have ? from_ordered(static_cast<uint32_t>(keys[i] >> 32)) : -INFINITY;
    }
    return;
  }
  for (uint32_t i = threadIdx.x; i < best; i += kSelectThreads) cand[i] = keys[i];
  if (threadIdx.x == 0) {
    st.counts[q] = best;
    st.thr[q] = best == topk ? from_ordered(static_cast<uint32_t>(sel_min >> 32)) : -INFINITY;
  }
}

void check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) throw Error(ST_ERR_HIP, cat(what, " launch failed: ", hipGetErrorString(e)));
}

// Scores docs [lo, hi) for every query; returns the number of workgroups
// (segments) used.  A workgroup scores at most docs_per_group docs, the bound
// on the entries of one segment that a round without a threshold can make.
template <int D>
int launch_score(const uint16_t* emb, const uint16_t* qv, const uint64_t* mask64,
                 int64_t num_columns, int64_t num_queries, int64_t lo, int64_t hi,
                 TopkState st, bool need_fit, hipStream_t s) {
  using SS = ScoreShape<D>;
  // One contiguous run of steps per workgroup, one workgroup per CU.
  const int64_t steps = (hi - lo + SS::kDocs - 1) / SS::kDocs;
  const int64_t groups = std::min<int64_t>(cu_count(), kMaxSegments);
  const int64_t per_group = (steps + groups - 1) / groups;
  const int grid = static_cast<int>(std::max<int64_t>(1, (steps + per_group - 1) / per_group));
  st.seg = kSegmentSlots / static_cast<uint32_t>(grid);
  if (need_fit && static_cast<int64_t>(st.seg) < per_group * SS::kDocs)
    fail("internal: a segment of ", st.seg, " slots cannot hold ", per_group * SS::kDocs, " docs");
  for (int64_t qb = 0; qb < num_queries; qb += SS::kQueries) {
    const int64_t qn = std::min<int64_t>(SS::kQueries, num_queries - qb);
    hipLaunchKernelGGL(topk_score_kernel<D>, dim3(grid), dim3(kScoreThreads), SS::kLds, s, emb,
                       qv, mask64, num_columns, qb, qn, lo, hi, per_group, st);
    check_launch("topk_score_kernel");
  }
  return grid;
}

using ScoreFn = int (*)(const uint16_t*, const uint16_t*, const uint64_t*, int64_t, int64_t,
                        int64_t, int64_t, TopkState, bool, hipStream_t);

ScoreFn score_fn(int64_t dim) {
  switch (dim) {
    case 64: return launch_score<64>;
    case 128: return launch_score<128>;
    case 256: return launch_score<256>;
    default: fail("embedding dimension ", dim, " is not supported (64, 128 or 256)");
  }
}

// The scoring kernel stages a step of doc rows and filter words in LDS
// (more than the 64 KB default limit).
void set_lds_limits() {
  static std::once_flag once;
  static hipError_t status = hipSuccess;
  std::call_once(once, [] {
    const std::pair<const void*, int> kernels[] = {
        {reinterpret_cast<const void*>(topk_score_kernel<64>), ScoreShape<64>::kLds},
        {reinterpret_cast<const void*>(topk_score_kernel<128>), ScoreShape<128>::kLds},
        {reinterpret_cast<const void*>(topk_score_kernel<256>), ScoreShape<256>::kLds}};
    for (const auto& k : kernels) {
      const hipError_t e = hipFuncSetAttribute(k.first, hipFuncAttributeMaxDynamicSharedMemorySize, k.second);
      if (e != hipSuccess && status == hipSuccess) status = e;
    }
  });
  if (status != hipSuccess)
    throw Error(ST_ERR_HIP, cat("hipFuncSetAttribute failed: ", hipGetErrorString(status)));
}

// Doc ranges of the rounds: a first round of 8192 docs, then each round
// eight times everything before it (rounds aligned to bundles), or, in the
// safe schedule, rounds no larger than the candidate segments can always hold.
std::vector<int64_t> round_bounds(int64_t num_docs, bool safe) {
  std::vector<int64_t> b{0};
  int64_t pos = 0;
  // A safe round gives each workgroup at most one segment's worth of docs.
  static_assert(kSegmentSlots % kRoundAlign == 0, "safe rounds stay aligned");
  const int64_t safe_step = kSegmentSlots;
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
  return num_queries * (4 + 4 + 8 * static_cast<int64_t>(st::kCandidateCapacity) +
                       4 * static_cast<int64_t>(st::kMaxSegments)) +
         256;
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
    state.segn = reinterpret_cast<uint32_t*>(state.cand + num_queries * static_cast<int64_t>(kCandidateCapacity));
    state.seg = 0;
    const uint16_t* emb = static_cast<const uint16_t*>(doc_embeddings);
    const uint16_t* qv = static_cast<const uint16_t*>(query_embeddings);
    const uint64_t* m64 = reinterpret_cast<const uint64_t*>(packed);
    const unsigned qgrid = static_cast<unsigned>(num_queries);

    for (int attempt = 0; attempt < 2; ++attempt) {
      const bool safe = attempt == 1;
      hipLaunchKernelGGL(topk_reset_kernel, dim3(static_cast<unsigned>((num_queries + 255) / 256)),
                         dim3(256), 0, s, state, num_queries);
      check_launch("topk_reset_kernel");
      const std::vector<int64_t> bounds = round_bounds(num_docs, safe);
      for (size_t r = 0; r + 1 < bounds.size(); ++r) {
        const int nseg = score(emb, qv, m64, num_columns, num_queries, bounds[r], bounds[r + 1],
                               state, safe, s);
        TopkState sel = state;
        sel.seg = kSegmentSlots / static_cast<uint32_t>(nseg);
        const bool last = r + 2 == bounds.size();
        hipLaunchKernelGGL(topk_select_kernel, dim3(qgrid), dim3(kSelectThreads), 0, s, sel,
                           topk, nseg, last ? 1 : 0, out_ids, out_scores);
        check_launch("topk_select_kernel");
      }
      if (bounds.size() == 1) {  // no docs: every output is padding
        hipLaunchKernelGGL(topk_select_kernel, dim3(qgrid), dim3(kSelectThreads), 0, s, state,
                           topk, 0, 1, out_ids, out_scores);
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
