// take_top_k_and_gather_from_main_and_fresh on gfx950: the top-k of the
// merged score row (fresh columns first, then main) and the gather of the
// caller's data rows through the fresh / main index tables.
//
// Replaces take_top_k_and_gather_from_main_and_fresh_cpu and
// gather_data_from_main_and_fresh_index_cpu_impl
// (fresh_index_post_processing.cpp:44-163, :231-270 of the reference):
//   merged[r] = cat(fresh_scores[r], main_scores[r]); k' = min(k, Nf + Nm);
//   top k' of merged[r], largest first (at::topk, sorted);
//   is_from_fresh = top index < Nf;
//   gathered[key][r * k' + j] = fresh_data[fresh_indices[r, t]]   (t <  Nf)
//                             = main_data[main_indices[r, t - Nf]] (t >= Nf)
//   with a source row outside the data's rows read as row 0.
// Order among equal scores: at::topk leaves it open; this build returns the
// lower merged index first.  NaN ranks above every number (at::topk's CPU
// comparator); -0.0 and +0.0 are equal.
//
// Selection, rows of at most 16,384 entries with k' <= 4,096: one workgroup
// per row holds the row in registers, finds the k'-th best key by a radix
// select and sorts the k' best in LDS (fresh_select_kernel).  Other rows:
// one workgroup per row keeps the row's best P = pow2 >= k'
// entries (key, index) sorted, best first.  The row is read 1024 entries at
// a time; entries better than the running k'-th best are compacted into a
// candidate buffer (wave ballot + per-wave counts), and a full buffer is
// sorted (bitonic) and merged into the kept list (bitonic merge of the kept
// list with the reversed candidates).  Most of a long row never reaches a
// sort.  The kept list lives in LDS for k' <= kFreshLdsMaxK and in the
// caller's workspace above that; the candidate buffer is always in LDS.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "../../include/silvertorch_hip.h"
#include "st_common.hpp"
#include "st_errors.hpp"

namespace st {
namespace {

constexpr int kFreshThreads = 1024;
constexpr int kFreshWaves = kFreshThreads / 64;
constexpr int kFreshCand = 4096;      // candidate buffer entries (LDS)
constexpr int kFreshLdsMaxK = 8192;   // kept list in LDS up to this many
constexpr uint32_t kNoIndex = 0xFFFFFFFFu;

// Order-preserving 64-bit keys: a larger key is a larger score.
__device__ __forceinline__ uint64_t f32_key(uint32_t u) {
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0xFFFFFFFFull;  // NaN: above all
  if (u == 0x80000000u) u = 0u;                                 // -0.0 == +0.0
  return (u & 0x80000000u) ? static_cast<uint64_t>(~u) : static_cast<uint64_t>(u | 0x80000000u);
}
__device__ __forceinline__ uint64_t f64_key(uint64_t u) {
  if ((u & 0x7FFFFFFFFFFFFFFFull) > 0x7FF0000000000000ull) return ~0ull;
  if (u == 0x8000000000000000ull) u = 0ull;
  return (u >> 63) ? ~u : (u | 0x8000000000000000ull);
}

template <int kType>
__device__ __forceinline__ uint64_t score_key(const void* base, int64_t i) {
  if constexpr (kType == ST_SCORE_F32) {
    return f32_key(static_cast<const uint32_t*>(base)[i]);
  } else if constexpr (kType == ST_SCORE_F16) {
    const _Float16 h = static_cast<const _Float16*>(base)[i];
    return f32_key(__builtin_bit_cast(uint32_t, static_cast<float>(h)));
  } else if constexpr (kType == ST_SCORE_BF16) {
    return f32_key(static_cast<uint32_t>(static_cast<const uint16_t*>(base)[i]) << 16);
  } else if constexpr (kType == ST_SCORE_F64) {
    return f64_key(static_cast<const uint64_t*>(base)[i]);
  } else if constexpr (kType == ST_SCORE_I64) {
    return static_cast<uint64_t>(static_cast<const int64_t*>(base)[i]) ^ 0x8000000000000000ull;
  } else if constexpr (kType == ST_SCORE_I32) {
    return static_cast<uint64_t>(static_cast<int64_t>(static_cast<const int32_t*>(base)[i])) ^
           0x8000000000000000ull;
  } else if constexpr (kType == ST_SCORE_I16) {
    return static_cast<uint64_t>(static_cast<int64_t>(static_cast<const int16_t*>(base)[i])) ^
           0x8000000000000000ull;
  } else if constexpr (kType == ST_SCORE_I8) {
    return static_cast<uint64_t>(static_cast<int64_t>(static_cast<const int8_t*>(base)[i])) ^
           0x8000000000000000ull;
  } else {
    static_assert(kType == ST_SCORE_U8, "score type");
    return static_cast<uint64_t>(static_cast<const uint8_t*>(base)[i]);
  }
}

// score_key of a 4-byte score from its bits.
template <int kType>
__device__ __forceinline__ uint64_t key_of_bits4(uint32_t u) {
  if constexpr (kType == ST_SCORE_F32) {
    return f32_key(u);
  } else {
    static_assert(kType == ST_SCORE_I32, "4-byte score type");
    return static_cast<uint64_t>(static_cast<int64_t>(static_cast<int32_t>(u))) ^ 0x8000000000000000ull;
  }
}

constexpr int score_bytes(int t) {
  return t == ST_SCORE_F64 || t == ST_SCORE_I64 ? 8
         : t == ST_SCORE_F32 || t == ST_SCORE_I32 ? 4
         : t == ST_SCORE_F16 || t == ST_SCORE_BF16 || t == ST_SCORE_I16 ? 2
                                                                       : 1;
}

// (key, merged index) pairs; `a` ranks before `b`.  The empty entry (key 0,
// index kNoIndex) ranks after every real entry (a real key-0 entry wins on
// its index).
__device__ __forceinline__ bool before(uint64_t ka, uint32_t ia, uint64_t kb, uint32_t ib) {
  return ka > kb || (ka == kb && ia < ib);
}

struct FreshTopkArgs {
  const void* fresh_scores;
  const void* main_scores;
  int64_t rows, num_fresh, num_main, k;
  int64_t p;            // kept list length: pow2 >= k
  uint64_t* ws_keys;    // rows * p (kept list outside LDS)
  uint32_t* ws_index;   // rows * p
  void* top_scores;     // rows * k, the score type
  int64_t* top_index;   // rows * k
  uint8_t* from_fresh;  // rows * k
};

// Sorts keys[0, n) / idx[0, n) best first (n a power of two, >= 2).
__device__ void bitonic_sort(uint64_t* keys, uint32_t* idx, int n) {
  const int tid = threadIdx.x;
  for (int size = 2; size <= n; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const int ls = __builtin_ctz(stride);
      for (int p = tid; p < n / 2; p += kFreshThreads) {
        const int i = ((p >> ls) << (ls + 1)) | (p & (stride - 1));
        const int l = i + stride;
        const bool best_first = (i & size) == 0;
        const uint64_t ki = keys[i], kl = keys[l];
        const uint32_t ii = idx[i], il = idx[l];
        if (before(kl, il, ki, ii) == best_first) {
          keys[i] = kl;
          keys[l] = ki;
          idx[i] = il;
          idx[l] = ii;
        }
      }
      __syncthreads();
    }
  }
}

// Merges the sorted candidates c[0, n) (n a power of two, padded with empty
// entries) into the sorted kept list r[0, P): pairwise best of r[i] and
// c[P - 1 - i] is bitonic and holds the best P of both; a bitonic merge
// sorts it.
template <typename KeyPtr, typename IdxPtr>
__device__ void merge_into(KeyPtr rk, IdxPtr ri, int64_t P, const uint64_t* ck,
                           const uint32_t* ci, int n) {
  const int tid = threadIdx.x;
  for (int64_t i = tid; i < P; i += kFreshThreads) {
    const int64_t j = P - 1 - i;
    if (j < n) {
      const uint64_t kc = ck[j];
      const uint32_t ic = ci[j];
      if (before(kc, ic, rk[i], ri[i])) {
        rk[i] = kc;
        ri[i] = ic;
      }
    }
  }
  __syncthreads();
  for (int64_t stride = P >> 1; stride > 0; stride >>= 1) {
    const int ls = __builtin_ctzll(static_cast<uint64_t>(stride));
    for (int64_t p = tid; p < P / 2; p += kFreshThreads) {
      const int64_t i = ((p >> ls) << (ls + 1)) | (p & (stride - 1));
      const int64_t l = i + stride;
      const uint64_t ki = rk[i], kl = rk[l];
      const uint32_t ii = ri[i], il = ri[l];
      if (before(kl, il, ki, ii)) {
        rk[i] = kl;
        rk[l] = ki;
        ri[i] = il;
        ri[l] = ii;
      }
    }
    __syncthreads();
  }
}

template <int kType, bool kLds>
__global__ __launch_bounds__(kFreshThreads) void fresh_topk_kernel(FreshTopkArgs a) {
  __shared__ uint64_t cand_key[kFreshCand];
  __shared__ uint32_t cand_idx[kFreshCand];
  __shared__ uint64_t lds_key[kLds ? kFreshLdsMaxK : 1];
  __shared__ uint32_t lds_idx[kLds ? kFreshLdsMaxK : 1];
  __shared__ uint32_t wave_count[kFreshWaves];
  __shared__ uint64_t thr_key;
  __shared__ uint32_t thr_idx;

  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t P = a.p;
  const int64_t N = a.num_fresh + a.num_main;
  uint64_t* rk;
  uint32_t* ri;
  if constexpr (kLds) {
    rk = lds_key;
    ri = lds_idx;
  } else {
    rk = a.ws_keys + row * P;
    ri = a.ws_index + row * P;
  }
  for (int64_t i = tid; i < P; i += kFreshThreads) {
    rk[i] = 0ull;
    ri[i] = kNoIndex;
  }
  if (tid == 0) {
    thr_key = 0ull;
    thr_idx = kNoIndex;
  }
  __syncthreads();

  const void* fs = static_cast<const char*>(a.fresh_scores) + row * a.num_fresh * score_bytes(kType);
  const void* ms = static_cast<const char*>(a.main_scores) + row * a.num_main * score_bytes(kType);
  auto flush = [&](int fill) {
    int n = 2;
    while (n < fill) n <<= 1;
    for (int i = fill + tid; i < n; i += kFreshThreads) {
      cand_key[i] = 0ull;
      cand_idx[i] = kNoIndex;
    }
    __syncthreads();
    bitonic_sort(cand_key, cand_idx, n);
    merge_into(rk, ri, P, cand_key, cand_idx, n);
    if (tid == 0) {
      thr_key = rk[a.k - 1];
      thr_idx = ri[a.k - 1];
    }
    __syncthreads();
  };

  int fill = 0;  // uniform
  for (int64_t base = 0; base < N; base += kFreshThreads) {
    const int64_t m = base + tid;
    uint64_t key = 0ull;
    uint32_t id = kNoIndex;
    if (m < N) {
      key = m < a.num_fresh ? score_key<kType>(fs, m) : score_key<kType>(ms, m - a.num_fresh);
      id = static_cast<uint32_t>(m);
    }
    for (int attempt = 0; attempt < 2; ++attempt) {
      const bool pass = m < N && before(key, id, thr_key, thr_idx);
      const uint64_t bal = __ballot(pass);
      if (lane == 0) wave_count[wave] = static_cast<uint32_t>(__popcll(bal));
      __syncthreads();
      uint32_t before_me = 0, total = 0;
      for (int w = 0; w < kFreshWaves; ++w) {
        const uint32_t c = wave_count[w];
        before_me += w < wave ? c : 0u;
        total += c;
      }
      __syncthreads();  // wave_count is rewritten by the next pass
      if (fill + static_cast<int>(total) <= kFreshCand) {
        if (pass) {
          const uint32_t at = static_cast<uint32_t>(fill) + before_me +
                              static_cast<uint32_t>(__popcll(bal & ((1ull << lane) - 1ull)));
          cand_key[at] = key;
          cand_idx[at] = id;
        }
        fill += static_cast<int>(total);
        __syncthreads();
        break;
      }
      // the buffer is full: merge it, then filter this block again against
      // the raised threshold (the second attempt always fits: the buffer is
      // empty and a block is kFreshThreads <= kFreshCand entries)
      flush(fill);
      fill = 0;
    }
  }
  if (fill > 0) flush(fill);

  const int64_t k = a.k;
  for (int64_t j = tid; j < k; j += kFreshThreads) {
    const uint32_t m = ri[j];
    const int64_t o = row * k + j;
    a.top_index[o] = static_cast<int64_t>(m);
    a.from_fresh[o] = static_cast<int64_t>(m) < a.num_fresh ? 1 : 0;
    constexpr int B = score_bytes(kType);
    const char* src = m < a.num_fresh ? static_cast<const char*>(fs) + static_cast<int64_t>(m) * B
                                      : static_cast<const char*>(ms) + (static_cast<int64_t>(m) - a.num_fresh) * B;
    char* dst = static_cast<char*>(a.top_scores) + o * B;
    if constexpr (B == 8) {
      *reinterpret_cast<uint64_t*>(dst) = *reinterpret_cast<const uint64_t*>(src);
    } else if constexpr (B == 4) {
      *reinterpret_cast<uint32_t*>(dst) = *reinterpret_cast<const uint32_t*>(src);
    } else if constexpr (B == 2) {
      *reinterpret_cast<uint16_t*>(dst) = *reinterpret_cast<const uint16_t*>(src);
    } else {
      *dst = *src;
    }
  }
}

// Rows of at most kSelectThreads * kSelectMaxPer entries with k <= kSelectMaxK
// take a selection instead of the streaming merge: each thread holds kPer
// consecutive entries of the row in registers; a radix select over the
// bits in which the row's keys differ (8 bits a pass, histogram in LDS)
// finds the k-th best key T and how many keys exceed it; the entries above
// T and the lowest-indexed entries equal to T (as many as k needs) are
// compacted in index order into LDS and sorted best first: up to 1,024 of
// them as 64-entry runs sorted within each wave (bitonic, by shuffles) and
// merged pairwise through LDS; more by a bitonic network in LDS.
constexpr int kSelectThreads = 1024;
constexpr int kSelectWaves = kSelectThreads / 64;
constexpr int kSelectMaxPer = 16;  // keys per thread (64-bit, in registers)
constexpr int kSelectMaxK = 4096;
static_assert(kSelectMaxK >= 2 * kSelectThreads && (kSelectThreads & (kSelectThreads - 1)) == 0,
              "the merge rounds' two run buffers fit s_key / s_idx");

// Exclusive prefix sum over the workgroup of one value per thread (in
// thread order); *total receives the sum.  Uses scratch[kSelectWaves + 1].
__device__ __forceinline__ uint32_t select_scan(uint32_t v, uint32_t* scratch, uint32_t* total) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t incl = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t y = __shfl_up(incl, d, 64);
    if (lane >= d) incl += y;
  }
  if (lane == 63) scratch[wave] = incl;
  __syncthreads();
  uint32_t before = 0, sum = 0;
#pragma unroll
  for (int w = 0; w < kSelectWaves; ++w) {
    const uint32_t c = scratch[w];
    before += w < wave ? c : 0u;
    sum += c;
  }
  __syncthreads();  // scratch is reused by the next scan
  *total = sum;
  return before + incl - v;
}

template <int kType, int kPer>
__global__ __launch_bounds__(kSelectThreads) void fresh_select_kernel(FreshTopkArgs a) {
  __shared__ __align__(16) uint32_t hist[kSelectWaves][256];  // one histogram per wave
  __shared__ uint32_t scan_scratch[kSelectWaves + 1];
  __shared__ uint64_t red_and[kSelectWaves], red_or[kSelectWaves];
  __shared__ uint64_t s_key[kSelectMaxK];
  __shared__ uint32_t s_idx[kSelectMaxK];
  __shared__ uint64_t s_prefix;
  __shared__ uint32_t s_remaining, s_above;

  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t N = a.num_fresh + a.num_main;
  const int64_t k = a.k;
  const void* fs = static_cast<const char*>(a.fresh_scores) + row * a.num_fresh * score_bytes(kType);
  const void* ms = static_cast<const char*>(a.main_scores) + row * a.num_main * score_bytes(kType);

  // entries m = tid * kPer + j of the merged row
  uint64_t key[kPer];
  const int64_t m0 = static_cast<int64_t>(tid) * kPer;
  bool vec = false;
  if constexpr (score_bytes(kType) == 4 && kPer % 4 == 0) {
    // 16-byte loads of 4 entries each (a thread's entries are consecutive,
    // so 4-byte loads would put 64 lanes' accesses 4 * kPer bytes apart):
    // each piece lies in one part when both parts' lengths are multiples of
    // 4, and N is then one too
    vec = a.num_fresh % 4 == 0 && a.num_main % 4 == 0 &&
          (reinterpret_cast<uintptr_t>(fs) & 15u) == 0 && (reinterpret_cast<uintptr_t>(ms) & 15u) == 0;
    if (vec) {
#pragma unroll
      for (int u = 0; u < kPer / 4; ++u) {
        const int64_t m = m0 + 4 * u;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (m < N)
          v = *reinterpret_cast<const uint4*>(m < a.num_fresh
                                                  ? static_cast<const uint32_t*>(fs) + m
                                                  : static_cast<const uint32_t*>(ms) + (m - a.num_fresh));
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) key[4 * u + e] = m < N ? key_of_bits4<kType>(w[e]) : 0ull;
      }
    }
  }
  if (!vec) {
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int64_t m = m0 + j;
      key[j] = m >= N ? 0ull : (m < a.num_fresh ? score_key<kType>(fs, m) : score_key<kType>(ms, m - a.num_fresh));
    }
  }
  // bits in which the row's keys differ
  uint64_t kand = ~0ull, kor = 0ull;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    if (m0 + j < N) {
      kand &= key[j];
      kor |= key[j];
    }
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
  for (int i = tid; i < kSelectWaves * 256; i += kSelectThreads) (&hist[0][0])[i] = 0u;
  __syncthreads();
  kand = ~0ull;
  kor = 0ull;
#pragma unroll
  for (int w = 0; w < kSelectWaves; ++w) {
    kand &= red_and[w];
    kor |= red_or[w];
  }
  const uint64_t diff = kand ^ kor;
  // Radix select: prefix holds the bits of T above `shift` (bits above the
  // highest differing bit are common to every key); `remaining` is how many
  // entries of the current prefix k still needs.
  uint64_t prefix = kand & ~((diff == 0ull) ? 0ull : ((~0ull) >> __builtin_clzll(diff)));
  uint32_t remaining = static_cast<uint32_t>(k), above = 0u;
  int shift = diff == 0ull ? -1 : ((63 - __builtin_clzll(diff)) / 8) * 8;
  for (; shift >= 0; shift -= 8) {
    const uint64_t hi_mask = shift + 8 >= 64 ? 0ull : (~0ull << (shift + 8));
    // each wave counts the digits of its keys under the current prefix in
    // its own histogram (score rows are often narrow in their top digits:
    // one histogram for the workgroup would serialize on a few bins)
#pragma unroll
    for (int j = 0; j < kPer; ++j)
      if (m0 + j < N && (key[j] & hi_mask) == (prefix & hi_mask))
        atomicAdd(&hist[wave][(key[j] >> shift) & 0xFFu], 1u);
    __syncthreads();
    if (wave == 0) {
      // bins from the top digit down: 4 per lane, lane 0 holding 255..252
      uint32_t c[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int w = 0; w < kSelectWaves; ++w) {  // bins 252 - 4 lane .. 255 - 4 lane at once
        const uint4 h = *reinterpret_cast<const uint4*>(&hist[w][252 - lane * 4]);
        c[0] += h.w;
        c[1] += h.z;
        c[2] += h.y;
        c[3] += h.x;
      }
      const uint32_t sum = c[0] + c[1] + c[2] + c[3];
      uint32_t incl = sum;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const uint32_t y = __shfl_up(incl, d, 64);
        if (lane >= d) incl += y;
      }
      // the digit where the count from the top reaches `remaining`
      uint32_t run = incl - sum;
      int digit = -1;
      uint32_t run_before = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (digit < 0 && run + c[i] >= remaining && run < remaining) {
          digit = 255 - (lane * 4 + i);
          run_before = run;
        }
        run += c[i];
      }
      if (digit >= 0) {
        s_prefix = (prefix & hi_mask) | (static_cast<uint64_t>(digit) << shift);
        s_remaining = remaining - run_before;
        s_above = above + run_before;
      }
    }
    __syncthreads();
    prefix = s_prefix;
    remaining = s_remaining;
    above = s_above;
    for (int i = tid; i < kSelectWaves * 256; i += kSelectThreads) (&hist[0][0])[i] = 0u;
    __syncthreads();
  }
  const uint64_t T = prefix;  // the k-th best key; `above` keys exceed it
  const uint32_t ties_taken = static_cast<uint32_t>(k) - above;
  // in index order: every key above T, and the first ties_taken keys == T
  uint32_t n_tie = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) n_tie += (m0 + j < N && key[j] == T) ? 1u : 0u;
  uint32_t tie_total;
  uint32_t tie_before = select_scan(n_tie, scan_scratch, &tie_total);
  uint32_t mine = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    if (m0 + j >= N) continue;
    if (key[j] > T) {
      ++mine;
    } else if (key[j] == T) {
      if (tie_before < ties_taken) ++mine;
      ++tie_before;
    }
  }
  uint32_t total;
  uint32_t at = select_scan(mine, scan_scratch, &total);
  tie_before -= n_tie;
  int n = 2;
  while (n < static_cast<int>(k)) n <<= 1;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    if (m0 + j >= N) continue;
    bool take = key[j] > T;
    if (key[j] == T) {
      take = tie_before < ties_taken;
      ++tie_before;
    }
    if (take) {
      s_key[at] = key[j];
      s_idx[at] = static_cast<uint32_t>(m0 + j);
      ++at;
    }
  }
  for (int i = static_cast<int>(k) + tid; i < n; i += kSelectThreads) {
    s_key[i] = 0ull;
    s_idx[i] = kNoIndex;
  }
  __syncthreads();
  constexpr int B = score_bytes(kType);
  auto emit = [&](int64_t j, uint32_t m) {
    if (static_cast<int64_t>(m) >= N) m = 0;  // never: exactly k entries were taken
    const int64_t o = row * k + j;
    a.top_index[o] = static_cast<int64_t>(m);
    a.from_fresh[o] = static_cast<int64_t>(m) < a.num_fresh ? 1 : 0;
    const char* src = m < a.num_fresh ? static_cast<const char*>(fs) + static_cast<int64_t>(m) * B
                                      : static_cast<const char*>(ms) + (static_cast<int64_t>(m) - a.num_fresh) * B;
    char* dst = static_cast<char*>(a.top_scores) + o * B;
    if constexpr (B == 8) {
      *reinterpret_cast<uint64_t*>(dst) = *reinterpret_cast<const uint64_t*>(src);
    } else if constexpr (B == 4) {
      *reinterpret_cast<uint32_t*>(dst) = *reinterpret_cast<const uint32_t*>(src);
    } else if constexpr (B == 2) {
      *reinterpret_cast<uint16_t*>(dst) = *reinterpret_cast<const uint16_t*>(src);
    } else {
      *dst = *src;
    }
  };
  if (n <= kSelectThreads) {
    // Entry t in thread t's registers.  Each wave sorts its 64 entries best
    // first (bitonic, lanes exchange by shuffles); then the sorted runs are
    // merged pairwise through LDS: an entry's place in the merged run is its
    // place in its own run plus how many entries of the other run go before
    // it (a binary search; entries of the second run also count the equal
    // ones, so that equal entries -- the empty padding -- keep distinct
    // places).
    uint64_t mk = 0ull;
    uint32_t mi = kNoIndex;
    if (tid < n) {
      mk = s_key[tid];
      mi = s_idx[tid];
    }
    const int wn = n < 64 ? n : 64;
    for (int size = 2; size <= wn; size <<= 1) {
      const bool best_first = size == wn || (tid & size) == 0;
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        const uint64_t pk = __shfl_xor(mk, stride, 64);
        const uint32_t pi = __shfl_xor(mi, stride, 64);
        // the lower thread of a pair keeps the entry that goes first in its
        // block's direction
        const bool first = ((tid & stride) == 0) == best_first;
        const bool take = first ? before(pk, pi, mk, mi) : before(mk, mi, pk, pi);
        if (tid < n && take) {
          mk = pk;
          mi = pi;
        }
      }
    }
    if (n > 64) {
      // runs in s_key / s_idx [cur, cur + n), merged into the other half
      int cur = 0;
      __syncthreads();  // every thread has read its entry
      if (tid < n) {
        s_key[tid] = mk;
        s_idx[tid] = mi;
      }
      __syncthreads();
      for (int len = 64; len < n; len <<= 1) {
        if (tid < n) {
          const int pos = tid & (len - 1);
          const int other = (tid & ~(len - 1)) ^ len;  // first entry of the other run
          const bool second = (tid & len) != 0;
          const uint64_t* ok = s_key + cur + other;
          const uint32_t* oi = s_idx + cur + other;
          int lo = 0, hi = len;  // entries of the other run that go first: [0, lo)
          while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            const bool goes_first = second ? !before(mk, mi, ok[mid], oi[mid])
                                           : before(ok[mid], oi[mid], mk, mi);
            if (goes_first) lo = mid + 1;
            else hi = mid;
          }
          const int at = (cur ^ kSelectThreads) + (tid & ~(2 * len - 1)) + pos + lo;
          s_key[at] = mk;
          s_idx[at] = mi;
        }
        __syncthreads();
        cur ^= kSelectThreads;
        if (tid < n) {
          mk = s_key[cur + tid];
          mi = s_idx[cur + tid];
        }
      }
    }
    if (tid < k) emit(tid, mi);
    return;
  }
  // bitonic sort of s_key / s_idx [0, n), best first
  for (int size = 2; size <= n; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const int ls = __builtin_ctz(stride);
      for (int p = tid; p < n / 2; p += kSelectThreads) {
        const int i = ((p >> ls) << (ls + 1)) | (p & (stride - 1));
        const int l = i + stride;
        const bool best_first = (i & size) == 0;
        const uint64_t ki = s_key[i], kl = s_key[l];
        const uint32_t ii = s_idx[i], il = s_idx[l];
        if (before(kl, il, ki, ii) == best_first) {
          s_key[i] = kl;
          s_key[l] = ki;
          s_idx[i] = il;
          s_idx[l] = ii;
        }
      }
      __syncthreads();
    }
  }
  for (int64_t j = tid; j < k; j += kSelectThreads) emit(j, s_idx[j]);
}

template <int kType>
void launch_topk_typed(const FreshTopkArgs& a, hipStream_t s) {
  const int64_t N = a.num_fresh + a.num_main;
  if (a.k <= kSelectMaxK && N <= static_cast<int64_t>(kSelectThreads) * kSelectMaxPer) {
    const dim3 g(static_cast<unsigned>(a.rows)), b(kSelectThreads);
    if (N <= kSelectThreads * 4)
      hipLaunchKernelGGL((fresh_select_kernel<kType, 4>), g, b, 0, s, a);
    else if (N <= kSelectThreads * 8)
      hipLaunchKernelGGL((fresh_select_kernel<kType, 8>), g, b, 0, s, a);
    else
      hipLaunchKernelGGL((fresh_select_kernel<kType, 16>), g, b, 0, s, a);
    return;
  }
  if (a.p <= kFreshLdsMaxK)
    hipLaunchKernelGGL((fresh_topk_kernel<kType, true>), dim3(a.rows), dim3(kFreshThreads), 0, s, a);
  else
    hipLaunchKernelGGL((fresh_topk_kernel<kType, false>), dim3(a.rows), dim3(kFreshThreads), 0, s, a);
}

int64_t kept_length(int64_t k) {
  int64_t p = 2;
  while (p < k) p <<= 1;
  return p;
}

// Gather of one data tensor: unit e of the output is unit e % D of the
// source row chosen for output row e / D (D units per row).  A thread moves
// kGatherPer units a grid apart and issues every load (the top-k entry, the
// index entry, the data unit) for all of them before its stores, so that
// kGatherPer dependent load chains are in flight per thread (2 or 8 per
// thread, or non-temporal row loads, measured slower).  Index arithmetic is
// 32-bit when the unit count fits (Narrow).
constexpr int kGatherPer = 4;
constexpr int kGatherThreads = 256;

template <typename Idx, typename Elem, bool Narrow>
__global__ __launch_bounds__(kGatherThreads) void fresh_gather_kernel(
    const int64_t* __restrict__ top_index, int64_t k, int64_t total,
    const Idx* __restrict__ fresh_idx, int64_t fresh_stride, const Idx* __restrict__ main_idx,
    int64_t main_stride, int64_t num_fresh, const Elem* __restrict__ fresh_data,
    int64_t fresh_rows, const Elem* __restrict__ main_data, int64_t main_rows, int64_t dim,
    Elem* __restrict__ out) {
  using U = typename std::conditional<Narrow, uint32_t, int64_t>::type;
  const U nt = static_cast<U>(gridDim.x) * kGatherThreads;
  const U e0 = static_cast<U>(blockIdx.x) * kGatherThreads + threadIdx.x;
  const U tot = static_cast<U>(total), D = static_cast<U>(dim), K = static_cast<U>(k);
  int64_t t[kGatherPer];
  U item[kGatherPer];
#pragma unroll
  for (int j = 0; j < kGatherPer; ++j) {
    const U e = e0 + static_cast<U>(j) * nt;
    item[j] = e / D;
    t[j] = e < tot ? top_index[item[j]] : 0;
  }
  int64_t src[kGatherPer];
#pragma unroll
  for (int j = 0; j < kGatherPer; ++j) {
    const U e = e0 + static_cast<U>(j) * nt;
    const int64_t row = static_cast<int64_t>(item[j] / K);
    const bool fresh = t[j] < num_fresh;
    src[j] = e >= tot ? 0
             : fresh  ? static_cast<int64_t>(fresh_idx[row * fresh_stride + t[j]])
                      : static_cast<int64_t>(main_idx[row * main_stride + (t[j] - num_fresh)]);
  }
  Elem v[kGatherPer];
#pragma unroll
  for (int j = 0; j < kGatherPer; ++j) {
    const U e = e0 + static_cast<U>(j) * nt;
    const U d = e - item[j] * D;
    const bool fresh = t[j] < num_fresh;
    const int64_t rows = fresh ? fresh_rows : main_rows;
    int64_t r = src[j];
    if (r < 0 || r >= rows) r = 0;  // padded offsets read row 0
    const Elem* data = fresh ? fresh_data : main_data;
    v[j] = e < tot && rows > 0
               ? data[r * static_cast<int64_t>(D) + static_cast<int64_t>(d)]
               : Elem{};
  }
#pragma unroll
  for (int j = 0; j < kGatherPer; ++j) {
    const U e = e0 + static_cast<U>(j) * nt;
    if (e < tot) out[e] = v[j];
  }
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// The rows are moved in the widest unit (16, 8, 4, 2 or 1 bytes) that
// divides a row and the alignment of the three data pointers.
template <typename Idx>
void launch_gather_idx(const int64_t* top_index, int64_t rows, int64_t k, const void* fi,
                       int64_t fs, const void* mi, int64_t ms, int64_t num_fresh,
                       const void* fd, int64_t frows, const void* md, int64_t mrows,
                       int64_t dim, int elem_bytes, void* out, hipStream_t s) {
  ST_CHECK(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8,
           "unsupported element size ", elem_bytes);
  const int64_t row_bytes = dim * elem_bytes;
  const uintptr_t align = reinterpret_cast<uintptr_t>(fd) | reinterpret_cast<uintptr_t>(md) |
                          reinterpret_cast<uintptr_t>(out);
  int unit = 16;
  while (unit > 1 && (row_bytes % unit != 0 || align % unit != 0)) unit >>= 1;
  const int64_t units = row_bytes / unit;
  const int64_t total = rows * k * units;
  const int64_t per_block = static_cast<int64_t>(kGatherThreads) * kGatherPer;
  ST_CHECK((total + per_block - 1) / per_block <= 0x7FFFFFFF, "gather of ", total, " units is too large");
  const dim3 grid(static_cast<unsigned>((total + per_block - 1) / per_block));
  // 32-bit arithmetic when every unit number a thread forms (below the
  // grid's threads x kGatherPer) fits
  const bool narrow = static_cast<int64_t>(grid.x) * per_block <= static_cast<int64_t>(UINT32_MAX);
  auto go = [&](auto tag) {
    using E = decltype(tag);
    if (narrow)
      hipLaunchKernelGGL((fresh_gather_kernel<Idx, E, true>), grid, dim3(kGatherThreads), 0, s,
                         top_index, k, total, static_cast<const Idx*>(fi), fs,
                         static_cast<const Idx*>(mi), ms, num_fresh, static_cast<const E*>(fd),
                         frows, static_cast<const E*>(md), mrows, units, static_cast<E*>(out));
    else
      hipLaunchKernelGGL((fresh_gather_kernel<Idx, E, false>), grid, dim3(kGatherThreads), 0, s,
                         top_index, k, total, static_cast<const Idx*>(fi), fs,
                         static_cast<const Idx*>(mi), ms, num_fresh, static_cast<const E*>(fd),
                         frows, static_cast<const E*>(md), mrows, units, static_cast<E*>(out));
  };
  switch (unit) {
    case 1: go(uint8_t{}); break;
    case 2: go(uint16_t{}); break;
    case 4: go(uint32_t{}); break;
    case 8: go(uint64_t{}); break;
    default: go(u32x4{}); break;
  }
}

}  // namespace
}  // namespace st

extern "C" int64_t st_fresh_topk_workspace_bytes(int64_t rows, int64_t k) {
  if (rows <= 0 || k <= 0) return 0;
  const int64_t p = st::kept_length(k);
  if (p <= st::kFreshLdsMaxK) return 0;
  return rows * p * 12 + 256;
}

extern "C" int st_fresh_topk(const void* main_scores, const void* fresh_scores, int score_type,
                             int64_t rows, int64_t num_main, int64_t num_fresh, int64_t k,
                             void* workspace, void* top_scores, int64_t* top_index,
                             uint8_t* is_from_fresh, void* stream) {
  using namespace st;
  return guarded([&] {
    ST_CHECK(rows >= 0 && num_main >= 0 && num_fresh >= 0, "negative sizes");
    ST_CHECK(k >= 0 && k <= num_main + num_fresh, "k = ", k, " must lie in [0, ",
             num_main + num_fresh, "]");
    ST_CHECK(num_main + num_fresh < static_cast<int64_t>(kNoIndex),
             "merged rows of ", num_main + num_fresh, " columns exceed the 32-bit index range");
    if (rows == 0 || k == 0) return;
    ST_CHECK(top_scores != nullptr && top_index != nullptr && is_from_fresh != nullptr,
             "null output");
    ST_CHECK(num_fresh == 0 || fresh_scores != nullptr, "fresh_scores is null");
    ST_CHECK(num_main == 0 || main_scores != nullptr, "main_scores is null");
    ST_CHECK(rows <= 0x7FFFFFFF, "too many rows: ", rows);
    FreshTopkArgs a;
    a.fresh_scores = fresh_scores;
    a.main_scores = main_scores;
    a.rows = rows;
    a.num_fresh = num_fresh;
    a.num_main = num_main;
    a.k = k;
    a.p = kept_length(k);
    a.ws_keys = nullptr;
    a.ws_index = nullptr;
    if (a.p > kFreshLdsMaxK) {
      ST_CHECK(workspace != nullptr, "workspace is null (st_fresh_topk_workspace_bytes)");
      a.ws_keys = static_cast<uint64_t*>(workspace);
      a.ws_index = reinterpret_cast<uint32_t*>(a.ws_keys + rows * a.p);
    }
    a.top_scores = top_scores;
    a.top_index = top_index;
    a.from_fresh = is_from_fresh;
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (score_type) {
      case ST_SCORE_F32: launch_topk_typed<ST_SCORE_F32>(a, s); break;
      case ST_SCORE_F16: launch_topk_typed<ST_SCORE_F16>(a, s); break;
      case ST_SCORE_BF16: launch_topk_typed<ST_SCORE_BF16>(a, s); break;
      case ST_SCORE_F64: launch_topk_typed<ST_SCORE_F64>(a, s); break;
      case ST_SCORE_I64: launch_topk_typed<ST_SCORE_I64>(a, s); break;
      case ST_SCORE_I32: launch_topk_typed<ST_SCORE_I32>(a, s); break;
      case ST_SCORE_I16: launch_topk_typed<ST_SCORE_I16>(a, s); break;
      case ST_SCORE_I8: launch_topk_typed<ST_SCORE_I8>(a, s); break;
      case ST_SCORE_U8: launch_topk_typed<ST_SCORE_U8>(a, s); break;
      default: fail("unknown score type ", score_type);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) throw Error(ST_ERR_HIP, cat("fresh top-k launch failed: ", hipGetErrorString(e)));
  });
}

extern "C" int st_fresh_gather(const int64_t* top_index, int64_t rows, int64_t k,
                               const void* fresh_indices, const void* main_indices,
                               int index_bytes, int64_t fresh_index_cols,
                               int64_t main_index_cols, int64_t num_fresh, int64_t num_main,
                               const void* fresh_data, int64_t fresh_rows,
                               const void* main_data, int64_t main_rows, int64_t dim,
                               int elem_bytes, void* out, void* stream) {
  using namespace st;
  return guarded([&] {
    ST_CHECK(rows >= 0 && k >= 0 && dim >= 0 && fresh_rows >= 0 && main_rows >= 0,
             "negative sizes");
    ST_CHECK(index_bytes == 4 || index_bytes == 8, "indices must be int32 or int64");
    ST_CHECK(fresh_index_cols >= num_fresh, "fresh_indices has ", fresh_index_cols,
             " columns for ", num_fresh, " fresh scores");
    ST_CHECK(main_index_cols >= num_main, "main_indices has ", main_index_cols,
             " columns for ", num_main, " main scores");
    if (rows == 0 || k == 0 || dim == 0) return;
    ST_CHECK(top_index != nullptr && out != nullptr, "null pointer");
    ST_CHECK(num_fresh == 0 || fresh_indices != nullptr, "fresh_indices is null");
    ST_CHECK(num_main == 0 || main_indices != nullptr, "main_indices is null");
    ST_CHECK(fresh_rows == 0 || fresh_data != nullptr, "fresh data is null");
    ST_CHECK(main_rows == 0 || main_data != nullptr, "main data is null");
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (index_bytes == 4)
      launch_gather_idx<int32_t>(top_index, rows, k, fresh_indices, fresh_index_cols,
                                 main_indices, main_index_cols, num_fresh, fresh_data,
                                 fresh_rows, main_data, main_rows, dim, elem_bytes, out, s);
    else
      launch_gather_idx<int64_t>(top_index, rows, k, fresh_indices, fresh_index_cols,
                                 main_indices, main_index_cols, num_fresh, fresh_data,
                                 fresh_rows, main_data, main_rows, dim, elem_bytes, out, s);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) throw Error(ST_ERR_HIP, cat("fresh gather launch failed: ", hipGetErrorString(e)));
  });
}
