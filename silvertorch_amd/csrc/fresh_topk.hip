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
// Selection: one workgroup per row keeps the row's best P = pow2 >= k'
// entries (key, index) sorted, best first.  The row is read 1024 entries at
// a time; entries better than the running k'-th best are compacted into a
// candidate buffer (wave ballot + per-wave counts), and a full buffer is
// sorted (bitonic) and merged into the kept list (bitonic merge of the kept
// list with the reversed candidates).  Most of a long row never reaches a
// sort.  The kept list lives in LDS for k' <= kFreshLdsMaxK and in the
// caller's workspace above that; the candidate buffer is always in LDS.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/silvertorch_hip.h"
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
      for (int p = tid; p < n / 2; p += kFreshThreads) {
        const int i = (p / stride) * 2 * stride + (p % stride);
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
    for (int64_t p = tid; p < P / 2; p += kFreshThreads) {
      const int64_t i = (p / stride) * 2 * stride + (p % stride);
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

template <int kType>
void launch_topk_typed(const FreshTopkArgs& a, hipStream_t s) {
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

// Gather of one data tensor: element e of the output is element e % D of the
// source row chosen for output row e / D.
template <typename Idx, typename Elem>
__global__ void fresh_gather_kernel(const int64_t* __restrict__ top_index, int64_t k,
                                    int64_t total, const Idx* __restrict__ fresh_idx,
                                    int64_t fresh_stride, const Idx* __restrict__ main_idx,
                                    int64_t main_stride, int64_t num_fresh,
                                    const Elem* __restrict__ fresh_data, int64_t fresh_rows,
                                    const Elem* __restrict__ main_data, int64_t main_rows,
                                    int64_t dim, Elem* __restrict__ out) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= total) return;
  const int64_t item = e / dim, d = e - item * dim;
  const int64_t row = item / k;
  const int64_t t = top_index[item];
  const bool fresh = t < num_fresh;
  int64_t src = fresh ? static_cast<int64_t>(fresh_idx[row * fresh_stride + t])
                      : static_cast<int64_t>(main_idx[row * main_stride + (t - num_fresh)]);
  const int64_t rows = fresh ? fresh_rows : main_rows;
  if (src < 0 || src >= rows) src = 0;  // padded offsets read row 0
  const Elem* data = fresh ? fresh_data : main_data;
  out[e] = rows > 0 ? data[src * dim + d] : Elem{};
}

template <typename Idx>
void launch_gather_idx(const int64_t* top_index, int64_t rows, int64_t k, const void* fi,
                       int64_t fs, const void* mi, int64_t ms, int64_t num_fresh,
                       const void* fd, int64_t frows, const void* md, int64_t mrows,
                       int64_t dim, int elem_bytes, void* out, hipStream_t s) {
  const int64_t total = rows * k * dim;
  const int threads = 256;
  const dim3 grid(static_cast<unsigned>((total + threads - 1) / threads));
  auto go = [&](auto tag) {
    using E = decltype(tag);
    hipLaunchKernelGGL((fresh_gather_kernel<Idx, E>), grid, dim3(threads), 0, s, top_index, k,
                       total, static_cast<const Idx*>(fi), fs, static_cast<const Idx*>(mi), ms,
                       num_fresh, static_cast<const E*>(fd), frows, static_cast<const E*>(md),
                       mrows, dim, static_cast<E*>(out));
  };
  switch (elem_bytes) {
    case 1: go(uint8_t{}); break;
    case 2: go(uint16_t{}); break;
    case 4: go(uint32_t{}); break;
    case 8: go(uint64_t{}); break;
    default: fail("unsupported element size ", elem_bytes);
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
