// Cluster-restricted search for gfx950: the plan of each (row, cluster) work
// item evaluated on the columns that cover the cluster's docs.
//
// Replaces bloom_index_search_batch_return_partial_response
// (bloom_index_search.cpp:246-395 on CPU, bloom_index_search_cuda.cu:617-1648
// on CUDA).  The host (st_search_plan_partial_items) lays out the response;
// here one wave takes one item at a time and each lane one 64-bit column
// word: the program is wave-uniform (scalar loads), the bundle width and so
// the row positions are the lane's own, resolved from the term hashes as
// signature_match does (bloom_index_search.cpp:40-61).
#include <hip/hip_runtime.h>

#include "search_plan.hpp"
#include "st_common.hpp"
#include "st_errors.hpp"

namespace st {
namespace {

constexpr int kPartialThreads = 256;

#define ST_CONST __attribute__((address_space(4)))

struct PartialArgs {
  const int64_t* index;
  int64_t index_numel;
  const int64_t* bbo;
  const ST_CONST uint32_t* blob32;
  const ST_CONST uint64_t* blob64;
  int32_t hash_k;
  uint32_t pos_bytes;  // program term references are term * pos_bytes
};

// Where this lane's column sits.
struct Column {
  int64_t start;  // first row of the bundle
  int64_t b;      // bundle width
  int64_t cib;    // column within the bundle
  FastMod64 fm;
};

// Word of one term on the lane's column: the AND of the rows at its first K
// distinct positions (int16)(h[p] % b), p < hash_k; a bundle of width 0
// matches nothing, a row outside the index reads as zero.
template <int K>
__device__ __forceinline__ uint64_t term_word(const PartialArgs& a, const Column& c,
                                              const ST_CONST uint64_t* h) {
  if constexpr (K == 0) {
    return ~0ull;
  } else {
    if (c.b <= 0) return 0;
    int16_t found[K];
    int cnt = 0;
    uint64_t r = ~0ull;
    for (int p = 0; p < a.hash_k && cnt < K; ++p) {
      const int16_t bp = static_cast<int16_t>(fast_mod(h[p], c.fm));
      bool dup = false;
#pragma unroll
      for (int j = 0; j < K; ++j) dup |= (j < cnt) && (found[j] == bp);
      if (dup) continue;
#pragma unroll
      for (int j = 0; j < K; ++j)
        if (j == cnt) found[j] = bp;
      ++cnt;
      const int64_t w = (c.start + bp) * kColumnsPerBundle + c.cib;
      r &= (w >= 0 && w < a.index_numel) ? static_cast<uint64_t>(a.index[w]) : 0ull;
    }
    return r;
  }
}

__device__ __forceinline__ uint64_t combine64(uint32_t op, uint64_t acc, uint64_t v) {
  if (op & 32u) v = ~v;
  const uint32_t mode = (op >> 3) & 3u;
  return mode == kModeSet ? v : (mode == kModeAnd ? (acc & v) : (acc | v));
}

// The row's program (search_plan.hpp forms) on the lane's column.
template <int K>
__device__ uint64_t eval_program(const PartialArgs& a, const Column& c,
                                 const ST_CONST uint32_t* prog,
                                 const ST_CONST uint64_t* hashes) {
  const uint32_t hdr = prog[0];
  const uint32_t T = hdr & 0xFFFFu;
  auto term_hashes = [&](uint32_t ref) {
    return hashes + static_cast<uint64_t>(ref / a.pos_bytes) * a.hash_k;
  };
  if (hdr & kFlatForm) {  // OR of AND-groups: [term ref, negate, group, 0]
    const ST_CONST uint32_t* lit = prog + kProgHeaderWords;
    uint64_t res = 0, acc = 0;
    for (uint32_t j = 0; j < T; ++j, lit += kFlatLiteralWords) {
      const uint64_t w = term_word<K>(a, c, term_hashes(lit[0]));
      const uint64_t neg = lit[1] ? ~0ull : 0ull;
      const uint64_t grp = lit[2] ? ~0ull : 0ull;
      res |= acc & grp;
      acc = (acc | grp) & (w ^ neg);
    }
    res |= acc;
    return (hdr & kFlatComplement) ? ~res : res;
  }
  // stack form: T term references, then the operations
  const ST_CONST uint32_t* tref = prog + kProgHeaderWords;
  const ST_CONST uint32_t* ops = tref + T;
  const uint32_t nops = prog[2];
  uint64_t acc = 0;
  uint64_t stk[kSearchMaxStack];
  uint32_t sp = 0, t = 0;
  for (uint32_t i = 0; i < nops; ++i) {
    const uint32_t op = ops[i];
    const uint32_t code = op & 7u;
    if (code == kInsTerm) {
      acc = combine64(op, acc, term_word<K>(a, c, term_hashes(tref[t++])));
    } else if (code == kInsConst) {
      acc = combine64(op, acc, ~0ull);
    } else if (code == kInsPush) {
      stk[sp++] = acc;
    } else if (code == kInsPop) {
      const uint64_t v = acc;
      acc = stk[--sp];
      acc = combine64(op, acc, v);
    } else {  // kInsNot
      acc = ~acc;
    }
  }
  return acc;
}

template <int K>
__global__ __launch_bounds__(kPartialThreads) void partial_search_kernel(
    const int64_t* __restrict__ index, int64_t index_numel, const int64_t* __restrict__ bbo,
    const uint32_t* __restrict__ blob, const st_partial_item* __restrict__ items,
    int64_t num_items, int32_t hash_k, uint32_t pos_bytes, int64_t* __restrict__ out) {
  PartialArgs a;
  a.index = index;
  a.index_numel = index_numel;
  a.bbo = bbo;
  a.blob32 = (const ST_CONST uint32_t*)(blob);
  a.blob64 = (const ST_CONST uint64_t*)(blob);
  a.hash_k = hash_k;
  a.pos_bytes = pos_bytes;
  const int lane = threadIdx.x & 63;
  const int64_t waves = static_cast<int64_t>(gridDim.x) * (kPartialThreads / 64);
  const int64_t first_wave = static_cast<int64_t>(blockIdx.x) * (kPartialThreads / 64) +
                             __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // st_partial_item as 8 words: first_column, out_offset (2 each),
  // num_columns, program, hashes, reserved
  static_assert(sizeof(st_partial_item) == 32, "st_partial_item layout");
  const ST_CONST uint32_t* words = (const ST_CONST uint32_t*)(items);
  auto i64_at = [](const ST_CONST uint32_t* w) {
    return static_cast<int64_t>((static_cast<uint64_t>(w[1]) << 32) | w[0]);
  };
  for (int64_t i = first_wave; i < num_items; i += waves) {
    const ST_CONST uint32_t* w = words + i * 8;
    const int64_t first_column = i64_at(w), out_offset = i64_at(w + 2);
    const int32_t num_columns = static_cast<int32_t>(w[4]);
    const ST_CONST uint32_t* prog = a.blob32 + w[5];
    const ST_CONST uint64_t* hashes = a.blob64 + w[6];
    for (int32_t j0 = 0; j0 < num_columns; j0 += 64) {
      const int32_t j = j0 + lane;
      if (j >= num_columns) break;
      const int64_t col = first_column + j;
      const int64_t bundle = col / kColumnsPerBundle;
      Column c;
      c.start = bbo[bundle];
      c.b = bbo[bundle + 1] - c.start;
      if (c.b < 0) c.b = 0;
      c.cib = col % kColumnsPerBundle;
      c.fm = make_fastmod_dev(static_cast<uint64_t>(c.b > 0 ? c.b : 1));
      out[out_offset + j] = static_cast<int64_t>(eval_program<K>(a, c, prog, hashes));
    }
  }
}

using PartialFn = void (*)(const int64_t*, int64_t, const int64_t*, const uint32_t*,
                           const st_partial_item*, int64_t, int32_t, uint32_t, int64_t*);

PartialFn select_partial(int k) {
  switch (k) {
    case 0: return partial_search_kernel<0>;
    case 1: return partial_search_kernel<1>;
    case 2: return partial_search_kernel<2>;
    case 3: return partial_search_kernel<3>;
    case 4: return partial_search_kernel<4>;
    case 5: return partial_search_kernel<5>;
    case 6: return partial_search_kernel<6>;
    case 7: return partial_search_kernel<7>;
    case 8: return partial_search_kernel<8>;
    case 9: return partial_search_kernel<9>;
    case 10: return partial_search_kernel<10>;
    default: fail("unsupported k_eff ", k);
  }
}

int cu_count_here() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    n = 256;
  return n;
}

}  // namespace
}  // namespace st

extern "C" int st_bloom_index_search_partial(const int64_t* bloom_index,
                                             int64_t bloom_index_numel,
                                             const int64_t* bundle_b_offsets,
                                             int64_t num_bundles, const st_search_plan* plan,
                                             const void* plan_blob_device,
                                             const st_partial_item* items_device,
                                             int64_t num_items, int64_t* out, void* stream) {
  using namespace st;
  return guarded([&] {
    ST_CHECK(plan != nullptr, "plan is null");
    ST_CHECK(num_items >= 0 && num_bundles >= 0 && bloom_index_numel >= 0, "negative sizes");
    if (num_items == 0) return;
    ST_CHECK(items_device != nullptr && out != nullptr && bundle_b_offsets != nullptr &&
                 plan_blob_device != nullptr,
             "null device pointer");
    ST_CHECK(bloom_index != nullptr || bloom_index_numel == 0, "bloom_index is null");
    const int64_t per_block = kPartialThreads / 64;
    const int64_t blocks =
        std::min<int64_t>((num_items + per_block - 1) / per_block, 8ll * cu_count_here());
    hipLaunchKernelGGL(select_partial(plan->k_eff), dim3(static_cast<unsigned>(blocks)),
                       dim3(kPartialThreads), 0, static_cast<hipStream_t>(stream), bloom_index,
                       bloom_index_numel, bundle_b_offsets,
                       static_cast<const uint32_t*>(plan_blob_device), items_device, num_items,
                       static_cast<int32_t>(plan->hash_k), static_cast<uint32_t>(plan->kp) * 4u,
                       out);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
      throw Error(ST_ERR_HIP, cat("partial search kernel launch failed: ", hipGetErrorString(e)));
  });
}
