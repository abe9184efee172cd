// Generic search kernel for gfx950: the queries the batch kernels do not
// take -- programs needing more than kSearchMaxStack stack slots, or more
// terms or operations than a batch program holds, or more distinct terms
// than a batch's position area -- each evaluated on every column by the
// per-lane evaluator of plan_eval.hpp (positions resolved by each lane from
// the term hashes, a stack of kGenericMaxStack words).  Together with the
// batch kernels this evaluates every plan the reference's CPU search does
// (run_query_plan, bloom_index_search.cpp:72-171, whose std::stack has no
// bound).  Such queries are rare; this path trades speed for generality.
#include <hip/hip_runtime.h>

#include "bloom_generic.hpp"
#include "plan_eval.hpp"
#include "search_plan.hpp"
#include "st_common.hpp"
#include "st_errors.hpp"

namespace st {
namespace {

constexpr int kGenericThreads = 256;  // 4 waves, 2 bundles each

#define ST_GCONST __attribute__((address_space(4)))

// Lane l of wave w serves column l & 31 of bundle 2 w + (l >> 5).
template <int K, int kOut>
__global__ __launch_bounds__(kGenericThreads) void generic_search_kernel(
    const int64_t* __restrict__ index, int64_t index_numel, const int64_t* __restrict__ bbo,
    int64_t num_bundles, const uint32_t* __restrict__ prog, const uint64_t* __restrict__ hashes,
    int32_t hash_k, uint32_t pos_bytes, uint32_t row, int64_t out_cols, void* __restrict__ out,
    int64_t* __restrict__ counts, int64_t num_docs) {
  EvalArgs a;
  a.index = index;
  a.index_numel = index_numel;
  a.hash_k = hash_k;
  a.pos_bytes = pos_bytes;
  const int lane = threadIdx.x & 63;
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * (kGenericThreads / 64) + (threadIdx.x >> 6);
  const int64_t bundle = wave * 2 + (lane >> 5);
  if (bundle >= num_bundles) return;
  const int64_t col = bundle * kColumnsPerBundle + (lane & 31);
  const Column c = column_of(bbo, col);
  const uint64_t w = eval_program<K, kGenericMaxStack>(
      a, c, (const ST_GCONST uint32_t*)(prog), (const ST_GCONST uint64_t*)(hashes));
  if constexpr (kOut == kGenericBool) {
    // doc 64 col + i at byte i: bit 63 - i of the word
    typedef uint32_t v4 __attribute__((ext_vector_type(4)));
    v4* dst = reinterpret_cast<v4*>(static_cast<uint8_t*>(out) +
                                    static_cast<int64_t>(row) * out_cols * 64 + col * 64);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t nib = static_cast<uint32_t>(__builtin_bitreverse64(w) >> (16 * q + 4 * e)) & 0xFu;
        o[e] = (nib * 0x00204081u) & 0x01010101u;
      }
      dst[q] = o;
    }
  } else {
    static_cast<int64_t*>(out)[static_cast<int64_t>(row) * out_cols + col] = static_cast<int64_t>(w);
    if constexpr (kOut == kGenericCounts) {
      const int64_t first = col * kBitsPerColumn;
      uint64_t valid = 0;
      if (num_docs > first) valid = num_docs - first >= 64 ? ~0ull : ~((~0ull) >> (num_docs - first));
      uint32_t n = static_cast<uint32_t>(__popcll(w & valid));
#pragma unroll
      for (int m = 16; m >= 1; m >>= 1) n += __shfl_xor(n, m, 32);
      if ((lane & 31) == 0) counts[static_cast<int64_t>(row) * num_bundles + bundle] = n;
    }
  }
}

using GenericFn = void (*)(const int64_t*, int64_t, const int64_t*, int64_t, const uint32_t*,
                           const uint64_t*, int32_t, uint32_t, uint32_t, int64_t, void*, int64_t*,
                           int64_t);

template <int kOut>
GenericFn select_generic_out(int k) {
  switch (k) {
    case 0: return generic_search_kernel<0, kOut>;
    case 1: return generic_search_kernel<1, kOut>;
    case 2: return generic_search_kernel<2, kOut>;
    case 3: return generic_search_kernel<3, kOut>;
    case 4: return generic_search_kernel<4, kOut>;
    case 5: return generic_search_kernel<5, kOut>;
    case 6: return generic_search_kernel<6, kOut>;
    case 7: return generic_search_kernel<7, kOut>;
    case 8: return generic_search_kernel<8, kOut>;
    case 9: return generic_search_kernel<9, kOut>;
    case 10: return generic_search_kernel<10, kOut>;
    default: fail("unsupported k_eff ", k);
  }
}

}  // namespace

void launch_generic_batch(const int64_t* index, int64_t index_numel, const int64_t* bbo,
                          int64_t num_bundles, const void* plan_blob_device,
                          const SearchBatch& bt, const std::vector<uint32_t>& starts,
                          const std::vector<uint32_t>& insns, int k_eff, int hash_k, int kp,
                          int out_mode, void* out, int64_t* counts, int64_t num_docs,
                          hipStream_t stream) {
  if (num_bundles == 0 || bt.num_slots == 0) return;
  const char* blob = static_cast<const char*>(plan_blob_device);
  const uint32_t start = starts[0];
  const uint32_t row = insns[start + 1];
  const int64_t waves = (num_bundles + 1) / 2;
  const int64_t blocks = (waves + kGenericThreads / 64 - 1) / (kGenericThreads / 64);
  GenericFn fn = out_mode == kGenericBool ? select_generic_out<kGenericBool>(k_eff)
                 : out_mode == kGenericCounts ? select_generic_out<kGenericCounts>(k_eff)
                                              : select_generic_out<kGenericPacked>(k_eff);
  hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(blocks)), dim3(kGenericThreads), 0, stream,
                     index, index_numel, bbo, num_bundles,
                     reinterpret_cast<const uint32_t*>(blob + bt.off_insns) + start,
                     reinterpret_cast<const uint64_t*>(blob + bt.off_hashes), hash_k,
                     static_cast<uint32_t>(kp) * 4u, row, num_bundles * kColumnsPerBundle, out,
                     counts, num_docs);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    throw Error(ST_ERR_HIP, cat("generic search kernel launch failed: ", hipGetErrorString(e)));
}

}  // namespace st
