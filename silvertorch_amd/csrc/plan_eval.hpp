// Evaluation of one compiled program (search_plan.hpp layouts) on one
// 64-bit column word per lane, with the row positions resolved by the lane
// itself from the term hashes (no width binding, no LDS).  Used by the
// cluster-restricted search and by the generic search kernel, which runs
// the programs the batch kernels do not take (deep stacks, very long
// queries).
#pragma once

#include <hip/hip_runtime.h>

#include "search_plan.hpp"
#include "st_common.hpp"

namespace st {

#define ST_EVAL_CONST __attribute__((address_space(4)))

struct EvalArgs {
  const int64_t* index;
  int64_t index_numel;
  int32_t hash_k;
  uint32_t pos_bytes;  // program term references are term * pos_bytes
};

// Where a lane's column sits.
struct Column {
  int64_t start;  // first row of the bundle
  int64_t b;      // bundle width
  int64_t cib;    // column within the bundle
  FastMod64 fm;
};

__device__ __forceinline__ Column column_of(const int64_t* bbo, int64_t col) {
  Column c;
  const int64_t bundle = col / kColumnsPerBundle;
  c.start = bbo[bundle];
  c.b = bbo[bundle + 1] - c.start;
  if (c.b < 0) c.b = 0;
  c.cib = col % kColumnsPerBundle;
  c.fm = make_fastmod_dev(static_cast<uint64_t>(c.b > 0 ? c.b : 1));
  return c;
}

// Word of one term on the lane's column: the AND of the rows at its first K
// distinct positions (int16)(h[p] % b), p < hash_k (signature_match,
// bloom_index_search.cpp:40-61); a bundle of width 0 matches nothing, a row
// outside the index reads as zero.
template <int K>
__device__ __forceinline__ uint64_t eval_term_word(const EvalArgs& a, const Column& c,
                                                   const ST_EVAL_CONST uint64_t* h) {
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

__device__ __forceinline__ uint64_t eval_combine(uint32_t op, uint64_t acc, uint64_t v) {
  if (op & 32u) v = ~v;
  const uint32_t mode = (op >> 3) & 3u;
  return mode == kModeSet ? v : (mode == kModeAnd ? (acc & v) : (acc | v));
}

// The program on the lane's column: flat form (OR of AND-groups) or stack
// form (accumulator machine with a stack of at most kStack words).
template <int K, int kStack>
__device__ uint64_t eval_program(const EvalArgs& a, const Column& c,
                                 const ST_EVAL_CONST uint32_t* prog,
                                 const ST_EVAL_CONST uint64_t* hashes) {
  const uint32_t hdr = prog[0];
  const uint32_t T = program_terms(hdr);
  auto term_hashes = [&](uint32_t ref) {
    return hashes + static_cast<uint64_t>(ref / a.pos_bytes) * a.hash_k;
  };
  if (hdr & kFlatForm) {  // OR of AND-groups: [term ref, negate, group, 0]
    const ST_EVAL_CONST uint32_t* lit = prog + kProgHeaderWords;
    uint64_t res = 0, acc = 0;
    for (uint32_t j = 0; j < T; ++j, lit += kFlatLiteralWords) {
      const uint64_t w = eval_term_word<K>(a, c, term_hashes(lit[0]));
      const uint64_t neg = lit[1] ? ~0ull : 0ull;
      const uint64_t grp = lit[2] ? ~0ull : 0ull;
      res |= acc & grp;
      acc = (acc | grp) & (w ^ neg);
    }
    res |= acc;
    return (hdr & kFlatComplement) ? ~res : res;
  }
  // stack form: T term references, then the operations
  const ST_EVAL_CONST uint32_t* tref = prog + kProgHeaderWords;
  const ST_EVAL_CONST uint32_t* ops = tref + T;
  const uint32_t nops = prog[2];
  uint64_t acc = 0;
  uint64_t stk[kStack];
  uint32_t sp = 0, t = 0;
  for (uint32_t i = 0; i < nops; ++i) {
    const uint32_t op = ops[i];
    const uint32_t code = op & 7u;
    if (code == kInsTerm) {
      acc = eval_combine(op, acc, eval_term_word<K>(a, c, term_hashes(tref[t++])));
    } else if (code == kInsConst) {
      acc = eval_combine(op, acc, ~0ull);
    } else if (code == kInsPush) {
      stk[sp < kStack ? sp : kStack - 1] = acc;  // the compiler bounds sp by kStack
      ++sp;
    } else if (code == kInsPop) {
      const uint64_t v = acc;
      --sp;
      acc = stk[sp < kStack ? sp : kStack - 1];
      acc = eval_combine(op, acc, v);
    } else {  // kInsNot
      acc = ~acc;
    }
  }
  return acc;
}

}  // namespace st
