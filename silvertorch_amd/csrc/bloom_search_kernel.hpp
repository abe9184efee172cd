// Batched boolean search over the bundled bloom index, for gfx950: device
// code and the kernel template.  Each K is instantiated in its own
// translation unit (bloom_search_k.hip); the host side is bloom_search.hip.
//
// Replaces process_documents / bloom_index_search_common
// (bloom_index_search_cuda.cu:575-615, :940-1029) and the CPU loop
// bloom_index_search_common_cpu (bloom_index_search.cpp:173-243).
//
// Layout (unchanged from the reference, bloom_indexer.cpp:72-110): bundle i
// owns rows [off[i], off[i+1]) of 32 int64 words; word (row, c) holds the
// bloom bit `row` of the 64 docs of column c, doc 64c+j at bit 63-j.
//
// Work decomposition: one 1024-thread workgroup per CU walks bundles
// blockIdx.x, blockIdx.x + gridDim.x, ... of the visiting order, loading each
// bundle's extent and width slot one bundle ahead.  For each bundle it
//   1. moves the bundle's rows (prefetched into registers while the previous
//      bundle was evaluated) into LDS, so the index is read from HBM once per
//      query batch;
//   2. resolves every distinct batch term to its k row positions for this
//      bundle's width b -- once per bundle instead of once per (query,
//      column) -- skipping the step when b equals the previous bundle's;
//   3. has each wave run its queries' programs.  Flat (OR-of-AND) programs
//      of a width-bound batch whose literal stream fits the LDS area after
//      the tile run four at a time in quad lanes (eval_quads: the stream is
//      staged in LDS with the tile, each 16-lane group serves one program
//      and every lane reads 16 bytes of a row); the other programs run one
//      per wave instruction, lane l owning the 32-bit half (l & 1) of column
//      l >> 1, with wave-uniform control flow.
// Bundles wider than the LDS tile are evaluated from global memory with the
// same programs.
#pragma once

#include <hip/hip_runtime.h>


#include "search_plan.hpp"
#include "st_common.hpp"
#include "st_errors.hpp"
#include "wave_ops.hpp"

namespace st {
namespace {

// Native 4 x u32 vector (usable with the nontemporal builtins).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// The plan arrays and bundle offsets are read-only for the kernel's lifetime.
// Reading them through the constant address space lets every uniform read
// become a scalar load: a vector load there would share the in-order vmcnt
// counter with the next bundle's tile prefetch, and waiting for it would wait
// for the whole prefetch.
#define ST_CONST __attribute__((address_space(4)))
// Output stores go through the global address space explicitly (a pointer
// rebuilt from an integer would otherwise be a flat pointer, and flat stores
// also count against the LDS wait counter).
#define ST_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ const ST_CONST T* as_const(const T* p) {
  return (const ST_CONST T*)(p);  // addrspacecast: only a C-style cast spells it
}

constexpr int kPrefetch = kSearchTileRows * 16 / kSearchThreads;  // uint4/thread
static_assert(kPrefetch * kSearchThreads == kSearchTileRows * 16, "tile split");

struct SearchArgs {
  const int64_t* index;
  int64_t index_numel;
  const ST_CONST int64_t* bundle_offsets;
  int64_t num_bundles;
  const ST_CONST uint32_t* wave_off;
  const ST_CONST uint32_t* insn_start;
  const ST_CONST uint32_t* insns;
  const ST_CONST uint64_t* hashes;
  const ST_CONST uint32_t* bundle_slot;   // nullptr when the plan is not width-bound
  const ST_CONST uint32_t* bundle_order;  // visiting order (nullptr: index order)
  const ST_CONST uint32_t* bound_start;
  const ST_CONST uint32_t* bound;
  uint32_t bound_words;
  uint32_t stream_off;                    // literal stream within a width block
  uint32_t stream_words;                  // 0: no stream
  uint32_t stream_masks;                  // records carry group masks
  uint32_t num_terms;
  int32_t hash_k;
  int64_t out_cols;  // columns per output row = num_bundles * 32
  void* out;
  int64_t* counts;   // kOutCounts: matches per (query row, bundle)
  int64_t num_docs;  // kOutCounts: docs at or past it are not counted
};

// Output modes of the search kernel.
constexpr int kOutPacked = 0;  // int64 words
constexpr int kOutBool = 1;    // one byte per doc
constexpr int kOutCounts = 2;  // int64 words, plus per-(row, bundle) match counts

__device__ __forceinline__ uint32_t uniform(uint32_t v) {
  return __builtin_amdgcn_readfirstlane(v);
}

// Width and first row of bundle `bnd`; a negative width (malformed offsets)
// reads as an empty bundle.
__device__ __forceinline__ void bundle_extent(const SearchArgs& a, int64_t bnd,
                                              int64_t& start, int64_t& b) {
  start = a.bundle_offsets[bnd];
  b = a.bundle_offsets[bnd + 1] - start;
  if (b < 0) b = 0;
}

// Where a bundle sits and which width block evaluates it; which share of
// its programs a visit evaluates (part of parts: rounds and programs whose
// index is part mod parts).  bundle < 0: no bundle.
struct BundleMeta {
  int64_t bundle;
  int64_t start;  // first row
  int64_t b;      // rows
  uint32_t slot;  // width slot (kNoWidthSlot: none)
  uint32_t part, parts;
};

// The bundles of the grid's last, partial round are split among up to this
// many workgroups each, by program.
constexpr int kTailParts = 4;

// Cycles a program or round counter through the parts of a split visit.
struct PartFilter {
  uint32_t part, parts, at;
  __device__ __forceinline__ bool take() {
    const bool mine = at == part;
    at = at + 1 == parts ? 0u : at + 1;
    return mine;
  }
};

// Issues this thread's share of the loads of the rows [start, start + b)
// into `pre` (nothing when the bundle is wider than the LDS tile).  The
// bound is one uniform limit on the 16-byte chunks (of a bundle whose rows
// pass the end of the index, which only malformed offsets describe, the
// chunks inside the index are loaded), so the per-load test is a 32-bit
// compare.
__device__ __forceinline__ void prefetch_tile(const SearchArgs& a, int64_t start, int64_t b,
                                              u32x4 (&pre)[kPrefetch]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < kPrefetch; ++i) pre[i] = u32x4{0, 0, 0, 0};
  if (b > kSearchTileRows || start < 0) return;
  const int64_t avail = (a.index_numel - start * 32) / 2;  // whole chunks left in the index
  const int lim = static_cast<int>(b * 16 < avail ? b * 16 : (avail > 0 ? avail : 0));
  const u32x4* src = reinterpret_cast<const u32x4*>(a.index + start * 32);
#pragma unroll
  for (int i = 0; i < kPrefetch; ++i) {
    const int c = tid + i * kSearchThreads;
    if (c < lim) pre[i] = __builtin_nontemporal_load(src + c);
  }
}

// Resolves term u's positions for width b, as signature_match does
// (bloom_index_search.cpp:40-61): over hashes p < hash_k, while fewer than K
// are resolved, b_p = (int16)(h[p] % b); repeats of an earlier b_p are
// skipped.  Unused slots repeat slot 0 (AND is idempotent).
template <int K>
__device__ __forceinline__ int resolve_positions(const ST_CONST uint64_t* h, int hash_k,
                                                 const FastMod64& fm,
                                                 int16_t (&found)[K]) {
  int cnt = 0;
  for (int p = 0; p < hash_k && cnt < K; ++p) {
    const int16_t bp = static_cast<int16_t>(fast_mod(h[p], fm));
    bool dup = false;
#pragma unroll
    for (int j = 0; j < K; ++j) dup |= (j < cnt) && (found[j] == bp);
    if (!dup) {
#pragma unroll
      for (int j = 0; j < K; ++j)
        if (j == cnt) found[j] = bp;
      ++cnt;
    }
  }
  return cnt;
}

// Expands a 32-bit match half into 32 bool bytes, most significant bit
// first (the doc order of bloom_index_search.cpp:231-236).
__device__ __forceinline__ void store_bool32(ST_GLOBAL char* dst, uint32_t bits) {
  const uint32_t y = __builtin_bitreverse32(bits);
  uint32_t w[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) w[j] = (((y >> (4 * j)) & 0xFu) * 0x00204081u) & 0x01010101u;
  ST_GLOBAL u32x4* d = (ST_GLOBAL u32x4*)(dst);
  __builtin_nontemporal_store(u32x4{w[0], w[1], w[2], w[3]}, d);
  __builtin_nontemporal_store(u32x4{w[4], w[5], w[6], w[7]}, d + 1);
}

// Executes one non-TERM operation on the accumulator machine.
__device__ __forceinline__ void exec_op(uint32_t op, uint32_t& acc,
                                        uint32_t (&stk)[kSearchMaxStack],
                                        uint32_t& sp) {
  const uint32_t code = op & 7u;
  uint32_t v;
  if (code == kInsConst) {
    v = ~0u;
  } else if (code == kInsPush) {
    stk[sp++] = acc;
    return;
  } else if (code == kInsPop) {
    v = acc;
    acc = stk[--sp];
  } else {  // kInsNot
    acc = ~acc;
    return;
  }
  if (op & 32u) v = ~v;
  const uint32_t mode = (op >> 3) & 3u;
  acc = mode == kModeSet ? v : (mode == kModeAnd ? (acc & v) : (acc | v));
}

__device__ __forceinline__ uint32_t combine(uint32_t op, uint32_t acc, uint32_t v) {
  if (op & 32u) v = ~v;
  const uint32_t mode = (op >> 3) & 3u;
  return mode == kModeSet ? v : (mode == kModeAnd ? (acc & v) : (acc | v));
}

// Where the rows of the current bundle are read from.
struct RowSource {
  const uint32_t* pos;    // LDS position lists
  const char* tile_lane;  // LDS tile + this lane's byte offset
  const uint32_t* index32;
  int64_t index_numel;
  int64_t start;          // first row of the bundle
  int64_t b;              // rows of the bundle
  int lane;
  bool staged;            // rows in the LDS tile (else global memory)
};

// Position list of the term whose list starts at byte `off` of the LDS
// position area.
template <int KP>
__device__ __forceinline__ void load_positions(const RowSource& rs, uint32_t off,
                                               uint32_t (&p)[KP]) {
  const uint32_t* pp = reinterpret_cast<const uint32_t*>(
      reinterpret_cast<const char*>(rs.pos) + off);
#pragma unroll
  for (int r = 0; r < KP; r += 4) {
    const u32x4 q4 = *reinterpret_cast<const u32x4*>(pp + r);
    p[r] = q4.x;
    p[r + 1] = q4.y;
    p[r + 2] = q4.z;
    p[r + 3] = q4.w;
  }
}

// Word of one term for this lane's 32-bit half column: AND of its K rows.
// STAGED selects the LDS tile or global memory at compile time, so the row
// reads of several terms form one straight-line block.
template <int K, int KP, bool STAGED>
__device__ __forceinline__ uint32_t term_word(const RowSource& rs, const uint32_t (&p)[KP]) {
  uint32_t v = ~0u;
  if constexpr (STAGED) {
#pragma unroll
    for (int j = 0; j < K; ++j) v &= *reinterpret_cast<const uint32_t*>(rs.tile_lane + p[j]);
  } else {
#pragma unroll
    for (int j = 0; j < K; ++j) {
      const int32_t r = static_cast<int32_t>(p[j]);
      uint32_t word = 0;
      if (r != kPosZeros) {
        const int64_t row = rs.start + r;
        if (row >= 0 && (row * 32 + (rs.lane >> 1)) < rs.index_numel)
          word = rs.index32[row * 64 + rs.lane];
      }
      v &= word;
    }
  }
  return v;
}

// Flat-form query with exactly T literals: every position list, then every
// row word, then the branch-free OR-of-ANDs fold.
template <int K, int KP, bool STAGED, int T>
__device__ __forceinline__ uint32_t eval_flat_fixed(const RowSource& rs, const ST_CONST u32x4* lit) {
  uint32_t p[T > 0 ? T : 1][KP];
#pragma unroll
  for (int j = 0; j < T; ++j) load_positions<KP>(rs, lit[j].x, p[j]);
  uint32_t w[T > 0 ? T : 1];
#pragma unroll
  for (int j = 0; j < T; ++j) w[j] = term_word<K, KP, STAGED>(rs, p[j]);
  uint32_t res = 0, acc = 0;
#pragma unroll
  for (int j = 0; j < T; ++j) {
    const u32x4 L = lit[j];
    res |= acc & L.z;
    acc = (acc | L.z) & (w[j] ^ L.y);
  }
  return res | acc;
}

// Flat-form query of any length, in groups of G literals.
template <int K, int KP, bool STAGED, int G>
__device__ __forceinline__ uint32_t eval_flat_loop(const RowSource& rs, const ST_CONST u32x4* lit,
                                                   uint32_t T) {
  uint32_t res = 0, acc = 0;
  for (uint32_t base = 0; base < T; base += G) {
    const uint32_t n = min(static_cast<uint32_t>(G), T - base);
    uint32_t p[G][KP];
#pragma unroll
    for (int j = 0; j < G; ++j)
      if (j < n) load_positions<KP>(rs, lit[base + j].x, p[j]);
    uint32_t w[G];
#pragma unroll
    for (int j = 0; j < G; ++j)
      if (j < n) w[j] = term_word<K, KP, STAGED>(rs, p[j]);
#pragma unroll
    for (int j = 0; j < G; ++j) {
      if (j < n) {
        const u32x4 L = lit[base + j];
        res |= acc & L.z;
        acc = (acc | L.z) & (w[j] ^ L.y);
      }
    }
  }
  return res | acc;
}

// Flat query dispatch: fully unrolled blocks for short queries (T * KP
// position registers bounded), the grouped loop otherwise.
template <int K, int KP, bool STAGED, int G, int T>
__device__ __forceinline__ uint32_t eval_flat_t(const RowSource& rs, const ST_CONST u32x4* lit, uint32_t n) {
  if constexpr (T * KP <= 24) {
    return eval_flat_fixed<K, KP, STAGED, T>(rs, lit);
  } else {
    return eval_flat_loop<K, KP, STAGED, G>(rs, lit, n);
  }
}

template <int K, int KP, bool STAGED, int G>
__device__ __forceinline__ uint32_t eval_flat(const RowSource& rs, const ST_CONST u32x4* lit, uint32_t T) {
  switch (T) {
    case 0: return 0;
    case 1: return eval_flat_t<K, KP, STAGED, G, 1>(rs, lit, T);
    case 2: return eval_flat_t<K, KP, STAGED, G, 2>(rs, lit, T);
    case 3: return eval_flat_t<K, KP, STAGED, G, 3>(rs, lit, T);
    case 4: return eval_flat_t<K, KP, STAGED, G, 4>(rs, lit, T);
    case 5: return eval_flat_t<K, KP, STAGED, G, 5>(rs, lit, T);
    case 6: return eval_flat_t<K, KP, STAGED, G, 6>(rs, lit, T);
    default: return eval_flat_loop<K, KP, STAGED, G>(rs, lit, T);
  }
}

// Stack-form query: term words in groups of G, operations walked in order.
template <int K, int KP, bool STAGED, int G>
__device__ __forceinline__ uint32_t eval_stack(const RowSource& rs, const ST_CONST uint32_t* prog,
                                               uint32_t T, uint32_t nops) {
  const ST_CONST uint32_t* tref = prog + kProgHeaderWords;
  const ST_CONST uint32_t* ops = tref + T;
  uint32_t acc = 0;
  uint32_t stk[kSearchMaxStack];
  uint32_t sp = 0;
  uint32_t i = 0;
  for (uint32_t base = 0; base < T; base += G) {
    const uint32_t n = min(static_cast<uint32_t>(G), T - base);
    uint32_t p[G][KP];
#pragma unroll
    for (int j = 0; j < G; ++j)
      if (j < n) load_positions<KP>(rs, tref[base + j], p[j]);
    uint32_t w[G];
#pragma unroll
    for (int j = 0; j < G; ++j)
      if (j < n) w[j] = term_word<K, KP, STAGED>(rs, p[j]);
#pragma unroll
    for (int j = 0; j < G; ++j) {
      if (j < n) {
        for (;;) {
          const uint32_t op = ops[i++];
          if ((op & 7u) == kInsTerm) {
            acc = combine(op, acc, w[j]);
            break;
          }
          exec_op(op, acc, stk, sp);
        }
      }
    }
  }
  for (; i < nops; ++i) exec_op(ops[i], acc, stk, sp);
  return acc;
}

// ----------------------------------------------------- width-bound programs

// This lane's 32-bit half of row position p of the current bundle.
template <bool STAGED>
__device__ __forceinline__ uint32_t row_word(const RowSource& rs, uint32_t p) {
  if constexpr (STAGED) {
    return *reinterpret_cast<const uint32_t*>(rs.tile_lane + p);
  } else {
    int32_t r = static_cast<int32_t>(p);
    if (r == kPosZeros) return 0;
    if (r == kPosOnes) return ~0u;
    if (wide_width(rs.b)) {  // a slice-tile byte offset; rows past b are no-op rows
      r /= kWideSliceBytes;
      if (r >= rs.b) return r == kWideOnesRow ? ~0u : 0u;
    }
    const int64_t row = rs.start + r;
    if (row < 0 || (row * 32 + (rs.lane >> 1)) >= rs.index_numel) return 0;
    return rs.index32[row * 64 + rs.lane];
  }
}

template <int K, bool STAGED>
__device__ __forceinline__ uint32_t bound_term_word(const RowSource& rs, const ST_CONST uint32_t* rec) {
  uint32_t v = ~0u;
#pragma unroll
  for (int q = 0; q < K; ++q) v &= row_word<STAGED>(rs, rec[q]);
  return v;
}

// Bound flat query with exactly T literals: all row reads of the query are
// issued before the OR-of-ANDs fold.
template <int K, bool STAGED, int T>
__device__ __forceinline__ uint32_t eval_bound_flat_fixed(const RowSource& rs, const ST_CONST uint32_t* recs) {
  constexpr int RW = ((K + 1 + 3) / 4) * 4;
  uint32_t w[T > 0 ? T : 1];
#pragma unroll
  for (int j = 0; j < T; ++j) w[j] = bound_term_word<K, STAGED>(rs, recs + j * RW);
  uint32_t res = 0, acc = 0;
#pragma unroll
  for (int j = 0; j < T; ++j) {
    const uint32_t f = recs[j * RW + K];
    const uint32_t neg = 0u - (f & 1u);
    const uint32_t grp = 0u - ((f >> 1) & 1u);
    res |= acc & grp;
    acc = (acc | grp) & (w[j] ^ neg);
  }
  return res | acc;
}

// Two bound flat queries with the same literal count T, evaluated together
// so that both queries' row reads are in flight at once.
template <int K, bool STAGED, int T>
__device__ __forceinline__ void eval_bound_pair_fixed(const RowSource& rs, const ST_CONST uint32_t* ra,
                                                      const ST_CONST uint32_t* rb, uint32_t& out_a,
                                                      uint32_t& out_b) {
  constexpr int RW = ((K + 1 + 3) / 4) * 4;
  uint32_t wa[T], wb[T];
#pragma unroll
  for (int j = 0; j < T; ++j) {
    wa[j] = bound_term_word<K, STAGED>(rs, ra + j * RW);
    wb[j] = bound_term_word<K, STAGED>(rs, rb + j * RW);
  }
  uint32_t res_a = 0, acc_a = 0, res_b = 0, acc_b = 0;
#pragma unroll
  for (int j = 0; j < T; ++j) {
    const uint32_t fa = ra[j * RW + K], fb = rb[j * RW + K];
    const uint32_t neg_a = 0u - (fa & 1u), grp_a = 0u - ((fa >> 1) & 1u);
    const uint32_t neg_b = 0u - (fb & 1u), grp_b = 0u - ((fb >> 1) & 1u);
    res_a |= acc_a & grp_a;
    acc_a = (acc_a | grp_a) & (wa[j] ^ neg_a);
    res_b |= acc_b & grp_b;
    acc_b = (acc_b | grp_b) & (wb[j] ^ neg_b);
  }
  out_a = res_a | acc_a;
  out_b = res_b | acc_b;
}

// Pair dispatch on the shared literal count; false when T is beyond the
// unrolled range (the caller then evaluates the two queries one by one).
template <int K, bool STAGED>
__device__ __forceinline__ bool eval_bound_pair(const RowSource& rs, const ST_CONST uint32_t* ra,
                                                const ST_CONST uint32_t* rb, uint32_t T, uint32_t& out_a,
                                                uint32_t& out_b) {
  switch (T) {
    case 0: out_a = 0; out_b = 0; return true;
    case 1: eval_bound_pair_fixed<K, STAGED, 1>(rs, ra, rb, out_a, out_b); return true;
    case 2: eval_bound_pair_fixed<K, STAGED, 2>(rs, ra, rb, out_a, out_b); return true;
    case 3: eval_bound_pair_fixed<K, STAGED, 3>(rs, ra, rb, out_a, out_b); return true;
    case 4: eval_bound_pair_fixed<K, STAGED, 4>(rs, ra, rb, out_a, out_b); return true;
    case 5: eval_bound_pair_fixed<K, STAGED, 5>(rs, ra, rb, out_a, out_b); return true;
    case 6: eval_bound_pair_fixed<K, STAGED, 6>(rs, ra, rb, out_a, out_b); return true;
    default: return false;
  }
}

template <int K, bool STAGED, int G>
__device__ __forceinline__ uint32_t eval_bound_flat_loop(const RowSource& rs, const ST_CONST uint32_t* recs,
                                                         uint32_t T) {
  constexpr int RW = ((K + 1 + 3) / 4) * 4;
  uint32_t res = 0, acc = 0;
  for (uint32_t base = 0; base < T; base += G) {
    const uint32_t n = min(static_cast<uint32_t>(G), T - base);
    const ST_CONST uint32_t* r0 = recs + base * RW;
    uint32_t w[G];
#pragma unroll
    for (int j = 0; j < G; ++j)
      if (j < n) w[j] = bound_term_word<K, STAGED>(rs, r0 + j * RW);
#pragma unroll
    for (int j = 0; j < G; ++j) {
      if (j < n) {
        const uint32_t f = r0[j * RW + K];
        const uint32_t neg = 0u - (f & 1u);
        const uint32_t grp = 0u - ((f >> 1) & 1u);
        res |= acc & grp;
        acc = (acc | grp) & (w[j] ^ neg);
      }
    }
  }
  return res | acc;
}

template <int K, bool STAGED, int G>
__device__ __forceinline__ uint32_t eval_bound_flat(const RowSource& rs, const ST_CONST uint32_t* recs,
                                                    uint32_t T) {
  switch (T) {
    case 0: return 0;
    case 1: return eval_bound_flat_fixed<K, STAGED, 1>(rs, recs);
    case 2: return eval_bound_flat_fixed<K, STAGED, 2>(rs, recs);
    case 3: return eval_bound_flat_fixed<K, STAGED, 3>(rs, recs);
    case 4: return eval_bound_flat_fixed<K, STAGED, 4>(rs, recs);
    case 5: return eval_bound_flat_fixed<K, STAGED, 5>(rs, recs);
    case 6: return eval_bound_flat_fixed<K, STAGED, 6>(rs, recs);
    case 7: return eval_bound_flat_fixed<K, STAGED, 7>(rs, recs);
    case 8: return eval_bound_flat_fixed<K, STAGED, 8>(rs, recs);
    default: return eval_bound_flat_loop<K, STAGED, G>(rs, recs, T);
  }
}

// Bound stack query: term position lists of KP words, then the operations.
template <int K, int KP, bool STAGED, int G>
__device__ __forceinline__ uint32_t eval_bound_stack(const RowSource& rs, const ST_CONST uint32_t* prog,
                                                     uint32_t T, uint32_t nops) {
  const ST_CONST uint32_t* tpos = prog + kProgHeaderWords;
  const ST_CONST uint32_t* ops = tpos + T * KP;
  uint32_t acc = 0;
  uint32_t stk[kSearchMaxStack];
  uint32_t sp = 0;
  uint32_t i = 0;
  for (uint32_t base = 0; base < T; base += G) {
    const uint32_t n = min(static_cast<uint32_t>(G), T - base);
    uint32_t w[G];
#pragma unroll
    for (int j = 0; j < G; ++j)
      if (j < n) w[j] = bound_term_word<K, STAGED>(rs, tpos + (base + j) * KP);
#pragma unroll
    for (int j = 0; j < G; ++j) {
      if (j < n) {
        for (;;) {
          const uint32_t op = ops[i++];
          if ((op & 7u) == kInsTerm) {
            acc = combine(op, acc, w[j]);
            break;
          }
          exec_op(op, acc, stk, sp);
        }
      }
    }
  }
  for (; i < nops; ++i) exec_op(ops[i], acc, stk, sp);
  return acc;
}

// Where a wave stores its results on one bundle: a per-lane byte offset
// (constant over the bundle) plus a uniform base per output row, so the
// address math of a store is scalar.
struct OutCursor {
  char* base;            // output byte address of row 0 on this bundle
  int64_t row_bytes;     // bytes per output row
  uint32_t lane_off;     // this lane's byte offset within its row's slice
  uint32_t count_mask;   // kOutCounts: docs of this lane that count
};

template <int kOut>
__device__ __forceinline__ OutCursor out_cursor(const SearchArgs& a, int lane, int64_t bundle) {
  OutCursor c;
  if constexpr (kOut == kOutBool) {
    // doc 64c + i at byte 64c + i; the lane's u32 holds docs 0-31 (odd
    // lanes) or 32-63 (even lanes) of column lane >> 1
    c.base = static_cast<char*>(a.out) + bundle * kDocsPerBundle;
    c.row_bytes = a.out_cols * 64;
    c.lane_off = static_cast<uint32_t>((lane >> 1) * 64 + ((lane & 1) ? 0 : 32));
  } else {
    c.base = static_cast<char*>(a.out) + bundle * 256;
    c.row_bytes = a.out_cols * 8;
    c.lane_off = static_cast<uint32_t>(lane) * 4u;
  }
  c.count_mask = 0u;
  if constexpr (kOut == kOutCounts) {
    // The lane's u32 is half (lane & 1) of little-endian word lane >> 1: odd
    // lanes hold the word's high half (docs 0-31), even lanes docs 32-63.
    const int64_t first_doc =
        bundle * kDocsPerBundle + (lane >> 1) * kBitsPerColumn + ((lane & 1) ? 0 : 32);
    c.count_mask = valid_doc_mask(first_doc, a.num_docs);
  }
  return c;
}

// Stores this lane's 32-bit half of output row `row` on the bundle (and the
// row's match count on the bundle in kOutCounts mode).
template <int kOut>
__device__ __forceinline__ void store_result(const SearchArgs& a, const OutCursor& c, int lane,
                                             int64_t bundle, uint32_t row, uint32_t acc) {
  // The row's base is computed in scalar registers and kept there (the empty
  // asm), so the store takes the scalar-base + per-lane-offset form.
  const uint64_t addr = reinterpret_cast<uint64_t>(c.base) +
                        static_cast<uint64_t>(row) * static_cast<uint64_t>(c.row_bytes);
  uint32_t lo = static_cast<uint32_t>(addr), hi = static_cast<uint32_t>(addr >> 32);
  asm volatile("" : "+s"(lo), "+s"(hi));
  ST_GLOBAL char* row_base = (ST_GLOBAL char*)((static_cast<uint64_t>(hi) << 32) | lo);
  if constexpr (kOut == kOutBool) {
    store_bool32(row_base + c.lane_off, acc);
  } else {
    __builtin_nontemporal_store(acc, (ST_GLOBAL uint32_t*)(row_base + c.lane_off));
  }
  if constexpr (kOut == kOutCounts) {
    const uint32_t n = wave_total_small(static_cast<uint32_t>(__builtin_popcount(acc & c.count_mask)));
    if (lane == 0) a.counts[static_cast<int64_t>(row) * a.num_bundles + bundle] = n;
  }
}

// ------------------------------------------------- literal stream, quad lanes
//
// When a batch's literal stream fits the LDS area after the tile and a step
// holds at least four records (k <= 7), the stream of the bundle's width slot
// is staged in LDS with the tile and evaluated four programs at a time: lane
// l serves slot 4 * quad + (l >> 4) of the round and owns bytes
// 16 * (l & 15) .. +15 of every row, so one 16-byte LDS read per lane fetches
// a row for four programs at once, each 16-lane group reading its own
// record.  Per literal and four programs that is one record read, k row reads
// and their address adds, and the OR-of-ANDs fold on four words.

// Record words, u32x4 per record, records per step and quads per step.
template <int K>
struct QuadShape {
  static constexpr int RW = ((K + 1 + 3) / 4) * 4;
  static constexpr int RV = RW / 4;
  static constexpr int NB = 32 / RW;
  static constexpr int NQ = NB / 4;
};

// LDS words a staged literal stream may take (the area after the tile).
constexpr uint32_t kQuadStreamMaxWords = kSearchPosSlots;
// u32x4 registers per thread that carry a stream of that size.
constexpr int kStreamPrefetch = (kQuadStreamMaxWords / 4 + kSearchThreads - 1) / kSearchThreads;

__device__ __forceinline__ uint32_t u32x4_get(const u32x4& v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

// Stores this lane's 16 bytes of packed output row `row` on the bundle (and,
// in kOutCounts mode, the row's match count on the bundle, summed over the
// lane's 16-lane group; called with the whole group active).  The u32s are, in order, the low and high halves of
// words 2s and 2s + 1 (s = lane & 15); a word's high half holds its first 32
// docs.
template <int kOut>
__device__ __forceinline__ void store_quad(const SearchArgs& a, int lane, int64_t bundle,
                                           uint32_t row, u32x4 v) {
  const uint32_t s = static_cast<uint32_t>(lane & 15);
  static_assert(kOut != kOutBool, "bool output of a quad goes through store_quad_bool");
  ST_GLOBAL u32x4* dst = (ST_GLOBAL u32x4*)(static_cast<char*>(a.out) +
                                            static_cast<int64_t>(row) * (a.out_cols * 8) +
                                            bundle * 256 + s * 16);
  __builtin_nontemporal_store(v, dst);
  if constexpr (kOut == kOutCounts) {
    uint32_t n;
    if ((bundle + 1) * kDocsPerBundle <= a.num_docs) {  // every doc of the bundle counts
      n = __builtin_popcount(v.x) + __builtin_popcount(v.y) + __builtin_popcount(v.z) +
          __builtin_popcount(v.w);
    } else {
      const int64_t first = bundle * kDocsPerBundle + static_cast<int64_t>(s) * 128;
      n = __builtin_popcount(v.y & valid_doc_mask(first, a.num_docs)) +
          __builtin_popcount(v.x & valid_doc_mask(first + 32, a.num_docs)) +
          __builtin_popcount(v.w & valid_doc_mask(first + 64, a.num_docs)) +
          __builtin_popcount(v.z & valid_doc_mask(first + 96, a.num_docs));
    }
    // the 16-lane group is one DPP row: its last lane holds the group's sum
    n = row16_inclusive_sum(n);
    if (s == 15) a.counts[static_cast<int64_t>(row) * a.num_bundles + bundle] = n;
  }
}

// Bool output of a quad: the four 2 KB rows of the wave's four programs,
// each written as two 1 KB stores of 16 consecutive bytes per lane (plain
// stores: at cfg2, whose bool output is 2.56 GB against 563 MB of index,
// they measured 633-639 us against 646-649 us non-temporal).  Lane l
// of a store covers docs 1024 j + 16 l .. +15, i.e. one half of a packed
// 32-doc word that sits in another lane of the program's group: the four
// components of that lane are fetched with ds_bpermute and the lane's one is
// kept.  Called by all lanes (the permutes need the whole wave).
__device__ __forceinline__ void store_quad_bool(const SearchArgs& a, int lane, int64_t bundle,
                                                uint32_t info, u32x4 v) {
  const uint32_t t = ((static_cast<uint32_t>(lane) >> 1) ^ 1u) & 3u;  // component wanted
  const uint32_t shift = (lane & 1) * 16;                             // docs 0-15 or 16-31
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const uint32_t gi = __builtin_amdgcn_readlane(info, 16 * g);
    if (!(gi & kSlotValid)) continue;
    ST_GLOBAL char* base = (ST_GLOBAL char*)(static_cast<char*>(a.out) +
                                             static_cast<int64_t>(gi >> kSlotRowShift) *
                                                 (a.out_cols * 64) +
                                             bundle * kDocsPerBundle);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int src = 16 * g + (((32 * j + (lane >> 1)) ^ 1) >> 2);
      const int addr = src * 4;
      const uint32_t c0 = __builtin_amdgcn_ds_bpermute(addr, v.x);
      const uint32_t c1 = __builtin_amdgcn_ds_bpermute(addr, v.y);
      const uint32_t c2 = __builtin_amdgcn_ds_bpermute(addr, v.z);
      const uint32_t c3 = __builtin_amdgcn_ds_bpermute(addr, v.w);
      const uint32_t p = t == 0 ? c0 : (t == 1 ? c1 : (t == 2 ? c2 : c3));
      const uint32_t y = __builtin_bitreverse32(p) >> shift;
      u32x4 o;
      o.x = ((y & 0xFu) * 0x00204081u) & 0x01010101u;
      o.y = (((y >> 4) & 0xFu) * 0x00204081u) & 0x01010101u;
      o.z = (((y >> 8) & 0xFu) * 0x00204081u) & 0x01010101u;
      o.w = (((y >> 12) & 0xFu) * 0x00204081u) & 0x01010101u;
      *(ST_GLOBAL u32x4*)(base + 1024 * j + 16 * lane) = o;
    }
  }
}

// Evaluates a wave's rounds of the LDS-staged literal stream `sw`, words
// [w_begin, w_end), on the bundle in the LDS tile.  Layout as the scalar
// path reads it (search_plan.hpp): per round a 16-word header (T, slot infos
// from word kRoundSlotInfo), then T steps of NB records of RW words.
template <int K, bool MASKS, int kOut>
__device__ __forceinline__ void eval_quads(const SearchArgs& a, const u32x4* tile,
                                           const uint32_t* sw, uint32_t w_begin,
                                           uint32_t w_end, int64_t bundle, int lane,
                                           PartFilter pf) {
  using S = QuadShape<K>;
  const int g = lane >> 4;
  const char* tb = reinterpret_cast<const char*>(tile) + (lane & 15) * 16;
  for (uint32_t w = w_begin; w < w_end;) {
    const uint32_t* hdr = sw + w;
    const uint32_t T = uniform(hdr[0]);
    if (!pf.take()) {  // another workgroup's share of a split bundle
      w += kRoundHeaderWords + T * S::NB * S::RW;
      continue;
    }
#pragma unroll
    for (int qd = 0; qd < S::NQ; ++qd) {
      const uint32_t info = hdr[kRoundSlotInfo + qd * 4 + g];
      u32x4 res{0, 0, 0, 0}, acc{0, 0, 0, 0};
      const u32x4* rec =
          reinterpret_cast<const u32x4*>(hdr + kRoundHeaderWords) + (qd * 4 + g) * S::RV;
      for (uint32_t j = 0; j < T; ++j, rec += S::NB * S::RV) {
        u32x4 r[S::RV];
#pragma unroll
        for (int v = 0; v < S::RV; ++v) r[v] = rec[v];
        u32x4 t = *reinterpret_cast<const u32x4*>(tb + u32x4_get(r[0], 0));
#pragma unroll
        for (int k = 1; k < K; ++k)
          t &= *reinterpret_cast<const u32x4*>(tb + u32x4_get(r[k >> 2], k & 3));
        const uint32_t f = u32x4_get(r[K >> 2], K & 3);
        if constexpr (MASKS) {  // f is the group mask; nothing is negated
          res |= acc & f;
          acc = (acc | f) & t;
        } else {
          const uint32_t neg = 0u - (f & kStreamNeg);
          const uint32_t grp = 0u - ((f >> 1) & 1u);
          res |= acc & grp;
          acc = (acc | grp) & (t ^ neg);
        }
      }
      u32x4 v = res | acc;
      if (info & kSlotComplement) v = ~v;
      if constexpr (kOut == kOutBool) {
        store_quad_bool(a, lane, bundle, info, v);
      } else if (info & kSlotValid) {
        store_quad<kOut>(a, lane, bundle, info >> kSlotRowShift, v);
      }
    }
    w += kRoundHeaderWords + T * S::NB * S::RW;
  }
}

// Evaluates a wave's rounds of the literal stream, words [w_begin, w_end):
// per step, one record of each of the NB slots arrives with scalar loads,
// then all NB * K row words are read from the tile, then the NB independent
// OR-of-ANDs folds run; the round's results are stored after its last step.
// No per-query decoding and no per-literal branches.
template <int K, bool STAGED, bool MASKS, int kOut>
__device__ __forceinline__ void eval_rounds(const SearchArgs& a, const RowSource& rs,
                                            const ST_CONST uint32_t* stream, uint32_t w_begin,
                                            uint32_t w_end, int64_t bundle, PartFilter pf) {
  constexpr int RW = ((K + 1 + 3) / 4) * 4;
  constexpr int NB = 32 / RW;  // slots per round
  const OutCursor oc = out_cursor<kOut>(a, rs.lane, bundle);
  for (uint32_t w = w_begin; w < w_end;) {
    const ST_CONST uint32_t* hdr = stream + w;
    const uint32_t T = hdr[0];
    if (!pf.take()) {  // another workgroup's share of a split bundle
      w += kRoundHeaderWords + T * NB * RW;
      continue;
    }
    uint32_t info[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) info[i] = hdr[kRoundSlotInfo + i];
    const ST_CONST uint32_t* step = hdr + kRoundHeaderWords;
    uint32_t res[NB], acc[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) res[i] = acc[i] = 0;
    for (uint32_t j = 0; j < T; ++j, step += NB * RW) {
      uint32_t rec[NB][K + 1];
#pragma unroll
      for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int v = 0; v <= K; ++v) rec[i][v] = step[i * RW + v];
      uint32_t t[NB];
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        uint32_t x = ~0u;
#pragma unroll
        for (int k = 0; k < K; ++k) x &= row_word<STAGED>(rs, rec[i][k]);
        t[i] = x;
      }
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const uint32_t f = rec[i][K];
        if constexpr (MASKS) {  // f is the group mask; nothing is negated
          res[i] |= acc[i] & f;
          acc[i] = (acc[i] | f) & t[i];
        } else {
          const uint32_t neg = 0u - (f & kStreamNeg);
          const uint32_t grp = 0u - ((f >> 1) & 1u);
          res[i] |= acc[i] & grp;
          acc[i] = (acc[i] | grp) & (t[i] ^ neg);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      if (info[i] & kSlotValid) {
        uint32_t v = res[i] | acc[i];
        if (info[i] & kSlotComplement) v = ~v;
        store_result<kOut>(a, oc, rs.lane, bundle, info[i] >> kSlotRowShift, v);
      }
    }
    w += kRoundHeaderWords + T * NB * RW;
  }
}

// Evaluates this wave's queries [s_begin, s_end) on one bundle and stores
// their 32-bit halves of the bundle's 32 output words.
// LITE (the quad instance, whose prefetch registers leave less room):
// programs one by one, literals in groups of G, no fully unrolled forms.
template <int K, int KP, bool STAGED, bool BOUND, int G, int kOut, bool LITE = false>
__device__ __forceinline__ void eval_queries(const SearchArgs& a, const RowSource& rs,
                                             uint32_t s_begin, uint32_t s_end,
                                             int64_t bundle, uint32_t slot, PartFilter pf) {
  const int lane = rs.lane;
  const OutCursor oc = out_cursor<kOut>(a, lane, bundle);
  auto store = [&](uint32_t row, uint32_t acc) {
    store_result<kOut>(a, oc, lane, bundle, row, acc);
  };
  if constexpr (BOUND) {
    constexpr int RW = ((K + 1 + 3) / 4) * 4;
    const ST_CONST uint32_t* progs = a.bound + static_cast<uint64_t>(slot) * a.bound_words;
    for (uint32_t s = s_begin; s < s_end;) {
      const ST_CONST uint32_t* prog = progs + a.bound_start[s];
      const uint32_t hdr = prog[0];
      const uint32_t T = hdr & 0xFFFFu;
      if (!pf.take()) {  // another workgroup's share of a split bundle
        s += (!LITE && (hdr & kPairedWithNext)) ? 2 : 1;
        continue;
      }
      if (!LITE && (hdr & kPairedWithNext)) {
        const ST_CONST uint32_t* prog_b = progs + a.bound_start[s + 1];
        const uint32_t hdr_b = prog_b[0];
        uint32_t acc_a, acc_b;
        if (!eval_bound_pair<K, STAGED>(rs, prog + kProgHeaderWords, prog_b + kProgHeaderWords,
                                        T, acc_a, acc_b)) {
          acc_a = eval_bound_flat_loop<K, STAGED, G>(rs, prog + kProgHeaderWords, T);
          acc_b = eval_bound_flat_loop<K, STAGED, G>(rs, prog_b + kProgHeaderWords, T);
        }
        if (hdr & kFlatComplement) acc_a = ~acc_a;
        if (hdr_b & kFlatComplement) acc_b = ~acc_b;
        store(prog[1], acc_a);
        store(prog_b[1], acc_b);
        s += 2;
        continue;
      }
      uint32_t acc;
      if (hdr & kFlatForm) {
        if constexpr (LITE)
          acc = eval_bound_flat_loop<K, STAGED, G>(rs, prog + kProgHeaderWords, T);
        else
          acc = eval_bound_flat<K, STAGED, G>(rs, prog + kProgHeaderWords, T);
        if (hdr & kFlatComplement) acc = ~acc;
      } else {
        acc = eval_bound_stack<K, KP, STAGED, G>(rs, prog, T, prog[2]);
      }
      store(prog[1], acc);
      ++s;
    }
    (void)RW;
    return;
  }
  const ST_CONST uint32_t* progs = a.insns;
  const ST_CONST uint32_t* starts = a.insn_start;
  for (uint32_t s = s_begin; s < s_end; ++s) {
    if (!pf.take()) continue;  // another workgroup's share of a split bundle
    const ST_CONST uint32_t* prog = progs + starts[s];
    const uint32_t hdr = prog[0];
    const uint32_t row = prog[1];
    const uint32_t T = hdr & 0xFFFFu;
    uint32_t acc;
    if (hdr & kFlatForm) {
      const ST_CONST u32x4* lits = reinterpret_cast<const ST_CONST u32x4*>(prog + kProgHeaderWords);
      if constexpr (LITE)
        acc = eval_flat_loop<K, KP, STAGED, G>(rs, lits, T);
      else
        acc = eval_flat<K, KP, STAGED, G>(rs, lits, T);
      if (hdr & kFlatComplement) acc = ~acc;
    } else {
      acc = eval_stack<K, KP, STAGED, G>(rs, prog, T, prog[2]);
    }
    store(row, acc);
  }
}

template <int K>
__device__ __forceinline__ void wide_phase(
    u32x4* tile, const int64_t* __restrict__ index, int64_t index_numel,
    const int64_t* __restrict__ bundle_offsets, int64_t num_bundles,
    const uint32_t* __restrict__ bundle_slot, const uint32_t* __restrict__ bundle_order,
    const uint32_t* __restrict__ blob, const uint32_t* __restrict__ table, int64_t out_cols,
    int64_t* __restrict__ out);

// The arrays arrive as separate __restrict__ parameters (not inside
// SearchArgs) so the compiler can prove the output stores never alias the
// program and offset arrays and fetch those with scalar loads.
template <int K, int kOut, bool kQuad>
__global__ __launch_bounds__(kSearchThreads) void bloom_search_kernel(
    const int64_t* __restrict__ index, int64_t index_numel,
    const int64_t* __restrict__ bundle_offsets, int64_t num_bundles,
    const uint32_t* __restrict__ wave_off,
    const uint32_t* __restrict__ insn_start, const uint32_t* __restrict__ insns,
    const uint64_t* __restrict__ hashes, const uint32_t* __restrict__ bundle_slot,
    const uint32_t* __restrict__ bundle_order,
    const uint32_t* __restrict__ bound_start, const uint32_t* __restrict__ bound,
    uint32_t bound_words, const uint32_t* __restrict__ stream_wave,
    const uint32_t* __restrict__ stream_skip, uint32_t stream_off, uint32_t stream_words,
    uint32_t stream_masks,
    uint32_t num_terms, int32_t hash_k,
    int64_t out_cols, void* __restrict__ out, int64_t* __restrict__ counts, int64_t num_docs,
    uint32_t wide_skip, const uint32_t* __restrict__ census,
    const uint32_t* __restrict__ wide_table, const uint32_t* __restrict__ wide_order,
    const uint32_t* __restrict__ blob) {
  // wide_skip == 2: the wide-bundle phase evaluates every program of this
  // batch on wide bundles; census[1] (device binding) says every bundle is
  // one, so the search phase has nothing to do; 3: the host knows so
  const bool search_phase =
      wide_skip != 3 && !(wide_skip == 2 && census != nullptr && as_const(census)[1] != 0u);
  SearchArgs a;
  a.index = index;
  a.index_numel = index_numel;
  a.bundle_offsets = as_const(bundle_offsets);
  a.num_bundles = num_bundles;
  a.wave_off = as_const(wave_off);
  a.insn_start = as_const(insn_start);
  a.insns = as_const(insns);
  a.hashes = as_const(hashes);
  a.bundle_slot = as_const(bundle_slot);
  a.bundle_order = as_const(bundle_order);
  a.bound_start = as_const(bound_start);
  a.bound = as_const(bound);
  a.bound_words = bound_words;
  a.stream_off = stream_off;
  a.stream_words = stream_words;
  a.stream_masks = stream_masks;
  a.num_terms = num_terms;
  a.hash_k = hash_k;
  a.out_cols = out_cols;
  a.out = out;
  a.counts = counts;
  a.num_docs = num_docs;
  constexpr int KP = K <= 4 ? 4 : (K <= 8 ? 8 : 12);
  constexpr int G = KP == 4 ? 4 : (KP == 8 ? 2 : 1);  // terms fetched together
  constexpr int GL = G > 2 ? 2 : G;                    // the same, LITE
  __shared__ u32x4 tile[(kSearchTileRows + 2) * 16];
  __shared__ __attribute__((aligned(16))) uint32_t pos[kSearchPosSlots];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const uint32_t wave = uniform(tid >> 6);

  if (tid < 32) {
    const uint32_t fill = tid < 16 ? ~0u : 0u;
    tile[kSearchOnesRow * 16 + (tid & 15) + (tid & 16)] = u32x4{fill, fill, fill, fill};
  }

  // Bundle visited at step i of the grid-stride walk, with its extent and
  // width slot.  Each bundle's metadata is loaded one bundle ahead of its
  // tile prefetch, so that neither the prefetch nor the evaluation waits on
  // a chain of dependent scalar loads.
  auto meta_at = [&](int64_t i) -> BundleMeta {
    BundleMeta m;
    m.bundle = a.bundle_order ? static_cast<int64_t>(a.bundle_order[i]) : i;
    bundle_extent(a, m.bundle, m.start, m.b);
    m.slot = a.bundle_slot ? a.bundle_slot[m.bundle] : kNoWidthSlot;
    m.part = 0;
    m.parts = 1;
    return m;
  };
  const int64_t grid = gridDim.x;
  // Visit v of this workgroup: order index blockIdx.x + v * grid while every
  // workgroup has one; the `tail` bundles of the last, partial round are
  // split `parts` ways by program among the first tail * parts workgroups,
  // so that round takes a fraction of a bundle's time instead of a whole one.
  const int64_t full = a.num_bundles / grid;
  const int64_t tail = a.num_bundles - full * grid;
  const int64_t parts = tail > 0 ? min<int64_t>(grid / tail, kTailParts) : 1;
  auto visit = [&](int64_t v) -> BundleMeta {
    if (v < full) return meta_at(blockIdx.x + v * grid);
    if (v == full && static_cast<int64_t>(blockIdx.x) < tail * parts) {
      BundleMeta m = meta_at(full * grid + blockIdx.x % tail);
      m.part = static_cast<uint32_t>(blockIdx.x / tail);
      m.parts = static_cast<uint32_t>(parts);
      return m;
    }
    return BundleMeta{-1, 0, 0, kNoWidthSlot, 0, 1};
  };
  // Quad-lane evaluation of the literal stream (eval_quads): the batch's
  // stream fits the LDS area after the tile and a step holds whole quads.
  const bool quad = kQuad && a.stream_words != 0 && a.stream_words <= kQuadStreamMaxWords &&
                    QuadShape<K>::NB >= 4;
  auto quad_bundle = [&](const BundleMeta& m) {
    return quad && m.slot != kNoWidthSlot && m.b <= kSearchTileRows;
  };
  // This thread's share of a quad bundle's stream, loaded with its tile.
  auto prefetch_stream = [&](const BundleMeta& m, u32x4 (&sp)[kQuad ? kStreamPrefetch : 1]) {
    const u32x4* src = reinterpret_cast<const u32x4*>(
        bound + static_cast<uint64_t>(m.slot) * a.bound_words + a.stream_off);
    const uint32_t chunks = a.stream_words / 4;
#pragma unroll
    for (int i = 0; i < (kQuad ? kStreamPrefetch : 1); ++i) {
      const uint32_t c = static_cast<uint32_t>(tid) + static_cast<uint32_t>(i) * kSearchThreads;
      sp[i] = c < chunks ? src[c] : u32x4{0, 0, 0, 0};
    }
  };
  u32x4 pre[kPrefetch];
  u32x4 spre[kQuad ? kStreamPrefetch : 1];
  const BundleMeta none{-1, 0, 0, kNoWidthSlot, 0, 1};
  BundleMeta cur = search_phase ? visit(0) : none, nxt = search_phase ? visit(1) : none;
  if (cur.bundle >= 0) {
    prefetch_tile(a, cur.start, cur.b, pre);
    if (quad_bundle(cur)) prefetch_stream(cur, spre);
  }

  int64_t prev_b = -1;  // width whose term positions are in pos
  uint32_t staged_slot = kNoWidthSlot;  // width slot whose literal stream is in pos
  const uint32_t s_begin = uniform(a.wave_off[wave]);
  const uint32_t s_end = uniform(a.wave_off[wave + 1]);
  const bool streamed = a.stream_words != 0;
  const uint32_t r_begin = streamed ? uniform(stream_wave[wave]) : 0u;
  const uint32_t r_end = streamed ? uniform(stream_wave[wave + 1]) : 0u;
  // the flat programs the stream covers are the wave's first ones
  const uint32_t s_rest = s_begin + (streamed ? uniform(stream_skip[wave]) : 0u);
  const char* tile_lane = reinterpret_cast<const char*>(tile) + lane * 4;
  const uint32_t* index32 = reinterpret_cast<const uint32_t*>(a.index);

  uint32_t warm = 0;  // scalar-cache warming loads of the next stream (see below)
  for (int64_t v = 0; cur.bundle >= 0; ++v) {
    const int64_t bundle = cur.bundle;
    const PartFilter pf{cur.part, cur.parts, 0u};
    const int64_t start = cur.start, b = cur.b;
    const uint32_t slot = cur.slot;
    const bool staged = b <= kSearchTileRows;

    const bool quad_here = quad_bundle(cur);
    // the wide-bundle kernel evaluates the literal stream of this bundle
    const bool wide_here = wide_skip != 0 && slot != kNoWidthSlot && wide_width(b);
    // ... and every program of this batch is in the stream: nothing to do here
    const bool skip = wide_here && wide_skip == 2;

    if (!skip) __syncthreads();  // previous bundle's readers are done with tile and pos
    if (staged) {
      const int64_t chunks = b * 16;
#pragma unroll
      for (int i = 0; i < kPrefetch; ++i) {
        const int c = tid + i * kSearchThreads;
        if (c < chunks) tile[c] = pre[i];
      }
    }
    if (quad_here && slot != staged_slot) {  // the stream goes where unbound bundles keep positions
      const uint32_t chunks = a.stream_words / 4;
      u32x4* dst = reinterpret_cast<u32x4*>(pos);
#pragma unroll
      for (int i = 0; i < (kQuad ? kStreamPrefetch : 1); ++i) {
        const uint32_t c = static_cast<uint32_t>(tid) + static_cast<uint32_t>(i) * kSearchThreads;
        if (c < chunks) dst[c] = spre[i];
      }
      staged_slot = slot;
      prev_b = -1;
    }
    // the positions of an unbound bundle replace the staged stream below
    if (!skip && slot == kNoWidthSlot && b != prev_b) staged_slot = kNoWidthSlot;
    // The next bundle's loads go out as soon as this thread's registers are
    // in LDS, before the barrier, so the HBM queue is not left empty while the
    // workgroup finishes storing the tile.  Its stream is loaded only when
    // another slot's is in LDS.
    const bool has_next = nxt.bundle >= 0;
    if (has_next) {
      prefetch_tile(a, nxt.start, nxt.b, pre);
      if (quad_bundle(nxt) && nxt.slot != staged_slot) prefetch_stream(nxt, spre);
    }
    if (!skip && slot == kNoWidthSlot && b != prev_b) {
      const FastMod64 fm = make_fastmod_dev(static_cast<uint64_t>(b));
      for (uint32_t u = tid; u < a.num_terms; u += kSearchThreads) {
        int16_t found[K];
#pragma unroll
        for (int j = 0; j < K; ++j) found[j] = 0;
        int cnt = 0;
        if (b > 0) cnt = resolve_positions<K>(a.hashes + static_cast<uint64_t>(u) * a.hash_k,
                                              a.hash_k, fm, found);
        uint32_t* dst = pos + u * KP;
#pragma unroll
        for (int j = 0; j < KP; ++j) {
          const int16_t r = (j < K && j < cnt) ? found[j < K ? j : 0] : found[0];
          uint32_t v;
          if (staged) {
            v = (cnt == 0 ? kSearchZerosRow : static_cast<int>(r)) * 256u;
          } else {
            v = cnt == 0 ? static_cast<uint32_t>(kPosZeros)
                         : static_cast<uint32_t>(static_cast<int32_t>(r));
          }
          dst[j] = v;
        }
      }
      prev_b = b;
    }
    if (!skip) __syncthreads();
    asm volatile("" ::"s"(warm));  // the warming loads are complete by now

    const BundleMeta after = visit(v + 2);

    // Evaluate this wave's queries on the bundle.
    RowSource rs;
    rs.pos = pos;
    rs.tile_lane = tile_lane;
    rs.index32 = index32;
    rs.index_numel = a.index_numel;
    rs.start = start;
    rs.b = b;
    rs.lane = lane;
    rs.staged = staged;
    if (skip) {
      // evaluated by the wide-bundle kernel
    } else if constexpr (kQuad) {
      // Quad instance: stream programs of staged slot bundles in quads, all
      // other bundles' programs from the width block one by one.
      if (quad_here) {
        if (a.stream_masks)
          eval_quads<K, true, kOut>(a, tile, pos, r_begin, r_end, bundle, lane, pf);
        else
          eval_quads<K, false, kOut>(a, tile, pos, r_begin, r_end, bundle, lane, pf);
        eval_queries<K, KP, true, true, GL, kOut, true>(a, rs, s_rest, s_end, bundle, slot, pf);
      } else if (slot != kNoWidthSlot) {
        if (staged)
          eval_queries<K, KP, true, true, GL, kOut, true>(a, rs, s_begin, s_end, bundle, slot, pf);
        else
          eval_queries<K, KP, false, true, GL, kOut, true>(a, rs, wide_here ? s_rest : s_begin,
                                                           s_end, bundle, slot, pf);
      } else if (staged) {
        eval_queries<K, KP, true, false, GL, kOut, true>(a, rs, s_begin, s_end, bundle, slot, pf);
      } else {
        eval_queries<K, KP, false, false, GL, kOut, true>(a, rs, s_begin, s_end, bundle, slot, pf);
      }
    } else if (slot != kNoWidthSlot) {
      const ST_CONST uint32_t* stream =
          a.bound + static_cast<uint64_t>(slot) * a.bound_words + a.stream_off;
      if (staged) {
        if (streamed) {
          if (a.stream_masks)
            eval_rounds<K, true, true, kOut>(a, rs, stream, r_begin, r_end, bundle, pf);
          else
            eval_rounds<K, true, false, kOut>(a, rs, stream, r_begin, r_end, bundle, pf);
        }
        eval_queries<K, KP, true, true, G, kOut>(a, rs, s_rest, s_end, bundle, slot, pf);
      } else {
        if (streamed && !wide_here) {
          if (a.stream_masks)
            eval_rounds<K, false, true, kOut>(a, rs, stream, r_begin, r_end, bundle, pf);
          else
            eval_rounds<K, false, false, kOut>(a, rs, stream, r_begin, r_end, bundle, pf);
        }
        eval_queries<K, KP, false, true, G, kOut>(a, rs, s_rest, s_end, bundle, slot, pf);
      }
    } else if (staged) {
      eval_queries<K, KP, true, false, G, kOut>(a, rs, s_begin, s_end, bundle, slot, pf);
    } else {
      eval_queries<K, KP, false, false, G, kOut>(a, rs, s_begin, s_end, bundle, slot, pf);
    }
    // The next bundle's first round header and records (this wave's part of
    // its width block) are read into the scalar cache now; the loads complete
    // while the workgroup waits at the barriers and stores the next tile.
    warm = 0;
    if (!kQuad && has_next && streamed && nxt.slot != kNoWidthSlot && r_begin < r_end) {
      const ST_CONST uint32_t* w =
          a.bound + static_cast<uint64_t>(nxt.slot) * a.bound_words + a.stream_off + r_begin;
      // a round is a 16-word header and at least one 32-word step
      warm = w[0] ^ w[kRoundHeaderWords] ^ w[kRoundHeaderWords + 16];
    }
    cur = nxt;
    nxt = after;
  }
  // The wide-bundle phase (packed output, k <= 7) of the call's last search
  // launch: skipped at once when the census found no wide slot width.
  if constexpr (kOut == kOutPacked && K <= 7) {
    if (wide_table != nullptr && (census == nullptr || as_const(census)[2] != 0u)) {
      __syncthreads();  // the search phase's readers are done with the LDS
      wide_phase<K>(reinterpret_cast<u32x4*>(tile), index, index_numel, bundle_offsets, num_bundles,
                    bundle_slot, wide_order, blob, wide_table, out_cols, static_cast<int64_t*>(out));
    }
  }
}

// ------------------------------------------------ wide bundles, column slices
//
// Width-bound bundles of kSearchTileRows < b <= kWideRows rows do not fit the
// LDS tile.  bloom_wide_kernel searches them in kWideSlices column slices:
// the slice's 64 bytes of every row (512 docs) are staged in LDS, followed by
// the all-ones and all-zeros rows (kWideOnesRow, kWideZerosRow), and the
// literal streams of every batch are evaluated on it 16 programs per wave
// instruction: the four lanes of quad p serve program p of the wave's current
// group (round p / NB, slot p % NB), each owning 16 bytes of every slice row
// (one 16-byte LDS read per row position).  The quad loads its program's
// stream record together (a quarter each; values reach the other lanes by
// DPP, fused into the LDS address add) from the width block in global
// memory, shared by every bundle of the width and so L2-resident, three
// steps ahead.  The index is read once per search, whatever the number of
// batches.  Packed output only.

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
constexpr int kWidePieces = kWideSliceBytes / 16;  // u32x4 per slice row
constexpr int kWidePrefetch = kWideRows * kWidePieces / kSearchThreads;
static_assert(kWidePrefetch * kSearchThreads == kWideRows * kWidePieces, "slice split");
static_assert((kWideRows + 2) * kWidePieces <= (kSearchTileRows + 2) * 16,
              "the search kernel's LDS tile holds the wide phase's slice tile");

// LDS pointers (address space 3): reads through them are ds_read, and a
// byte offset added to one is a 32-bit add.
#define ST_LDS __attribute__((address_space(3)))

// Word i of a quad's stream record as every lane of the quad sees it: lane q
// holds words WPL * q .. WPL * q + WPL - 1, and the value moves by DPP
// (quad_perm broadcast, with bound_ctrl so that a following add absorbs
// the move).
template <int WPL>
__device__ __forceinline__ uint32_t quad_word(const uint32_t (&r)[WPL], int i) {
  const uint32_t v = r[i % WPL];
  switch (i / WPL) {
    case 0: return __builtin_amdgcn_mov_dpp(v, 0x00, 0xF, 0xF, true);
    case 1: return __builtin_amdgcn_mov_dpp(v, 0x55, 0xF, 0xF, true);
    case 2: return __builtin_amdgcn_mov_dpp(v, 0xAA, 0xF, 0xF, true);
    default: return __builtin_amdgcn_mov_dpp(v, 0xFF, 0xF, 0xF, true);
  }
}

// 3-input bitwise functions (v_bitop3_b32 truth tables over a = 0xF0,
// b = 0xCC, c = 0xAA).
__device__ __forceinline__ uint32_t and_xor(uint32_t a, uint32_t b, uint32_t c) {
  return __builtin_amdgcn_bitop3_b32(a, b, c, 0x6A);  // (a & b) ^ c
}
__device__ __forceinline__ uint32_t or_and(uint32_t a, uint32_t b, uint32_t c) {
  return __builtin_amdgcn_bitop3_b32(a, b, c, 0xA8);  // (a | b) & c
}
__device__ __forceinline__ uint32_t or_andb(uint32_t a, uint32_t b, uint32_t c) {
  return __builtin_amdgcn_bitop3_b32(a, b, c, 0xF8);  // a | (b & c)
}

// One literal step of a lane's program: K row positions (slice-tile byte
// offsets) and the flags from the quad's record, K LDS reads of the lane's
// 16 bytes, the OR-of-ANDs fold.
template <int K, bool MASKS, int WPL>
__device__ __forceinline__ void wide_step(const uint32_t (&r)[WPL], const ST_LDS char* tile_lane,
                                          u32x4& res, u32x4& acc) {
  u32x4 row[K];
#pragma unroll
  for (int k = 0; k < K; ++k)
    row[k] = *reinterpret_cast<const ST_LDS u32x4*>(tile_lane + quad_word<WPL>(r, k));
  const uint32_t f = quad_word<WPL>(r, K);
  u32x4 t = row[0];
#pragma unroll
  for (int k = 1; k + 1 < K; ++k) t &= row[k];
  // negated literal (mask neg) folded into the last AND; group mask g
  const uint32_t neg = MASKS ? 0u : 0u - (f & kStreamNeg);
  const uint32_t g = MASKS ? f : 0u - ((f >> 1) & 1u);
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    uint32_t tc = u32x4_get(t, c);
    if constexpr (K > 1)
      tc = MASKS ? (tc & u32x4_get(row[K - 1], c)) : and_xor(tc, u32x4_get(row[K - 1], c), neg);
    else if constexpr (!MASKS)
      tc ^= neg;
    const uint32_t ac = u32x4_get(acc, c), rc = u32x4_get(res, c);
    const uint32_t nres = or_andb(rc, ac, g);
    const uint32_t nacc = or_and(ac, g, tc);
    if (c == 0) { res.x = nres; acc.x = nacc; }
    if (c == 1) { res.y = nres; acc.y = nacc; }
    if (c == 2) { res.z = nres; acc.z = nacc; }
    if (c == 3) { res.w = nres; acc.w = nacc; }
  }
}

// One group of 16 programs on the staged slice: each lane folds its
// program's literals over its 16 bytes and stores them to output row
// (info >> kSlotRowShift).  `stream` is the batch's stream in this bundle's
// width block; `out_lane` the lane's byte address in output row 0.  The loop
// runs the group's longest round (its first) with uniform control; a lane
// whose round is shorter repeats its last record, which leaves the
// OR-of-ANDs fold unchanged.  Each lane loads its share of the record three
// steps ahead into one of three buffers.
template <int K, bool MASKS>
__device__ __forceinline__ void wide_eval_group(const char* stream, const ST_CONST uint32_t* grp,
                                                const ST_LDS char* tile_lane, int lane,
                                                int64_t row_bytes, char* out_lane) {
  using S = QuadShape<K>;
  constexpr int WPL = S::RW / 4;  // record words per lane
  constexpr int kRounds = kWidePrograms / S::NB;
  constexpr uint32_t kStepBytes = S::NB * S::RW * 4;  // 128
  const int pg = lane >> 2;
  const int rr = pg / S::NB;
  const int sl = pg % S::NB;
  uint32_t roff = grp[2], T = grp[2 + kWideMaxRounds];
#pragma unroll
  for (int i = 1; i < kRounds; ++i) {
    if (rr == i) {
      roff = grp[2 + i];
      T = grp[2 + kWideMaxRounds + i];
    }
  }
  const bool valid = roff != ~0u;
  if (!valid) {  // compute on a real round, store nothing
    roff = grp[2];
    T = grp[2 + kWideMaxRounds];
  }
  const uint32_t rb = roff * 4;
  const uint32_t info = *reinterpret_cast<const uint32_t*>(stream + rb + (kRoundSlotInfo + sl) * 4);
  const uint32_t steps = grp[1];
  const uint32_t o_first = rb + kRoundHeaderWords * 4 + sl * S::RW * 4 + (lane & 3) * WPL * 4;
  const uint32_t o_last = o_first + (T > 0 ? T - 1 : 0) * kStepBytes;
  uint32_t o = o_first;
  typedef uint32_t Share[WPL];
  auto next = [&](Share& r) {
    if constexpr (WPL == 1) {
      r[0] = *reinterpret_cast<const uint32_t*>(stream + o);
    } else {
      const u32x2 v = *reinterpret_cast<const u32x2*>(stream + o);
      r[0] = v.x;
      r[1] = v.y;
    }
    o = min(o + kStepBytes, o_last);
  };
  Share b0, b1, b2;
  next(b0);
  next(b1);
  next(b2);
  u32x4 res{0, 0, 0, 0}, acc{0, 0, 0, 0};
  // whole triples with a branch-free body (loads stay three steps ahead),
  // then the one or two steps left
  uint32_t j = 0;
  for (; j + 3 <= steps; j += 3) {
    wide_step<K, MASKS, WPL>(b0, tile_lane, res, acc);
    next(b0);
    wide_step<K, MASKS, WPL>(b1, tile_lane, res, acc);
    next(b1);
    wide_step<K, MASKS, WPL>(b2, tile_lane, res, acc);
    next(b2);
  }
  if (j < steps) wide_step<K, MASKS, WPL>(b0, tile_lane, res, acc);
  if (j + 1 < steps) wide_step<K, MASKS, WPL>(b1, tile_lane, res, acc);
  u32x4 v = res | acc;
  if (info & kSlotComplement) v = ~v;
  // A plain (cached) store: the pair's other workgroup writes the other
  // 64-byte half of the same 128-byte output line at about the same time,
  // and the halves can meet in L2 (non-temporal stores went out as partial
  // lines: 3% slower at cfg3).
  if (valid && (info & kSlotValid))
    *(ST_GLOBAL u32x4*)(out_lane + static_cast<int64_t>(info >> kSlotRowShift) * row_bytes) = v;
}

// Grid: 1024-thread workgroups, one per CU.  When the grid is a multiple
// of 16, workgroups w and w + 8 (dispatched to the same XCD) form a pair
// that walks the wide bundles p, p + grid / 2, ... of the visiting order
// `bundle_order` (bundles grouped by width slot, so that the workgroups
// working at one time share the slot's literal stream in L2), one member
// taking slices 0 and 2, the other 1 and 3, so the two halves of each
// 128-byte index line are read by the same XCD at about the same time;
// otherwise workgroup w takes bundles w, w + grid, ... with all slices.  Each
// wave issues its share of the next slice's loads when it has evaluated the
// current one.  `tile` is the workgroup's LDS (kWideRows + 2 slice rows); the
// phase runs as a kernel of its own (bloom_wide_kernel) or after the search
// phase of a packed search launch (bloom_search_kernel), saving the call a
// launch.
template <int K>
__device__ __forceinline__ void wide_phase(
    u32x4* tile, const int64_t* __restrict__ index, int64_t index_numel,
    const int64_t* __restrict__ bundle_offsets, int64_t num_bundles,
    const uint32_t* __restrict__ bundle_slot, const uint32_t* __restrict__ bundle_order,
    const uint32_t* __restrict__ blob, const uint32_t* __restrict__ table, int64_t out_cols,
    int64_t* __restrict__ out) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const uint32_t wave = uniform(tid >> 6);
  const ST_CONST int64_t* boff = as_const(bundle_offsets);
  const ST_CONST uint32_t* bslot = as_const(bundle_slot);
  const ST_CONST uint32_t* border = as_const(bundle_order);
  const ST_CONST uint32_t* tab = as_const(table);

  if (tid < 2 * kWidePieces) {
    const uint32_t fill = tid < kWidePieces ? ~0u : 0u;
    tile[kWideOnesRow * kWidePieces + tid] = u32x4{fill, fill, fill, fill};
  }
  const uint32_t nbt = tab[0];
  const uint32_t g_begin = uniform(tab[4 + wave]), g_end = uniform(tab[5 + wave]);
  const ST_CONST uint32_t* batches = tab + kWideTableHead;
  const ST_CONST uint32_t* groups = batches + 4 * nbt;
  const int64_t grid = gridDim.x;
  const bool paired = grid % 16 == 0;
  const int64_t first = paired ? (blockIdx.x >> 4) * 8 + (blockIdx.x & 7) : blockIdx.x;
  const int64_t stride = paired ? grid / 2 : grid;
  const int s_first = paired ? static_cast<int>((blockIdx.x >> 3) & 1) : 0;
  const int s_step = paired ? 2 : 1;

  // first wide bundle at or after visiting position i on this workgroup's
  // stride: (position, bundle), position num_bundles when there is none
  auto next_wide = [&](int64_t i, int64_t& bnd) -> int64_t {
    for (; i < num_bundles; i += stride) {
      bnd = border[i];
      const int64_t b = boff[bnd + 1] - boff[bnd];
      if (bslot[bnd] != kNoWidthSlot && wide_width(b)) return i;
    }
    return num_bundles;
  };
  const u32x4* src = reinterpret_cast<const u32x4*>(index);
  auto prefetch = [&](int64_t bnd, int slice, u32x4 (&pre)[kWidePrefetch]) {
    const int64_t start = boff[bnd];
    const int64_t b = boff[bnd + 1] - start;
#pragma unroll
    for (int i = 0; i < kWidePrefetch; ++i) {
      const int c = tid + i * kSearchThreads;
      const int64_t row = c / kWidePieces;
      const int64_t word = (start + row) * 32 + slice * (kWideSliceBytes / 8) +
                           (c % kWidePieces) * 2;
      pre[i] = u32x4{0, 0, 0, 0};
      if (row < b && word >= 0 && word + 1 < index_numel) pre[i] = src[word / 2];
    }
  };

  int64_t cbnd = 0;  // bundle at visiting position cp
  int64_t cp = next_wide(first, cbnd);
  if (cp >= num_bundles) return;
  int cs = s_first;
  u32x4 pre[kWidePrefetch];
  prefetch(cbnd, cs, pre);
  const ST_LDS char* tile_lane = (const ST_LDS char*)(tile) + (lane & 3) * 16;
  const int64_t row_bytes = out_cols * 8;
  for (;;) {
    const int64_t cb = cbnd;
    const int64_t b = boff[cb + 1] - boff[cb];
    const uint32_t slot = bslot[cb];
    int64_t np = cp, nbnd = cb;
    int ns = cs + s_step;
    if (ns >= kWideSlices) {
      np = next_wide(cp + stride, nbnd);
      ns = s_first;
    }
    const bool has_next = np < num_bundles;
    __syncthreads();  // the previous slice's readers are done
#pragma unroll
    for (int i = 0; i < kWidePrefetch; ++i) {
      const int c = tid + i * kSearchThreads;
      if (c < b * kWidePieces) tile[c] = pre[i];
    }
    __syncthreads();
    char* out_lane =
        reinterpret_cast<char*>(out) + cb * 256 + cs * kWideSliceBytes + (lane & 3) * 16;
    for (uint32_t g = g_begin; g < g_end; ++g) {
      const ST_CONST uint32_t* grp = groups + static_cast<uint64_t>(g) * kWideGroupWords;
      const ST_CONST uint32_t* bt = batches + 4 * grp[0];
      const char* stream = reinterpret_cast<const char*>(
          blob + bt[0] + static_cast<uint64_t>(slot) * bt[1] + bt[2]);
      if (bt[3])
        wide_eval_group<K, true>(stream, grp, tile_lane, lane, row_bytes, out_lane);
      else
        wide_eval_group<K, false>(stream, grp, tile_lane, lane, row_bytes, out_lane);
    }
    // The next slice's loads go out after this wave's evaluation: issued
    // earlier, every wait for a stream record (in-order vmcnt) would also
    // wait for them.
    if (has_next) prefetch(nbnd, ns, pre);
    if (!has_next) break;
    cp = np;
    cbnd = nbnd;
    cs = ns;
  }
}

// The wide-bundle evaluation as a launch of its own (when no search launch
// of the call carries it).  `num_slots` (device binding; nullptr when the
// host decided to launch) lets it return at once when no slot width is wide
// (its word 2).
template <int K>
__global__ __launch_bounds__(kSearchThreads) void bloom_wide_kernel(
    const int64_t* __restrict__ index, int64_t index_numel,
    const int64_t* __restrict__ bundle_offsets, int64_t num_bundles,
    const uint32_t* __restrict__ bundle_slot, const uint32_t* __restrict__ bundle_order,
    const uint32_t* __restrict__ num_slots, const uint32_t* __restrict__ blob,
    const uint32_t* __restrict__ table, int64_t out_cols, int64_t* __restrict__ out) {
  __shared__ u32x4 tile[(kWideRows + 2) * kWidePieces];
  if (num_slots != nullptr && as_const(num_slots)[2] == 0u) return;
  wide_phase<K>(tile, index, index_numel, bundle_offsets, num_bundles, bundle_slot, bundle_order,
                blob, table, out_cols, out);
}

}  // namespace

using WideFn = void (*)(const int64_t*, int64_t, const int64_t*, int64_t, const uint32_t*,
                        const uint32_t*, const uint32_t*, const uint32_t*, const uint32_t*, int64_t,
                        int64_t*);
// The wide-bundle kernel of one K (nullptr for K > 7), defined in the
// translation unit compiled with ST_SEARCH_K = K.
template <int K>
WideFn wide_kernel_for();
template <> WideFn wide_kernel_for<1>();
template <> WideFn wide_kernel_for<2>();
template <> WideFn wide_kernel_for<3>();
template <> WideFn wide_kernel_for<4>();
template <> WideFn wide_kernel_for<5>();
template <> WideFn wide_kernel_for<6>();
template <> WideFn wide_kernel_for<7>();
template <> WideFn wide_kernel_for<8>();
template <> WideFn wide_kernel_for<9>();
template <> WideFn wide_kernel_for<10>();

using KernelFn = void (*)(const int64_t*, int64_t, const int64_t*, int64_t,
                          const uint32_t*, const uint32_t*,
                          const uint32_t*, const uint64_t*, const uint32_t*,
                          const uint32_t*, const uint32_t*, const uint32_t*, uint32_t,
                          const uint32_t*, const uint32_t*, uint32_t, uint32_t, uint32_t,
                          uint32_t, int32_t,
                          int64_t, void*, int64_t*, int64_t, uint32_t, const uint32_t*,
                          const uint32_t*, const uint32_t*, const uint32_t*);

// The kernels of one K (all output modes; the quad instance evaluates the
// literal stream in quad lanes and needs a stream that fits the LDS and k <= 7),
// defined in the translation unit compiled with ST_SEARCH_K = K.
template <int K>
KernelFn search_kernel_for(int mode, bool quad);
template <> KernelFn search_kernel_for<1>(int mode, bool quad);
template <> KernelFn search_kernel_for<2>(int mode, bool quad);
template <> KernelFn search_kernel_for<3>(int mode, bool quad);
template <> KernelFn search_kernel_for<4>(int mode, bool quad);
template <> KernelFn search_kernel_for<5>(int mode, bool quad);
template <> KernelFn search_kernel_for<6>(int mode, bool quad);
template <> KernelFn search_kernel_for<7>(int mode, bool quad);
template <> KernelFn search_kernel_for<8>(int mode, bool quad);
template <> KernelFn search_kernel_for<9>(int mode, bool quad);
template <> KernelFn search_kernel_for<10>(int mode, bool quad);

}  // namespace st
