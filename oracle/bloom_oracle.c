/*
 * bloom_oracle.c -- CPU restatement of the reference bloom retrieval path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * implementation in silvertorch_amd/.  Only tests/, __graft_entry__.smoke()
 * and the cpu_baseline leg of bench.py may load it; the product never does.
 *
 * It restates, single-threaded and in plain C, the reference CPU algorithm
 * (paths relative to silvertorch/ops/csrc/ of the reference tree):
 *   or_murmur3_pair        bloom_index_util.cuh:59-106
 *   or_build_positions     bloom_index_util.cuh:183-207
 *   or_bundle_b_offsets    bloom_indexer.cpp:43-70
 *   or_bloom_build         bloom_indexer.cpp:72-110
 *   or_search_batch        bloom_index_search.cpp:27-171 (signature_match,
 *                          run_query_plan) and :173-243 (the q x column loop)
 *   or_partial_response    bloom_index_search.cpp:246-395 (the cluster-
 *                          restricted search: per (query, cluster) the
 *                          columns covering the cluster's docs)
 *   or_unpack_bool         bloom_index_search.cpp:231-236
 *   or_compact             README.md:191 (mask[:, :num_docs].nonzero())
 *   or_filtered_topk       no reference op; top-k by (score desc, id asc) of
 *                          fp64 dot products over filter-passing docs
 *
 * Pinning (what each function is checked against, see tests/):
 *   murmur      sklearn's independent MurmurHash3_x64_128 vectors
 *               (tests/golden/murmur_x64_128.json) and the reference build.
 *   positions   brute force from the hash; reference golden fixtures.
 *   build       reference CPU build (oracle/_ref) golden fixtures, README
 *               known answers, invariants (exact bit counts per doc).
 *   search      reference CPU search golden fixtures, README known answers,
 *               bitwise identities (De Morgan, EMPTY = all ones).
 *   partial     reference CPU partial-response golden fixtures; every
 *               returned column equals the full search's word there.
 *   compact     numpy nonzero on the unpacked mask.
 *   topk        brute-force numpy sort on tiny inputs.
 * Defined where the reference is undefined (the HIP kernels do the same):
 *   a search term in a bundle of width 0 matches nothing (reference divides
 *   by zero); a row index that falls outside the index reads as zero.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define OR_COLS 32
#define OR_BITS 64
#define OR_DOCS_PER_BUNDLE 2048
#define OR_MAX_SEARCH_K 10
#define OR_MAX_BUILD_K 64

enum { OR_AND = 1, OR_OR = 2, OR_NOT = 3, OR_TERM = 4, OR_EMPTY = 5 };

static uint64_t rotl(uint64_t v, int r) { return (v << r) | (v >> (64 - r)); }

static uint64_t fmix(uint64_t h) {
  h ^= h >> 33;
  h *= 0xff51afd7ed558ccdULL;
  h ^= h >> 33;
  h *= 0xc4ceb9fe1a85ec53ULL;
  h ^= h >> 33;
  return h;
}

/* MurmurHash3_x64_128 of the 16-byte key LE(x) || LE(y) under `seed`,
 * folded to h1 ^ h2 (bloom_index_util.cuh:59-106). */
uint64_t or_murmur3_pair(uint64_t x, uint64_t y, uint64_t seed) {
  const uint64_t c1 = 0x87c37b91114253d5ULL;
  const uint64_t c2 = 0x4cf5ad432745937fULL;
  uint64_t h1 = seed, h2 = seed;
  uint64_t k1 = x * c1;
  k1 = rotl(k1, 31);
  k1 *= c2;
  h1 ^= k1;
  h1 = rotl(h1, 27);
  h1 += h2;
  h1 = h1 * 5 + 0x52dce729ULL;
  uint64_t k2 = y * c2;
  k2 = rotl(k2, 33);
  k2 *= c1;
  h2 ^= k2;
  h2 = rotl(h2, 31);
  h2 += h1;
  h2 = h2 * 5 + 0x38495ab5ULL;
  h1 ^= 16; /* key length */
  h2 ^= 16;
  h1 += h2;
  h2 += h1;
  h1 = fmix(h1);
  h2 = fmix(h2);
  h1 += h2;
  h2 += h1;
  return h1 ^ h2;
}

/* First k distinct murmur(fid, value, seed) % b over seeds 0, 1, 2, ...
 * (bloom_index_util.cuh:183-207).  Returns 0, or -1 if the arguments could
 * not terminate (b < k with k > 0, or b <= 0). */
int or_build_positions(int64_t fid, int64_t value, int64_t b, int64_t k,
                       int32_t* out) {
  if (k <= 0) return 0;
  if (b <= 0 || b < k) return -1;
  int64_t n = 0;
  uint64_t seed = 0;
  while (n < k) {
    uint64_t p = or_murmur3_pair((uint64_t)fid, (uint64_t)value, seed++) % (uint64_t)b;
    int dup = 0;
    for (int64_t j = 0; j < n; ++j) dup |= ((uint64_t)out[j] == p);
    if (!dup) out[n++] = (int32_t)p;
  }
  return 0;
}

/* bundle_b_offsets[nb + 1] from the jagged offsets (bloom_indexer.cpp:43-70):
 * b_i = (int64)((double)(max over docs of the bundle of the doc's term count
 * times k) * b_multiplier). */
void or_bundle_b_offsets(const int64_t* offsets, int64_t num_docs,
                         int64_t num_features, int64_t k, double b_multiplier,
                         int64_t* out) {
  const int64_t nb = (num_docs + OR_DOCS_PER_BUNDLE - 1) / OR_DOCS_PER_BUNDLE;
  out[0] = 0;
  for (int64_t i = 0; i < nb; ++i) {
    int64_t best = 0;
    for (int64_t d = i * OR_DOCS_PER_BUNDLE;
         d < (i + 1) * OR_DOCS_PER_BUNDLE && d < num_docs; ++d) {
      int64_t cnt = 0;
      for (int64_t f = 0; f < num_features; ++f)
        cnt += offsets[d * num_features + f + 1] - offsets[d * num_features + f];
      if (cnt > best) best = cnt;
    }
    out[i + 1] = out[i] + (int64_t)((double)(best * k) * b_multiplier);
  }
}

/* Sets every term's k bits (bloom_indexer.cpp:72-110).  `index` holds
 * bundle_b_offsets[nb] * 32 words and is zeroed here.  Returns 0 or -1. */
int or_bloom_build(const int32_t* feature_ids, const int64_t* offsets,
                   const int64_t* values, int64_t num_features,
                   int64_t num_docs, int64_t k, const int64_t* bundle_b_offsets,
                   int64_t* index) {
  if (k < 0 || k > OR_MAX_BUILD_K) return -1;
  const int64_t nb = (num_docs + OR_DOCS_PER_BUNDLE - 1) / OR_DOCS_PER_BUNDLE;
  memset(index, 0, sizeof(int64_t) * (size_t)bundle_b_offsets[nb] * OR_COLS);
  int32_t pos[OR_MAX_BUILD_K];
  for (int64_t d = 0; d < num_docs; ++d) {
    const int64_t bundle = d / OR_DOCS_PER_BUNDLE;
    const int64_t col = (d % OR_DOCS_PER_BUNDLE) / OR_BITS;
    const uint64_t bit = 1ULL << (63 - d % OR_BITS);
    const int64_t start = bundle_b_offsets[bundle];
    const int64_t b = bundle_b_offsets[bundle + 1] - start;
    for (int64_t f = 0; f < num_features; ++f) {
      const int64_t fid = (int64_t)feature_ids[f];
      for (int64_t j = offsets[d * num_features + f];
           j < offsets[d * num_features + f + 1]; ++j) {
        if (or_build_positions(fid, values[j], b, k, pos) != 0) return -1;
        for (int64_t t = 0; t < k; ++t)
          index[(start + pos[t]) * OR_COLS + col] |= (int64_t)bit;
      }
    }
  }
  return 0;
}

/* ------------------------------------------------------------------ search */

typedef struct {
  const uint8_t* ops;
  int64_t n_ops;
  const uint8_t* offsets; /* int32 entries, possibly unaligned */
  int64_t n_offsets;
  const uint8_t* hashes; /* uint64 entries */
  int64_t n_hashes;
} or_plan;

static int32_t rd_i32(const uint8_t* p) {
  int32_t v;
  memcpy(&v, p, 4);
  return v;
}
static uint64_t rd_u64(const uint8_t* p) {
  uint64_t v;
  memcpy(&v, p, 8);
  return v;
}

/* TERM word of one column (signature_match, bloom_index_search.cpp:40-61):
 * positions are (int16)(h[p] % b) over p < hash_k, first k distinct kept. */
static uint64_t term_word(const int64_t* index, int64_t index_numel,
                          int64_t start, int64_t b, int64_t col_in_bundle,
                          const uint8_t* h, int64_t k, int64_t hash_k) {
  uint64_t r = ~0ULL;
  if (b <= 0) return (k > 0 && hash_k > 0) ? 0 : r;
  int16_t used[OR_MAX_SEARCH_K];
  int64_t n = 0;
  for (int64_t p = 0; p < hash_k && n < k; ++p) {
    const int16_t bp = (int16_t)(rd_u64(h + 8 * p) % (uint64_t)b);
    int dup = 0;
    for (int64_t j = 0; j < n; ++j) dup |= (used[j] == bp);
    if (dup) continue;
    used[n++] = bp;
    const int64_t w = (start + bp) * OR_COLS + col_in_bundle;
    r &= (w >= 0 && w < index_numel) ? (uint64_t)index[w] : 0;
  }
  return r;
}

/* Stack evaluation of one plan on one column (run_query_plan,
 * bloom_index_search.cpp:72-171).  Returns 0 or -1 on a malformed plan. */
static int eval_plan(const or_plan* pl, const int64_t* index,
                     int64_t index_numel, int64_t start, int64_t b,
                     int64_t col_in_bundle, int64_t k, int64_t hash_k,
                     uint64_t* stack, uint64_t* result) {
  int64_t sp = 0, term = 0;
  for (int64_t i = 0; i < pl->n_ops; ++i) {
    const uint8_t op = pl->ops[i];
    int32_t children = 0;
    if (op == OR_AND || op == OR_OR || op == OR_NOT) {
      if (i + 1 >= pl->n_offsets) return -1;
      children = rd_i32(pl->offsets + 4 * (i + 1)) - rd_i32(pl->offsets + 4 * i);
    }
    switch (op) {
      case OR_TERM: {
        if (hash_k > 0 && k > 0 && (term + 1) * hash_k > pl->n_hashes) return -1;
        const uint8_t* h = pl->hashes + 8 * term * (hash_k > 0 ? hash_k : 0);
        stack[sp++] = term_word(index, index_numel, start, b, col_in_bundle, h,
                                k, hash_k);
        ++term;
        break;
      }
      case OR_AND:
      case OR_OR: {
        uint64_t v = op == OR_AND ? ~0ULL : 0;
        for (int32_t j = 0; j < children; ++j) {
          if (sp == 0) return -1;
          v = op == OR_AND ? (v & stack[--sp]) : (v | stack[--sp]);
        }
        stack[sp++] = v;
        break;
      }
      case OR_NOT:
        if (children != 1 || sp == 0) return -1;
        stack[sp - 1] = ~stack[sp - 1];
        break;
      case OR_EMPTY:
        stack[sp++] = ~0ULL;
        break;
      default:
        return -1;
    }
  }
  if (sp == 0) return -1;
  *result = stack[sp - 1];
  return 0;
}

/* The four byte ranges of one encoded plan (bloom_index_util.cpp:81-124:
 * operators, child-count offsets, parameters, hashes); -1 when a range lies
 * outside plans_data. */
static int decode_plan(const int8_t* plans_data, int64_t plans_data_len,
                       const int64_t* o, or_plan* pl) {
  for (int j = 0; j < 8; j += 2)
    if (o[j] < 0 || o[j] > o[j + 1] || o[j + 1] > plans_data_len) return -1;
  pl->ops = (const uint8_t*)plans_data + o[0];
  pl->n_ops = o[1] - o[0];
  pl->offsets = (const uint8_t*)plans_data + o[2];
  pl->n_offsets = (o[3] - o[2]) / 4;
  pl->hashes = (const uint8_t*)plans_data + o[6];
  pl->n_hashes = (o[7] - o[6]) / 8;
  return 0;
}

/* Packed search: out[q * (nb * 32) + c] for every plan q and column c
 * (bloom_index_search.cpp:173-243 with return_bool_mask = false).
 * Returns 0, or -1 - q for the first malformed plan q. */
int or_search_batch(const int64_t* index, int64_t index_numel,
                    const int64_t* bundle_b_offsets, int64_t num_bundles,
                    const int8_t* plans_data, int64_t plans_data_len,
                    const int64_t* plans_offsets, int64_t num_plans, int64_t k,
                    int64_t hash_k, int64_t* out) {
  if (k > OR_MAX_SEARCH_K && hash_k > OR_MAX_SEARCH_K) return -1;
  const int64_t C = num_bundles * OR_COLS;
  for (int64_t q = 0; q < num_plans; ++q) {
    or_plan pl;
    if (decode_plan(plans_data, plans_data_len, plans_offsets + 8 * q, &pl) != 0)
      return -1 - (int)q;
    uint64_t* stack = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)(pl.n_ops + 1));
    if (!stack) return -1 - (int)q;
    for (int64_t c = 0; c < C; ++c) {
      const int64_t bundle = c / OR_COLS;
      const int64_t start = bundle_b_offsets[bundle];
      int64_t b = bundle_b_offsets[bundle + 1] - start;
      if (b < 0) b = 0;
      uint64_t r;
      if (eval_plan(&pl, index, index_numel, start, b, c % OR_COLS, k, hash_k,
                    stack, &r) != 0) {
        free(stack);
        return -1 - (int)q;
      }
      out[q * C + c] = (int64_t)r;
    }
    free(stack);
  }
  return 0;
}

/* Cluster-restricted search (bloom_index_search_common_return_partial_response,
 * bloom_index_search.cpp:246-395).  For row q and cluster c of the
 * [rows, clusters] arrays: first column start / 64 (C++ truncation),
 * first_offsets[q, c] = (int8)(start % 64), ncol = length > 0 ?
 * (length + offset + 63) / 64 : 0 columns, cumsum[q, c] the running int32
 * column total, and mask[...] the plan's word on each of those columns, in
 * (q, c, column) order.  The plan is plan_index[q] when plan_index is given,
 * else q.  Where the reference reads out of bounds this returns an error:
 * -1 a plan index outside [0, num_plans), -2 a column outside the index,
 * -3 an int32 running total overflow, -4 capacity too small (*total still
 * set), -5 a malformed plan. */
int or_partial_response(const int64_t* index, int64_t index_numel,
                        const int64_t* bundle_b_offsets, int64_t num_bundles,
                        const int8_t* plans_data, int64_t plans_data_len,
                        const int64_t* plans_offsets, int64_t num_plans, int64_t k,
                        int64_t hash_k, const int64_t* cluster_offsets,
                        const int64_t* cluster_lengths, int64_t rows,
                        int64_t clusters, const int64_t* plan_index,
                        int32_t* cumsum, int8_t* first_offsets, int64_t* mask,
                        int64_t capacity, int64_t* total) {
  const int64_t C = num_bundles * OR_COLS;
  int64_t acc = 0;
  *total = 0;
  for (int64_t q = 0; q < rows; ++q) {
    for (int64_t c = 0; c < clusters; ++c) {
      const int64_t start = cluster_offsets[q * clusters + c];
      const int64_t length = cluster_lengths[q * clusters + c];
      const int8_t off = (int8_t)(start % OR_BITS);
      const int64_t first_col = start / OR_BITS;
      const int64_t ncol = length > 0 ? (length + off + OR_BITS - 1) / OR_BITS : 0;
      first_offsets[q * clusters + c] = off;
      acc += ncol;
      if (acc > INT32_MAX) return -3;
      cumsum[q * clusters + c] = (int32_t)acc;
      if (ncol == 0) continue;
      if (first_col < 0 || first_col + ncol > C) return -2;
      const int64_t p = plan_index ? plan_index[q] : q;
      if (p < 0 || p >= num_plans) return -1;
      or_plan pl;
      if (decode_plan(plans_data, plans_data_len, plans_offsets + 8 * p, &pl) != 0) return -5;
      uint64_t* stack = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)(pl.n_ops + 1));
      if (!stack) return -5;
      for (int64_t j = 0; j < ncol; ++j, ++*total) {
        if (*total >= capacity) continue;
        const int64_t col = first_col + j;
        const int64_t bundle = col / OR_COLS;
        const int64_t bstart = bundle_b_offsets[bundle];
        int64_t b = bundle_b_offsets[bundle + 1] - bstart;
        if (b < 0) b = 0;
        uint64_t r;
        if (eval_plan(&pl, index, index_numel, bstart, b, col % OR_COLS, k, hash_k, stack,
                      &r) != 0) {
          free(stack);
          return -5;
        }
        mask[*total] = (int64_t)r;
      }
      free(stack);
    }
  }
  return *total > capacity ? -4 : 0;
}

/* Bool mask from the packed words: mask[q, 64c + i] = bit (63 - i). */
void or_unpack_bool(const int64_t* packed, int64_t rows, int64_t cols,
                    uint8_t* mask) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c) {
      const uint64_t w = (uint64_t)packed[r * cols + c];
      for (int i = 0; i < OR_BITS; ++i)
        mask[(r * cols + c) * OR_BITS + i] = (uint8_t)((w >> (63 - i)) & 1);
    }
}

/* Ascending matching doc ids below num_docs per query, CSR layout:
 * ids[row_offsets[q] .. row_offsets[q+1]).  `ids` must hold the total match
 * count (pass NULL to only fill row_offsets). */
void or_compact(const int64_t* packed, int64_t rows, int64_t cols,
                int64_t num_docs, int64_t* row_offsets, int64_t* ids) {
  int64_t n = 0;
  row_offsets[0] = 0;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c = 0; c < cols; ++c) {
      const uint64_t w = (uint64_t)packed[r * cols + c];
      for (int i = 0; i < OR_BITS; ++i) {
        const int64_t d = c * OR_BITS + i;
        if (d < num_docs && ((w >> (63 - i)) & 1)) {
          if (ids) ids[n] = d;
          ++n;
        }
      }
    }
    row_offsets[r + 1] = n;
  }
}

/* ----------------------------------------------------------- filtered top-k */

typedef struct {
  double score;
  int64_t id;
} or_scored;

static int by_score_then_id(const void* a, const void* b) {
  const or_scored* x = (const or_scored*)a;
  const or_scored* y = (const or_scored*)b;
  if (x->score > y->score) return -1;
  if (x->score < y->score) return 1;
  return (x->id > y->id) - (x->id < y->id);
}

/* For every query q: score[d] = sum_j emb[d, j] * qv[q, j] in fp64 over docs
 * d < num_docs whose packed filter bit is set; top `topk` by (score desc,
 * id asc); missing entries are id -1, score -inf.  emb / qv are fp32 copies
 * of the bf16 inputs. */
int or_filtered_topk(const float* emb, int64_t num_docs, int64_t dim,
                     const float* qv, int64_t num_queries,
                     const int64_t* packed, int64_t cols, int64_t topk,
                     int64_t* out_ids, float* out_scores) {
  or_scored* buf = (or_scored*)malloc(sizeof(or_scored) * (size_t)(num_docs > 0 ? num_docs : 1));
  if (!buf) return -1;
  for (int64_t q = 0; q < num_queries; ++q) {
    int64_t n = 0;
    for (int64_t d = 0; d < num_docs; ++d) {
      const uint64_t w = (uint64_t)packed[q * cols + d / OR_BITS];
      if (!((w >> (63 - d % OR_BITS)) & 1)) continue;
      double s = 0.0;
      for (int64_t j = 0; j < dim; ++j)
        s += (double)emb[d * dim + j] * (double)qv[q * dim + j];
      buf[n].score = s;
      buf[n].id = d;
      ++n;
    }
    qsort(buf, (size_t)n, sizeof(or_scored), by_score_then_id);
    for (int64_t t = 0; t < topk; ++t) {
      out_ids[q * topk + t] = t < n ? buf[t].id : -1;
      out_scores[q * topk + t] = t < n ? (float)buf[t].score : -INFINITY;
    }
  }
  free(buf);
  return 0;
}
