/*
 * silvertorch_hip.h -- C ABI of the MI355X (gfx950) bloom-index retrieval path.
 *
 * Plain pointers and sizes only; no torch types.  Every device pointer is a
 * HIP device allocation on the current device, and every `stream` argument is
 * a hipStream_t passed as void* (NULL = the legacy default stream).  Work is
 * enqueued on that stream and ordered with the caller's other work on it.
 *
 * Status convention: every function returning int returns 0 on success and a
 * negative code on failure; st_last_error() then returns a message for the
 * calling thread (valid until that thread's next call into this library).
 *
 * Reference interfaces replaced (paths relative to the reference tree
 * silvertorch/ops/csrc/):
 *   st::bloom_index_build             bloom_indexer.cpp:115-125 (schema),
 *                                     bloom_indexer.cpp:26-113 (CPU impl),
 *                                     bloom_indexer_cuda.cu:880-904 (CUDA impl)
 *   st::bloom_index_search_batch      bloom_index_search.cpp:549-558 (schema),
 *                                     bloom_index_search.cpp:378-395 (CPU impl),
 *                                     bloom_index_search_cuda.cu:1031-1109 (CUDA)
 *   st::parse_expression_query_batch  expression_query_parser.cpp:456-472
 *   st::generate_column_info_for_clusters
 *                                     bloom_index_search.cpp:489-540, :543-547
 *   st::take_top_k_and_gather_from_main_and_fresh
 *                                     fresh_index_post_processing.cpp:231-287
 */
#ifndef SILVERTORCH_HIP_H_
#define SILVERTORCH_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ST_OK 0
#define ST_ERR_INVALID_ARGUMENT (-1)
#define ST_ERR_HIP (-2)
#define ST_ERR_UNSUPPORTED (-3)

/* Geometry of the bloom index (bloom_index_util.h:41-45 of the reference). */
#define ST_BITS_PER_COLUMN 64
#define ST_COLUMNS_PER_BUNDLE 32
#define ST_DOCS_PER_BUNDLE 2048
/* Largest number of distinct positions a search term may resolve
 * (MAX_K_V2, bloom_index_util.h:45). */
#define ST_MAX_SEARCH_K 10
/* Largest k the build accepts (MAX_K, bloom_index_util.h:39). */
#define ST_MAX_BUILD_K 64

/* Message describing the last failure on the calling thread. */
const char* st_last_error(void);

/* Library version string. */
const char* st_version(void);

/* ---------------------------------------------------------------------------
 * Hash.  MurmurHash3_x64_128 of the 16-byte key LE(x)||LE(y) with both lanes
 * seeded by `seed`, folded as h1 ^ h2.  Host-side twin of the device routine
 * the kernels use; replaces murmur_hash3_2x64 (bloom_index_util.cuh:59-106).
 * ------------------------------------------------------------------------- */
uint64_t st_murmur_hash3_2x64(uint64_t x, uint64_t y, uint64_t seed);

/* ---------------------------------------------------------------------------
 * Build, step 1 of 2: per-bundle bloom widths.
 *
 * Replaces the width pass of bloom_index_build (bloom_indexer.cpp:43-70 and
 * bloom_indexer_cuda.cu:253-389):
 *   b_i = (int64)((double)(max_{doc in bundle i} terms(doc) * k) * b_multiplier)
 *   bundle_b_offsets[0] = 0, bundle_b_offsets[i+1] = bundle_b_offsets[i] + b_i
 *
 *   feature_offsets   device int64[num_docs * num_features + 1]
 *   bundle_b_offsets  device int64[ceil(num_docs / 2048) + 1]      (output)
 *   stats             device int64[6]                              (output)
 *                     stats[0] = total rows (bundle_b_offsets[last]),
 *                     stats[1] = largest single-bundle width,
 *                     stats[2] = 1 if feature_offsets ever decreases, else 0,
 *                     stats[3] = feature_offsets[0],
 *                     stats[4] = feature_offsets[num_docs * num_features],
 *                     stats[5] = 0 (reserved).
 * The caller must check stats[2] == 0 and 0 <= stats[3] <= stats[4] <=
 * num_values before st_bloom_index_build; values outside [0, num_values) are
 * never read.
 * Requires num_features >= 1, num_docs >= 0, 0 <= k <= ST_MAX_BUILD_K and
 * b_multiplier > 1.0.
 * ------------------------------------------------------------------------- */
int st_bloom_build_bundle_offsets(const int64_t* feature_offsets,
                                  int64_t num_docs, int64_t num_features,
                                  int64_t k, double b_multiplier,
                                  int64_t* bundle_b_offsets, int64_t* stats,
                                  void* stream);

/* ---------------------------------------------------------------------------
 * Build, step 2 of 2: set the bloom bits.
 *
 * Replaces the scatter of bloom_index_build (bloom_indexer.cpp:72-110 and
 * bloom_indexer_cuda.cu:137-251 / :506-711).  For every doc d, feature slot f
 * and value v of that slot, the first k distinct murmur(feature_ids[f], v,
 * seed = 0, 1, 2, ...) % b positions p set bit (63 - d % 64) of
 *   bloom_index[(bundle_b_offsets[d / 2048] + p) * 32 + (d % 2048) / 64].
 *
 *   feature_ids       device int32[num_features]
 *   feature_offsets   device int64[num_docs * num_features + 1]
 *   feature_values    device int64[num_values]
 *   bundle_b_offsets  device int64[nb + 1] from st_bloom_build_bundle_offsets
 *   max_b             stats[1] of that call (host value)
 *   bloom_index       device int64[bloom_index_numel] (output, fully written;
 *                     bloom_index_numel must equal total rows * 32)
 * ------------------------------------------------------------------------- */
int st_bloom_index_build(const int32_t* feature_ids,
                         const int64_t* feature_offsets,
                         const int64_t* feature_values, int64_t num_features,
                         int64_t num_docs, int64_t num_values, int64_t k,
                         const int64_t* bundle_b_offsets, int64_t max_b,
                         int64_t* bloom_index, int64_t bloom_index_numel,
                         void* stream);

/* ---------------------------------------------------------------------------
 * Search plan: a host-side compilation of a batch of encoded query plans
 * (the plans_data / plans_offsets pair produced by
 * st::parse_expression_query_batch; format of bloom_index_util.cpp:81-124)
 * into the flat accumulator programs the search kernel runs.
 *
 * st_search_plan_create validates the plans exactly where the reference CPU
 * search would fail or read out of bounds (bloom_index_search.cpp:72-171):
 * unknown operators, NOT with a child count other than 1, stack underflow,
 * empty programs and hash reads past the plan's hash array are errors.
 *
 *   plans_data     host int8[plans_data_len]
 *   plans_offsets  host int64[plans_offsets_len], 8 per query
 *   k, hash_k      as passed to bloom_index_search_batch
 *
 * The blob (st_search_plan_blob, st_search_plan_blob_bytes bytes) must be
 * copied verbatim to device memory, which is then passed to
 * st_bloom_index_search_batch together with the plan.
 * ------------------------------------------------------------------------- */
typedef struct st_search_plan st_search_plan;

int st_search_plan_create(const int8_t* plans_data, int64_t plans_data_len,
                          const int64_t* plans_offsets,
                          int64_t plans_offsets_len, int64_t k, int64_t hash_k,
                          st_search_plan** out);
/* Optional, after create: binds the plan to an index's bundle widths.
 * bundle_b_offsets is a HOST copy of the index's int64[num_bundles + 1]
 * offsets.  The most frequent widths (up to 64) get programs whose term
 * references are replaced by the terms' row positions at that width, which
 * removes the per-bundle position step from the kernel; bundles of other
 * widths keep the unbound path.  A bound plan may only be used with an index
 * of num_bundles bundles.  Call at most once per plan. */
int st_search_plan_bind_widths(st_search_plan* plan,
                               const int64_t* bundle_b_offsets,
                               int64_t num_bundles);
/* Width binding on the device instead: the search call itself derives the
 * slots from the device bundle offsets (a census kernel) and expands
 * host-built width-independent templates (a fill kernel), so that no copy of
 * the bundle offsets to the host and no synchronisation is needed.  After
 * this call the device copy of the plan must hold
 * st_search_plan_device_bytes(plan) bytes: the first
 * st_search_plan_blob_bytes(plan) copied from st_search_plan_blob(plan), the
 * rest written by the search call.  Exclusive with
 * st_search_plan_bind_widths. */
int st_search_plan_prepare_device_binding(st_search_plan* plan,
                                          int64_t num_bundles);
int64_t st_search_plan_device_bytes(const st_search_plan* plan);
/* Optional: the search calls with this plan copy the blob into
 * plan_blob_device themselves, in their first kernel, from `pinned_host` --
 * pinned, device-accessible host memory (hipHostMalloc, e.g. a pinned torch
 * tensor), 16-byte aligned, holding st_search_plan_blob_bytes bytes of the
 * blob, unchanged until the stream has run the call.  The caller then does
 * not copy the blob.  No reference counterpart (the reference copies its
 * plans with two host-to-device copies per call,
 * bloom_index_search_cuda.cu:1043-1098). */
int st_search_plan_upload_source(st_search_plan* plan, const void* pinned_host);
/* Optional, with st_search_plan_upload_source: the search call's copy runs
 * in st_search_plan_upload_groups(plan) workgroups, and each workgroup g,
 * once its loads of `pinned_host` have returned, stores `value` to
 * pinned_words[g] (pinned, device-accessible host memory, 8-byte aligned,
 * that many words).  A caller that sees every word equal to `value` may
 * reuse `pinned_host` without an event on the stream.  Null turns it off.
 * No reference counterpart. */
int st_search_plan_upload_signal(st_search_plan* plan, void* pinned_words, uint64_t value);
int64_t st_search_plan_upload_groups(const st_search_plan* plan);
int64_t st_search_plan_num_queries(const st_search_plan* plan);
int64_t st_search_plan_blob_bytes(const st_search_plan* plan);
const void* st_search_plan_blob(const st_search_plan* plan);
void st_search_plan_destroy(st_search_plan* plan);

/* ---------------------------------------------------------------------------
 * Batched boolean search.  Replaces bloom_index_search_batch
 * (bloom_index_search.cpp:173-243, bloom_index_search_cuda.cu:575-615,
 * :940-1029).  With C = num_bundles * 32 columns:
 *   return_bool_mask == 0: out is device int64[Q, C], out[q, c] = the 64-bit
 *                          match word of column c (doc 64c+i is bit 63-i);
 *   return_bool_mask != 0: out is device bool (uint8)[Q, C * 64],
 *                          out[q, 64c + i] = bit (63 - i) of that word.
 * Docs past the real doc count are included, as in the reference.
 *
 *   bloom_index        device int64[bloom_index_numel]
 *   bundle_b_offsets   device int64[num_bundles + 1]
 *   plan_blob_device   device copy of st_search_plan_blob(plan)
 * ------------------------------------------------------------------------- */
int st_bloom_index_search_batch(const int64_t* bloom_index,
                                int64_t bloom_index_numel,
                                const int64_t* bundle_b_offsets,
                                int64_t num_bundles,
                                const st_search_plan* plan,
                                const void* plan_blob_device,
                                int return_bool_mask, void* out,
                                void* stream);

/* ---------------------------------------------------------------------------
 * Expression parser (host).  Replaces parse_expression_query_batch
 * (expression_query_parser.cpp:30-430): grammar of EXPRESSION_SYNTAX.md,
 * precedence NOT > AND > OR, runs of more than max_sub_queries operands
 * folded into nested operators, every term carrying hash_k murmur hashes
 * (seeds 0..hash_k-1), "" compiling to a single EMPTY operator.  The encoded
 * bytes are identical to the reference's.
 * ------------------------------------------------------------------------- */
typedef struct st_parsed_plans st_parsed_plans;

int st_parse_expression_query_batch(const char* const* expressions,
                                    int64_t num_expressions, int64_t hash_k,
                                    int return_query_plan,
                                    int64_t max_sub_queries,
                                    st_parsed_plans** out);
int64_t st_parsed_plans_max_stack(const st_parsed_plans* plans);
int64_t st_parsed_plans_data_bytes(const st_parsed_plans* plans);
const int8_t* st_parsed_plans_data(const st_parsed_plans* plans);
int64_t st_parsed_plans_offsets_len(const st_parsed_plans* plans);
const int64_t* st_parsed_plans_offsets(const st_parsed_plans* plans);
void st_parsed_plans_destroy(st_parsed_plans* plans);

/* ---------------------------------------------------------------------------
 * Cluster column geometry (companion op of the same operator surface).
 * Replaces generate_column_info_for_clusters (bloom_index_search.cpp:489-540,
 * bloom_index_search_cuda.cu:617-645).  For cluster i with first doc
 * offsets[i] and length lengths[i]:
 *   start_columns[i] = offsets[i] / 64, first_offsets[i] = offsets[i] % 64,
 *   column_counts[i] = lengths[i] > 0
 *       ? (lengths[i] + first_offsets[i] + 63) / 64 : 0.
 * All pointers are device pointers; n entries each.
 * ------------------------------------------------------------------------- */
int st_generate_column_info_for_clusters(const int64_t* offsets,
                                         const int64_t* lengths, int64_t n,
                                         int32_t* column_counts,
                                         int32_t* start_columns,
                                         int8_t* first_offsets, void* stream);

/* ---------------------------------------------------------------------------
 * Cluster-restricted search.  Replaces
 * bloom_index_search_batch_return_partial_response (bloom_index_search.cpp:
 * 246-418, bloom_index_search_cuda.cu:617-1648); the _multiple variant
 * (bloom_index_search.cpp:420-487) is the same per index chunk.  For row q and
 * cluster c of the HOST int64[rows, clusters] arrays cluster_offsets (first
 * doc) and cluster_lengths:
 *   first_offsets[q, c] = (int8)(offset % 64)  (C++ truncating division),
 *   ncol = length > 0 ? (length + first_offset + 63) / 64 : 0 columns from
 *   column offset / 64, column_counts_cumsum[q, c] = running int32 total;
 * the response holds, in (q, c, column) order, the 64-bit match word of plan
 * plan_index[q] (or q when plan_index is NULL) on each of those columns.
 *
 * st_search_plan_partial_items (host) validates the arrays and writes the
 * two host outputs above (rows * clusters entries each) and one work item per
 * cluster with columns into items (capacity rows * clusters), with the item
 * count and the response length (total columns).  Where the reference reads
 * out of bounds it fails: a plan index outside [0, queries), columns outside
 * [0, num_bundles * 32), an int32 running total that overflows.
 * st_bloom_index_search_partial then fills the device int64[total] response
 * from a device copy of the items and of st_search_plan_blob(plan); the plan
 * need not be width-bound (widths are resolved per column).
 * ------------------------------------------------------------------------- */
typedef struct st_partial_item {
  int64_t first_column;  /* first column of the cluster */
  int64_t out_offset;    /* first response entry */
  int32_t num_columns;
  uint32_t program;      /* word offset of the plan's program in the blob */
  uint32_t hashes;       /* uint64 offset of its batch's term hashes */
  uint32_t reserved;
} st_partial_item;

int st_search_plan_partial_items(const st_search_plan* plan,
                                 const int64_t* cluster_offsets,
                                 const int64_t* cluster_lengths, int64_t rows,
                                 int64_t clusters, const int64_t* plan_index,
                                 int64_t num_bundles,
                                 int32_t* column_counts_cumsum,
                                 int8_t* first_offsets, st_partial_item* items,
                                 int64_t* num_items, int64_t* total_columns);
int st_bloom_index_search_partial(const int64_t* bloom_index,
                                  int64_t bloom_index_numel,
                                  const int64_t* bundle_b_offsets,
                                  int64_t num_bundles,
                                  const st_search_plan* plan,
                                  const void* plan_blob_device,
                                  const st_partial_item* items_device,
                                  int64_t num_items, int64_t* out,
                                  void* stream);

/* ---------------------------------------------------------------------------
 * Compaction of matching doc ids.  No reference operator: the reference's
 * users call mask[:, :num_docs].nonzero() on the search output (README.md:
 * 191-193, :265-266 of the reference).  `packed` is a packed search output,
 * int64[num_queries, num_columns] (device).  The ids of query q are the
 * ascending d < num_docs whose bit is set, stored at
 * ids[row_offsets[q] .. row_offsets[q+1]).
 *   1. st_bloom_compact_offsets: counts and scans; writes row_offsets
 *      (device int64[num_queries + 1]) and the per-chunk output positions into
 *      `workspace` (device, st_bloom_compact_workspace_bytes bytes).
 *   2. the caller reads row_offsets[num_queries] (the total) and allocates ids.
 *   3. st_bloom_compact_ids: writes the ids (int32 unless ids_int64; int32
 *      requires doc ids below 2^31).  Needs the workspace of step 1 unchanged.
 * ------------------------------------------------------------------------- */
int64_t st_bloom_compact_workspace_bytes(int64_t num_queries, int64_t num_columns);
int st_bloom_compact_offsets(const int64_t* packed, int64_t num_queries,
                             int64_t num_columns, int64_t num_docs,
                             void* workspace, int64_t* row_offsets, void* stream);
/* Search plus step 1 of the compaction in one pass over the index: writes
 * the packed output int64[num_queries, 32 * num_bundles] to packed_out, the
 * per-(query, bundle) match counts of docs < num_docs into the workspace
 * (st_bloom_compact_workspace_bytes(num_queries, 32 * num_bundles) bytes) and
 * scans them into row_offsets, as st_bloom_compact_offsets would.  Step 3 is
 * st_bloom_compact_ids on packed_out with the same workspace. */
int st_bloom_index_search_batch_counts(const int64_t* bloom_index,
                                       int64_t bloom_index_numel,
                                       const int64_t* bundle_b_offsets,
                                       int64_t num_bundles,
                                       const st_search_plan* plan,
                                       const void* plan_blob_device,
                                       int64_t num_docs, int64_t* packed_out,
                                       void* workspace, int64_t* row_offsets,
                                       void* stream);
int st_bloom_compact_ids(const int64_t* packed, int64_t num_queries,
                         int64_t num_columns, int64_t num_docs,
                         const void* workspace, void* ids, int ids_int64,
                         void* stream);

/* ---------------------------------------------------------------------------
 * Fused filter + top-k.  No reference operator; relatives are the bloom-
 * filtered scoring of fused_kmean_ann (fused_kmean_ann_cuda.cu:545-551,
 * :1797-1926) and at::topk (fresh_index_post_processing.cpp:245-250).
 * For each query q, among docs d < num_docs whose bit is set in `packed`
 * (int64[num_queries, num_columns], the packed search output), the `topk`
 * best by score = sum_j doc_embeddings[d, j] * query_embeddings[q, j]
 * (bf16 inputs, row-major [*, dim], fp32 accumulation), ordered by score
 * descending then doc id ascending, into out_ids int64[num_queries, topk]
 * and out_scores float[num_queries, topk]; missing entries are -1 / -inf.
 * dim is 64, 128 or 256; 1 <= topk <= 2048; doc ids below 2^32; embeddings
 * 16-byte aligned with at least num_docs rows.  workspace: device memory of
 * st_filtered_topk_workspace_bytes(num_queries) bytes.  Synchronises the
 * stream once (to learn whether a candidate list overflowed; if one did, the
 * selection is redone with smaller rounds).
 * ------------------------------------------------------------------------- */
int64_t st_filtered_topk_workspace_bytes(int64_t num_queries);
int st_filtered_topk(const int64_t* packed, int64_t num_queries,
                     int64_t num_columns, int64_t num_docs,
                     const void* doc_embeddings, const void* query_embeddings,
                     int64_t dim, int64_t topk, void* workspace,
                     int64_t* out_ids, float* out_scores, void* stream);

/* ---------------------------------------------------------------------------
 * Clustered nearest-neighbour scoring, the consumer step after the search.
 * Replaces fused_kmean_ann (fused_kmean_ann.cpp:85-227; CUDA op
 * fused_kmean_ann_cuda.cu:1797-1926).  For each query row b, over the probes
 * p in order, the docs cluster_offsets[cluster_ids[b][p]] + i,
 * 0 <= i < cluster_length[b][p] (int64 arrays; cluster_ids / cluster_length
 * [batch, probes]) that pass the row's filter take consecutive output slots
 * until max_per_row are filled; the rest is padding (score dtype minimum,
 * invalid_index_value).  Filter (optional): int64 filter_mask
 * [filter_rows, filter_cols], row filter_index[b] (or b when filter_index is
 * null; then filter_rows >= batch); doc d passes when bit 63 - d % 64 of
 * word d / 64 is set, or when that word is past filter_cols.  A
 * filter_index[b] outside [0, filter_rows) passes no doc (the reference
 * reads out of bounds there).  embeddings [total_docs, dim] and queries [batch, dim]
 * share emb_dtype: 0 float32, 1 float16, 2 bfloat16, 3 int8.  Scores
 * (st_kmean_ann_score_dtype: the embedding dtype; for int8, int32 (code 4),
 * or float16 when divisor_for_int8 != -1 or per_embedding_scale (float16
 * [total_docs]) is given) are float64 dot products converted to the score
 * dtype (int8: exact int32 sums, divided as float when scaled); indices are
 * int32 doc ids.  1 <= dim <= 1280.  A cluster id outside
 * [0, num_offsets) or a negative length selects nothing.  workspace: device
 * memory of st_fused_kmean_ann_workspace_bytes(batch, probes) bytes (the
 * per-(row, probe) counts of passing docs, then the per-row totals and group
 * starts that calls of 2,048 pairs or more use to spread the scoring).
 * ------------------------------------------------------------------------- */
int64_t st_fused_kmean_ann_workspace_bytes(int64_t batch, int64_t probes);
int st_kmean_ann_score_dtype(int emb_dtype, int64_t divisor_for_int8,
                             int has_per_embedding_scale);
int st_fused_kmean_ann(const int64_t* cluster_offsets, int64_t num_offsets,
                       const int64_t* cluster_ids, const int64_t* cluster_length,
                       int64_t batch, int64_t probes, const void* embeddings,
                       int64_t total_docs, int64_t dim, int emb_dtype,
                       const void* queries, int64_t max_per_row,
                       const int64_t* filter_mask, int64_t filter_rows,
                       int64_t filter_cols, const int64_t* filter_index,
                       const uint16_t* per_embedding_scale,
                       int64_t divisor_for_int8, int64_t invalid_index_value,
                       void* workspace, void* scores, int32_t* indices,
                       void* stream);

/* ---------------------------------------------------------------------------
 * Merge of a main and a fresh candidate list.  Replaces
 * take_top_k_and_gather_from_main_and_fresh (schema
 * fresh_index_post_processing.cpp:275-287, CPU impl :231-270, gather
 * :44-163).  Two calls:
 *
 * st_fresh_topk: row r's merged scores are fresh_scores[r, 0..num_fresh)
 * followed by main_scores[r, 0..num_main) (both row-major, contiguous, of
 * score_type); the k best (0 <= k <= num_fresh + num_main), best first, go
 * to top_scores [rows, k] (score_type, the input values), top_index int64
 * [rows, k] (merged column) and is_from_fresh uint8 [rows, k] (top_index <
 * num_fresh).  Larger scores rank first; NaN above every number; -0.0 and
 * +0.0 are equal; equal scores in merged-column order.  workspace: device
 * memory of st_fresh_topk_workspace_bytes(rows, k) bytes (0 for k <= 8192).
 *
 * st_fresh_gather: one data tensor.  For output row o = r * k + j with
 * t = top_index[o]: source row s = fresh_indices[r * fresh_index_cols + t]
 * when t < num_fresh, else main_indices[r * main_index_cols + t - num_fresh]
 * (indices int32 or int64: index_bytes 4 or 8); s outside [0, data rows)
 * reads row 0 (an empty data tensor gives zeros); out[o, 0..dim) =
 * data[s, 0..dim) with elements of elem_bytes (1, 2, 4 or 8) bytes.
 * ------------------------------------------------------------------------- */
#define ST_SCORE_F32 0
#define ST_SCORE_F16 1
#define ST_SCORE_BF16 2
#define ST_SCORE_F64 3
#define ST_SCORE_I64 4
#define ST_SCORE_I32 5
#define ST_SCORE_I16 6
#define ST_SCORE_I8 7
#define ST_SCORE_U8 8
int64_t st_fresh_topk_workspace_bytes(int64_t rows, int64_t k);
int st_fresh_topk(const void* main_scores, const void* fresh_scores, int score_type,
                  int64_t rows, int64_t num_main, int64_t num_fresh, int64_t k,
                  void* workspace, void* top_scores, int64_t* top_index,
                  uint8_t* is_from_fresh, void* stream);
int st_fresh_gather(const int64_t* top_index, int64_t rows, int64_t k,
                    const void* fresh_indices, const void* main_indices,
                    int index_bytes, int64_t fresh_index_cols, int64_t main_index_cols,
                    int64_t num_fresh, int64_t num_main, const void* fresh_data,
                    int64_t fresh_rows, const void* main_data, int64_t main_rows,
                    int64_t dim, int elem_bytes, void* out, void* stream);

/* ---------------------------------------------------------------------------
 * st_fused_kmean_ann without allocation.  No counterpart in the reference:
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments and results as st_fused_kmean_ann minus `workspace`: the
 * per-(row, probe) counts (and, when they fit after them, the row totals and
 * group starts of calls of 2,048 pairs or more) go to a fixed device array
 * of the library, one copy per GPU (8 MiB, held until the process ends), so
 * batch x probes must not exceed ST_KMEAN_NOALLOC_MAX_PAIRS (larger calls
 * are rejected before any launch).  The device current on the calling thread must be the one
 * the buffers and the stream belong to.  Allocates nothing (no hipMalloc,
 * hipFree or allocating library call).  Calls on one GPU share the array, so
 * they never overlap: calls on one stream run in stream order, and a call on
 * another stream than the device's previous call waits (hipStreamWaitEvent)
 * for that call's event, recorded after every call; the event is created
 * with the array's address on the device's first call.  Under graph capture,
 * capture every call on one stream (a wait on an event recorded outside the
 * capture is not part of the graph).
 * ------------------------------------------------------------------------- */
#define ST_KMEAN_NOALLOC_MAX_PAIRS (1 << 20)
int st_fused_kmean_ann_noalloc(const int64_t* cluster_offsets, int64_t num_offsets,
                               const int64_t* cluster_ids,
                               const int64_t* cluster_length, int64_t batch,
                               int64_t probes, const void* embeddings,
                               int64_t total_docs, int64_t dim, int emb_dtype,
                               const void* queries, int64_t max_per_row,
                               const int64_t* filter_mask, int64_t filter_rows,
                               int64_t filter_cols, const int64_t* filter_index,
                               const uint16_t* per_embedding_scale,
                               int64_t divisor_for_int8,
                               int64_t invalid_index_value, void* scores,
                               int32_t* indices, void* stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* SILVERTORCH_HIP_H_ */
