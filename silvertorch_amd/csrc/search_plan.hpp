// Compiled form of a batch of encoded query plans, shared by the host plan
// compiler (search_plan.cpp) and the search kernels (bloom_search.hip).
//
// Each query plan arrives as the postfix operator list of
// bloom_index_util.h:70-93 (ops, child counts via offsets, hash_k hashes per
// TERM).  The compiler rebuilds the expression tree, flattens nested
// AND/AND and OR/OR, removes double negation, deduplicates terms across the
// batch, and emits a straight-line program for a one-accumulator machine
// with a small push/pop stack.  All of that preserves the bitwise result of
// the reference's stack evaluation (bloom_index_search.cpp:72-171) exactly,
// since AND and OR over 64-bit words are associative, commutative and
// idempotent.
#pragma once

#include <climits>
#include <cstdint>
#include <vector>

namespace st {

// Search kernel geometry.
constexpr int kSearchWaves = 16;                 // waves per workgroup
constexpr int kSearchThreads = kSearchWaves * 64;
constexpr int kSearchTileRows = 512;             // bundle rows staged in LDS
constexpr int kSearchOnesRow = kSearchTileRows;  // virtual all-ones row
constexpr int kSearchZerosRow = kSearchTileRows + 1;  // virtual all-zeros row
constexpr int kSearchTileBytes = (kSearchTileRows + 2) * 256;
constexpr int kSearchLdsBytes = 160 * 1024;
constexpr int kSearchPosSlots = (kSearchLdsBytes - kSearchTileBytes) / 4;
constexpr int kSearchMaxStack = 8;

// Position codes of the global-memory path (bundles wider than the tile).
constexpr int32_t kPosOnes = INT32_MIN;  // (no-op literals of width-bound pairs)
constexpr int32_t kPosZeros = INT32_MIN + 1;

// A query program is a 16-byte aligned run of uint32 words with a 4-word
// header [form | T, output row, n_ops, 0], in one of two forms.  Term
// references are byte offsets of the term's position list in the kernel's
// LDS position area (term id * positions_per_term * 4), so the kernel never
// decodes them.
//
// Flat form (kFlatForm set): the query as an OR of AND-groups of literals,
// optionally complemented as a whole.  T literal records of 4 words follow:
//   [position byte offset, negate mask, group mask, 0]
// (masks are 0 or ~0; the group mask is ~0 on the first literal of each
// group).  Evaluated with no decoding: per literal w = word ^ negate,
// res |= acc & group, acc = (acc | group) & w; then res | acc, complemented
// if kFlatComplement is set.
//
// Stack form (kFlatForm clear), for queries whose flat form would be large:
// T term references (1 word each, in the order the TERM ops consume them)
// then n_ops operations: [2:0] opcode, [4:3] combine mode, [5] negate.
constexpr uint32_t kFlatForm = 1u << 31;
constexpr uint32_t kFlatComplement = 1u << 30;
// Set on the first of two consecutive flat programs of a wave that the
// width-bound kernel evaluates together; their bound copies are padded to the
// same literal count with no-op literals (all-ones row, same group).
constexpr uint32_t kPairedWithNext = 1u << 29;
constexpr int kFlatMaxLiterals = 64;
constexpr int kProgHeaderWords = 4;
constexpr int kFlatLiteralWords = 4;

enum InsnOp : uint32_t {
  kInsTerm = 0,   // acc = mode(acc, [~]next term word)
  kInsConst = 1,  // acc = mode(acc, [~]all_ones)
  kInsPush = 2,   // stack[sp++] = acc
  kInsPop = 3,    // acc = mode(stack[--sp], acc)
  kInsNot = 4,    // acc = ~acc
};
enum InsnMode : uint32_t { kModeSet = 0, kModeAnd = 1, kModeOr = 2 };

inline uint32_t encode_insn(uint32_t op, uint32_t mode, bool neg) {
  return op | (mode << 3) | (static_cast<uint32_t>(neg) << 5);
}

// Largest program the batch kernels run; larger ones, and programs needing
// more than kSearchMaxStack slots, run in generic batches (one query each,
// evaluated by the generic kernel with its positions resolved per lane).
constexpr uint32_t kMaxTermsPerQuery = 0xFFFF;
constexpr uint32_t kMaxOpsPerQuery = 0x7FFF;
constexpr int kGenericMaxStack = 32;
// Term and operation counts of a generic program stay below this (the
// stack-form header's term count keeps clear of the flag bits).
constexpr uint32_t kGenericMaxTerms = 1u << 29;

// Term count of a program header (stack form: the whole word below the
// flags; flat form: the low 16 bits).
constexpr uint32_t program_terms(uint32_t hdr) {
  return (hdr & (1u << 31)) ? (hdr & 0xFFFFu) : (hdr & (kGenericMaxTerms - 1u));
}

// Positions stored per term in LDS, padded so a term's list is read with
// 16-byte loads.
inline int positions_per_term(int k_eff) {
  return k_eff <= 4 ? 4 : (k_eff <= 8 ? 8 : 12);
}

// Width-bound programs.  Once the bundle widths are known on the host
// (st_search_plan_bind_widths), every distinct width among the most frequent
// kMaxWidthSlots gets a copy of the batch's programs with each term
// reference replaced by the term's row positions at that width, so the
// kernel needs neither the per-bundle positions step nor the LDS position
// lookup.  Bundles of other widths (bundle_slot == kNoWidthSlot) use the
// term-reference programs.
//
// Bound flat form: header as above, then T records of
// bound_record_words(K) words: [row position 0 .. K-1, flags, pad...]
// with flags bit 0 = negate, bit 1 = first of its group.
// Bound stack form: header, T position lists of positions_per_term(K)
// words, then the operations.
// Positions are LDS byte offsets (row * 256) for bundles staged in LDS and
// signed rows relative to the bundle start otherwise (no-op rows: kPosOnes /
// kPosZeros), except at wide widths (see below): slice-tile byte offsets.
constexpr int kMaxWidthSlots = 64;
constexpr uint32_t kNoWidthSlot = 0xFFFFFFFFu;

constexpr int bound_record_words(int k_eff) { return ((k_eff + 1 + 3) / 4) * 4; }

// Literal stream.  Every width block also carries the batch's flat programs
// as rounds of literal records, which the kernel reads with scalar loads and
// evaluates without per-query decoding.  A wave's flat programs are taken
// longest first, stream_block_records(K) at a time, into rounds; a round
// evaluates its programs (its slots) in lockstep, one literal of every slot
// per step:
//   header, kRoundHeaderWords words: [T, 0 x 7, slot 0 info, slot 1 info,
//     ...], slot info = bit 0 valid, bit 1 complement the result,
//     bits 2..31 output row;
//   then T steps of stream_block_records(K) records (one per slot) of
//     bound_record_words(K) words: [row position 0 .. K-1, flags, pad...],
//     flags bit 0 = negate, bit 1 = first of its group; in a batch with no
//     negated literal (stream_masks set) the flags word is the group mask
//     itself (~0 on the first literal of a group, else 0).
// T is the longest program of the round; shorter ones (and empty slots) are
// padded with no-op records (all-ones row, flags 0).  A program with no
// literal is one record on the all-zeros row.  The flat programs a wave's
// rounds cover are its first ones; the rest are evaluated from the width
// block.
constexpr uint32_t kStreamNeg = 1u;
constexpr uint32_t kStreamFirst = 2u;
constexpr uint32_t kSlotValid = 1u;
constexpr uint32_t kSlotComplement = 2u;
constexpr int kSlotRowShift = 2;
constexpr int64_t kStreamMaxRows = int64_t{1} << (32 - kSlotRowShift);
constexpr int kRoundHeaderWords = 16;
constexpr int kRoundSlotInfo = 8;  // header word of slot 0's info
// Slots of a round: 32 words of records per step.
inline int stream_block_records(int k_eff) { return 32 / bound_record_words(k_eff); }

// One kernel launch worth of queries.  Offsets are byte offsets into the
// plan blob.
struct SearchBatch {
  bool generic = false;     // one query for the generic kernel (no width blocks)
  uint32_t num_slots = 0;   // queries in this batch
  uint32_t num_terms = 0;   // distinct terms in this batch
  uint64_t off_wave = 0;    // uint32[kSearchWaves + 1]: slot range per wave
  uint64_t off_insn_start = 0;  // uint32[num_slots]: first word of each program
  uint64_t off_insns = 0;   // uint32[...]: query programs
  uint64_t off_hashes = 0;  // uint64[num_terms * hash_k]
  // width-bound programs (valid when the plan is bound)
  uint64_t off_bound_start = 0;  // uint32[num_slots]: first word within a width block
  uint64_t off_bound = 0;        // uint32[width_slots * bound_words]
  uint32_t bound_words = 0;      // words per width block
  // device binding: one width block as a template (host-written) whose
  // position words are codes resolved per slot width on the device
  uint64_t off_tmpl = 0;         // uint32[bound_words]: words copied as they are
  uint64_t off_tmpl_code = 0;    // uint32[bound_words]: kTmplCopy / kTmplOnes / term code
  // literal stream (stream_words == 0: none): words [stream_off,
  // stream_off + stream_words) of every width block
  uint32_t stream_off = 0;
  uint32_t stream_words = 0;
  uint32_t stream_masks = 0;     // 1: records carry group masks (no negation)
  uint64_t off_stream_wave = 0;  // uint32[kSearchWaves + 1]: first stream word of each wave
  uint64_t off_stream_skip = 0;  // uint32[kSearchWaves]: flat programs each run covers
  // device binding: the stream's balance units, the block word of the first
  // of four records one 16-lane group of the wide-bundle kernel reads
  // together (none unless the records hold 2 .. 7 positions)
  uint64_t off_units = 0;        // uint32[n_units]
  uint32_t n_units = 0;
};

// Wide bundles (kSearchTileRows < b <= kWideRows rows, width-bound) are
// searched by a second kernel in column slices: 64 bytes (8 words, 512
// docs) of every row staged in LDS at a time, four slices per bundle, the
// literal streams of all batches evaluated on each slice.  Their bound
// positions are byte offsets in that slice tile (row * kWideSliceBytes);
// the all-ones and all-zeros no-op rows are the tile's rows kWideOnesRow and
// kWideZerosRow.
constexpr int kWideRows = 2048;
constexpr int kWideOnesRow = kWideRows;
constexpr int kWideZerosRow = kWideRows + 1;
constexpr int kWideSliceBytes = 64;
constexpr int kWideSlices = 256 / kWideSliceBytes;
constexpr bool wide_width(int64_t b) { return b > kSearchTileRows && b <= kWideRows; }

// Work table of the wide-bundle kernel (uint32 words at
// st_search_plan::off_wide, absent when off_wide == 0):
//   [0] batches, [1] groups, [2] rounds per group, [3] 0,
//   [4 .. 4 + kSearchWaves] first group of each wave (groups are stored
//     wave by wave), padded to kWideTableHead words;
//   per batch, 4 words: [word offset of its width blocks in the device blob,
//     words per width block, stream offset within a block, stream_masks];
//   per group, kWideGroupWords words: [batch, longest round's steps,
//     round 0 .. 3 word offsets within the stream (~0u: none),
//     round 0 .. 3 steps, 0, 0].
// A group is stream_block_records(k) * rounds-per-group = 16 programs, one
// per lane quad of a wave.
constexpr int kWideTableHead = 24;
constexpr int kWideGroupWords = 12;
constexpr int kWidePrograms = 16;
constexpr int kWideMaxRounds = 4;

// Batch table of the device binding kernel (uint64 words at
// st_search_plan::off_bind_table), per batch: byte offsets of its template,
// template codes, term hashes and width blocks in the device blob, words per
// width block, distinct terms, byte offset of its balance units, their
// number, and its literal stream's words within a block (first | count << 32).
constexpr int kBindTableWords = 9;

// Codes of a width-block template word.
constexpr uint32_t kTmplCopy = 0u;           // the template word itself
constexpr uint32_t kTmplOnes = 0xFFFFFFFFu;  // the all-ones row at the slot's width
constexpr uint32_t kTmplZeros = 0xFFFFFFFEu; // the all-zeros row at the slot's width
// otherwise ((term + 1) << 4) | r: position r of batch term `term`
inline uint32_t tmpl_position_code(uint32_t term, uint32_t r) { return ((term + 1u) << 4) | r; }

}  // namespace st

// Host object behind the opaque st_search_plan handle.
struct st_search_plan {
  int64_t num_queries = 0;
  int64_t hash_k = 0;
  int k_eff = 0;        // distinct positions resolved per term
  int kp = 4;           // padded positions per term in LDS
  int max_stack = 0;    // deepest push in any program
  std::vector<st::SearchBatch> batches;
  std::vector<uint8_t> blob;
  // term-reference programs and term hashes of each batch, kept for binding
  std::vector<std::vector<uint32_t>> batch_insns;
  std::vector<std::vector<uint32_t>> batch_starts;
  std::vector<std::vector<uint64_t>> batch_hashes;
  // set by st_search_plan_bind_widths
  int64_t bound_bundles = -1;        // -1: not bound
  uint64_t off_bundle_slot = 0;      // uint32[bound_bundles]
  uint64_t off_bundle_order = 0;     // uint32[bound_bundles]: visiting order
  std::vector<int64_t> slot_width;   // width of each slot
  // set by st_search_plan_prepare_device_binding: the search call binds the
  // widths on the device into the part of the device copy past the host blob
  bool device_bind = false;
  uint64_t device_bytes = 0;         // size of the device copy
  uint64_t off_num_slots = 0;        // uint32[3] (device-written): slots, all wide, some wide
  uint64_t off_slot_width = 0;       // int64[kMaxWidthSlots] (device-written)
  uint64_t off_bind_table = 0;       // uint64[batches * kBindTableWords]
  // set by st_search_plan_upload_source: the search calls copy the blob
  // from this pinned host buffer (device address upload_device_src)
  const void* upload_source = nullptr;
  const void* upload_device_src = nullptr;
  // set by st_search_plan_upload_signal: after copying its part of the blob
  // each upload workgroup g stores upload_signal_value to
  // upload_signal_device[g] (pinned host memory, device address)
  void* upload_signal_device = nullptr;
  uint64_t upload_signal_value = 0;
  // work table of the wide-bundle kernel (0: none), set by either binding
  uint64_t off_wide = 0;
  // host binding: every bundle has a slot and every slot width is wide
  bool all_wide = false;
};
