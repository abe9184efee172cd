// Host compiler from encoded query plans to accumulator programs.
//
// Input format (bloom_index_util.cpp:81-124 of the reference): for query q,
// plans_offsets[8q .. 8q+7] are byte ranges in plans_data of
//   operators  uint8[n_ops]       (PlanOp codes)
//   offsets    int32[n_ops + 1]   (children of op i = offsets[i+1]-offsets[i])
//   parameters int32[...]         (not needed: the reference CPU search
//                                  evaluates by stack order, not by index)
//   hashes     uint64[n_terms * hash_k]
// Evaluation semantics restated from run_query_plan
// (bloom_index_search.cpp:72-171): TERMs take hash groups in program order;
// AND pops `children` values and ANDs them into all-ones; OR ORs them into
// zero; NOT needs exactly one child; EMPTY pushes all-ones; the answer is the
// top of the stack.
#include <algorithm>
#include <climits>
#include <cstring>
#include <memory>
#include <string>
#include <unordered_map>

#include "search_plan.hpp"
#include "st_common.hpp"
#include "st_errors.hpp"

namespace st {
namespace {

enum class NodeKind { kTerm, kConst, kAnd, kOr, kNot };

struct Node {
  NodeKind kind;
  bool ones = true;        // kConst: value is all ones (true) or zero
  uint32_t term = 0;       // kTerm: batch-local term id
  std::vector<int> kids;   // kAnd / kOr / kNot
  int need = 0;            // stack slots needed to evaluate
};

struct Tree {
  std::vector<Node> nodes;
  int add(Node n) {
    nodes.push_back(std::move(n));
    return static_cast<int>(nodes.size()) - 1;
  }
};

template <typename T>
T load_le(const int8_t* p) {
  T v;
  std::memcpy(&v, p, sizeof(T));
  return v;
}

// Interns each distinct hash_k-tuple once per batch.
struct TermTable {
  int64_t hash_k = 0;
  std::unordered_map<std::string, uint32_t> ids;
  std::vector<uint64_t> hashes;
  std::vector<std::string> added;  // keys interned since the last commit()
  uint32_t intern(const int8_t* h) {
    std::string key(reinterpret_cast<const char*>(h),
                    static_cast<size_t>(hash_k) * 8);
    auto it = ids.find(key);
    if (it != ids.end()) return it->second;
    uint32_t id = static_cast<uint32_t>(ids.size());
    ids.emplace(key, id);
    added.push_back(std::move(key));
    for (int64_t j = 0; j < hash_k; ++j) hashes.push_back(load_le<uint64_t>(h + 8 * j));
    return id;
  }
  void commit() { added.clear(); }
  void rollback() {
    for (const auto& key : added) ids.erase(key);
    hashes.resize(ids.size() * static_cast<size_t>(hash_k));
    added.clear();
  }
  void clear() {
    ids.clear();
    hashes.clear();
    added.clear();
  }
};

bool is_leaf(const Tree& t, int id) {
  const Node& n = t.nodes[id];
  if (n.kind == NodeKind::kTerm || n.kind == NodeKind::kConst) return true;
  if (n.kind == NodeKind::kNot) {
    const Node& c = t.nodes[n.kids[0]];
    return c.kind == NodeKind::kTerm || c.kind == NodeKind::kConst;
  }
  return false;
}

// Simplifies in place (flatten same-kind children, drop double negation) and
// computes `need`.  Returns the id that replaces `id`.
int normalize(Tree& t, int id) {
  Node& n0 = t.nodes[id];
  if (n0.kind == NodeKind::kTerm || n0.kind == NodeKind::kConst) {
    t.nodes[id].need = 0;
    return id;
  }
  if (n0.kind == NodeKind::kNot) {
    int c = normalize(t, t.nodes[id].kids[0]);
    if (t.nodes[c].kind == NodeKind::kNot) return t.nodes[c].kids[0];
    if (t.nodes[c].kind == NodeKind::kConst) {
      Node k;
      k.kind = NodeKind::kConst;
      k.ones = !t.nodes[c].ones;
      return t.add(k);
    }
    t.nodes[id].kids[0] = c;
    t.nodes[id].need = t.nodes[c].need;
    return id;
  }
  const NodeKind kind = n0.kind;
  std::vector<int> flat;
  std::vector<int> pending = t.nodes[id].kids;
  for (int c : pending) {
    int nc = normalize(t, c);
    if (t.nodes[nc].kind == kind) {
      for (int g : t.nodes[nc].kids) flat.push_back(g);
    } else {
      flat.push_back(nc);
    }
  }
  if (flat.empty()) {
    Node k;
    k.kind = NodeKind::kConst;
    k.ones = (kind == NodeKind::kAnd);
    return t.add(k);
  }
  // Evaluation order: the most demanding subtree first, the other
  // subtrees by decreasing demand, leaves last.
  std::stable_sort(flat.begin(), flat.end(), [&](int a, int b) {
    bool la = is_leaf(t, a), lb = is_leaf(t, b);
    if (la != lb) return !la;
    return t.nodes[a].need > t.nodes[b].need;
  });
  int need = t.nodes[flat[0]].need;
  for (size_t i = 1; i < flat.size(); ++i) {
    if (!is_leaf(t, flat[i])) need = std::max(need, 1 + t.nodes[flat[i]].need);
  }
  t.nodes[id].kids = std::move(flat);
  t.nodes[id].need = need;
  return id;
}

void emit_leaf(const Tree& t, int id, uint32_t mode, std::vector<uint32_t>& out) {
  const Node& n = t.nodes[id];
  bool neg = false;
  const Node* leaf = &n;
  if (n.kind == NodeKind::kNot) {
    neg = true;
    leaf = &t.nodes[n.kids[0]];
  }
  if (leaf->kind == NodeKind::kTerm) {
    out.push_back(encode_insn(kInsTerm, mode, neg, leaf->term));
  } else {
    out.push_back(encode_insn(kInsConst, mode, neg != !leaf->ones, 0));
  }
}

void emit(const Tree& t, int id, std::vector<uint32_t>& out) {
  if (is_leaf(t, id)) {
    emit_leaf(t, id, kModeSet, out);
    return;
  }
  const Node& n = t.nodes[id];
  if (n.kind == NodeKind::kNot) {
    emit(t, n.kids[0], out);
    out.push_back(encode_insn(kInsNot, 0, false, 0));
    return;
  }
  const uint32_t mode = n.kind == NodeKind::kAnd ? kModeAnd : kModeOr;
  emit(t, n.kids[0], out);
  for (size_t i = 1; i < n.kids.size(); ++i) {
    int c = n.kids[i];
    if (is_leaf(t, c)) {
      emit_leaf(t, c, mode, out);
    } else {
      out.push_back(encode_insn(kInsPush, 0, false, 0));
      emit(t, c, out);
      out.push_back(encode_insn(kInsPop, mode, false, 0));
    }
  }
}

struct CompiledQuery {
  std::vector<uint32_t> insns;
  int need = 0;
  int term_refs = 0;
};

// Decodes query q, builds its tree and returns its program.  Terms are
// interned in `terms` (ids are batch-local).
CompiledQuery compile_query(const int8_t* data, int64_t data_len,
                            const int64_t* offs, int64_t q, int64_t hash_k,
                            int k_eff, TermTable& terms) {
  const int64_t* o = offs + 8 * q;
  for (int j = 0; j < 8; j += 2) {
    ST_CHECK(o[j] >= 0 && o[j] <= o[j + 1] && o[j + 1] <= data_len,
             "query plan ", q, ": byte range [", o[j], ", ", o[j + 1],
             ") of section ", j / 2, " lies outside plans_data (",
             data_len, " bytes)");
  }
  const int64_t n_ops = o[1] - o[0];
  const int64_t n_offsets = (o[3] - o[2]) / 4;
  const int64_t n_hashes = (o[7] - o[6]) / 8;
  const int8_t* ops = data + o[0];
  const int8_t* offsets = data + o[2];
  const int8_t* hashes = data + o[6];
  ST_CHECK(n_ops > 0, "query plan ", q, " has no operators");

  Tree tree;
  std::vector<int> stack;
  int64_t term_counter = 0;
  auto child_count = [&](int64_t i) -> int32_t {
    ST_CHECK(i + 1 < n_offsets, "query plan ", q, ": operator ", i,
             " has no child count (offsets array holds ", n_offsets,
             " entries)");
    return load_le<int32_t>(offsets + 4 * (i + 1)) -
           load_le<int32_t>(offsets + 4 * i);
  };
  for (int64_t i = 0; i < n_ops; ++i) {
    const uint8_t op = static_cast<uint8_t>(ops[i]);
    switch (op) {
      case kOpTerm: {
        Node n;
        if (k_eff == 0) {
          // No position is ever resolved: the term word stays all ones.
          n.kind = NodeKind::kConst;
          n.ones = true;
        } else {
          ST_CHECK((term_counter + 1) * hash_k <= n_hashes, "query plan ", q,
                   ": term ", term_counter, " needs hashes [",
                   term_counter * hash_k, ", ", (term_counter + 1) * hash_k,
                   ") but the plan holds ", n_hashes);
          n.kind = NodeKind::kTerm;
          n.term = terms.intern(hashes + 8 * term_counter * hash_k);
          ST_CHECK(n.term <= kInsnMaxArg, "too many distinct terms");
        }
        ++term_counter;
        stack.push_back(tree.add(n));
        break;
      }
      case kOpEmpty: {
        Node n;
        n.kind = NodeKind::kConst;
        n.ones = true;
        stack.push_back(tree.add(n));
        break;
      }
      case kOpAnd:
      case kOpOr: {
        int32_t children = child_count(i);
        Node n;
        n.kind = op == kOpAnd ? NodeKind::kAnd : NodeKind::kOr;
        for (int32_t j = 0; j < children; ++j) {
          ST_CHECK(!stack.empty(), "query plan ", q, ": operator ", i,
                   " pops ", children, " values from a shorter stack");
          n.kids.push_back(stack.back());
          stack.pop_back();
        }
        stack.push_back(tree.add(n));
        break;
      }
      case kOpNot: {
        int32_t children = child_count(i);
        ST_CHECK(children == 1, "NOT query should have 1 parameter, but got ",
                 children);
        ST_CHECK(!stack.empty(), "query plan ", q, ": NOT operator ", i,
                 " applied to an empty stack");
        Node n;
        n.kind = NodeKind::kNot;
        n.kids.push_back(stack.back());
        stack.pop_back();
        stack.push_back(tree.add(n));
        break;
      }
      default:
        fail("unknown operator: ", static_cast<int>(op));
    }
  }
  ST_CHECK(!stack.empty(), "query plan ", q, " leaves an empty stack");
  int root = normalize(tree, stack.back());
  CompiledQuery cq;
  emit(tree, root, cq.insns);
  cq.need = tree.nodes[root].need;
  for (uint32_t w : cq.insns) cq.term_refs += ((w & 7u) == kInsTerm);
  ST_CHECK(cq.need <= kSearchMaxStack, "query plan ", q, " needs ", cq.need,
           " stack slots; this build evaluates at most ", kSearchMaxStack);
  return cq;
}

void append_bytes(std::vector<uint8_t>& blob, const void* p, size_t n) {
  const uint8_t* b = static_cast<const uint8_t*>(p);
  blob.insert(blob.end(), b, b + n);
  while (blob.size() % 16) blob.push_back(0);
}

}  // namespace
}  // namespace st

extern "C" int st_search_plan_create(const int8_t* plans_data,
                                     int64_t plans_data_len,
                                     const int64_t* plans_offsets,
                                     int64_t plans_offsets_len, int64_t k,
                                     int64_t hash_k, st_search_plan** out) {
  using namespace st;
  return guarded([&] {
    ST_CHECK(out != nullptr, "out is null");
    *out = nullptr;
    ST_CHECK(plans_data_len >= 0 && plans_offsets_len >= 0,
             "negative plan sizes");
    ST_CHECK(plans_data != nullptr || plans_data_len == 0, "plans_data is null");
    ST_CHECK(plans_offsets != nullptr || plans_offsets_len == 0,
             "plans_offsets is null");
    const int64_t num_queries = plans_offsets_len / 8;
    int64_t k_eff = std::max<int64_t>(0, std::min(k, hash_k));
    ST_CHECK(k_eff <= kMaxSearchK, "k = ", k, " with hash_k = ", hash_k,
             " resolves up to ", k_eff,
             " positions per term; at most ", kMaxSearchK, " are supported");

    auto plan = std::make_unique<st_search_plan>();
    plan->num_queries = num_queries;
    plan->hash_k = hash_k;
    plan->k_eff = static_cast<int>(k_eff);
    plan->kp = positions_per_term(plan->k_eff);
    const int64_t term_capacity = kSearchPosSlots / plan->kp;

    // Compile queries in order, cutting a new batch whenever the distinct
    // terms of the running batch would overflow the LDS position area.
    struct Pending {
      int64_t row;
      CompiledQuery cq;
    };
    std::vector<Pending> cur;
    TermTable terms;
    terms.hash_k = std::max<int64_t>(hash_k, 0);

    auto flush = [&]() {
      if (cur.empty()) return;
      SearchBatch b;
      b.num_slots = static_cast<uint32_t>(cur.size());
      b.num_terms = static_cast<uint32_t>(terms.ids.size());
      // Longest-processing-time assignment of queries to the waves of a
      // workgroup; cost ~ LDS word reads plus instruction count.
      std::vector<int> order(cur.size());
      for (size_t i = 0; i < order.size(); ++i) order[i] = static_cast<int>(i);
      auto cost = [&](int i) {
        return static_cast<int64_t>(cur[i].cq.insns.size()) +
               static_cast<int64_t>(cur[i].cq.term_refs) * (k_eff + 1);
      };
      std::stable_sort(order.begin(), order.end(),
                       [&](int a, int c) { return cost(a) > cost(c); });
      std::vector<std::vector<int>> per_wave(kSearchWaves);
      std::vector<int64_t> load(kSearchWaves, 0);
      for (int i : order) {
        int w = static_cast<int>(std::min_element(load.begin(), load.end()) -
                                 load.begin());
        per_wave[w].push_back(i);
        load[w] += cost(i);
      }
      std::vector<uint32_t> wave_off(kSearchWaves + 1, 0), rows, starts,
          insns;
      for (int w = 0; w < kSearchWaves; ++w) {
        for (int i : per_wave[w]) {
          rows.push_back(static_cast<uint32_t>(cur[i].row));
          starts.push_back(static_cast<uint32_t>(insns.size()));
          insns.insert(insns.end(), cur[i].cq.insns.begin(),
                       cur[i].cq.insns.end());
        }
        wave_off[w + 1] = static_cast<uint32_t>(rows.size());
      }
      starts.push_back(static_cast<uint32_t>(insns.size()));
      auto& blob = plan->blob;
      b.off_wave = blob.size();
      append_bytes(blob, wave_off.data(), wave_off.size() * 4);
      b.off_row = blob.size();
      append_bytes(blob, rows.data(), rows.size() * 4);
      b.off_insn_start = blob.size();
      append_bytes(blob, starts.data(), starts.size() * 4);
      b.off_insns = blob.size();
      append_bytes(blob, insns.data(), insns.size() * 4);
      b.off_hashes = blob.size();
      append_bytes(blob, terms.hashes.data(), terms.hashes.size() * 8);
      plan->batches.push_back(b);
      cur.clear();
      terms.clear();
    };

    for (int64_t q = 0; q < num_queries; ++q) {
      CompiledQuery cq = compile_query(plans_data, plans_data_len,
                                       plans_offsets, q, hash_k,
                                       plan->k_eff, terms);
      if (static_cast<int64_t>(terms.ids.size()) > term_capacity) {
        terms.rollback();
        flush();
        cq = compile_query(plans_data, plans_data_len, plans_offsets, q,
                           hash_k, plan->k_eff, terms);
        ST_CHECK(static_cast<int64_t>(terms.ids.size()) <= term_capacity,
                 "query plan ", q, " has ", terms.ids.size(),
                 " distinct terms; at most ", term_capacity,
                 " fit one search pass at k = ", plan->k_eff);
      }
      terms.commit();
      plan->max_stack = std::max(plan->max_stack, cq.need);
      cur.push_back(Pending{q, std::move(cq)});
    }
    flush();
    *out = plan.release();
  });
}

extern "C" int64_t st_search_plan_num_queries(const st_search_plan* plan) {
  return plan ? plan->num_queries : 0;
}

extern "C" int64_t st_search_plan_blob_bytes(const st_search_plan* plan) {
  return plan ? static_cast<int64_t>(plan->blob.size()) : 0;
}

extern "C" const void* st_search_plan_blob(const st_search_plan* plan) {
  return plan ? plan->blob.data() : nullptr;
}

extern "C" void st_search_plan_destroy(st_search_plan* plan) { delete plan; }
