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

struct CompiledQuery {
  std::vector<uint32_t> terms;  // stack form: term ids in consumption order
  std::vector<uint32_t> ops;    // stack form: operations
  int need = 0;
  bool flat = false;            // flat form: OR of AND-groups
  bool complement = false;
  struct FlatLit {
    uint32_t term;
    bool neg;
    bool first;
  };
  std::vector<FlatLit> lits;    // flat form: literals, group by group
};

// ---------------------------------------------------------------- flat form
// Disjunctive normal form of a (sub)tree or of its complement, with the
// negations pushed onto the terms (De Morgan).  Exact for 64-bit words since
// every bit obeys Boolean algebra independently.  Groups holding a term and
// its negation are dropped (their AND is 0), repeated literals are merged.

struct Lit {
  uint32_t term;
  bool neg;
  bool operator<(const Lit& o) const {
    return term != o.term ? term < o.term : neg < o.neg;
  }
  bool operator==(const Lit& o) const { return term == o.term && neg == o.neg; }
};

struct Dnf {
  bool is_true = false;             // the constant all-ones
  std::vector<std::vector<Lit>> groups;  // empty and !is_true: constant zero
  size_t literals() const {
    size_t n = 0;
    for (const auto& g : groups) n += g.size();
    return n;
  }
};

Dnf dnf_true() {
  Dnf d;
  d.is_true = true;
  return d;
}

// Conjunction of two DNFs by distribution; false when the result exceeds cap.
bool dnf_and(const Dnf& a, const Dnf& b, size_t cap, Dnf& out) {
  if (a.is_true) { out = b; return true; }
  if (b.is_true) { out = a; return true; }
  Dnf r;
  for (const auto& ga : a.groups) {
    for (const auto& gb : b.groups) {
      std::vector<Lit> g(ga);
      g.insert(g.end(), gb.begin(), gb.end());
      std::sort(g.begin(), g.end());
      g.erase(std::unique(g.begin(), g.end()), g.end());
      bool contradiction = false;
      for (size_t i = 1; i < g.size(); ++i)
        contradiction |= g[i].term == g[i - 1].term;  // t and ~t
      if (contradiction) continue;
      r.groups.push_back(std::move(g));
      if (r.literals() > cap) return false;
    }
  }
  out = std::move(r);
  return true;
}

bool to_dnf(const Tree& t, int id, bool negated, size_t cap, Dnf& out) {
  const Node& n = t.nodes[id];
  switch (n.kind) {
    case NodeKind::kTerm:
      out = Dnf();
      out.groups.push_back({Lit{n.term, negated}});
      return true;
    case NodeKind::kConst:
      out = (n.ones != negated) ? dnf_true() : Dnf();
      return true;
    case NodeKind::kNot:
      return to_dnf(t, n.kids[0], !negated, cap, out);
    case NodeKind::kAnd:
    case NodeKind::kOr: {
      const bool conj = (n.kind == NodeKind::kAnd) != negated;
      Dnf acc = conj ? dnf_true() : Dnf();
      for (int c : n.kids) {
        Dnf d;
        if (!to_dnf(t, c, negated, cap, d)) return false;
        if (conj) {
          Dnf next;
          if (!dnf_and(acc, d, cap, next)) return false;
          acc = std::move(next);
        } else {
          if (acc.is_true) continue;
          if (d.is_true) {
            acc = dnf_true();
            continue;
          }
          for (auto& g : d.groups) acc.groups.push_back(std::move(g));
          if (acc.literals() > cap) return false;
        }
      }
      out = std::move(acc);
      return true;
    }
  }
  return false;
}

// Fills cq's flat form when the query (or its complement) has a DNF of at
// most kFlatMaxLiterals literals.
bool try_flat(const Tree& t, int root, CompiledQuery& cq) {
  Dnf direct, inverse;
  const bool ok_d = to_dnf(t, root, false, kFlatMaxLiterals, direct);
  const bool ok_i = to_dnf(t, root, true, kFlatMaxLiterals, inverse);
  if (!ok_d && !ok_i) return false;
  const bool use_inverse =
      !ok_d || (ok_i && inverse.literals() < direct.literals());
  const Dnf& d = use_inverse ? inverse : direct;
  cq.flat = true;
  cq.lits.clear();
  if (d.is_true) {
    cq.complement = !use_inverse;  // empty OR is zero; complement gives ones
    return true;
  }
  cq.complement = use_inverse;
  for (const auto& g : d.groups) {
    for (size_t i = 0; i < g.size(); ++i)
      cq.lits.push_back(CompiledQuery::FlatLit{g[i].term, g[i].neg, i == 0});
  }
  return true;
}

void emit_leaf(const Tree& t, int id, uint32_t mode, CompiledQuery& out) {
  const Node& n = t.nodes[id];
  bool neg = false;
  const Node* leaf = &n;
  if (n.kind == NodeKind::kNot) {
    neg = true;
    leaf = &t.nodes[n.kids[0]];
  }
  if (leaf->kind == NodeKind::kTerm) {
    out.terms.push_back(leaf->term);
    out.ops.push_back(encode_insn(kInsTerm, mode, neg));
  } else {
    out.ops.push_back(encode_insn(kInsConst, mode, neg != !leaf->ones));
  }
}

void emit(const Tree& t, int id, CompiledQuery& out) {
  if (is_leaf(t, id)) {
    emit_leaf(t, id, kModeSet, out);
    return;
  }
  const Node& n = t.nodes[id];
  if (n.kind == NodeKind::kNot) {
    emit(t, n.kids[0], out);
    out.ops.push_back(encode_insn(kInsNot, 0, false));
    return;
  }
  const uint32_t mode = n.kind == NodeKind::kAnd ? kModeAnd : kModeOr;
  emit(t, n.kids[0], out);
  for (size_t i = 1; i < n.kids.size(); ++i) {
    int c = n.kids[i];
    if (is_leaf(t, c)) {
      emit_leaf(t, c, mode, out);
    } else {
      out.ops.push_back(encode_insn(kInsPush, 0, false));
      emit(t, c, out);
      out.ops.push_back(encode_insn(kInsPop, mode, false));
    }
  }
}

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
  if (try_flat(tree, root, cq)) return cq;
  emit(tree, root, cq);
  cq.need = tree.nodes[root].need;
  ST_CHECK(cq.need <= kSearchMaxStack, "query plan ", q, " needs ", cq.need,
           " stack slots; this build evaluates at most ", kSearchMaxStack);
  ST_CHECK(cq.terms.size() <= kMaxTermsPerQuery && cq.ops.size() <= kMaxOpsPerQuery,
           "query plan ", q, " is too long (", cq.terms.size(), " terms, ",
           cq.ops.size(), " operations)");
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
        const CompiledQuery& c = cur[i].cq;
        if (c.flat) return 4 + static_cast<int64_t>(c.lits.size()) * (k_eff + 3);
        return 8 + 6 * static_cast<int64_t>(c.ops.size()) +
               static_cast<int64_t>(c.terms.size()) * (k_eff + 3);
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
      std::vector<uint32_t> wave_off(kSearchWaves + 1, 0), starts, insns;
      const uint32_t pos_bytes = static_cast<uint32_t>(plan->kp) * 4;
      for (int w = 0; w < kSearchWaves; ++w) {
        // Within a wave: flat programs by decreasing literal count, paired
        // neighbour by neighbour, then the stack-form ones.
        auto& list = per_wave[w];
        std::stable_sort(list.begin(), list.end(), [&](int x, int y) {
          const CompiledQuery& a = cur[x].cq;
          const CompiledQuery& c = cur[y].cq;
          if (a.flat != c.flat) return a.flat;
          return a.flat && a.lits.size() > c.lits.size();
        });
        size_t n_flat = 0;
        while (n_flat < list.size() && cur[list[n_flat]].cq.flat) ++n_flat;
        for (size_t li = 0; li < list.size(); ++li) {
          const int i = list[li];
          const CompiledQuery& cq = cur[i].cq;
          while (insns.size() % 4) insns.push_back(0);  // 16-byte aligned programs
          starts.push_back(static_cast<uint32_t>(insns.size()));
          const uint32_t row = static_cast<uint32_t>(cur[i].row);
          const bool paired = cq.flat && li % 2 == 0 && li + 1 < n_flat;
          if (cq.flat) {
            insns.insert(insns.end(),
                         {static_cast<uint32_t>(cq.lits.size()) | kFlatForm |
                              (cq.complement ? kFlatComplement : 0u) |
                              (paired ? kPairedWithNext : 0u),
                          row, 0u, 0u});
            for (const auto& l : cq.lits) {
              insns.insert(insns.end(), {l.term * pos_bytes, l.neg ? ~0u : 0u,
                                         l.first ? ~0u : 0u, 0u});
            }
          } else {
            insns.insert(insns.end(), {static_cast<uint32_t>(cq.terms.size()), row,
                                       static_cast<uint32_t>(cq.ops.size()), 0u});
            for (uint32_t t : cq.terms) insns.push_back(t * pos_bytes);
            insns.insert(insns.end(), cq.ops.begin(), cq.ops.end());
          }
        }
        wave_off[w + 1] = static_cast<uint32_t>(starts.size());
      }
      auto& blob = plan->blob;
      b.off_wave = blob.size();
      append_bytes(blob, wave_off.data(), wave_off.size() * 4);
      b.off_insn_start = blob.size();
      append_bytes(blob, starts.data(), starts.size() * 4);
      b.off_insns = blob.size();
      append_bytes(blob, insns.data(), insns.size() * 4);
      b.off_hashes = blob.size();
      append_bytes(blob, terms.hashes.data(), terms.hashes.size() * 8);
      plan->batches.push_back(b);
      plan->batch_insns.push_back(insns);
      plan->batch_starts.push_back(starts);
      plan->batch_hashes.push_back(terms.hashes);
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
    plan->blob.resize(plan->blob.size() + 256, 0);  // slack for scalar loads
    *out = plan.release();
  });
}

namespace st {
namespace {

// Row positions of one term at width b, as the kernel's positions step and
// signature_match (bloom_index_search.cpp:40-61) resolve them: over hashes
// p < hash_k, b_p = (int16)(h[p] % b), repeats skipped, at most k_eff kept;
// unused slots repeat the first.  Staged bundles get LDS byte offsets
// (row * 256, the all-zeros row when nothing resolves); others get signed
// rows relative to the bundle start (kPosZeros when nothing resolves).
void term_positions(const uint64_t* h, int64_t hash_k, int k_eff, int64_t b,
                    int slots, uint32_t* out) {
  int16_t found[kMaxSearchK] = {0};
  int cnt = 0;
  if (b > 0) {
    for (int64_t p = 0; p < hash_k && cnt < k_eff; ++p) {
      const int16_t bp = static_cast<int16_t>(h[p] % static_cast<uint64_t>(b));
      bool dup = false;
      for (int j = 0; j < cnt; ++j) dup |= found[j] == bp;
      if (!dup) found[cnt++] = bp;
    }
  }
  const bool staged = b <= kSearchTileRows;
  for (int j = 0; j < slots; ++j) {
    const int16_t r = j < cnt ? found[j] : found[0];
    if (staged) {
      out[j] = static_cast<uint32_t>(cnt == 0 ? kSearchZerosRow : r) * 256u;
    } else {
      out[j] = cnt == 0 ? static_cast<uint32_t>(kPosZeros)
                        : static_cast<uint32_t>(static_cast<int32_t>(r));
    }
  }
}

}  // namespace
}  // namespace st

extern "C" int st_search_plan_bind_widths(st_search_plan* plan,
                                          const int64_t* bundle_b_offsets,
                                          int64_t num_bundles) {
  using namespace st;
  return guarded([&] {
    ST_CHECK(plan != nullptr, "plan is null");
    ST_CHECK(plan->bound_bundles < 0, "plan is already bound to bundle widths");
    ST_CHECK(num_bundles >= 0, "negative bundle count");
    ST_CHECK(num_bundles == 0 || bundle_b_offsets != nullptr,
             "bundle_b_offsets is null");
    const int k_eff = plan->k_eff;
    const int kp = plan->kp;
    const int rw = bound_record_words(k_eff);
    const uint32_t pos_bytes = static_cast<uint32_t>(kp) * 4;

    // Most frequent widths get slots (ties to the smaller width).
    std::vector<int64_t> width(num_bundles);
    std::unordered_map<int64_t, int64_t> freq;
    for (int64_t i = 0; i < num_bundles; ++i) {
      width[i] = std::max<int64_t>(bundle_b_offsets[i + 1] - bundle_b_offsets[i], 0);
      ++freq[width[i]];
    }
    std::vector<std::pair<int64_t, int64_t>> by_freq(freq.begin(), freq.end());
    std::sort(by_freq.begin(), by_freq.end(), [](const auto& a, const auto& c) {
      return a.second != c.second ? a.second > c.second : a.first < c.first;
    });
    if (by_freq.size() > static_cast<size_t>(kMaxWidthSlots)) by_freq.resize(kMaxWidthSlots);
    std::unordered_map<int64_t, uint32_t> slot_of;
    plan->slot_width.clear();
    for (const auto& wf : by_freq) {
      slot_of[wf.first] = static_cast<uint32_t>(plan->slot_width.size());
      plan->slot_width.push_back(wf.first);
    }
    std::vector<uint32_t> bundle_slot(num_bundles);
    for (int64_t i = 0; i < num_bundles; ++i) {
      auto it = slot_of.find(width[i]);
      bundle_slot[i] = it == slot_of.end() ? kNoWidthSlot : it->second;
    }
    // Visiting order: bundles grouped by slot (then by width), so that a
    // workgroup striding through it meets long runs of one width and reuses
    // that width's programs from the scalar cache.
    std::vector<uint32_t> order(num_bundles);
    for (int64_t i = 0; i < num_bundles; ++i) order[i] = static_cast<uint32_t>(i);
    std::stable_sort(order.begin(), order.end(), [&](uint32_t x, uint32_t y) {
      if (bundle_slot[x] != bundle_slot[y]) return bundle_slot[x] < bundle_slot[y];
      return width[x] < width[y];
    });
    auto& blob = plan->blob;
    plan->off_bundle_slot = blob.size();
    append_bytes(blob, bundle_slot.data(), bundle_slot.size() * 4);
    plan->off_bundle_order = blob.size();
    append_bytes(blob, order.data(), order.size() * 4);

    const size_t nslots = plan->slot_width.size();
    for (size_t bi = 0; bi < plan->batches.size(); ++bi) {
      SearchBatch& bt = plan->batches[bi];
      const auto& insns = plan->batch_insns[bi];
      const auto& starts = plan->batch_starts[bi];
      const auto& hashes = plan->batch_hashes[bi];
      // positions of every term at every slot width
      std::vector<uint32_t> pos(nslots * bt.num_terms * kp);
      for (size_t s = 0; s < nslots; ++s)
        for (uint32_t u = 0; u < bt.num_terms; ++u)
          term_positions(hashes.data() + static_cast<size_t>(u) * plan->hash_k,
                         plan->hash_k, k_eff, plan->slot_width[s], kp,
                         &pos[(s * bt.num_terms + u) * kp]);
      // Literal count of each bound program: paired flat programs are padded
      // to the larger count of the pair.
      std::vector<uint32_t> bound_T(bt.num_slots);
      for (uint32_t q = 0; q < bt.num_slots; ++q) bound_T[q] = insns[starts[q]] & 0xFFFFu;
      for (uint32_t q = 0; q + 1 < bt.num_slots; ++q) {
        if (insns[starts[q]] & kPairedWithNext) {
          const uint32_t t = std::max(bound_T[q], bound_T[q + 1]);
          bound_T[q] = bound_T[q + 1] = t;
        }
      }
      // layout of one width block (identical for every slot)
      std::vector<uint32_t> bstart(bt.num_slots);
      uint32_t words = 0;
      for (uint32_t q = 0; q < bt.num_slots; ++q) {
        bstart[q] = words;
        const uint32_t hdr = insns[starts[q]];
        const uint32_t T = hdr & 0xFFFFu;
        uint32_t n = kProgHeaderWords;
        if (hdr & kFlatForm) {
          n += bound_T[q] * rw;
        } else {
          n += T * kp + insns[starts[q] + 2];
        }
        words += (n + 3) & ~3u;
      }
      std::vector<uint32_t> block(nslots * words, 0);
      for (size_t s = 0; s < nslots; ++s) {
        uint32_t* base = block.data() + s * words;
        const uint32_t* spos = pos.data() + s * bt.num_terms * kp;
        for (uint32_t q = 0; q < bt.num_slots; ++q) {
          const uint32_t* src = insns.data() + starts[q];
          uint32_t* dst = base + bstart[q];
          const uint32_t hdr = src[0];
          const uint32_t T = hdr & 0xFFFFu;
          for (int w = 0; w < kProgHeaderWords; ++w) dst[w] = src[w];
          if (hdr & kFlatForm) {
            dst[0] = (hdr & ~0xFFFFu) | bound_T[q];
            for (uint32_t j = 0; j < T; ++j) {
              const uint32_t* lit = src + kProgHeaderWords + j * kFlatLiteralWords;
              const uint32_t* tp = spos + (lit[0] / pos_bytes) * kp;
              uint32_t* rec = dst + kProgHeaderWords + j * rw;
              for (int r = 0; r < k_eff; ++r) rec[r] = tp[r];
              rec[k_eff] = (lit[1] ? 1u : 0u) | (lit[2] ? 2u : 0u);
            }
            // no-op padding: AND with the all-ones row inside the last group
            const bool staged = plan->slot_width[s] <= kSearchTileRows;
            const uint32_t ones = staged ? static_cast<uint32_t>(kSearchOnesRow) * 256u
                                         : static_cast<uint32_t>(kPosOnes);
            for (uint32_t j = T; j < bound_T[q]; ++j) {
              uint32_t* rec = dst + kProgHeaderWords + j * rw;
              for (int r = 0; r < k_eff; ++r) rec[r] = ones;
              rec[k_eff] = 0;
            }
          } else {
            const uint32_t nops = src[2];
            for (uint32_t j = 0; j < T; ++j) {
              const uint32_t* tp = spos + (src[kProgHeaderWords + j] / pos_bytes) * kp;
              for (int r = 0; r < kp; ++r) dst[kProgHeaderWords + j * kp + r] = tp[r];
            }
            for (uint32_t o = 0; o < nops; ++o)
              dst[kProgHeaderWords + T * kp + o] = src[kProgHeaderWords + T + o];
          }
        }
      }
      bt.bound_words = words;
      bt.off_bound_start = blob.size();
      append_bytes(blob, bstart.data(), bstart.size() * 4);
      bt.off_bound = blob.size();
      append_bytes(blob, block.data(), block.size() * 4);
    }
    // Scalar loads may read a few words past the last program.
    blob.resize(blob.size() + 256, 0);
    plan->bound_bundles = num_bundles;
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
