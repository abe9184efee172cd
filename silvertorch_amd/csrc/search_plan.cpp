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
#include <cstdlib>
#include <cstring>
#include <exception>
#include <functional>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>

#include "search_plan.hpp"
#include "st_common.hpp"
#include "host_pool.hpp"
#include "st_errors.hpp"
#include "wide_balance.hpp"

namespace st {
namespace {

enum class NodeKind { kTerm, kConst, kAnd, kOr, kNot };

// Expression tree of one query.  Child lists live in one shared pool
// (kids[kb .. kb+kn)), so building and simplifying a tree allocates nothing
// once the pools have grown to the largest query seen.
struct Node {
  NodeKind kind;
  bool ones = true;        // kConst: value is all ones (true) or zero
  uint32_t term = 0;       // kTerm: batch-local term id
  int kb = 0, kn = 0;      // kAnd / kOr / kNot: children
  int need = 0;            // stack slots needed to evaluate
};

struct Tree {
  std::vector<Node> nodes;
  std::vector<int> kids;
  void clear() {
    nodes.clear();
    kids.clear();
  }
  int add(const Node& n) {
    nodes.push_back(n);
    return static_cast<int>(nodes.size()) - 1;
  }
  int kid(int id, int j) const { return kids[nodes[id].kb + j]; }
};

// Deepest subtree the flat-form search descends into.
constexpr int kMaxFlatDepth = 64;

template <typename T>
T load_le(const int8_t* p) {
  T v;
  std::memcpy(&v, p, sizeof(T));
  return v;
}

// Interns each distinct hash_k-tuple once per batch: open addressing on a
// 64-bit digest of the tuple, verified against the stored hashes.
struct TermTable {
  int64_t hash_k = 0;
  std::vector<uint64_t> hashes;  // hash_k words per interned term
  std::vector<uint32_t> slots;   // id + 1 (0 = empty); power-of-two size
  uint32_t count = 0, committed = 0;

  uint64_t digest(const int8_t* h) const {
    uint64_t d = 0x9E3779B97F4A7C15ull;
    for (int64_t j = 0; j < hash_k; ++j) {
      d = (d ^ load_le<uint64_t>(h + 8 * j)) * 0xFF51AFD7ED558CCDull;
      d ^= d >> 29;
    }
    return d;
  }
  void place(uint32_t id) {
    const size_t mask = slots.size() - 1;
    size_t i = digest(reinterpret_cast<const int8_t*>(hashes.data() + id * hash_k)) & mask;
    while (slots[i] != 0) i = (i + 1) & mask;
    slots[i] = id + 1;
  }
  void rehash(size_t n) {
    slots.assign(n, 0);
    for (uint32_t id = 0; id < count; ++id) place(id);
  }
  uint32_t intern(const int8_t* h) { return intern(h, digest(h)); }
  // with the digest of h already known
  uint32_t intern(const int8_t* h, uint64_t dg) {
    if ((static_cast<size_t>(count) + 1) * 2 > slots.size())
      rehash(std::max<size_t>(256, slots.size() * 2));
    const size_t mask = slots.size() - 1;
    const size_t bytes = static_cast<size_t>(hash_k) * 8;
    for (size_t i = dg & mask;; i = (i + 1) & mask) {
      const uint32_t s = slots[i];
      if (s == 0) {
        slots[i] = count + 1;
        hashes.resize(hashes.size() + hash_k);
        std::memcpy(hashes.data() + count * hash_k, h, bytes);
        return count++;
      }
      if (std::memcmp(hashes.data() + (s - 1) * hash_k, h, bytes) == 0) return s - 1;
    }
  }
  uint32_t size() const { return count; }
  // room for n terms without growing
  void reserve(size_t n) {
    size_t want = 256;
    while (want < 2 * n + 2) want *= 2;
    if (want > slots.size()) rehash(want);
  }
  void commit() { committed = count; }
  void rollback() {  // forget the terms interned since the last commit()
    count = committed;
    hashes.resize(static_cast<size_t>(count) * hash_k);
    rehash(slots.size());
  }
  void clear() {
    count = committed = 0;
    hashes.clear();
    std::fill(slots.begin(), slots.end(), 0u);
  }
};

bool is_leaf(const Tree& t, int id) {
  const Node& n = t.nodes[id];
  if (n.kind == NodeKind::kTerm || n.kind == NodeKind::kConst) return true;
  if (n.kind == NodeKind::kNot) {
    const Node& c = t.nodes[t.kid(id, 0)];
    return c.kind == NodeKind::kTerm || c.kind == NodeKind::kConst;
  }
  return false;
}

int add_const(Tree& t, bool ones) {
  Node k;
  k.kind = NodeKind::kConst;
  k.ones = ones;
  return t.add(k);
}

// Simplifies one node whose children are already simplified (their ids in
// `repl`): flattens same-kind children, drops double negation, folds
// constants under NOT, orders the children and computes `need`.  Returns
// the id that replaces `id`.
int normalize_node(Tree& t, int id, const std::vector<int>& repl) {
  const NodeKind kind = t.nodes[id].kind;
  if (kind == NodeKind::kTerm || kind == NodeKind::kConst) {
    t.nodes[id].need = 0;
    return id;
  }
  if (kind == NodeKind::kNot) {
    const int c = repl[t.kid(id, 0)];
    if (t.nodes[c].kind == NodeKind::kNot) return t.kid(c, 0);
    if (t.nodes[c].kind == NodeKind::kConst) return add_const(t, !t.nodes[c].ones);
    t.kids[t.nodes[id].kb] = c;
    t.nodes[id].need = t.nodes[c].need;
    return id;
  }
  const int kb = t.nodes[id].kb, kn = t.nodes[id].kn;
  for (int j = 0; j < kn; ++j) t.kids[kb + j] = repl[t.kids[kb + j]];
  // Flattened child list, appended to the pool.
  const int fb = static_cast<int>(t.kids.size());
  for (int j = 0; j < kn; ++j) {
    const int c = t.kids[kb + j];
    if (t.nodes[c].kind == kind) {
      const int cb = t.nodes[c].kb, cn = t.nodes[c].kn;
      for (int g = 0; g < cn; ++g) {
        const int v = t.kids[cb + g];
        t.kids.push_back(v);
      }
    } else {
      t.kids.push_back(c);
    }
  }
  const int fn = static_cast<int>(t.kids.size()) - fb;
  if (fn == 0) return add_const(t, kind == NodeKind::kAnd);
  // Evaluation order: the most demanding subtree first, the other subtrees
  // by decreasing demand, leaves last (stable: equal demands keep their order).
  auto before = [&](int a, int b) {
    const bool la = is_leaf(t, a), lb = is_leaf(t, b);
    if (la != lb) return !la;
    return t.nodes[a].need > t.nodes[b].need;
  };
  int* f = t.kids.data() + fb;
  if (fn > 32) {
    std::stable_sort(f, f + fn, before);
  } else {  // insertion sort (stable; child lists are short)
    for (int i = 1; i < fn; ++i) {
      const int v = f[i];
      int j = i;
      while (j > 0 && before(v, f[j - 1])) {
        f[j] = f[j - 1];
        --j;
      }
      f[j] = v;
    }
  }
  int need = t.nodes[f[0]].need;
  for (int i = 1; i < fn; ++i) {
    if (!is_leaf(t, f[i])) need = std::max(need, 1 + t.nodes[f[i]].need);
  }
  t.nodes[id].kb = fb;
  t.nodes[id].kn = fn;
  t.nodes[id].need = need;
  return id;
}

// Simplifies the tree under `root` bottom-up with an explicit stack (no
// recursion: plans may nest without limit).  Returns the new root.
int normalize(Tree& t, int root, std::vector<int>& repl, std::vector<std::pair<int, int>>& st) {
  repl.assign(t.nodes.size(), -1);
  st.clear();
  st.emplace_back(root, 0);
  while (!st.empty()) {
    const int id = st.back().first;
    const int j = st.back().second;
    const NodeKind kind = t.nodes[id].kind;
    const int kn = (kind == NodeKind::kAnd || kind == NodeKind::kOr || kind == NodeKind::kNot)
                       ? t.nodes[id].kn : 0;
    if (j < kn) {
      st.back().second = j + 1;
      st.emplace_back(t.kid(id, j), 0);
      continue;
    }
    repl[id] = normalize_node(t, id, repl);  // ids on the stack are nodes of the built tree
    st.pop_back();
  }
  return repl[root];
}

struct CompiledQuery {
  std::vector<uint32_t> terms;  // stack form: term ids in consumption order
  std::vector<uint32_t> ops;    // stack form: operations
  int need = 0;
  bool generic = false;         // stack form beyond the batch kernels' limits
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

// At most kFlatMaxLiterals literals, hence at most as many groups.  Copies
// move only the used prefix of the arrays.
struct Dnf {
  bool is_true = false;  // the constant all-ones
  int nlits = 0, ngroups = 0;  // ngroups == 0 and !is_true: constant zero
  uint8_t gend[kFlatMaxLiterals];  // end of group g in lits
  Lit lits[kFlatMaxLiterals];

  Dnf() = default;
  explicit Dnf(bool ones) : is_true(ones) {}
  Dnf(const Dnf& o) { *this = o; }
  Dnf& operator=(const Dnf& o) {
    is_true = o.is_true;
    nlits = o.nlits;
    ngroups = o.ngroups;
    std::memcpy(gend, o.gend, static_cast<size_t>(ngroups));
    std::memcpy(lits, o.lits, sizeof(Lit) * static_cast<size_t>(nlits));
    return *this;
  }
  int gbegin(int g) const { return g ? gend[g - 1] : 0; }
  // Appends a group; false when the literal budget would be exceeded.
  bool push(const Lit* g, int n) {
    if (nlits + n > kFlatMaxLiterals) return false;
    for (int i = 0; i < n; ++i) lits[nlits + i] = g[i];
    nlits += n;
    gend[ngroups++] = static_cast<uint8_t>(nlits);
    return true;
  }
};

// Conjunction of two DNFs by distribution, built in `out` (which must be
// neither operand); false when it exceeds the budget.
bool dnf_and(const Dnf& a, const Dnf& b, Dnf& out) {
  if (a.is_true) { out = b; return true; }
  if (b.is_true) { out = a; return true; }
  Dnf& r = out;
  r.is_true = false;
  r.nlits = r.ngroups = 0;
  Lit g[2 * kFlatMaxLiterals];
  for (int ia = 0; ia < a.ngroups; ++ia) {
    for (int ib = 0; ib < b.ngroups; ++ib) {
      int n = 0;
      for (int i = a.gbegin(ia); i < a.gend[ia]; ++i) g[n++] = a.lits[i];
      for (int i = b.gbegin(ib); i < b.gend[ib]; ++i) g[n++] = b.lits[i];
      for (int i = 1; i < n; ++i) {  // sort (insertion: groups are short)
        const Lit v = g[i];
        int j = i;
        while (j > 0 && v < g[j - 1]) {
          g[j] = g[j - 1];
          --j;
        }
        g[j] = v;
      }
      n = static_cast<int>(std::unique(g, g + n) - g);
      bool contradiction = false;
      for (int i = 1; i < n; ++i) contradiction |= g[i].term == g[i - 1].term;  // t, ~t
      if (contradiction) continue;
      if (!r.push(g, n)) return false;
    }
  }
  return true;
}

bool to_dnf(const Tree& t, int id, bool negated, int depth, Dnf& out) {
  if (depth > kMaxFlatDepth) return false;
  const Node& n = t.nodes[id];
  switch (n.kind) {
    case NodeKind::kTerm: {
      out = Dnf(false);
      const Lit l{n.term, negated};
      out.push(&l, 1);
      return true;
    }
    case NodeKind::kConst:
      out = Dnf(n.ones != negated);
      return true;
    case NodeKind::kNot:
      return to_dnf(t, t.kid(id, 0), !negated, depth + 1, out);
    case NodeKind::kAnd:
    case NodeKind::kOr: {
      // accumulated in `out`; conjunctions alternate between `out` and a
      // second buffer (no copies of the running DNF)
      const bool conj = (n.kind == NodeKind::kAnd) != negated;
      out.is_true = conj;
      out.nlits = out.ngroups = 0;
      Dnf d, other;
      Dnf* acc = &out;
      Dnf* spare = &other;
      for (int j = 0; j < n.kn; ++j) {
        if (!to_dnf(t, t.kid(id, j), negated, depth + 1, d)) return false;
        if (conj) {
          if (!dnf_and(*acc, d, *spare)) return false;
          std::swap(acc, spare);
        } else {
          if (acc->is_true) continue;
          if (d.is_true) {
            acc->is_true = true;
            acc->nlits = acc->ngroups = 0;
            continue;
          }
          for (int g = 0; g < d.ngroups; ++g)
            if (!acc->push(d.lits + d.gbegin(g), d.gend[g] - d.gbegin(g))) return false;
        }
      }
      if (acc != &out) out = *acc;
      return true;
    }
  }
  return false;
}

// Fills cq's flat form when the query (or its complement) has a DNF of at
// most kFlatMaxLiterals literals.  A direct form with no more literals than
// the query has term leaves repeats no term, and the complement cannot be
// shorter, so it is not tried then.
bool try_flat(const Tree& t, int root, int term_leaves, CompiledQuery& cq) {
  Dnf direct, inverse;
  const bool ok_d = to_dnf(t, root, false, 0, direct);
  const bool ok_i = !(ok_d && direct.nlits <= term_leaves) &&
                    to_dnf(t, root, true, 0, inverse);
  if (!ok_d && !ok_i) return false;
  const bool use_inverse = !ok_d || (ok_i && inverse.nlits < direct.nlits);
  const Dnf& d = use_inverse ? inverse : direct;
  cq.flat = true;
  cq.lits.clear();
  if (d.is_true) {
    cq.complement = !use_inverse;  // empty OR is zero; complement gives ones
    return true;
  }
  cq.complement = use_inverse;
  cq.lits.reserve(d.nlits);
  for (int g = 0; g < d.ngroups; ++g) {
    for (int i = d.gbegin(g); i < d.gend[g]; ++i)
      cq.lits.push_back(CompiledQuery::FlatLit{d.lits[i].term, d.lits[i].neg,
                                               i == d.gbegin(g)});
  }
  return true;
}

void emit_leaf(const Tree& t, int id, uint32_t mode, CompiledQuery& out) {
  const Node& n = t.nodes[id];
  bool neg = false;
  const Node* leaf = &n;
  if (n.kind == NodeKind::kNot) {
    neg = true;
    leaf = &t.nodes[t.kid(id, 0)];
  }
  if (leaf->kind == NodeKind::kTerm) {
    out.terms.push_back(leaf->term);
    out.ops.push_back(encode_insn(kInsTerm, mode, neg));
  } else {
    out.ops.push_back(encode_insn(kInsConst, mode, neg != !leaf->ones));
  }
}

// Stack-form program of the tree under `root`: a leaf is loaded into the
// accumulator; a NOT complements it; an AND / OR evaluates its first child
// into the accumulator and combines each further child -- a leaf directly,
// a subtree by PUSH, the subtree, POP.  Explicit stack of (node, state):
// state -1 = not started, else (next child << 1) | (a POP is due).
void emit(const Tree& t, int root, CompiledQuery& out, std::vector<std::pair<int, int>>& st) {
  st.clear();
  st.emplace_back(root, -1);
  while (!st.empty()) {
    const int id = st.back().first;
    const int state = st.back().second;
    if (state == -1) {
      if (is_leaf(t, id)) {
        emit_leaf(t, id, kModeSet, out);
        st.pop_back();
        continue;
      }
      st.back().second = 1 << 1;
      st.emplace_back(t.kid(id, 0), -1);
      continue;
    }
    const Node& n = t.nodes[id];
    if (n.kind == NodeKind::kNot) {
      out.ops.push_back(encode_insn(kInsNot, 0, false));
      st.pop_back();
      continue;
    }
    const uint32_t mode = n.kind == NodeKind::kAnd ? kModeAnd : kModeOr;
    if (state & 1) out.ops.push_back(encode_insn(kInsPop, mode, false));
    int next = state >> 1;
    bool descended = false;
    for (; next < n.kn; ++next) {
      const int c = t.kid(id, next);
      if (is_leaf(t, c)) {
        emit_leaf(t, c, mode, out);
        continue;
      }
      out.ops.push_back(encode_insn(kInsPush, 0, false));
      st.back().second = ((next + 1) << 1) | 1;
      st.emplace_back(c, -1);
      descended = true;
      break;
    }
    if (!descended) st.pop_back();
  }
}

// Per-thread working storage of the compiler, kept between calls so that
// compiling a batch allocates only its results.
struct CompileScratch {
  Tree tree;
  std::vector<int> stack;
  std::vector<int> repl;                     // normalize: replacement of each node
  std::vector<std::pair<int, int>> walk;     // normalize / emit: explicit traversal stack
  // flat_direct: literals in stack order, and the stack of (kind, first literal)
  std::vector<CompiledQuery::FlatLit> lits;
  std::vector<std::pair<uint8_t, uint32_t>> items;
};

// Direct flat form of a query whose plan is already an OR of AND-groups of
// terms (nested ANDs / ORs of the same shape included, as the parser's
// max_sub_queries folding makes them): one pass over the postfix operators,
// no tree.  Literals are kept in stack order, so the operands an operator
// pops are one contiguous run: AND joins the run into one group, OR keeps
// the runs' groups.  Returns false (nothing interned is lost: interning is
// idempotent) for anything else -- NOT, EMPTY, an AND over an OR, a child
// count outside [1, stack size], more than kFlatMaxLiterals literals, a
// malformed plan -- and the general compiler then handles the query (and
// raises its errors).  The result equals the general DNF of such a plan up
// to the order of literals within a group and repeated literals, which do
// not change the OR-of-ANDs value.
bool flat_direct(const int8_t* ops, int64_t n_ops, const int8_t* offsets, int64_t n_offsets,
                 const int8_t* hashes, int64_t n_hashes, int64_t hash_k, int k_eff,
                 TermTable& terms, CompileScratch& cs, CompiledQuery& cq) {
  if (k_eff == 0 || hash_k <= 0 || n_offsets < n_ops + 1) return false;
  constexpr uint8_t kLit = 0, kAndGroup = 1, kOrGroups = 2;
  auto& lits = cs.lits;
  auto& items = cs.items;
  lits.clear();
  items.clear();
  int64_t term_counter = 0;
  for (int64_t i = 0; i < n_ops; ++i) {
    const uint8_t op = static_cast<uint8_t>(ops[i]);
    if (op == kOpTerm) {
      if ((term_counter + 1) * hash_k > n_hashes || lits.size() >= kFlatMaxLiterals) return false;
      const uint32_t t = terms.intern(hashes + 8 * term_counter * hash_k);
      ++term_counter;
      items.emplace_back(kLit, static_cast<uint32_t>(lits.size()));
      lits.push_back(CompiledQuery::FlatLit{t, false, true});
      continue;
    }
    if (op != kOpAnd && op != kOpOr) return false;
    const int32_t children = load_le<int32_t>(offsets + 4 * (i + 1)) - load_le<int32_t>(offsets + 4 * i);
    if (children < 1 || static_cast<size_t>(children) > items.size()) return false;
    const size_t first = items.size() - static_cast<size_t>(children);
    const uint32_t begin = items[first].second;
    if (op == kOpAnd) {
      for (size_t j = first; j < items.size(); ++j)
        if (items[j].first == kOrGroups) return false;
      for (size_t l = begin + 1; l < lits.size(); ++l) lits[l].first = false;
      items.resize(first);
      items.emplace_back(kAndGroup, begin);
    } else {
      items.resize(first);
      items.emplace_back(kOrGroups, begin);
    }
  }
  if (items.empty()) return false;
  const uint32_t begin = items.back().second;
  cq.flat = true;
  cq.complement = false;
  cq.lits.assign(lits.begin() + begin, lits.end());
  return true;
}

// Decodes query q, builds its tree and returns its program.  Terms are
// interned in `terms` (ids are batch-local).
CompiledQuery compile_query(const int8_t* data, int64_t data_len,
                            const int64_t* offs, int64_t q, int64_t hash_k,
                            int k_eff, TermTable& terms, CompileScratch& cs) {
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
  {
    CompiledQuery cq;
    if (flat_direct(ops, n_ops, offsets, n_offsets, hashes, n_hashes, hash_k, k_eff, terms, cs, cq))
      return cq;
  }

  Tree& tree = cs.tree;
  std::vector<int>& stack = cs.stack;
  tree.clear();
  stack.clear();
  int64_t term_counter = 0;
  auto child_count = [&](int64_t i) -> int32_t {
    ST_CHECK(i + 1 < n_offsets, "query plan ", q, ": operator ", i,
             " has no child count (offsets array holds ", n_offsets,
             " entries)");
    return load_le<int32_t>(offsets + 4 * (i + 1)) -
           load_le<int32_t>(offsets + 4 * i);
  };
  auto push = [&](const Node& n) { stack.push_back(tree.add(n)); };
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
        push(n);
        break;
      }
      case kOpEmpty: {
        Node n;
        n.kind = NodeKind::kConst;
        n.ones = true;
        push(n);
        break;
      }
      case kOpAnd:
      case kOpOr: {
        // A count below one pops nothing: the operator's identity results.
        const int32_t children = std::max<int32_t>(child_count(i), 0);
        ST_CHECK(static_cast<size_t>(children) <= stack.size(), "query plan ", q,
                 ": operator ", i, " pops ", child_count(i),
                 " values from a shorter stack");
        Node n;
        n.kind = op == kOpAnd ? NodeKind::kAnd : NodeKind::kOr;
        n.kb = static_cast<int>(tree.kids.size());
        n.kn = children;
        for (int32_t j = 0; j < children; ++j) {  // top of the stack first
          tree.kids.push_back(stack.back());
          stack.pop_back();
        }
        push(n);
        break;
      }
      case kOpNot: {
        const int32_t children = child_count(i);
        ST_CHECK(children == 1, "NOT query should have 1 parameter, but got ",
                 children);
        ST_CHECK(!stack.empty(), "query plan ", q, ": NOT operator ", i,
                 " applied to an empty stack");
        Node n;
        n.kind = NodeKind::kNot;
        n.kb = static_cast<int>(tree.kids.size());
        n.kn = 1;
        tree.kids.push_back(stack.back());
        stack.pop_back();
        push(n);
        break;
      }
      default:
        fail("unknown operator: ", static_cast<int>(op));
    }
  }
  ST_CHECK(!stack.empty(), "query plan ", q, " leaves an empty stack");
  const int root = normalize(tree, stack.back(), cs.repl, cs.walk);
  CompiledQuery cq;
  if (try_flat(tree, root, static_cast<int>(term_counter), cq)) return cq;
  emit(tree, root, cq, cs.walk);
  cq.need = tree.nodes[root].need;
  // Children are ordered by demand, so a program needs at most about
  // log2(leaves) + 1 slots: within the size limits below, at most 30.
  ST_CHECK(cq.need <= kGenericMaxStack, "query plan ", q, " needs ", cq.need,
           " stack slots; this build evaluates at most ", kGenericMaxStack);
  ST_CHECK(cq.terms.size() < kGenericMaxTerms && cq.ops.size() < kGenericMaxTerms,
           "query plan ", q, " is too long (", cq.terms.size(), " terms, ",
           cq.ops.size(), " operations)");
  cq.generic = cq.need > kSearchMaxStack || cq.terms.size() > kMaxTermsPerQuery ||
               cq.ops.size() > kMaxOpsPerQuery;
  return cq;
}

// Blob buffers of destroyed plans, kept with their capacity: a fresh buffer
// of a few hundred KB would be mapped anew by the allocator on every call and
// page-faulted in word by word.
std::mutex g_blob_pool_mu;
std::vector<std::vector<uint8_t>> g_blob_pool;
constexpr size_t kBlobPoolSize = 4;

std::vector<uint8_t> take_blob_buffer() {
  std::lock_guard<std::mutex> lock(g_blob_pool_mu);
  if (g_blob_pool.empty()) return {};
  std::vector<uint8_t> b = std::move(g_blob_pool.back());
  g_blob_pool.pop_back();
  b.clear();
  return b;
}

void return_blob_buffer(std::vector<uint8_t>&& b) {
  std::lock_guard<std::mutex> lock(g_blob_pool_mu);
  if (g_blob_pool.size() < kBlobPoolSize) g_blob_pool.push_back(std::move(b));
}

void append_bytes(std::vector<uint8_t>& blob, const void* p, size_t n) {
  const uint8_t* b = static_cast<const uint8_t*>(p);
  blob.insert(blob.end(), b, b + n);
  while (blob.size() % 16) blob.push_back(0);
}

}  // namespace
}  // namespace st

namespace st {
namespace {

// Appends query `row`'s program (search_plan.hpp layouts), 16-byte aligned;
// returns its first word.  Term references are term * pos_bytes.
uint32_t append_program(std::vector<uint32_t>& insns, const CompiledQuery& cq, uint32_t row,
                        uint32_t pos_bytes, bool paired) {
  while (insns.size() % 4) insns.push_back(0);
  const uint32_t start = static_cast<uint32_t>(insns.size());
  if (cq.flat) {
    insns.insert(insns.end(),
                 {static_cast<uint32_t>(cq.lits.size()) | kFlatForm |
                      (cq.complement ? kFlatComplement : 0u) | (paired ? kPairedWithNext : 0u),
                  row, 0u, 0u});
    for (const auto& l : cq.lits)
      insns.insert(insns.end(), {l.term * pos_bytes, l.neg ? ~0u : 0u, l.first ? ~0u : 0u, 0u});
  } else {
    insns.insert(insns.end(), {static_cast<uint32_t>(cq.terms.size()), row,
                               static_cast<uint32_t>(cq.ops.size()), 0u});
    for (uint32_t t : cq.terms) insns.push_back(t * pos_bytes);
    insns.insert(insns.end(), cq.ops.begin(), cq.ops.end());
  }
  return start;
}

}  // namespace
}  // namespace st

namespace st {
namespace {

// Plans of at least this many bytes are compiled on the pool (below it the
// workers' wake-up costs more than it saves: 256 flat queries take ~0.15 ms
// on one thread).
constexpr int64_t kParallelCompileBytes = 192 * 1024;

// One query compiled on its own: its term ids are local (first appearance
// in the query), local_hashes holds their hashes, and the batch ids replace
// them when the query joins a batch.  A query that fails keeps its error.
struct LocalQuery {
  CompiledQuery cq;
  std::vector<uint64_t> local_hashes;
  std::vector<uint64_t> digests;  // TermTable digest of each local term
  uint32_t local_terms = 0;
  std::exception_ptr error;
};

void compile_local(const int8_t* data, int64_t data_len, const int64_t* offs, int64_t q,
                   int64_t hash_k, int k_eff, LocalQuery& out) {
  static thread_local TermTable terms;
  static thread_local CompileScratch scratch;
  terms.hash_k = std::max<int64_t>(hash_k, 0);
  terms.clear();
  try {
    out.cq = compile_query(data, data_len, offs, q, hash_k, k_eff, terms, scratch);
    out.local_terms = terms.size();
    out.local_hashes.assign(terms.hashes.begin(), terms.hashes.end());
    out.digests.resize(out.local_terms);
    for (uint32_t i = 0; i < out.local_terms; ++i)
      out.digests[i] = terms.digest(reinterpret_cast<const int8_t*>(terms.hashes.data() + i * terms.hash_k));
  } catch (...) {
    out.error = std::current_exception();
  }
}

// Batch ids of a compiled query's local terms, interned into `terms`.
void intern_local(const LocalQuery& lq, int64_t hash_k, TermTable& terms, std::vector<uint32_t>& ids) {
  ids.resize(lq.local_terms);
  for (uint32_t i = 0; i < lq.local_terms; ++i)
    ids[i] = terms.intern(reinterpret_cast<const int8_t*>(lq.local_hashes.data() + i * hash_k),
                          lq.digests[i]);
}

void rename_terms(CompiledQuery& cq, const std::vector<uint32_t>& ids) {
  for (auto& l : cq.lits) l.term = ids[l.term];
  for (auto& t : cq.terms) t = ids[t];
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
    plan->blob = take_blob_buffer();
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
    cur.reserve(static_cast<size_t>(std::min<int64_t>(num_queries, 1 << 16)));
    static thread_local TermTable terms;
    terms.hash_k = std::max<int64_t>(hash_k, 0);
    terms.clear();

    auto flush = [&]() {
      if (cur.empty()) return;
      SearchBatch b;
      b.num_slots = static_cast<uint32_t>(cur.size());
      b.num_terms = terms.size();
      // Assignment of queries to the waves of a workgroup.  Flat programs,
      // longest first, are cut into rounds of as many programs as the
      // kernel's literal stream evaluates in lockstep (similar lengths, so
      // little padding); whole rounds go to the least loaded wave, longest
      // first, then the stack-form programs one by one.  Cost ~ literal
      // steps times the row reads and instructions of one step.
      const int per_round = stream_block_records(std::max(plan->k_eff, 1));
      auto cost = [&](int i) {
        const CompiledQuery& c = cur[i].cq;
        if (c.flat) return 4 + static_cast<int64_t>(c.lits.size()) * (k_eff + 3);
        return 8 + 6 * static_cast<int64_t>(c.ops.size()) +
               static_cast<int64_t>(c.terms.size()) * (k_eff + 3);
      };
      std::vector<int> flat_q, stack_q;
      for (size_t i = 0; i < cur.size(); ++i)
        (cur[i].cq.flat ? flat_q : stack_q).push_back(static_cast<int>(i));
      std::stable_sort(flat_q.begin(), flat_q.end(), [&](int a, int c) {
        return cur[a].cq.lits.size() > cur[c].cq.lits.size();
      });
      std::stable_sort(stack_q.begin(), stack_q.end(),
                       [&](int a, int c) { return cost(a) > cost(c); });
      struct Round {
        size_t first, count;
        int64_t cost;
      };
      std::vector<Round> rounds;
      for (size_t r0 = 0; r0 < flat_q.size(); r0 += per_round) {
        const size_t n = std::min<size_t>(per_round, flat_q.size() - r0);
        const int64_t steps = std::max<int64_t>(1, cur[flat_q[r0]].cq.lits.size());
        rounds.push_back({r0, n, 4 + steps * per_round * (k_eff + 3)});
      }
      // rounds arrive longest first already; a stable sort keeps the one
      // partial round behind the full rounds of its length
      std::stable_sort(rounds.begin(), rounds.end(),
                       [](const Round& x, const Round& y) { return x.cost > y.cost; });
      std::vector<std::vector<int>> per_wave(kSearchWaves);
      std::vector<std::vector<const Round*>> wave_rounds(kSearchWaves);
      std::vector<int64_t> load(kSearchWaves, 0);
      auto least_loaded = [&]() {
        return static_cast<int>(std::min_element(load.begin(), load.end()) - load.begin());
      };
      for (const Round& r : rounds) {
        const int w = least_loaded();
        wave_rounds[w].push_back(&r);
        load[w] += r.cost;
      }
      for (int w = 0; w < kSearchWaves; ++w) {
        // the batch's one partial round (if any) goes last in its wave, so
        // that cutting the wave's flat programs into rounds in order finds
        // the same rounds again
        std::stable_sort(wave_rounds[w].begin(), wave_rounds[w].end(),
                         [](const Round* x, const Round* y) { return x->count > y->count; });
        for (const Round* r : wave_rounds[w])
          for (size_t i = 0; i < r->count; ++i) per_wave[w].push_back(flat_q[r->first + i]);
      }
      for (int i : stack_q) {
        const int w = least_loaded();
        per_wave[w].push_back(i);
        load[w] += cost(i);
      }
      std::vector<uint32_t> wave_off(kSearchWaves + 1, 0), starts, insns;
      size_t insn_words = 0;
      for (const Pending& pq : cur)
        insn_words += 8 + (pq.cq.flat ? 4 * pq.cq.lits.size() : pq.cq.terms.size() + pq.cq.ops.size());
      insns.reserve(insn_words);
      starts.reserve(cur.size());
      const uint32_t pos_bytes = static_cast<uint32_t>(plan->kp) * 4;
      for (int w = 0; w < kSearchWaves; ++w) {
        // Within a wave: flat programs round by round, paired neighbour by
        // neighbour, then the stack-form ones.
        auto& list = per_wave[w];
        size_t n_flat = 0;
        while (n_flat < list.size() && cur[list[n_flat]].cq.flat) ++n_flat;
        for (size_t li = 0; li < list.size(); ++li) {
          const int i = list[li];
          const CompiledQuery& cq = cur[i].cq;
          starts.push_back(append_program(insns, cq, static_cast<uint32_t>(cur[i].row), pos_bytes,
                                          cq.flat && li % 2 == 0 && li + 1 < n_flat));
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
      plan->batch_insns.push_back(std::move(insns));
      plan->batch_starts.push_back(std::move(starts));
      plan->batch_hashes.push_back(std::move(terms.hashes));
      cur.clear();
      terms.clear();
    };

    // Queries are compiled in order, their terms interned into the running
    // batch.  Large plans are first compiled query by query on the pool with
    // local term ids; in query order, each query's terms then join the
    // batch and its program is renamed.  Queries beyond the batch kernels'
    // limits (stack depth, program size, or more distinct terms than a
    // batch's position area holds on their own) each become a generic batch,
    // after the regular ones.
    const bool parallel = plans_data_len >= kParallelCompileBytes && num_queries > 1;
    const int64_t hk = std::max<int64_t>(hash_k, 0);
    std::vector<LocalQuery> local;
    std::vector<int64_t> generic_q;
    std::vector<uint32_t> ids;
    if (parallel) {
      local.resize(static_cast<size_t>(num_queries));
      host_pool_run(num_queries, 32, [&](int64_t q) {
        compile_local(plans_data, plans_data_len, plans_offsets, q, hash_k, plan->k_eff,
                      local[static_cast<size_t>(q)]);
      });
      for (const LocalQuery& lq : local)  // the first failing query's error
        if (lq.error) std::rethrow_exception(lq.error);
      size_t leaves = 0;
      for (const LocalQuery& lq : local) leaves += lq.local_terms;
      terms.reserve(std::min<size_t>(leaves, static_cast<size_t>(term_capacity) + 1));
      for (int64_t q = 0; q < num_queries; ++q) {
        LocalQuery& lq = local[static_cast<size_t>(q)];
        intern_local(lq, hk, terms, ids);
        if (!lq.cq.generic && static_cast<int64_t>(terms.size()) > term_capacity) {
          terms.rollback();
          flush();
          intern_local(lq, hk, terms, ids);
        }
        if (lq.cq.generic || static_cast<int64_t>(terms.size()) > term_capacity) {
          terms.rollback();
          generic_q.push_back(q);
          continue;
        }
        terms.commit();
        rename_terms(lq.cq, ids);
        plan->max_stack = std::max(plan->max_stack, lq.cq.need);
        cur.push_back(Pending{q, std::move(lq.cq)});
      }
    } else {
      static thread_local CompileScratch scratch;
      for (int64_t q = 0; q < num_queries; ++q) {
        CompiledQuery cq = compile_query(plans_data, plans_data_len, plans_offsets, q, hash_k,
                                         plan->k_eff, terms, scratch);
        if (!cq.generic && static_cast<int64_t>(terms.size()) > term_capacity) {
          terms.rollback();
          flush();
          cq = compile_query(plans_data, plans_data_len, plans_offsets, q, hash_k, plan->k_eff,
                             terms, scratch);
        }
        if (cq.generic || static_cast<int64_t>(terms.size()) > term_capacity) {
          terms.rollback();
          generic_q.push_back(q);
          continue;
        }
        terms.commit();
        plan->max_stack = std::max(plan->max_stack, cq.need);
        cur.push_back(Pending{q, std::move(cq)});
      }
    }
    flush();
    for (const int64_t q : generic_q) {
      // alone in its batch: the local term ids are the batch's
      terms.clear();
      LocalQuery single;
      if (!parallel)
        compile_local(plans_data, plans_data_len, plans_offsets, q, hash_k, plan->k_eff, single);
      const LocalQuery& lq = parallel ? local[static_cast<size_t>(q)] : single;
      intern_local(lq, hk, terms, ids);
      const CompiledQuery& cq = lq.cq;
      plan->max_stack = std::max(plan->max_stack, cq.need);
      SearchBatch b;
      b.generic = true;
      b.num_slots = 1;
      b.num_terms = terms.size();
      std::vector<uint32_t> wave_off(kSearchWaves + 1, 1u), starts, insns;
      wave_off[0] = 0;
      starts.push_back(append_program(insns, cq, static_cast<uint32_t>(q),
                                      static_cast<uint32_t>(plan->kp) * 4, false));
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
      plan->batch_insns.push_back(std::move(insns));
      plan->batch_starts.push_back(std::move(starts));
      plan->batch_hashes.push_back(std::move(terms.hashes));
    }
    terms.clear();
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
                    const FastMod64& fm, int slots, uint32_t* out) {
  int16_t found[kMaxSearchK] = {0};
  int cnt = 0;
  if (b > 0) {
    for (int64_t p = 0; p < hash_k && cnt < k_eff; ++p) {
      const int16_t bp = static_cast<int16_t>(fast_mod(h[p], fm));
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
    } else if (wide_width(b)) {
      out[j] = static_cast<uint32_t>(cnt == 0 ? kWideZerosRow : r) * kWideSliceBytes;
    } else {
      out[j] = cnt == 0 ? static_cast<uint32_t>(kPosZeros)
                        : static_cast<uint32_t>(static_cast<int32_t>(r));
    }
  }
}

}  // namespace
}  // namespace st

namespace st {
namespace {

uint64_t align_to(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

// Template of one batch's width block: every bound program (the layout the
// kernel's per-query loop reads), then the batch's literal stream (absent
// only when an output row does not fit a record's row field).  Each position word is a code (term,
// position index) resolved at each slot width, on the host
// (st_search_plan_bind_widths) or on the device.  Sets bt.stream_off and
// bt.stream_words; wave_rec / wave_skip receive the per-wave stream tables
// (all zero without a stream), units the stream's balance units (the block
// word of every fourth record of a round step, when balance_applies).
void build_block_template(const st_search_plan& plan, SearchBatch& bt,
                          const std::vector<uint32_t>& insns,
                          const std::vector<uint32_t>& starts, std::vector<uint32_t>& bstart,
                          std::vector<uint32_t>& tmpl, std::vector<uint32_t>& code,
                          std::vector<uint32_t>& wave_rec, std::vector<uint32_t>& wave_skip,
                          std::vector<uint32_t>& units) {
  const int k_eff = plan.k_eff, kp = plan.kp, rw = bound_record_words(k_eff);
  const uint32_t pos_bytes = static_cast<uint32_t>(kp) * 4;
  std::vector<uint32_t> bound_T(bt.num_slots);
  for (uint32_t q = 0; q < bt.num_slots; ++q) bound_T[q] = insns[starts[q]] & 0xFFFFu;
  for (uint32_t q = 0; q + 1 < bt.num_slots; ++q) {
    if (insns[starts[q]] & kPairedWithNext) {
      const uint32_t t = std::max(bound_T[q], bound_T[q + 1]);
      bound_T[q] = bound_T[q + 1] = t;
    }
  }
  bstart.assign(bt.num_slots, 0);
  uint32_t words = 0;
  for (uint32_t q = 0; q < bt.num_slots; ++q) {
    bstart[q] = words;
    const uint32_t hdr = insns[starts[q]];
    uint32_t n = kProgHeaderWords;
    n += (hdr & kFlatForm) ? bound_T[q] * rw : (hdr & 0xFFFFu) * kp + insns[starts[q] + 2];
    words += (n + 3) & ~3u;
  }
  tmpl.assign(words, 0u);
  code.assign(words, kTmplCopy);
  for (uint32_t q = 0; q < bt.num_slots; ++q) {
    const uint32_t* src = insns.data() + starts[q];
    uint32_t* dst = tmpl.data() + bstart[q];
    uint32_t* dc = code.data() + bstart[q];
    const uint32_t hdr = src[0];
    const uint32_t T = hdr & 0xFFFFu;
    for (int w = 0; w < kProgHeaderWords; ++w) dst[w] = src[w];
    if (hdr & kFlatForm) {
      dst[0] = (hdr & ~0xFFFFu) | bound_T[q];
      for (uint32_t j = 0; j < T; ++j) {
        const uint32_t* lit = src + kProgHeaderWords + j * kFlatLiteralWords;
        const uint32_t term = lit[0] / pos_bytes;
        const uint32_t at = kProgHeaderWords + j * rw;
        for (int r = 0; r < k_eff; ++r) dc[at + r] = tmpl_position_code(term, r);
        dst[at + k_eff] = (lit[1] ? 1u : 0u) | (lit[2] ? 2u : 0u);
      }
      for (uint32_t j = T; j < bound_T[q]; ++j) {  // no-op padding records
        const uint32_t at = kProgHeaderWords + j * rw;
        for (int r = 0; r < k_eff; ++r) dc[at + r] = kTmplOnes;
        dst[at + k_eff] = 0u;
      }
    } else {
      const uint32_t nops = src[2];
      for (uint32_t j = 0; j < T; ++j) {
        const uint32_t term = src[kProgHeaderWords + j] / pos_bytes;
        for (int r = 0; r < kp; ++r)
          dc[kProgHeaderWords + j * kp + r] = tmpl_position_code(term, r);
      }
      for (uint32_t o = 0; o < nops; ++o)
        dst[kProgHeaderWords + T * kp + o] = src[kProgHeaderWords + T + o];
    }
  }

  // Literal stream: per wave, its leading flat programs in rounds of
  // per_block slots, in the order the compiler laid them out.  Records follow the kernel's K, which is 1
  // when no position resolves (k_eff 0: no term literals then).
  const uint32_t* wave_off = reinterpret_cast<const uint32_t*>(plan.blob.data() + bt.off_wave);
  const int ks = std::max(k_eff, 1);
  const int srw = bound_record_words(ks);
  const uint32_t per_block = static_cast<uint32_t>(stream_block_records(ks));
  wave_rec.assign(kSearchWaves + 1, 0u);
  wave_skip.assign(kSearchWaves, 0u);
  units.clear();
  const bool balance = balance_applies(ks);
  bt.stream_off = static_cast<uint32_t>(tmpl.size());
  bt.stream_words = 0;
  bool fits = true;
  // The stream's exact size first, so that it is written in place.
  size_t stream_total = 0;
  for (int w = 0; w < kSearchWaves; ++w) {
    uint32_t n_flat = 0;
    while (wave_off[w] + n_flat < wave_off[w + 1] && (insns[starts[wave_off[w] + n_flat]] & kFlatForm))
      ++n_flat;
    for (uint32_t r0 = 0; r0 < n_flat; r0 += per_block) {
      const uint32_t n = std::min(per_block, n_flat - r0);
      uint32_t T = 1;
      for (uint32_t i = 0; i < n; ++i) T = std::max(T, insns[starts[wave_off[w] + r0 + i]] & 0xFFFFu);
      stream_total += kRoundHeaderWords + static_cast<size_t>(T) * per_block * srw;
    }
  }
  size_t at = tmpl.size();
  tmpl.resize(at + stream_total, 0u);
  code.resize(at + stream_total, kTmplCopy);
  auto word = [&](uint32_t v) { tmpl[at++] = v; };
  auto record = [&](uint32_t pos_code, uint32_t term, uint32_t flags) {
    for (int r = 0; r < ks; ++r)
      code[at + r] = pos_code == kTmplCopy ? tmpl_position_code(term, r) : pos_code;
    tmpl[at + ks] = flags;
    at += srw;
  };
  // Group masks instead of flag bits when no literal of the batch's flat
  // programs is negated.
  bool masks = true;
  for (uint32_t q = 0; q < bt.num_slots && masks; ++q) {
    const uint32_t* src = insns.data() + starts[q];
    if (!(src[0] & kFlatForm)) continue;
    const uint32_t T = src[0] & 0xFFFFu;
    for (uint32_t j = 0; j < T; ++j)
      if (src[kProgHeaderWords + j * kFlatLiteralWords + 1]) masks = false;
  }
  auto lit_flags = [&](bool neg, bool first) -> uint32_t {
    if (masks) return first ? ~0u : 0u;
    return (neg ? kStreamNeg : 0u) | (first ? kStreamFirst : 0u);
  };
  bt.stream_masks = masks ? 1u : 0u;
  std::vector<uint32_t> flat;
  for (int w = 0; w < kSearchWaves && fits; ++w) {
    wave_rec[w] = static_cast<uint32_t>(at - bt.stream_off);
    flat.clear();
    for (uint32_t q = wave_off[w]; q < wave_off[w + 1]; ++q) {
      const uint32_t hdr = insns[starts[q]];
      if (!(hdr & kFlatForm)) break;  // flat programs lead each wave's list
      if (static_cast<int64_t>(insns[starts[q] + 1]) >= kStreamMaxRows) fits = false;
      flat.push_back(q);
    }
    if (!fits) break;
    // the compiler laid the wave's flat programs out round by round
    wave_skip[w] = static_cast<uint32_t>(flat.size());
    for (size_t r0 = 0; r0 < flat.size(); r0 += per_block) {
      const size_t n = std::min<size_t>(per_block, flat.size() - r0);
      uint32_t T = 1;  // an empty program still takes one (zeros-row) step
      for (size_t i = 0; i < n; ++i) T = std::max(T, insns[starts[flat[r0 + i]]] & 0xFFFFu);
      word(T);
      for (int i = 1; i < kRoundSlotInfo; ++i) word(0u);
      for (uint32_t i = 0; i < per_block; ++i) {
        if (i < n) {
          const uint32_t* src = insns.data() + starts[flat[r0 + i]];
          word(kSlotValid | ((src[0] & kFlatComplement) ? kSlotComplement : 0u) |
               (src[1] << kSlotRowShift));
        } else {
          word(0u);
        }
      }
      for (uint32_t i = per_block; kRoundSlotInfo + i < kRoundHeaderWords; ++i) word(0u);
      for (uint32_t j = 0; j < T; ++j) {
        for (uint32_t i = 0; i < per_block; ++i) {
          if (balance && i % kBalanceRecords == 0) units.push_back(static_cast<uint32_t>(at));
          if (i >= n) {
            record(kTmplOnes, 0, 0u);
            continue;
          }
          const uint32_t* src = insns.data() + starts[flat[r0 + i]];
          const uint32_t Tq = src[0] & 0xFFFFu;
          if (Tq == 0 && j == 0) {
            record(kTmplZeros, 0, lit_flags(false, true));
          } else if (j < Tq) {
            const uint32_t* lit = src + kProgHeaderWords + j * kFlatLiteralWords;
            record(kTmplCopy, lit[0] / pos_bytes, lit_flags(lit[1] != 0, lit[2] != 0));
          } else {
            record(kTmplOnes, 0, 0u);
          }
        }
      }
    }
  }
  wave_rec[kSearchWaves] = static_cast<uint32_t>(at - bt.stream_off);
  if (fits && wave_rec[kSearchWaves] > 0) {
    if (at != tmpl.size()) fail("literal stream size mismatch: ", at, " != ", tmpl.size());
    bt.stream_words = wave_rec[kSearchWaves];
  } else {  // no stream: every program runs from the width block
    bt.stream_masks = 0;
    tmpl.resize(bt.stream_off);
    code.resize(bt.stream_off);
    bt.stream_off = 0;
    wave_rec.assign(kSearchWaves + 1, 0u);
    wave_skip.assign(kSearchWaves, 0u);
    units.clear();
  }
}

// Balances the read order of every unit of a wide slot's width block
// (out: the block, expanded).
void balance_block(const std::vector<uint32_t>& units, int ks, uint32_t* out) {
  const int srw = bound_record_words(ks);
  for (const uint32_t u : units) {
    uint32_t res[kBalanceRecords] = {}, choice[kBalanceRecords], v[kBalanceMaxK];
    for (int i = 0; i < kBalanceRecords; ++i)
      for (int j = 0; j < ks; ++j) res[i] |= wide_bank_group(out[u + i * srw + j]) << (2 * j);
    balance_wide_choice(res, ks, choice);
    for (int i = 0; i < kBalanceRecords; ++i) {
      uint32_t* rec = out + u + i * srw;
      for (int k = 0; k < ks; ++k) v[k] = rec[balance_source(res[i], choice[i], k, ks)];
      for (int k = 0; k < ks; ++k) rec[k] = v[k];
    }
  }
}

// Width block of one slot from the batch's template; spos holds the kp
// positions of every batch term at the slot's width.
void expand_block(const std::vector<uint32_t>& tmpl, const std::vector<uint32_t>& code,
                  const uint32_t* spos, int kp, int64_t width, uint32_t* out) {
  const bool staged = width <= kSearchTileRows;
  const bool wide = wide_width(width);
  const uint32_t ones = staged ? static_cast<uint32_t>(kSearchOnesRow) * 256u
                       : wide ? static_cast<uint32_t>(kWideOnesRow) * kWideSliceBytes
                              : static_cast<uint32_t>(kPosOnes);
  const uint32_t zeros = staged ? static_cast<uint32_t>(kSearchZerosRow) * 256u
                        : wide ? static_cast<uint32_t>(kWideZerosRow) * kWideSliceBytes
                               : static_cast<uint32_t>(kPosZeros);
  for (size_t i = 0; i < tmpl.size(); ++i) {
    const uint32_t c = code[i];
    if (c == kTmplCopy) {
      out[i] = tmpl[i];
    } else if (c == kTmplOnes) {
      out[i] = ones;
    } else if (c == kTmplZeros) {
      out[i] = zeros;
    } else {
      out[i] = spos[static_cast<size_t>((c >> 4) - 1u) * kp + (c & 15u)];
    }
  }
}

// Rounds of a batch's literal stream, read from its width-block template:
// (first word within the stream, steps).
using RoundList = std::vector<std::pair<uint32_t, uint32_t>>;
void stream_rounds(const std::vector<uint32_t>& tmpl, const SearchBatch& bt, int k_eff,
                   RoundList& out) {
  out.clear();
  if (bt.stream_words == 0) return;
  const int ks = std::max(k_eff, 1);
  const uint32_t step_words =
      static_cast<uint32_t>(stream_block_records(ks) * bound_record_words(ks));
  for (uint32_t w = 0; w < bt.stream_words;) {
    const uint32_t T = tmpl[bt.stream_off + w];
    out.emplace_back(w, T);
    w += kRoundHeaderWords + T * step_words;
  }
}

// Appends the wide-bundle kernel's work table (layout in search_plan.hpp):
// each batch's rounds, longest first, in groups of 16 programs; groups go
// longest first to the least loaded wave.  The batches' block offsets are
// written by patch_wide_table once the blocks have their place.  No table
// (off_wide = 0) when a batch has no literal stream or k is outside 1..7
// (a step must hold four or eight records).
void append_wide_table(st_search_plan& plan, const std::vector<RoundList>& rounds) {
  plan.off_wide = 0;
  const int k = plan.k_eff;
  if (k < 1 || k > 7 || plan.batches.empty()) return;
  for (const SearchBatch& bt : plan.batches)
    if (!bt.generic && bt.stream_words == 0) return;
  const int rg = kWidePrograms / stream_block_records(k);
  struct Group {
    uint32_t batch, steps;
    uint32_t r[kWideMaxRounds], t[kWideMaxRounds];
  };
  std::vector<Group> groups;
  RoundList rs;
  for (size_t bi = 0; bi < rounds.size(); ++bi) {
    rs = rounds[bi];
    std::stable_sort(rs.begin(), rs.end(),
                     [](const auto& x, const auto& y) { return x.second > y.second; });
    for (size_t i = 0; i < rs.size(); i += rg) {
      Group g{static_cast<uint32_t>(bi), rs[i].second, {}};
      for (int j = 0; j < kWideMaxRounds; ++j) g.r[j] = ~0u, g.t[j] = 0;
      for (int j = 0; j < rg && i + j < rs.size(); ++j) {
        g.r[j] = rs[i + j].first;
        g.t[j] = rs[i + j].second;
      }
      groups.push_back(g);
    }
  }
  std::vector<int> order(groups.size());
  for (size_t i = 0; i < order.size(); ++i) order[i] = static_cast<int>(i);
  std::stable_sort(order.begin(), order.end(),
                   [&](int x, int y) { return groups[x].steps > groups[y].steps; });
  std::vector<std::vector<int>> per_wave(kSearchWaves);
  std::vector<int64_t> load(kSearchWaves, 0);
  for (int i : order) {
    const int w = static_cast<int>(std::min_element(load.begin(), load.end()) - load.begin());
    per_wave[w].push_back(i);
    load[w] += 2 + groups[i].steps;
  }
  const size_t nbt = plan.batches.size();
  std::vector<uint32_t> t(kWideTableHead + 4 * nbt + kWideGroupWords * groups.size(), 0u);
  t[0] = static_cast<uint32_t>(nbt);
  t[1] = static_cast<uint32_t>(groups.size());
  t[2] = static_cast<uint32_t>(rg);
  for (size_t bi = 0; bi < nbt; ++bi) {
    const SearchBatch& bt = plan.batches[bi];
    t[kWideTableHead + 4 * bi + 1] = bt.bound_words;
    t[kWideTableHead + 4 * bi + 2] = bt.stream_off;
    t[kWideTableHead + 4 * bi + 3] = bt.stream_masks;
  }
  size_t at = kWideTableHead + 4 * nbt;
  uint32_t g = 0;
  for (int w = 0; w < kSearchWaves; ++w) {
    t[4 + w] = g;
    for (int i : per_wave[w]) {
      const Group& gr = groups[i];
      t[at] = gr.batch;
      t[at + 1] = gr.steps;
      for (int j = 0; j < kWideMaxRounds; ++j) {
        t[at + 2 + j] = gr.r[j];
        t[at + 2 + kWideMaxRounds + j] = gr.t[j];
      }
      at += kWideGroupWords;
      ++g;
    }
  }
  t[4 + kSearchWaves] = g;
  plan.off_wide = plan.blob.size();
  append_bytes(plan.blob, t.data(), t.size() * 4);
}

// Writes each batch's width-block offset (in words of the device blob) into
// the wide-bundle table; drops the table if an offset does not fit 32 bits.
void patch_wide_table(st_search_plan& plan) {
  if (plan.off_wide == 0) return;
  uint32_t* t = reinterpret_cast<uint32_t*>(plan.blob.data() + plan.off_wide);
  for (size_t bi = 0; bi < plan.batches.size(); ++bi) {
    const uint64_t words = plan.batches[bi].off_bound / 4;
    if (words > UINT32_MAX) {
      plan.off_wide = 0;
      return;
    }
    t[kWideTableHead + 4 * bi] = static_cast<uint32_t>(words);
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

    // Most frequent widths get slots (ties to the smaller width).  Census in
    // an open-addressed table keyed by width (few distinct widths).
    std::vector<int64_t> width(num_bundles);
    std::vector<std::pair<int64_t, int64_t>> census;  // (width, bundles)
    std::vector<int32_t> cell(64, -1);  // index into census
    auto cell_of = [&](int64_t w) -> int32_t& {
      size_t m = cell.size() - 1;
      size_t i = static_cast<size_t>(static_cast<uint64_t>(w) * 0x9E3779B97F4A7C15ull >> 40) & m;
      while (cell[i] >= 0 && census[cell[i]].first != w) i = (i + 1) & m;
      return cell[i];
    };
    for (int64_t i = 0; i < num_bundles; ++i) {
      const int64_t w = std::max<int64_t>(bundle_b_offsets[i + 1] - bundle_b_offsets[i], 0);
      width[i] = w;
      int32_t& c = cell_of(w);
      if (c < 0) {
        c = static_cast<int32_t>(census.size());
        census.emplace_back(w, 0);
        if (census.size() * 2 > cell.size()) {  // grow and re-place
          cell.assign(cell.size() * 2, -1);
          for (size_t j = 0; j < census.size(); ++j) cell_of(census[j].first) = static_cast<int32_t>(j);
        }
      }
      ++census[cell_of(w)].second;
    }
    std::vector<std::pair<int64_t, int64_t>> by_freq = census;
    std::sort(by_freq.begin(), by_freq.end(), [](const auto& a, const auto& c) {
      return a.second != c.second ? a.second > c.second : a.first < c.first;
    });
    if (by_freq.size() > static_cast<size_t>(kMaxWidthSlots)) by_freq.resize(kMaxWidthSlots);
    // slot of each census entry
    std::vector<uint32_t> census_slot(census.size(), kNoWidthSlot);
    plan->slot_width.clear();
    for (const auto& wf : by_freq) {
      census_slot[cell_of(wf.first)] = static_cast<uint32_t>(plan->slot_width.size());
      plan->slot_width.push_back(wf.first);
    }
    std::vector<uint32_t> bundle_slot(num_bundles);
    plan->all_wide = true;
    for (int64_t i = 0; i < num_bundles; ++i) {
      bundle_slot[i] = census_slot[cell_of(width[i])];
      plan->all_wide &= bundle_slot[i] != kNoWidthSlot && wide_width(width[i]);
    }
    // Visiting order: bundles grouped by slot (then by width), so that a
    // workgroup striding through it meets long runs of one width and reuses
    // that width's programs from the scalar cache.
    // A slot fixes the width, so a counting sort by slot does it; bundles
    // without a slot (kNoWidthSlot) go last, stably sorted by width.
    std::vector<uint32_t> order(num_bundles);
    {
      const size_t nsl = plan->slot_width.size();
      std::vector<int64_t> first(nsl + 2, 0);
      for (int64_t i = 0; i < num_bundles; ++i)
        ++first[(bundle_slot[i] == kNoWidthSlot ? nsl : bundle_slot[i]) + 1];
      for (size_t j = 1; j < first.size(); ++j) first[j] += first[j - 1];
      const int64_t unslotted = first[nsl];  // start of the kNoWidthSlot bucket
      for (int64_t i = 0; i < num_bundles; ++i)
        order[first[bundle_slot[i] == kNoWidthSlot ? nsl : bundle_slot[i]]++] =
            static_cast<uint32_t>(i);
      std::stable_sort(order.begin() + unslotted, order.end(),
                       [&](uint32_t x, uint32_t y) { return width[x] < width[y]; });
    }
    auto& blob = plan->blob;
    plan->off_bundle_slot = blob.size();
    append_bytes(blob, bundle_slot.data(), bundle_slot.size() * 4);
    plan->off_bundle_order = blob.size();
    append_bytes(blob, order.data(), order.size() * 4);

    const size_t nslots = plan->slot_width.size();
    std::vector<RoundList> rounds(plan->batches.size());
    for (size_t bi = 0; bi < plan->batches.size(); ++bi) {
      SearchBatch& bt = plan->batches[bi];
      if (bt.generic) continue;  // no width blocks: the generic kernel resolves positions
      const auto& insns = plan->batch_insns[bi];
      const auto& starts = plan->batch_starts[bi];
      const auto& hashes = plan->batch_hashes[bi];
      // positions of every term at every slot width
      static thread_local std::vector<uint32_t> pos;
      pos.resize(nslots * bt.num_terms * kp);
      for (size_t s = 0; s < nslots; ++s) {
        const FastMod64 fm = make_fastmod(static_cast<uint64_t>(plan->slot_width[s]));
        for (uint32_t u = 0; u < bt.num_terms; ++u)
          term_positions(hashes.data() + static_cast<size_t>(u) * plan->hash_k,
                         plan->hash_k, k_eff, plan->slot_width[s], fm, kp,
                         &pos[(s * bt.num_terms + u) * kp]);
      }
      static thread_local std::vector<uint32_t> bstart, tmpl, code, wave_rec, wave_skip, units;
      build_block_template(*plan, bt, insns, starts, bstart, tmpl, code, wave_rec, wave_skip, units);
      stream_rounds(tmpl, bt, k_eff, rounds[bi]);
      const uint32_t words = static_cast<uint32_t>(tmpl.size());
      bt.bound_words = words;
      bt.off_bound_start = blob.size();
      append_bytes(blob, bstart.data(), bstart.size() * 4);
      bt.off_stream_wave = blob.size();
      append_bytes(blob, wave_rec.data(), wave_rec.size() * 4);
      bt.off_stream_skip = blob.size();
      append_bytes(blob, wave_skip.data(), wave_skip.size() * 4);
      // The width blocks are written in place at the end of the blob.
      bt.off_bound = blob.size();
      blob.resize(blob.size() + nslots * words * 4, 0);
      uint32_t* block = reinterpret_cast<uint32_t*>(blob.data() + bt.off_bound);
      for (size_t s = 0; s < nslots; ++s) {
        expand_block(tmpl, code, pos.data() + s * bt.num_terms * kp, kp, plan->slot_width[s],
                     block + s * words);
        if (wide_width(plan->slot_width[s]))
          balance_block(units, std::max(k_eff, 1), block + s * words);
      }
    }
    append_wide_table(*plan, rounds);
    patch_wide_table(*plan);
    // Scalar loads may read a few words past the last program.
    blob.resize(blob.size() + 256, 0);
    plan->bound_bundles = num_bundles;
  });
}


extern "C" int st_search_plan_prepare_device_binding(st_search_plan* plan,
                                                     int64_t num_bundles) {
  using namespace st;
  return guarded([&] {
    ST_CHECK(plan != nullptr, "plan is null");
    ST_CHECK(plan->bound_bundles < 0, "plan is already bound to bundle widths");
    ST_CHECK(num_bundles >= 0, "negative bundle count");
    auto& blob = plan->blob;
    // working vectors keep their capacity between calls on a thread
    static thread_local std::vector<uint32_t> bstart, tmpl, code, wave_rec, wave_skip, units;
    std::vector<RoundList> rounds(plan->batches.size());
    for (size_t bi = 0; bi < plan->batches.size(); ++bi) {
      SearchBatch& bt = plan->batches[bi];
      if (bt.generic) continue;  // no width blocks: the generic kernel resolves positions
      build_block_template(*plan, bt, plan->batch_insns[bi], plan->batch_starts[bi], bstart,
                           tmpl, code, wave_rec, wave_skip, units);
      stream_rounds(tmpl, bt, plan->k_eff, rounds[bi]);
      bt.bound_words = static_cast<uint32_t>(tmpl.size());
      bt.off_bound_start = blob.size();
      append_bytes(blob, bstart.data(), bstart.size() * 4);
      bt.off_stream_wave = blob.size();
      append_bytes(blob, wave_rec.data(), wave_rec.size() * 4);
      bt.off_stream_skip = blob.size();
      append_bytes(blob, wave_skip.data(), wave_skip.size() * 4);
      bt.off_tmpl = blob.size();
      append_bytes(blob, tmpl.data(), tmpl.size() * 4);
      bt.off_tmpl_code = blob.size();
      append_bytes(blob, code.data(), code.size() * 4);
      bt.off_units = blob.size();
      bt.n_units = static_cast<uint32_t>(units.size());
      append_bytes(blob, units.data(), units.size() * 4);
    }
    append_wide_table(*plan, rounds);
    blob.resize(align_to(blob.size(), 8), 0);
    plan->off_bind_table = blob.size();
    blob.resize(blob.size() + 8 * kBindTableWords * plan->batches.size(), 0);
    blob.resize(blob.size() + 256, 0);  // slack for scalar loads
    // The device-written part follows the uploaded bytes.
    uint64_t d = align_to(blob.size(), 256);
    plan->off_num_slots = d;
    d += 256;
    plan->off_slot_width = d;
    d = align_to(d + 8 * kMaxWidthSlots, 256);
    plan->off_bundle_slot = d;
    d = align_to(d + 4 * static_cast<uint64_t>(num_bundles), 256);
    plan->off_bundle_order = d;
    d = align_to(d + 4 * static_cast<uint64_t>(num_bundles), 256);
    for (size_t bi = 0; bi < plan->batches.size(); ++bi) {
      SearchBatch& bt = plan->batches[bi];
      bt.off_bound = d;
      d = align_to(d + 4ull * kMaxWidthSlots * bt.bound_words, 256);
      const uint64_t row[kBindTableWords] = {
          bt.off_tmpl, bt.off_tmpl_code, bt.off_hashes, bt.off_bound, bt.bound_words, bt.num_terms,
          bt.off_units, bt.n_units, bt.stream_off | (static_cast<uint64_t>(bt.stream_words) << 32)};
      std::memcpy(blob.data() + plan->off_bind_table + 8 * kBindTableWords * bi, row, sizeof(row));
    }
    patch_wide_table(*plan);
    plan->device_bytes = d + 256;  // slack after the last width block
    plan->bound_bundles = num_bundles;
    plan->device_bind = true;
  });
}

extern "C" int64_t st_search_plan_device_bytes(const st_search_plan* plan) {
  if (plan == nullptr) return 0;
  return static_cast<int64_t>(plan->device_bind ? plan->device_bytes : plan->blob.size());
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

extern "C" void st_search_plan_destroy(st_search_plan* plan) {
  if (plan == nullptr) return;
  st::return_blob_buffer(std::move(plan->blob));
  delete plan;
}

// Work items of the cluster-restricted search
// (bloom_index_search_common_return_partial_response,
// bloom_index_search.cpp:246-395): the reference's column bookkeeping per
// (row, cluster), and the location of each row's program in the blob.
extern "C" int st_search_plan_partial_items(const st_search_plan* plan,
                                            const int64_t* cluster_offsets,
                                            const int64_t* cluster_lengths, int64_t rows,
                                            int64_t clusters, const int64_t* plan_index,
                                            int64_t num_bundles,
                                            int32_t* column_counts_cumsum,
                                            int8_t* first_offsets, st_partial_item* items,
                                            int64_t* num_items, int64_t* total_columns) {
  using namespace st;
  return guarded([&] {
    ST_CHECK(plan != nullptr, "plan is null");
    ST_CHECK(rows >= 0 && clusters >= 0 && num_bundles >= 0, "negative sizes");
    ST_CHECK(num_items != nullptr && total_columns != nullptr, "null output");
    const int64_t n = rows * clusters;
    ST_CHECK(n == 0 || (cluster_offsets && cluster_lengths && column_counts_cumsum &&
                        first_offsets && items),
             "null array");
    // program word and hash offset of every plan, from the batches' layout
    std::vector<uint32_t> prog(plan->num_queries, 0), hash(plan->num_queries, 0);
    for (size_t bi = 0; bi < plan->batches.size(); ++bi) {
      const SearchBatch& bt = plan->batches[bi];
      const auto& insns = plan->batch_insns[bi];
      const auto& starts = plan->batch_starts[bi];
      for (uint32_t s = 0; s < bt.num_slots; ++s) {
        const uint32_t row = insns[starts[s] + 1];
        prog[row] = static_cast<uint32_t>(bt.off_insns / 4 + starts[s]);
        hash[row] = static_cast<uint32_t>(bt.off_hashes / 8);
      }
    }
    const int64_t C = num_bundles * kColumnsPerBundle;
    int64_t acc = 0, m = 0;
    for (int64_t q = 0; q < rows; ++q) {
      const int64_t p = plan_index ? plan_index[q] : q;
      for (int64_t c = 0; c < clusters; ++c) {
        const int64_t i = q * clusters + c;
        const int64_t start = cluster_offsets[i], length = cluster_lengths[i];
        const int64_t off = start % kBitsPerColumn;  // truncating, as in C++
        const int64_t first_col = start / kBitsPerColumn;
        const int64_t ncol = length > 0 ? (length + off + kBitsPerColumn - 1) / kBitsPerColumn : 0;
        first_offsets[i] = static_cast<int8_t>(off);
        acc += ncol;
        ST_CHECK(acc <= INT32_MAX, "the response of clusters up to row ", q, ", cluster ", c,
                 " holds more than 2^31 - 1 columns (the column counts are int32)");
        column_counts_cumsum[i] = static_cast<int32_t>(acc);
        if (ncol == 0) continue;
        ST_CHECK(first_col >= 0 && first_col + ncol <= C, "cluster (", q, ", ", c, ") at doc ",
                 start, " of length ", length, " covers columns [", first_col, ", ",
                 first_col + ncol, ") outside the index's ", C, " columns");
        ST_CHECK(p >= 0 && p < plan->num_queries, "query_plan_index[", q, "] = ", p,
                 " is outside the ", plan->num_queries, " query plans");
        st_partial_item& it = items[m++];
        it.first_column = first_col;
        it.out_offset = acc - ncol;
        it.num_columns = static_cast<int32_t>(ncol);
        it.program = prog[p];
        it.hashes = hash[p];
        it.reserved = 0;
      }
    }
    *num_items = m;
    *total_columns = acc;
  });
}
