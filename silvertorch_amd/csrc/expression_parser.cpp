// Text query parser: expressions -> encoded query plans.
//
// Restates parse_expression_query_batch (expression_query_parser.cpp:30-430
// of the reference, grammar in EXPRESSION_SYNTAX.md:67-77):
//   expression   = or_expr
//   or_expr      = and_expr { ("OR" | "|") and_expr }
//   and_expr     = unary    { ("AND" | "&") unary }
//   unary        = ("NOT" | "!") unary | primary
//   primary      = "(" expression ")" | feature_term
//   feature_term = NUMBER ":" NUMBER [ ":" (NUMBER | FLOAT) ]
// The plan is emitted in postfix while the text is parsed (no tree), with
// the reference's operand folding: an AND/OR run is cut into a nested
// operator each time its pending operand count reaches max_sub_queries
// (expression_query_parser.cpp:206-284), which fixes the exact plan bytes.
// Tokens are produced lazily so that errors surface at the same point, with
// the same text, as in the reference; the hash_k check of a term is made
// once the whole text has parsed, as the reference encodes after parsing.
#include <cstring>
#include <exception>
#include <memory>
#include <string>
#include <vector>

#include "host_pool.hpp"
#include "st_common.hpp"
#include "st_errors.hpp"

struct st_parsed_plans {
  int64_t max_stack = 0;
  std::vector<int8_t> data;
  std::vector<int64_t> offsets;
};

namespace st {
namespace {

enum class Tok { kNumber, kFloat, kColon, kLParen, kRParen, kAnd, kOr, kNot, kEnd };

// A token is a span of the expression text; its text is taken only for an
// error message or a number.
struct Token {
  Tok type;
  size_t pos, len;
};

bool is_space(char c) {
  return c == ' ' || c == '\t' || c == '\n' || c == '\v' || c == '\f' || c == '\r';
}
bool is_digit(char c) { return c >= '0' && c <= '9'; }
bool is_alpha(char c) { return (c >= 'a' && c <= 'z') || (c >= 'A' && c <= 'Z'); }

class Lexer {
 public:
  explicit Lexer(const std::string& s) : s_(s) {}

  Token next() {
    if (has_peek_) {
      has_peek_ = false;
      return peeked_;
    }
    return scan();
  }

  // The next token without consuming it (scanned once, kept until next()).
  const Token& peek() {
    if (!has_peek_) {
      peeked_ = scan();
      has_peek_ = true;
    }
    return peeked_;
  }

  std::string text(const Token& t) const { return s_.substr(t.pos, t.len); }

 private:
  Token scan() {
    while (i_ < s_.size() && is_space(s_[i_])) ++i_;
    if (i_ >= s_.size()) return {Tok::kEnd, i_, 0};
    const size_t at = i_;
    const char c = s_[i_];
    switch (c) {
      case '(': ++i_; return {Tok::kLParen, at, 1};
      case ')': ++i_; return {Tok::kRParen, at, 1};
      case ':': ++i_; return {Tok::kColon, at, 1};
      case '&': ++i_; return {Tok::kAnd, at, 1};
      case '|': ++i_; return {Tok::kOr, at, 1};
      case '!': ++i_; return {Tok::kNot, at, 1};
      default: break;
    }
    if (is_digit(c) || (c == '-' && i_ + 1 < s_.size() && is_digit(s_[i_ + 1]))) {
      if (c == '-') ++i_;
      bool dot = false;
      while (i_ < s_.size() && (is_digit(s_[i_]) || s_[i_] == '.')) {
        if (s_[i_] == '.') {
          if (dot) break;
          dot = true;
        }
        ++i_;
      }
      return {dot ? Tok::kFloat : Tok::kNumber, at, i_ - at};
    }
    if (is_alpha(c)) {
      while (i_ < s_.size() && is_alpha(s_[i_])) ++i_;
      const size_t n = i_ - at;
      const char* w = s_.data() + at;
      if (n == 3 && w[0] == 'A' && w[1] == 'N' && w[2] == 'D') return {Tok::kAnd, at, n};
      if (n == 2 && w[0] == 'O' && w[1] == 'R') return {Tok::kOr, at, n};
      if (n == 3 && w[0] == 'N' && w[1] == 'O' && w[2] == 'T') return {Tok::kNot, at, n};
      fail("Unknown keyword '", s_.substr(at, n), "' at position ", at);
    }
    fail("Unexpected character '", c, "' at position ", at);
  }

  const std::string& s_;
  size_t i_ = 0;
  bool has_peek_ = false;
  Token peeked_{Tok::kEnd, 0, 0};
};

// The value of an integer token ([-]digits), or the reference's error when
// it does not fit int64 (std::stoll's range).
int64_t to_int64(const Lexer& lx, const Token& t, const char* what, const std::string& s) {
  const char* p = s.data() + t.pos;
  const char* e = p + t.len;
  const bool neg = *p == '-';
  if (neg) ++p;
  // accumulate toward the sign's side so that INT64_MIN is reachable
  int64_t v = 0;
  bool ok = p < e;
  for (; p < e && ok; ++p) {
    const int d = *p - '0';
    if (neg) {
      ok = v >= (INT64_MIN + d) / 10 && v * 10 >= INT64_MIN + d;
      if (ok) v = v * 10 - d;
    } else {
      ok = v <= (INT64_MAX - d) / 10;
      if (ok) v = v * 10 + d;
    }
  }
  if (!ok)
    fail(what, " '", lx.text(t), "' at position ", t.pos, " does not fit a signed 64-bit integer");
  return v;
}

// One plan under construction (the QueryPlan of bloom_index_util.h:70-93).
struct PlanBuf {
  std::vector<uint8_t> ops;
  std::vector<int32_t> offsets{0};
  std::vector<int32_t> params;
  std::vector<uint64_t> hashes;
  int64_t hash_k = 0;
  int32_t terms = 0;

  int32_t last() const { return static_cast<int32_t>(ops.size()) - 1; }

  void compound(uint8_t op, const int32_t* kids, size_t n) {
    params.insert(params.end(), kids, kids + n);
    ops.push_back(op);
    offsets.push_back(offsets.back() + static_cast<int32_t>(n));
  }

  // hash_k < 1 is reported by the caller once the text has parsed
  void term(int64_t fid, int64_t value) {
    if (hash_k >= 1) {
      const uint64_t mx = murmur_mix_x(static_cast<uint64_t>(fid));
      const uint64_t my = murmur_mix_y(static_cast<uint64_t>(value));
      for (int64_t seed = 0; seed < hash_k; ++seed)
        hashes.push_back(murmur_finish(mx, my, static_cast<uint64_t>(seed)));
    }
    ops.push_back(kOpTerm);
    offsets.push_back(offsets.back() + 1);
    params.push_back(terms++);
  }
};

// Recursive descent over the grammar above, emitting each operand's postfix
// as it is parsed; each rule returns the op index of its root.  An AND/OR
// run with more than one operand becomes one operator over the operand
// roots, except that whenever the pending operand count reaches
// max_sub_queries the pending operands are closed into an operator which
// then stands as the first pending operand.
class Parser {
 public:
  Parser(const std::string& s, int64_t max_sub, PlanBuf& p) : s_(s), lex_(s), max_sub_(max_sub), p_(p) {}

  void parse() {
    or_expr();
    const Token& t = lex_.peek();
    ST_CHECK(t.type == Tok::kEnd, "Unexpected token '", lex_.text(t), "' at position ",
             t.pos, ", expected end of expression");
  }

 private:
  int32_t list(uint8_t op, Tok sep, int32_t (Parser::*operand)()) {
    const int32_t first = (this->*operand)();
    if (lex_.peek().type != sep) return first;  // one operand: no operator
    const size_t base = pending_.size();  // this run's pending roots
    pending_.push_back(first);
    if (static_cast<int64_t>(pending_.size() - base) == max_sub_) close(op, base);
    while (lex_.peek().type == sep) {
      lex_.next();
      pending_.push_back((this->*operand)());
      if (static_cast<int64_t>(pending_.size() - base) == max_sub_) close(op, base);
    }
    p_.compound(op, pending_.data() + base, pending_.size() - base);
    pending_.resize(base);
    return p_.last();
  }
  // the pending operands into an operator, which becomes the first pending
  void close(uint8_t op, size_t base) {
    p_.compound(op, pending_.data() + base, pending_.size() - base);
    pending_.resize(base);
    pending_.push_back(p_.last());
  }
  int32_t or_expr() { return list(kOpOr, Tok::kOr, &Parser::and_expr); }
  int32_t and_expr() { return list(kOpAnd, Tok::kAnd, &Parser::unary); }

  int32_t unary() {
    if (lex_.peek().type == Tok::kNot) {
      lex_.next();
      const int32_t kid = unary();
      p_.compound(kOpNot, &kid, 1);
      return p_.last();
    }
    if (lex_.peek().type == Tok::kLParen) {
      lex_.next();
      const int32_t inner = or_expr();
      Token t = lex_.next();
      ST_CHECK(t.type == Tok::kRParen, "Expected ')' at position ", t.pos,
               ", got '", lex_.text(t), "'");
      return inner;
    }
    return term();
  }

  int32_t term() {
    Token id = lex_.next();
    ST_CHECK(id.type == Tok::kNumber, "Expected feature id (integer) at position ",
             id.pos, ", got '", lex_.text(id), "'");
    Token colon = lex_.next();
    ST_CHECK(colon.type == Tok::kColon, "Expected ':' after feature id at position ",
             colon.pos);
    Token val = lex_.next();
    ST_CHECK(val.type == Tok::kNumber, "Expected feature value (integer) at position ",
             val.pos, ", got '", lex_.text(val), "'");
    const int64_t fid = to_int64(lex_, id, "feature id", s_);
    const int64_t value = to_int64(lex_, val, "feature value", s_);
    if (lex_.peek().type == Tok::kColon) {  // optional weight, not used
      lex_.next();
      Token w = lex_.next();
      ST_CHECK(w.type == Tok::kFloat || w.type == Tok::kNumber,
               "Expected weight (number) at position ", w.pos, ", got '", lex_.text(w), "'");
    }
    p_.term(fid, value);
    return p_.last();
  }

  const std::string& s_;
  Lexer lex_;
  int64_t max_sub_;
  PlanBuf& p_;
  std::vector<int32_t> pending_;  // pending operand roots of the open runs
};

// Largest running stack depth of the postfix program
// (get_max_stack_size_impl, bloom_index_util.cpp:26-56).
int64_t stack_depth(const PlanBuf& p) {
  int64_t depth = 0, best = 0;
  for (size_t i = 0; i < p.ops.size(); ++i) {
    if (p.ops[i] == kOpTerm || p.ops[i] == kOpEmpty) {
      ++depth;
    } else {
      depth += 1 - (p.offsets[i + 1] - p.offsets[i]);
    }
    best = depth > best ? depth : best;
  }
  return best;
}

template <typename T>
void append_section(const std::vector<T>& v, std::vector<int8_t>& data,
                    std::vector<int64_t>& offsets) {
  const int64_t start = static_cast<int64_t>(data.size());
  const size_t bytes = v.size() * sizeof(T);
  data.resize(data.size() + ((bytes + 7) / 8) * 8, 0);
  if (bytes) std::memcpy(data.data() + start, v.data(), bytes);
  offsets.push_back(start);
  offsets.push_back(start + static_cast<int64_t>(bytes));
}

// One expression parsed and emitted on its own (the batch's queries are
// independent); a failure keeps its error.
struct ParsedOne {
  PlanBuf plan;
  int64_t depth = 0;
  std::exception_ptr error;
};

void parse_one(const char* expression, int64_t hash_k, int64_t max_sub, ParsedOne& out) {
  try {
    const std::string text = expression ? expression : "";
    PlanBuf& p = out.plan;
    p.hash_k = hash_k;
    if (text.empty()) {
      p.ops.push_back(kOpEmpty);
      p.offsets.push_back(p.offsets.back());
    } else {
      Parser(text, max_sub, p).parse();
      ST_CHECK(p.terms == 0 || hash_k >= 1, "bloom_hash_k must be at least 1, got ", hash_k);
    }
    out.depth = stack_depth(p);
  } catch (...) {
    out.error = std::current_exception();
  }
}

// Batches of at least this many expressions are parsed on the host pool.
constexpr int64_t kParallelParse = 128;

}  // namespace
}  // namespace st

extern "C" int st_parse_expression_query_batch(const char* const* expressions,
                                               int64_t num_expressions,
                                               int64_t hash_k,
                                               int return_query_plan,
                                               int64_t max_sub_queries,
                                               st_parsed_plans** out) {
  using namespace st;
  return guarded([&] {
    ST_CHECK(out != nullptr, "out is null");
    *out = nullptr;
    ST_CHECK(num_expressions >= 0, "negative expression count");
    ST_CHECK(num_expressions == 0 || expressions, "expressions is null");
    auto res = std::make_unique<st_parsed_plans>();
    // Every expression is parsed on its own (on the host pool for large
    // batches), then the plans are laid out in order; the error raised is
    // the first failing expression's, as in a query-by-query parse.
    std::vector<ParsedOne> parsed(static_cast<size_t>(num_expressions));
    const auto one = [&](int64_t q) {
      parse_one(expressions[q], hash_k, max_sub_queries, parsed[static_cast<size_t>(q)]);
    };
    if (num_expressions >= kParallelParse) {
      host_pool_run(num_expressions, 16, one);
    } else {
      for (int64_t q = 0; q < num_expressions; ++q) one(q);
    }
    for (const ParsedOne& r : parsed)
      if (r.error) std::rethrow_exception(r.error);
    if (return_query_plan) {
      const auto padded = [](size_t bytes) { return ((bytes + 7) / 8) * 8; };
      size_t total = 0;
      for (const ParsedOne& r : parsed)
        total += padded(r.plan.ops.size()) + padded(r.plan.offsets.size() * 4) +
                 padded(r.plan.params.size() * 4) + r.plan.hashes.size() * 8;
      res->data.reserve(total);
      res->offsets.reserve(parsed.size() * 8);
    }
    for (const ParsedOne& r : parsed) {
      res->max_stack = r.depth > res->max_stack ? r.depth : res->max_stack;
      if (return_query_plan) {
        append_section(r.plan.ops, res->data, res->offsets);
        append_section(r.plan.offsets, res->data, res->offsets);
        append_section(r.plan.params, res->data, res->offsets);
        append_section(r.plan.hashes, res->data, res->offsets);
      }
    }
    *out = res.release();
  });
}

extern "C" int64_t st_parsed_plans_max_stack(const st_parsed_plans* p) {
  return p ? p->max_stack : 0;
}
extern "C" int64_t st_parsed_plans_data_bytes(const st_parsed_plans* p) {
  return p ? static_cast<int64_t>(p->data.size()) : 0;
}
extern "C" const int8_t* st_parsed_plans_data(const st_parsed_plans* p) {
  return p ? p->data.data() : nullptr;
}
extern "C" int64_t st_parsed_plans_offsets_len(const st_parsed_plans* p) {
  return p ? static_cast<int64_t>(p->offsets.size()) : 0;
}
extern "C" const int64_t* st_parsed_plans_offsets(const st_parsed_plans* p) {
  return p ? p->offsets.data() : nullptr;
}
extern "C" void st_parsed_plans_destroy(st_parsed_plans* p) { delete p; }
