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
// The text is first parsed into a tree; the tree is then emitted in postfix
// with the reference's operand folding: an AND/OR run is cut into a nested
// operator each time its pending operand count reaches max_sub_queries
// (expression_query_parser.cpp:206-284), which fixes the exact plan bytes.
// Tokens are produced lazily so that errors surface at the same point, with
// the same text, as in the reference.
#include <cstring>
#include <memory>
#include <string>
#include <vector>

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

struct Token {
  Tok type;
  std::string text;
  size_t pos;
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
    while (i_ < s_.size() && is_space(s_[i_])) ++i_;
    if (i_ >= s_.size()) return {Tok::kEnd, "", i_};
    const size_t at = i_;
    const char c = s_[i_];
    switch (c) {
      case '(': ++i_; return {Tok::kLParen, "(", at};
      case ')': ++i_; return {Tok::kRParen, ")", at};
      case ':': ++i_; return {Tok::kColon, ":", at};
      case '&': ++i_; return {Tok::kAnd, "&", at};
      case '|': ++i_; return {Tok::kOr, "|", at};
      case '!': ++i_; return {Tok::kNot, "!", at};
      default: break;
    }
    if (is_digit(c) || (c == '-' && i_ + 1 < s_.size() && is_digit(s_[i_ + 1]))) {
      std::string num;
      if (c == '-') num += s_[i_++];
      bool dot = false;
      while (i_ < s_.size() && (is_digit(s_[i_]) || s_[i_] == '.')) {
        if (s_[i_] == '.') {
          if (dot) break;
          dot = true;
        }
        num += s_[i_++];
      }
      return {dot ? Tok::kFloat : Tok::kNumber, num, at};
    }
    if (is_alpha(c)) {
      std::string word;
      while (i_ < s_.size() && is_alpha(s_[i_])) word += s_[i_++];
      if (word == "AND") return {Tok::kAnd, word, at};
      if (word == "OR") return {Tok::kOr, word, at};
      if (word == "NOT") return {Tok::kNot, word, at};
      fail("Unknown keyword '", word, "' at position ", at);
    }
    fail("Unexpected character '", c, "' at position ", at);
  }

  Token peek() {
    const size_t saved = i_;
    Token t = next();
    i_ = saved;
    return t;
  }

 private:
  const std::string& s_;
  size_t i_ = 0;
};

enum class Kind { kTerm, kAnd, kOr, kNot };

struct Expr {
  Kind kind;
  int64_t feature_id = 0;
  int64_t value = 0;
  std::vector<std::unique_ptr<Expr>> kids;
};
using ExprPtr = std::unique_ptr<Expr>;

int64_t to_int64(const Token& t, const char* what) {
  try {
    size_t used = 0;
    long long v = std::stoll(t.text, &used);
    return static_cast<int64_t>(v);
  } catch (const std::exception&) {
    fail(what, " '", t.text, "' at position ", t.pos,
         " does not fit a signed 64-bit integer");
  }
}

class Parser {
 public:
  explicit Parser(const std::string& s) : lex_(s) {}

  ExprPtr parse() {
    ExprPtr e = or_expr();
    Token t = lex_.peek();
    ST_CHECK(t.type == Tok::kEnd, "Unexpected token '", t.text, "' at position ",
             t.pos, ", expected end of expression");
    return e;
  }

 private:
  ExprPtr list(Kind kind, Tok sep, ExprPtr (Parser::*operand)()) {
    auto node = std::make_unique<Expr>();
    node->kind = kind;
    node->kids.push_back((this->*operand)());
    while (lex_.peek().type == sep) {
      lex_.next();
      node->kids.push_back((this->*operand)());
    }
    return node;
  }
  ExprPtr or_expr() { return list(Kind::kOr, Tok::kOr, &Parser::and_expr); }
  ExprPtr and_expr() { return list(Kind::kAnd, Tok::kAnd, &Parser::unary); }

  ExprPtr unary() {
    if (lex_.peek().type == Tok::kNot) {
      lex_.next();
      auto node = std::make_unique<Expr>();
      node->kind = Kind::kNot;
      node->kids.push_back(unary());
      return node;
    }
    if (lex_.peek().type == Tok::kLParen) {
      lex_.next();
      ExprPtr inner = or_expr();
      Token t = lex_.next();
      ST_CHECK(t.type == Tok::kRParen, "Expected ')' at position ", t.pos,
               ", got '", t.text, "'");
      return inner;
    }
    return term();
  }

  ExprPtr term() {
    Token id = lex_.next();
    ST_CHECK(id.type == Tok::kNumber, "Expected feature id (integer) at position ",
             id.pos, ", got '", id.text, "'");
    Token colon = lex_.next();
    ST_CHECK(colon.type == Tok::kColon, "Expected ':' after feature id at position ",
             colon.pos);
    Token val = lex_.next();
    ST_CHECK(val.type == Tok::kNumber, "Expected feature value (integer) at position ",
             val.pos, ", got '", val.text, "'");
    auto node = std::make_unique<Expr>();
    node->kind = Kind::kTerm;
    node->feature_id = to_int64(id, "feature id");
    node->value = to_int64(val, "feature value");
    if (lex_.peek().type == Tok::kColon) {  // optional weight, not used
      lex_.next();
      Token w = lex_.next();
      ST_CHECK(w.type == Tok::kFloat || w.type == Tok::kNumber,
               "Expected weight (number) at position ", w.pos, ", got '", w.text, "'");
    }
    return node;
  }

  Lexer lex_;
};

// One plan under construction (the QueryPlan of bloom_index_util.h:70-93).
struct PlanBuf {
  std::vector<uint8_t> ops;
  std::vector<int32_t> offsets{0};
  std::vector<int32_t> params;
  std::vector<uint64_t> hashes;
  int64_t hash_k = 0;

  int32_t last() const { return static_cast<int32_t>(ops.size()) - 1; }

  void compound(uint8_t op, const std::vector<int32_t>& kids) {
    params.insert(params.end(), kids.begin(), kids.end());
    ops.push_back(op);
    offsets.push_back(offsets.back() + static_cast<int32_t>(kids.size()));
  }

  void term(int64_t fid, int64_t value) {
    ST_CHECK(hash_k >= 1, "bloom_hash_k must be at least 1, got ", hash_k);
    const uint64_t mx = murmur_mix_x(static_cast<uint64_t>(fid));
    const uint64_t my = murmur_mix_y(static_cast<uint64_t>(value));
    for (int64_t seed = 0; seed < hash_k; ++seed)
      hashes.push_back(murmur_finish(mx, my, static_cast<uint64_t>(seed)));
    ops.push_back(kOpTerm);
    offsets.push_back(offsets.back() + 1);
    params.push_back(static_cast<int32_t>(hashes.size() / hash_k) - 1);
  }
};

// Emits `e` in postfix.  An AND/OR run with more than one operand becomes one
// operator over the operand roots, except that whenever the pending operand
// count reaches max_sub_queries the pending operands are closed into an
// operator which then stands as the first pending operand.
void emit(const Expr& e, int64_t max_sub, PlanBuf& p) {
  switch (e.kind) {
    case Kind::kTerm:
      p.term(e.feature_id, e.value);
      return;
    case Kind::kNot:
      emit(*e.kids[0], max_sub, p);
      p.compound(kOpNot, {p.last()});
      return;
    case Kind::kAnd:
    case Kind::kOr: {
      const uint8_t op = e.kind == Kind::kAnd ? kOpAnd : kOpOr;
      if (e.kids.size() == 1) {
        emit(*e.kids[0], max_sub, p);
        return;
      }
      std::vector<int32_t> pending;
      for (const auto& kid : e.kids) {
        emit(*kid, max_sub, p);
        pending.push_back(p.last());
        if (static_cast<int64_t>(pending.size()) == max_sub) {
          p.compound(op, pending);
          pending.assign(1, p.last());
        }
      }
      p.compound(op, pending);
      return;
    }
  }
}

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
    for (int64_t q = 0; q < num_expressions; ++q) {
      const std::string text = expressions[q] ? expressions[q] : "";
      PlanBuf p;
      p.hash_k = hash_k;
      if (text.empty()) {
        p.ops.push_back(kOpEmpty);
        p.offsets.push_back(p.offsets.back());
      } else {
        ExprPtr e = Parser(text).parse();
        emit(*e, max_sub_queries, p);
      }
      const int64_t d = stack_depth(p);
      res->max_stack = d > res->max_stack ? d : res->max_stack;
      if (return_query_plan) {
        append_section(p.ops, res->data, res->offsets);
        append_section(p.offsets, res->data, res->offsets);
        append_section(p.params, res->data, res->offsets);
        append_section(p.hashes, res->data, res->offsets);
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
