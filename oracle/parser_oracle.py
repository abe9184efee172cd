"""Pure-Python restatement of the expression parser -- TEST INFRASTRUCTURE ONLY.

Restates parse_expression_query_batch (expression_query_parser.cpp:30-430 of
the reference, grammar EXPRESSION_SYNTAX.md:67-77) and the plan encoder
encode_query_plans (bloom_index_util.cpp:81-124), and carries its own murmur
(bloom_index_util.cuh:59-106) so that it shares no code with either the C
oracle or the product.  Pinned by tests/golden/ref_parser.json (bytes of the
reference parser compiled in oracle/_ref) and the reference's own structural
tests (test_expression_query_parser.py:44-179).
"""

from __future__ import annotations

import struct

M64 = (1 << 64) - 1

AND, OR, NOT, TERM, EMPTY = 1, 2, 3, 4, 5


class ParseError(RuntimeError):
    pass


def _rotl(v: int, r: int) -> int:
    return ((v << r) | (v >> (64 - r))) & M64


def _fmix(h: int) -> int:
    h ^= h >> 33
    h = (h * 0xFF51AFD7ED558CCD) & M64
    h ^= h >> 33
    h = (h * 0xC4CEB9FE1A85EC53) & M64
    h ^= h >> 33
    return h


def murmur3_pair(x: int, y: int, seed: int) -> int:
    """MurmurHash3_x64_128 of LE(x)||LE(y) under seed, folded to h1 ^ h2."""
    c1, c2 = 0x87C37B91114253D5, 0x4CF5AD432745937F
    x &= M64
    y &= M64
    h1 = h2 = seed & M64
    k1 = (_rotl((x * c1) & M64, 31) * c2) & M64
    h1 = (_rotl(h1 ^ k1, 27) + h2) & M64
    h1 = (h1 * 5 + 0x52DCE729) & M64
    k2 = (_rotl((y * c2) & M64, 33) * c1) & M64
    h2 = (_rotl(h2 ^ k2, 31) + h1) & M64
    h2 = (h2 * 5 + 0x38495AB5) & M64
    h1 ^= 16
    h2 ^= 16
    h1 = (h1 + h2) & M64
    h2 = (h2 + h1) & M64
    h1 = _fmix(h1)
    h2 = _fmix(h2)
    h1 = (h1 + h2) & M64
    h2 = (h2 + h1) & M64
    return h1 ^ h2


_SPACE = " \t\n\v\f\r"


class _Tokens:
    """Lazy tokenizer (expression_query_parser.cpp:48-155)."""

    def __init__(self, s: str):
        self.s = s
        self.i = 0

    def next(self):
        s = self.s
        while self.i < len(s) and s[self.i] in _SPACE:
            self.i += 1
        if self.i >= len(s):
            return ("END", "", self.i)
        at = self.i
        c = s[at]
        single = {"(": "LP", ")": "RP", ":": "COLON", "&": "AND", "|": "OR", "!": "NOT"}
        if c in single:
            self.i += 1
            return (single[c], c, at)
        if c.isascii() and (c.isdigit() or (c == "-" and at + 1 < len(s) and s[at + 1].isascii() and s[at + 1].isdigit())):
            j = at + (1 if c == "-" else 0)
            dot = False
            while j < len(s) and s[j].isascii() and (s[j].isdigit() or s[j] == "."):
                if s[j] == ".":
                    if dot:
                        break
                    dot = True
                j += 1
            self.i = j
            return ("FLOAT" if dot else "NUM", s[at:j], at)
        if c.isascii() and c.isalpha():
            j = at
            while j < len(s) and s[j].isascii() and s[j].isalpha():
                j += 1
            word = s[at:j]
            self.i = j
            if word in ("AND", "OR", "NOT"):
                return (word, word, at)
            raise ParseError(f"Unknown keyword '{word}' at position {at}")
        raise ParseError(f"Unexpected character '{c}' at position {at}")

    def peek(self):
        saved = self.i
        t = self.next()
        self.i = saved
        return t


class _Builder:
    """One-pass plan construction (expression_query_parser.cpp:170-380)."""

    def __init__(self, text: str, hash_k: int, max_sub: int):
        self.t = _Tokens(text)
        self.hash_k = hash_k
        self.max_sub = max_sub
        self.ops: list[int] = []
        self.offsets: list[int] = [0]
        self.params: list[int] = []
        self.hashes: list[int] = []

    def _compound(self, op: int, kids: list[int]) -> None:
        self.params.extend(kids)
        self.ops.append(op)
        self.offsets.append(self.offsets[-1] + len(kids))

    def _run(self, op: int, sep: str, operand) -> None:
        kids: list[int] = []
        count = 0
        folded = False

        def fold():
            nonlocal count, folded, kids
            if count == self.max_sub:
                self._compound(op, kids)
                kids = [len(self.ops) - 1]
                count = 1
                folded = True

        operand()
        kids.append(len(self.ops) - 1)
        count += 1
        if self.t.peek()[0] == sep:
            fold()
        while self.t.peek()[0] == sep:
            self.t.next()
            operand()
            kids.append(len(self.ops) - 1)
            count += 1
            fold()
        if len(kids) <= 1 and not folded:
            return
        self._compound(op, kids)

    def or_expr(self):
        self._run(OR, "OR", self.and_expr)

    def and_expr(self):
        self._run(AND, "AND", self.unary)

    def unary(self):
        if self.t.peek()[0] == "NOT":
            self.t.next()
            self.unary()
            self._compound(NOT, [len(self.ops) - 1])
            return
        if self.t.peek()[0] == "LP":
            self.t.next()
            self.or_expr()
            tok = self.t.next()
            if tok[0] != "RP":
                raise ParseError(f"Expected ')' at position {tok[2]}, got '{tok[1]}'")
            return
        self.term()

    def term(self):
        kind, text, at = self.t.next()
        if kind != "NUM":
            raise ParseError(f"Expected feature id (integer) at position {at}, got '{text}'")
        c = self.t.next()
        if c[0] != "COLON":
            raise ParseError(f"Expected ':' after feature id at position {c[2]}")
        v = self.t.next()
        if v[0] != "NUM":
            raise ParseError(f"Expected feature value (integer) at position {v[2]}, got '{v[1]}'")
        fid, val = int(text), int(v[1])
        for x in (fid, val):
            if not -(1 << 63) <= x < (1 << 63):
                raise ParseError("integer out of int64 range")
        if self.t.peek()[0] == "COLON":
            self.t.next()
            w = self.t.next()
            if w[0] not in ("FLOAT", "NUM"):
                raise ParseError(f"Expected weight (number) at position {w[2]}, got '{w[1]}'")
        if self.hash_k < 1:
            raise ParseError("bloom_hash_k must be at least 1")
        for seed in range(self.hash_k):
            self.hashes.append(murmur3_pair(fid, val, seed))
        self.ops.append(TERM)
        self.offsets.append(self.offsets[-1] + 1)
        self.params.append(len(self.hashes) // self.hash_k - 1)

    def build(self):
        self.or_expr()
        kind, text, at = self.t.peek()
        if kind != "END":
            raise ParseError(f"Unexpected token '{text}' at position {at}, expected end of expression")


def _max_stack(ops: list[int], offsets: list[int]) -> int:
    """get_max_stack_size_impl (bloom_index_util.cpp:26-56)."""
    depth = best = 0
    for i, op in enumerate(ops):
        if op in (TERM, EMPTY):
            depth += 1
        elif op in (AND, OR, NOT):
            depth += 1 - (offsets[i + 1] - offsets[i])
        best = max(best, depth)
    return best


def _section(buf: bytearray, offs: list[int], raw: bytes) -> None:
    start = len(buf)
    buf += raw
    buf += b"\x00" * ((-len(raw)) % 8)
    offs += [start, start + len(raw)]


def parse_batch(expressions: list[str], hash_k: int, return_query_plan: bool = True, max_sub_queries: int = 5):
    """-> (max_stack, plans_data bytes, plans_offsets list)."""
    buf = bytearray()
    offs: list[int] = []
    best = 0
    for text in expressions:
        b = _Builder(text, hash_k, max_sub_queries)
        if text == "":
            b.ops, b.offsets = [EMPTY], [0, 0]
        else:
            b.build()
        best = max(best, _max_stack(b.ops, b.offsets))
        if return_query_plan:
            _section(buf, offs, bytes(b.ops))
            _section(buf, offs, struct.pack(f"<{len(b.offsets)}i", *b.offsets))
            _section(buf, offs, struct.pack(f"<{len(b.params)}i", *b.params))
            _section(buf, offs, struct.pack(f"<{len(b.hashes)}Q", *b.hashes))
    return best, bytes(buf), offs
