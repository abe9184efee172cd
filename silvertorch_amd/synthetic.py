"""Seeded synthetic corpora and queries for the benchmark configurations.

Each component draws from its own numpy stream ``default_rng([seed, stream])``
so that, for example, the queries do not change when the corpus size does.

* per (doc, feature) value counts: ``integers(lo, hi + 1, (N, F))``, row major;
* values: Zipf(s) over ranks 1..V by inverse CDF (``p_r ~ r^-s``,
  ``searchsorted`` of ``random()``), value = per-feature offset + rank - 1,
  or uniform over [0, V) when ``s`` is None;
* ``feature_ids = 1..F``;
* query terms: feature uniform in 1..F, value from that feature's distribution.

Counts and values are drawn in fixed chunks of 2^22 entries, chunk c from
stream ``[seed, stream, c]``, on a thread pool; the output does not depend on
the number of threads.

The named configurations follow BASELINE.json (cfg1 ... cfg5).
"""

from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass, field

import numpy as np

CHUNK = 1 << 22

STREAM_COUNTS = 1
STREAM_VALUES = 2
STREAM_QUERIES = 3
STREAM_EMB = 4
STREAM_QEMB = 5


@dataclass(frozen=True)
class CorpusSpec:
    num_docs: int
    num_features: int
    count_lo: int
    count_hi: int
    vocab: int
    zipf_s: float | None  # None = uniform values
    feature_offsets: tuple[int, ...] | None = None  # value offset per feature
    k: int = 3
    hash_k: int = 7
    b_multiplier: float = 5.0


@dataclass(frozen=True)
class QuerySpec:
    num_queries: int
    kind: str  # "and2" | "flat" | "tree"
    min_terms: int = 2
    max_terms: int = 2
    not_prob: float = 0.0


@dataclass
class Corpus:
    feature_ids: np.ndarray  # int32[F]
    feature_offsets: np.ndarray  # int64[N*F+1]
    feature_values: np.ndarray  # int64[V]
    spec: CorpusSpec = field(repr=False)


CONFIGS: dict[str, tuple[CorpusSpec, QuerySpec | None]] = {
    "cfg1": (CorpusSpec(100_000, 2, 1, 3, 1_000, 1.2, (0, 10_000)), QuerySpec(32, "and2")),
    "cfg2": (CorpusSpec(10_000_000, 8, 1, 4, 100_000, 1.1), QuerySpec(256, "flat", 2, 6)),
    "cfg3": (CorpusSpec(50_000_000, 16, 1, 3, 1_000_000, 1.05, k=4, b_multiplier=10.0),
             QuerySpec(1024, "tree", 3, 12, 0.2)),
    "cfg4": (CorpusSpec(100_000_000, 4, 1, 8, 10_000_000, None), None),
    "cfg5": (CorpusSpec(20_000_000, 8, 1, 4, 100_000, 1.1), QuerySpec(512, "flat", 3, 3)),
}


def _rng(seed: int, stream: int) -> np.random.Generator:
    return np.random.default_rng([seed, stream])


def _zipf_cdf(vocab: int, s: float) -> np.ndarray:
    w = np.arange(1, vocab + 1, dtype=np.float64) ** (-s)
    cdf = np.cumsum(w)
    return cdf / cdf[-1]


def _draw_values(rng: np.random.Generator, n: int, spec: CorpusSpec, cdf) -> np.ndarray:
    if spec.zipf_s is None:
        return rng.integers(0, spec.vocab, n, dtype=np.int64)
    ranks = np.searchsorted(cdf, rng.random(n), side="right")
    return np.minimum(ranks, spec.vocab - 1).astype(np.int64)  # rank - 1


def _value_offset(spec: CorpusSpec, f: int) -> int:
    return spec.feature_offsets[f] if spec.feature_offsets else 0


def _chunked(total: int, fill, progress=None, what: str = "") -> None:
    """Runs fill(chunk_index, lo, hi) over [0, total) in CHUNK pieces; with
    `progress`, reports each tenth of the chunks as it completes."""
    n_chunks = (total + CHUNK - 1) // CHUNK
    workers = max(1, min(16, os.cpu_count() or 1, n_chunks))
    with ThreadPoolExecutor(workers) as ex:
        futs = [ex.submit(fill, c, c * CHUNK, min(total, (c + 1) * CHUNK)) for c in range(n_chunks)]
        step = max(1, n_chunks // 10)
        for i, f in enumerate(futs):
            f.result()
            if progress is not None and ((i + 1) % step == 0 or i + 1 == n_chunks):
                progress(f"{what}: {i + 1}/{n_chunks} chunks")


def make_corpus(spec: CorpusSpec, seed: int = 0, num_docs: int | None = None, progress=None) -> Corpus:
    """The seeded corpus of `spec` (its first `num_docs` docs); `progress`, if
    given, is called with a short message as the generation advances."""
    n = spec.num_docs if num_docs is None else num_docs
    F = spec.num_features
    flat = np.empty(n * F, dtype=np.int64)

    def fill_counts(c, lo, hi):
        flat[lo:hi] = np.random.default_rng([seed, STREAM_COUNTS, c]).integers(
            spec.count_lo, spec.count_hi + 1, hi - lo, dtype=np.int64)

    _chunked(n * F, fill_counts, progress, "value counts")
    offsets = np.empty(n * F + 1, dtype=np.int64)
    offsets[0] = 0
    np.cumsum(flat, out=offsets[1:])
    cdf = _zipf_cdf(spec.vocab, spec.zipf_s) if spec.zipf_s is not None else None
    values = np.empty(int(offsets[-1]), dtype=np.int64)

    def fill_values(c, lo, hi):
        values[lo:hi] = _draw_values(np.random.default_rng([seed, STREAM_VALUES, c]), hi - lo, spec, cdf)

    _chunked(values.size, fill_values, progress, "values")
    if spec.feature_offsets:
        feat_of_value = np.repeat(np.tile(np.arange(F), n), flat)
        values += np.asarray(spec.feature_offsets, dtype=np.int64)[feat_of_value]
    ids = np.arange(1, F + 1, dtype=np.int32)
    return Corpus(ids, offsets, values, spec)


def make_queries(cspec: CorpusSpec, qspec: QuerySpec, seed: int = 0) -> list[str]:
    rng = _rng(seed, STREAM_QUERIES)
    cdf = _zipf_cdf(cspec.vocab, cspec.zipf_s) if cspec.zipf_s is not None else None

    def term() -> str:
        f = int(rng.integers(0, cspec.num_features))
        v = int(_draw_values(rng, 1, cspec, cdf)[0]) + _value_offset(cspec, f)
        t = f"{f + 1}:{v}"
        if qspec.not_prob and rng.random() < qspec.not_prob:
            t = "NOT " + t
        return t

    def tree(leaves: int, depth: int) -> str:
        if leaves == 1 or depth == 0:
            return term() if leaves == 1 else " AND ".join(term() for _ in range(leaves))
        parts = int(rng.integers(2, min(leaves, 4) + 1))
        cuts = np.sort(rng.choice(np.arange(1, leaves), parts - 1, replace=False))
        sizes = np.diff(np.concatenate([[0], cuts, [leaves]]))
        op = " AND " if rng.random() < 0.5 else " OR "
        return op.join(f"({tree(int(s), depth - 1)})" if s > 1 else tree(1, 0) for s in sizes)

    out = []
    for _ in range(qspec.num_queries):
        if qspec.kind == "and2":
            out.append(f"{term()} AND {term()}")
        elif qspec.kind == "flat":
            t = int(rng.integers(qspec.min_terms, qspec.max_terms + 1))
            s = term()
            for _ in range(t - 1):
                s += (" AND " if rng.random() < 0.5 else " OR ") + term()
            out.append(s)
        elif qspec.kind == "tree":
            t = int(rng.integers(qspec.min_terms, qspec.max_terms + 1))
            out.append(tree(t, 3))
        else:
            raise ValueError(qspec.kind)
    return out


DIGEST_CHUNK = 1 << 26


def digest(a: np.ndarray) -> str:
    """sha256 over the sha256 digests of the array's bytes in 64 MiB pieces
    (hashed on a thread pool), so multi-GB outputs are digested in seconds;
    the same rule is applied to the reference's outputs and to this build's."""
    import hashlib

    buf = memoryview(np.ascontiguousarray(a).reshape(-1).view(np.uint8))
    pieces = [buf[i:i + DIGEST_CHUNK] for i in range(0, len(buf), DIGEST_CHUNK)] or [buf]
    workers = max(1, min(16, os.cpu_count() or 1, len(pieces)))
    with ThreadPoolExecutor(workers) as ex:
        parts = list(ex.map(lambda p: hashlib.sha256(p).digest(), pieces))
    return hashlib.sha256(b"".join(parts)).hexdigest()


def match_counts(packed: np.ndarray, num_docs: int) -> list[int]:
    """Per query, the set bits of a packed [Q, C] search output among docs
    d < num_docs (doc d at bit 63 - d % 64 of word d / 64)."""
    words = np.ascontiguousarray(packed).view(np.uint64)
    full, rest = divmod(num_docs, 64)
    out = [int(v) for v in np.bitwise_count(words[:, :full]).sum(axis=1, dtype=np.int64)]
    if rest:
        tail = words[:, full] >> np.uint64(64 - rest)
        out = [c + int(t) for c, t in zip(out, np.bitwise_count(tail))]
    return out


def make_corpus_device(spec: CorpusSpec, seed: int = 0, num_docs: int | None = None,
                       device: str = "cuda", chunk: int = 1 << 26):
    """Large-scale corpus drawn on the device with a seeded torch generator
    (same distributions as make_corpus, not the same draws): per (doc,
    feature) counts uniform in [lo, hi], values Zipf(s) by inverse CDF or
    uniform.  Returns device tensors (feature_ids, feature_offsets,
    feature_values)."""
    import torch

    n = spec.num_docs if num_docs is None else num_docs
    F = spec.num_features
    g = torch.Generator(device=device)
    g.manual_seed(seed * 1_000_003 + STREAM_COUNTS)
    counts = torch.randint(spec.count_lo, spec.count_hi + 1, (n * F,), generator=g, device=device)
    offsets = torch.zeros(n * F + 1, dtype=torch.long, device=device)
    torch.cumsum(counts, 0, out=offsets[1:])
    total = int(offsets[-1].item())
    g.manual_seed(seed * 1_000_003 + STREAM_VALUES)
    values = torch.empty(total, dtype=torch.long, device=device)
    cdf = None
    if spec.zipf_s is not None:
        cdf = torch.from_numpy(_zipf_cdf(spec.vocab, spec.zipf_s)).to(device)
    for lo in range(0, total, chunk):
        hi = min(total, lo + chunk)
        if cdf is None:
            values[lo:hi] = torch.randint(0, spec.vocab, (hi - lo,), generator=g, device=device)
        else:
            u = torch.rand(hi - lo, generator=g, device=device, dtype=torch.float64)
            values[lo:hi] = torch.clamp(torch.searchsorted(cdf, u, right=True), max=spec.vocab - 1)
    if spec.feature_offsets:
        fo = torch.tensor(spec.feature_offsets, dtype=torch.long, device=device)
        values += torch.repeat_interleave(fo.repeat(n), counts)
    ids = torch.arange(1, F + 1, dtype=torch.int32, device=device)
    return ids, offsets, values


def make_embeddings(num_docs: int, dim: int, num_queries: int, seed: int = 0):
    """bf16-representable fp32 embeddings: docs ~ N(0, 1/dim), queries ~ N(0, 1)."""
    import torch

    e = _rng(seed, STREAM_EMB).standard_normal((num_docs, dim), dtype=np.float32) / np.sqrt(dim)
    q = _rng(seed, STREAM_QEMB).standard_normal((num_queries, dim), dtype=np.float32)
    return (torch.from_numpy(e).to(torch.bfloat16), torch.from_numpy(q).to(torch.bfloat16))


def make_embeddings_device(num_docs: int, dim: int, num_queries: int, seed: int = 0,
                           device: str = "cuda", chunk: int = 1 << 21):
    """Large-scale variant of make_embeddings, drawn on the device with a
    seeded torch generator (docs ~ N(0, 1/dim), queries ~ N(0, 1), stored as
    bf16), chunk by chunk to bound the fp32 staging."""
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(seed * 1_000_003 + STREAM_EMB)
    emb = torch.empty((num_docs, dim), dtype=torch.bfloat16, device=device)
    for r0 in range(0, num_docs, chunk):
        r1 = min(num_docs, r0 + chunk)
        emb[r0:r1] = (torch.randn((r1 - r0, dim), generator=g, device=device) / dim ** 0.5).to(torch.bfloat16)
    g.manual_seed(seed * 1_000_003 + STREAM_QEMB)
    q = torch.randn((num_queries, dim), generator=g, device=device).to(torch.bfloat16)
    return emb, q
