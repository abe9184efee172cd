"""GPU parity of plans beyond the batch kernels' limits, which the reference
evaluates with an unbounded std::stack (run_query_plan,
bloom_index_search.cpp:72-171): programs needing more than 8 stack slots (a
balanced AND/OR tree of depth 10, 1024 leaves with NOTs), a single query of
3000 distinct terms, and a 5000-deep left chain ((t0 AND t1) OR t2) AND ...,
mixed in one call with ordinary queries (the chain is encoded directly: its
text form would nest 5000 parentheses).  Packed and bool outputs through
the C ABI (host-bound, device-bound and unbound plans), the ids op (counted
search) and the cluster-restricted search, all against the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from oracle import parser_oracle as P
from tests import gpu_helpers as H

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    import silvertorch_amd.ops._load_ops  # noqa: F401


def _corpus(rng, n, F, vocab):
    cnt = rng.integers(1, 5, (n, F))
    offs = np.concatenate([[0], np.cumsum(cnt.reshape(-1))]).astype(np.int64)
    vals = rng.integers(0, vocab, int(offs[-1])).astype(np.int64)
    return np.arange(1, F + 1, dtype=np.int32), offs, vals


def _balanced(rng, F, vocab, depth, op=0):
    if depth == 0:
        t = f"{int(rng.integers(1, F + 1))}:{int(rng.integers(0, vocab))}"
        return ("NOT " + t) if rng.random() < 0.15 else t
    j = " AND " if op % 2 == 0 else " OR "
    return "(" + _balanced(rng, F, vocab, depth - 1, op + 1) + j + _balanced(rng, F, vocab, depth - 1, op + 1) + ")"


def _queries(rng, F, vocab):
    qs = [_balanced(rng, F, vocab, 10)]                                               # needs 11 slots
    qs.append(" OR ".join(f"{1 + i % F}:{i}" for i in range(3000)))                   # 3000 terms
    for _ in range(20):  # ordinary queries around them
        t = int(rng.integers(1, 5))
        qs.append(" AND ".join(f"{int(rng.integers(1, F + 1))}:{int(rng.integers(0, vocab))}" for _ in range(t)))
    order = rng.permutation(len(qs))
    return [qs[i] for i in order]


def _chain_plan(rng, F, vocab, hash_k, depth):
    """Plan sections of ((t0 AND t1) OR t2) AND t3 ... (depth terms), in the
    reference's encoding (bloom_index_util.cpp:81-124), built directly: the
    text form would nest `depth` parentheses deep."""
    ops, offsets, hashes = [P.TERM], [0, 1], []
    terms = [(1 + i % F, int(rng.integers(0, vocab))) for i in range(depth)]
    for i in range(1, depth):
        ops += [P.TERM, P.AND if i % 2 else P.OR]
        offsets += [offsets[-1] + 1, offsets[-1] + 3]
    for fid, val in terms:
        hashes += [P.murmur3_pair(fid, val, s) for s in range(hash_k)]
    return ops, offsets, [0] * offsets[-1], hashes


def _plans(rng, queries, F, vocab, hash_k, chain_at):
    """Plans of `queries` with a 5000-deep chain inserted as query chain_at."""
    import struct

    _, data, po = P.parse_batch(queries, hash_k)
    buf, offs = bytearray(data), list(po)
    ops, ofs, params, hs = _chain_plan(rng, F, vocab, hash_k, 5000)
    chain = []
    P._section(buf, chain, bytes(ops))
    P._section(buf, chain, struct.pack(f"<{len(ofs)}i", *ofs))
    P._section(buf, chain, struct.pack(f"<{len(params)}i", *params))
    P._section(buf, chain, struct.pack(f"<{len(hs)}Q", *hs))
    offs = offs[:8 * chain_at] + chain + offs[8 * chain_at:]
    return np.frombuffer(bytes(buf), dtype=np.int8).copy(), np.array(offs, dtype=np.int64)


@pytest.mark.timeout(600)
@pytest.mark.parametrize("k,hash_k", [(3, 7), (1, 3), (7, 9)])
def test_generic_plans_vs_oracle(k, hash_k):
    rng = np.random.default_rng(1000 + k)
    F, vocab = 3, 4000
    ids, offs, vals = _corpus(rng, 9000, F, vocab)
    index, bbo = H.build(ids, offs, vals, 3.0, k)
    queries = _queries(rng, F, vocab)
    pd, po = _plans(rng, queries, F, vocab, hash_k, 5)
    H.note(f"[generic] k={k} hash_k={hash_k} queries={len(po) // 8} plan bytes={pd.size}")
    want = O.search_packed(index, bbo, pd, po, k, hash_k)
    np.testing.assert_array_equal(H.search(index, bbo, pd, po, k, hash_k), want)  # host, device, unbound
    np.testing.assert_array_equal(H.search(index, bbo, pd, po, k, hash_k, bool_mask=True, bind="device"),
                                  O.unpack_bool(want))
    # counted search (ids op) and the drop-in op
    n = (len(offs) - 1) // F
    ids_got, ro, packed = H.search_ids(index, bbo, pd, po, k, hash_k, n)
    np.testing.assert_array_equal(packed, want)
    want_ids, want_ro = O.compact(want, n)
    np.testing.assert_array_equal(ro, want_ro)
    np.testing.assert_array_equal(ids_got, want_ids)
    dev = torch.device("cuda")
    got = torch.ops.st.bloom_index_search_batch(torch.from_numpy(index).to(dev), torch.from_numpy(bbo).to(dev),
                                                torch.from_numpy(pd), torch.from_numpy(po), k, hash_k, False)
    np.testing.assert_array_equal(got.cpu().numpy(), want)


@pytest.mark.timeout(600)
def test_generic_plans_in_cluster_restricted_search():
    rng = np.random.default_rng(77)
    F, vocab = 2, 3000
    ids, offs, vals = _corpus(rng, 6000, F, vocab)
    index, bbo = H.build(ids, offs, vals, 3.0, 3)
    queries = _queries(rng, F, vocab)[:8] + [_balanced(rng, F, vocab, 10)]
    pd, po = _plans(rng, queries, F, vocab, 7, 2)
    rows, clusters = len(po) // 8, 3
    total = (bbo.size - 1) * 2048
    co = rng.integers(0, total, (rows, clusters)).astype(np.int64)
    cl = np.minimum(rng.integers(1, 2500, (rows, clusters)), total - co).astype(np.int64)
    want = O.partial_response(index, bbo, pd, po, 3, 7, co, cl)
    dev = torch.device("cuda")
    r = torch.ops.st.bloom_index_search_batch_return_partial_response(
        torch.from_numpy(index).to(dev), torch.from_numpy(bbo).to(dev), torch.from_numpy(pd), torch.from_numpy(po),
        torch.from_numpy(co).to(dev), torch.from_numpy(cl).to(dev), 3, 7, None)
    for g, w in zip(r, want):
        np.testing.assert_array_equal(g.cpu().numpy(), w)
