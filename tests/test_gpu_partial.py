"""GPU parity of the cluster-restricted search
(bloom_index_search_batch_return_partial_response and _multiple,
bloom_index_search.cpp:246-487) through torch.ops.st: the reference CPU op's
outputs (tests/golden/ref_partial.npz) and the oracle on random cases, bit for
bit, on both dispatch keys."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from oracle import parser_oracle as P
from tests import _fixtures as G
from tests import gpu_helpers as H

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    import silvertorch_amd.ops._load_ops  # noqa: F401


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _partial(dev, index, bbo, pd, po, co, cl, k, hk, pi=None):
    r = torch.ops.st.bloom_index_search_batch_return_partial_response(
        _t(index, dev), _t(bbo, dev), _t(pd, dev), _t(po, dev), _t(co, dev), _t(cl, dev), k, hk,
        None if pi is None else _t(pi, dev))
    for t in r:
        assert t.device.type == torch.device(dev).type
    return r[0].cpu().numpy(), r[1].cpu().numpy(), r[2].cpu().numpy()


@pytest.mark.parametrize("dev", ["cuda", "cpu"])
@pytest.mark.parametrize("name", G.partial_case_names())
def test_partial_matches_reference_fixture(name, dev):
    c = G.partial_case(name)
    k, hk = (int(v) for v in c["params"])
    H.note(f"[partial] case={name} dev={dev}")
    got = _partial(dev, c["index"], c["bundle_b_offsets"], c["plans_data"], c["plans_offsets"],
                   c["cluster_offsets"], c["cluster_lengths"], k, hk, c.get("plan_index"))
    for g, w in zip(got, (c["cumsum"], c["first"], c["mask"])):
        assert g.dtype == w.dtype
        np.testing.assert_array_equal(g, w)


@pytest.mark.parametrize("fuse", [False, True])
def test_partial_multiple_matches_reference_fixture(fuse):
    m = G.partial_multiple()
    H.note(f"[partial] multiple fuse={fuse}")
    res = torch.ops.st.bloom_index_search_batch_return_partial_response_multiple(
        [_t(ch["index"], "cuda") for ch in m["chunks"]], [_t(ch["bundle_b_offsets"], "cuda") for ch in m["chunks"]],
        _t(m["plans_data"], "cuda"), _t(m["plans_offsets"], "cuda"),
        [_t(ch["cluster_offsets"], "cuda") for ch in m["chunks"]],
        [_t(ch["cluster_lengths"], "cuda") for ch in m["chunks"]], 3, 7, None, fuse)
    for i, want in enumerate(m["outputs"][int(fuse)]):
        for out, w in zip((res[0][i], res[1][i], res[2][i]), want):
            np.testing.assert_array_equal(out.cpu().numpy(), w)


@pytest.mark.parametrize("seed", range(5))
def test_partial_random_vs_oracle(seed):
    """Random corpora (k / hash_k / widths including bundles wider than the
    search kernel's LDS tile), boolean queries, clusters at unaligned offsets
    crossing bundles, empty and negative lengths, a query_plan_index."""
    rng = np.random.default_rng(500 + seed)
    n = int(rng.integers(100, 12000))
    F = int(rng.integers(1, 4))
    hi = [3, 5, 30, 2, 6][seed]
    cnt = rng.integers(0, hi + 1, (n, F))
    offs = np.concatenate([[0], np.cumsum(cnt.reshape(-1))]).astype(np.int64)
    vocab = int(rng.integers(20, 800))
    vals = rng.integers(0, vocab, int(offs[-1])).astype(np.int64)
    ids = np.arange(1, F + 1, dtype=np.int32)
    kb = int(rng.integers(1, 8))
    index, bbo = H.build(ids, offs, vals, float(rng.choice([1.5, 3.0, 6.0])), kb)
    queries = []
    for _ in range(int(rng.integers(1, 12))):
        t = int(rng.integers(1, 5))
        parts = [f"{'NOT ' if rng.random() < 0.2 else ''}{int(rng.integers(1, F + 1))}:{int(rng.integers(0, vocab))}"
                 for _ in range(t)]
        q = parts[0]
        for p in parts[1:]:
            q += (" AND " if rng.random() < 0.5 else " OR ") + p
        queries.append("" if rng.random() < 0.05 else q)
    hk = int(rng.integers(1, 9))
    ks = int(rng.integers(0, 9))
    _, data, po = P.parse_batch(queries, hk)
    pd = np.frombuffer(data, dtype=np.int8).copy()
    po = np.array(po, dtype=np.int64)
    rows, clusters = int(rng.integers(1, 9)), int(rng.integers(1, 5))
    total_docs = (bbo.size - 1) * 2048
    co = rng.integers(0, total_docs, (rows, clusters)).astype(np.int64)
    cl = np.minimum(rng.integers(-3, 3000, (rows, clusters)), total_docs - co).astype(np.int64)
    pi = rng.integers(0, len(queries), rows).astype(np.int64)
    H.note(f"[partial] seed={seed} docs={n} k={ks} hash_k={hk} rows={rows} clusters={clusters} "
           f"widths={int(np.diff(bbo).min())}-{int(np.diff(bbo).max())}")
    want = O.partial_response(index, bbo, pd, po, ks, hk, co, cl, pi)
    got = _partial("cuda", index, bbo, pd, po, co, cl, ks, hk, pi)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)
    if rows == len(queries):  # no plan index: row q runs plan q
        want = O.partial_response(index, bbo, pd, po, ks, hk, co, cl)
        for g, w in zip(_partial("cuda", index, bbo, pd, po, co, cl, ks, hk), want):
            np.testing.assert_array_equal(g, w)


def test_partial_errors():
    c = G.partial_case("varied_plan_index")
    k, hk = (int(v) for v in c["params"])
    args = [c["index"], c["bundle_b_offsets"], c["plans_data"], c["plans_offsets"]]
    co, cl, pi = c["cluster_offsets"], c["cluster_lengths"], c["plan_index"]
    with pytest.raises(RuntimeError, match="outside the 6 query plans"):
        _partial("cuda", *args, co, cl, k, hk, np.full_like(pi, 6))
    bad = co.copy()
    bad[0, 0] = (c["bundle_b_offsets"].size - 1) * 2048 - 10
    with pytest.raises(RuntimeError, match="outside the index"):
        _partial("cuda", *args, bad, np.full_like(cl, 100), k, hk, pi)
    with pytest.raises(RuntimeError, match="query_plan count must be same"):
        _partial("cuda", *args, co, cl, k, hk, pi[:2])
    with pytest.raises(RuntimeError, match="query_plan_count must be equal"):
        _partial("cuda", *args, co, cl, k, hk, None)
