"""GPU parity: the HIP path against the reference's outputs and the oracle.

Integer work is compared bit-exactly:
  * golden fixtures of the reference's CPU ops (tests/golden/ref_cases.npz,
    ref_digests.json), through the C ABI;
  * the C oracle (oracle/) on seeded random corpora and query batches,
    including bundles wider than the LDS tile, int16 position wrap-around,
    k / hash_k variants and batches large enough to need several passes;
  * the reference's own test shapes through torch.ops.st (the drop-in path),
    after test_bloom_index_search.py:41-269 and test_bloom_indexer.py:31-150.
"""

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


def _plans(queries, hash_k, max_sub=5):
    _, data, offs = P.parse_batch(queries, hash_k, True, max_sub)
    return np.frombuffer(data, dtype=np.int8).copy(), np.array(offs, dtype=np.int64)


@pytest.mark.parametrize("name", G.case_names())
def test_build_matches_reference(name):
    c = G.case(name)
    H.note(f"[build] case={name} docs={(len(c['offsets']) - 1) // len(c['ids'])} k={c['build_k']}")
    index, bbo = H.build(c["ids"], c["offsets"], c["values"], c["b_multiplier"], c["build_k"])
    np.testing.assert_array_equal(bbo, c["bundle_b_offsets"])
    np.testing.assert_array_equal(index, c["index"])


@pytest.mark.parametrize("name", G.case_names())
@pytest.mark.parametrize("fast_build", [False, True])
def test_op_build_fast_build_flag_matches_reference(name, fast_build):
    """torch.ops.st.bloom_index_build with fast_build=True returns the same
    bits as the default build: the reference's flag selects another CUDA
    algorithm with identical output (bloom_indexer_cuda.cu:838-853) and is
    ignored by its CPU op (bloom_indexer.cpp:32), so both are checked against
    the reference CPU op's fixtures, on GPU and on CPU tensors."""
    c = G.case(name)
    H.note(f"[build op] case={name} fast_build={fast_build}")
    args = [torch.from_numpy(c["ids"]), torch.from_numpy(c["offsets"]), torch.from_numpy(c["values"])]
    for dev in ("cuda", "cpu"):
        bi, bo = torch.ops.st.bloom_index_build(*[a.to(dev) for a in args], c["b_multiplier"], c["build_k"],
                                                fast_build=fast_build)
        assert bi.device.type == dev
        np.testing.assert_array_equal(bo.cpu().numpy(), c["bundle_b_offsets"])
        np.testing.assert_array_equal(bi.cpu().numpy(), c["index"])


@pytest.mark.parametrize("name", G.case_names())
@pytest.mark.parametrize("bool_mask", [False, True])
def test_search_matches_reference(name, bool_mask):
    c = G.case(name)
    H.note(f"[search] case={name} k={c['k']} hash_k={c['hash_k']} bool={bool_mask}")
    out = H.search(c["index"], c["bundle_b_offsets"], c["plans_data"], c["plans_offsets"], c["k"], c["hash_k"], bool_mask)
    want = O.unpack_bool(c["packed"]) if bool_mask else c["packed"]
    np.testing.assert_array_equal(out, want)


def test_cfg1_digest():
    from silvertorch_amd import synthetic as S

    d = G.digests()["cfg1"]
    cspec, qspec = S.CONFIGS["cfg1"]
    corp = S.make_corpus(cspec, seed=0)
    H.note("[cfg1] build + search on GPU")
    index, bbo = H.build(corp.feature_ids, corp.feature_offsets, corp.feature_values, cspec.b_multiplier, cspec.k)
    assert G.sha(index) == d["index"] and G.sha(bbo) == d["bundle_b_offsets"]
    pd, po = _plans(S.make_queries(cspec, qspec, seed=0), cspec.hash_k)
    packed = H.search(index, bbo, pd, po, cspec.k, cspec.hash_k)
    assert G.sha(packed) == d["packed"]


def test_wide_bundles_global_path_and_int16_wrap():
    ids, offs, vals, w = G.wide_corpus()
    H.note("[wide] bundles of 32768 and 40000 rows")
    index, bbo = H.build(ids, offs, vals, w["b_multiplier"], w["k"])
    assert bbo.tolist() == w["bundle_b_offsets"]
    assert G.sha(index) == w["index"]
    pd, po = _plans(w["queries"], 7)
    assert G.sha(H.search(index, bbo, pd, po, w["k"], 7)) == w["packed"]


def _random_corpus(rng, n, F, lo, hi, vocab):
    cnt = rng.integers(lo, hi + 1, (n, F))
    offs = np.concatenate([[0], np.cumsum(cnt.reshape(-1))]).astype(np.int64)
    vals = rng.integers(-vocab // 4, vocab, int(offs[-1])).astype(np.int64)
    ids = (rng.permutation(50)[:F] - 10).astype(np.int32)
    return ids, offs, vals


def _random_queries(rng, ids, vocab, n, max_terms, deep=False):
    out = []
    for _ in range(n):
        def leaf():
            t = f"{int(rng.choice(ids))}:{int(rng.integers(-vocab // 4, vocab))}"
            return ("NOT " + t) if rng.random() < 0.2 else t

        def tree(d):
            if d == 0 or rng.random() < 0.3:
                return leaf()
            parts = [tree(d - 1) for _ in range(int(rng.integers(1, max_terms + 1)))]
            s = (" AND " if rng.random() < 0.5 else " OR ").join(parts)
            s = f"({s})"
            return ("NOT " + s) if rng.random() < 0.15 else s

        q = tree(4 if deep else 2)
        out.append("" if rng.random() < 0.03 else q)
    return out


@pytest.mark.parametrize("seed", range(6))
def test_random_vs_oracle(seed):
    rng = np.random.default_rng(1000 + seed)
    n = int(rng.integers(1, 20000))
    F = int(rng.integers(1, 6))
    hi = [3, 6, 40, 3, 8, 2][seed]  # seed 2 gives bundles wider than the LDS tile
    vocab = int(rng.integers(10, 5000))
    ids, offs, vals = _random_corpus(rng, n, F, 0, hi, vocab)
    kb = int(rng.integers(1, 11))
    bm = float(rng.choice([1.1, 2.0, 5.0, 9.5]))
    H.note(f"[random] seed={seed} docs={n} F={F} max_cnt={hi} k={kb} bm={bm}")
    index, bbo = H.build(ids, offs, vals, bm, kb)
    want_index, want_bbo = O.bloom_build(ids, offs, vals, bm, kb)
    np.testing.assert_array_equal(bbo, want_bbo)
    np.testing.assert_array_equal(index, want_index)
    queries = _random_queries(rng, ids, vocab, int(rng.integers(1, 300)), 5, deep=seed % 2 == 1)
    hk = int(rng.integers(1, 11))
    ks = int(rng.integers(0, 12))
    pd, po = _plans(queries, hk, int(rng.integers(1, 6)))
    if min(ks, hk) > 10:
        ks = 10
    H.note(f"[random] seed={seed} queries={len(queries)} k={ks} hash_k={hk}")
    got = H.search(index, bbo, pd, po, ks, hk)
    np.testing.assert_array_equal(got, O.search_packed(index, bbo, pd, po, ks, hk))


@pytest.mark.parametrize("F,n", [(1, 5000), (16, 3000), (17, 2500), (40, 2100), (3, 257)])
def test_build_feature_counts_vs_oracle(F, n):
    """Bundle widths for feature counts on both sides of the widths kernel's
    LDS staging limit (16), ragged last bundles and docs without terms;
    decreasing offsets are rejected."""
    rng = np.random.default_rng(40 + F)
    ids, offs, vals = _random_corpus(rng, n, F, 0, 4, 3000)
    H.note(f"[build widths] F={F} docs={n}")
    index, bbo = H.build(ids, offs, vals, 2.0, 3)
    want_index, want_bbo = O.bloom_build(ids, offs, vals, 2.0, 3)
    np.testing.assert_array_equal(bbo, want_bbo)
    np.testing.assert_array_equal(index, want_index)
    bad = offs.copy()
    bad[len(bad) // 2] = bad[len(bad) // 2 + 1] + 1  # one decrease
    with pytest.raises(RuntimeError, match="non-decreasing"):
        torch.ops.st.bloom_index_build(torch.from_numpy(ids).cuda(), torch.from_numpy(bad).cuda(),
                                       torch.from_numpy(vals).cuda(), 2.0, 3)


def test_many_terms_split_into_passes():
    """More distinct terms than one LDS position area holds -> several passes."""
    rng = np.random.default_rng(77)
    ids, offs, vals = _random_corpus(rng, 5000, 3, 1, 3, 100000)
    index, bbo = H.build(ids, offs, vals, 3.0, 3)
    queries = [" OR ".join(f"{int(rng.choice(ids))}:{int(rng.integers(0, 100000))}" for _ in range(40))
               for _ in range(120)]
    pd, po = _plans(queries, 7, 64)
    H.note("[passes] 4800 terms")
    np.testing.assert_array_equal(H.search(index, bbo, pd, po, 3, 7), O.search_packed(index, bbo, pd, po, 3, 7))


def test_program_forms():
    """Queries compiled to each program form: flat OR-of-ANDs, flat
    complement (AND-of-ORs) and the stack form (both flat forms too large)."""
    rng = np.random.default_rng(5)
    ids, offs, vals = _random_corpus(rng, 9000, 4, 1, 4, 60)
    index, bbo = H.build(ids, offs, vals, 4.0, 3)

    def t():
        return f"{int(rng.choice(ids))}:{int(rng.integers(-15, 60))}"

    def ors(n):
        return "(" + " OR ".join(t() for _ in range(n)) + ")"

    block = lambda: "(" + " AND ".join(ors(2) for _ in range(4)) + ")"
    queries = [
        " OR ".join(f"{t()} AND NOT {t()}" for _ in range(5)),      # flat
        " AND ".join(ors(2) for _ in range(8)),                      # flat complement
        " OR ".join(block() for _ in range(3)),                      # stack form
        "NOT (" + " OR ".join(block() for _ in range(3)) + ")",      # stack form, negated
        f"{t()} AND NOT {t()} AND ({t()} OR NOT ({t()} AND {t()}))",
        f"({t()} OR {t()}) AND NOT ({t()} OR {t()})",
    ]
    for hk, k in [(7, 3), (3, 3), (9, 9)]:
        pd, po = _plans(queries, hk, 3)
        H.note(f"[forms] hash_k={hk} k={k}")
        np.testing.assert_array_equal(H.search(index, bbo, pd, po, k, hk), O.search_packed(index, bbo, pd, po, k, hk))


def test_edge_cases():
    c = G.case("features10x3")
    # no queries
    out = H.search(c["index"], c["bundle_b_offsets"], np.zeros(0, np.int8), np.zeros(0, np.int64), 3, 7)
    assert out.shape == (0, 32)
    # zero docs
    ids = np.array([1], dtype=np.int32)
    index, bbo = H.build(ids, np.zeros(1, np.int64), np.zeros(0, np.int64), 2.0, 3)
    assert index.size == 0 and bbo.tolist() == [0]
    pd, po = _plans(["1:1", ""], 7)
    assert H.search(index, bbo, pd, po, 3, 7).shape == (2, 0)
    # docs without terms: width-0 bundles, terms match nothing, NOT / EMPTY match all
    index, bbo = H.build(ids, np.zeros(3001, np.int64), np.zeros(0, np.int64), 2.0, 3)
    assert bbo.tolist() == [0, 0, 0]
    pd, po = _plans(["1:1", "NOT 1:1", ""], 7)
    got = H.search(index, bbo, pd, po, 3, 7)
    np.testing.assert_array_equal(got, O.search_packed(index, bbo, pd, po, 3, 7))
    assert (got[0] == 0).all() and (got[1] == -1).all() and (got[2] == -1).all()


def test_hand_built_plans():
    """Plans the parser never writes: a negative child count (the operator
    pops nothing and pushes its identity), 4000 nested NOTs, and a query
    whose flat form repeats a term."""
    c = G.case("features10x3")
    index, bbo = c["index"], c["bundle_b_offsets"]
    _, data, offs = P.parse_batch(["1:2"], 7)
    h = list(np.frombuffer(data[offs[6]:offs[7]], dtype="<u8"))
    plans = [
        ([4, 1], [0, 1, -2], h),               # TERM, AND(-3 children) -> all ones
        ([4, 2], [0, 1, -1], h),               # TERM, OR(-2 children) -> zero
        ([4] + [3] * 4000, list(range(4002)), h),  # NOT^4000 TERM = TERM
        ([4, 4, 4, 1, 2], [0, 1, 2, 3, 5, 7], h * 3),  # t OR (t AND t)
    ]
    pd, po = bytearray(), []
    for ops, o, hs in plans:
        d, of = G.encode_plan(ops, o, hs)
        po += [x + len(pd) for x in of]
        pd += d
    pd = np.frombuffer(bytes(pd), dtype=np.int8).copy()
    po = np.array(po, dtype=np.int64)
    H.note("[hand-built plans]")
    got = H.search(index, bbo, pd, po, 3, 7)
    want = O.search_packed(index, bbo, pd, po, 3, 7)
    np.testing.assert_array_equal(got, want)
    assert (got[0] == -1).all() and (got[1] == 0).all()
    np.testing.assert_array_equal(got[2], got[3])


# ------------------------------------------------ drop-in path (torch.ops.st)

def _make_features(num_docs, num_features):  # test_bloom_index_search.py:41-53
    ids = torch.arange(num_features, dtype=torch.int32)
    vals, offs = [], [0]
    for d in range(num_docs):
        for f in range(num_features):
            vals.append(d * 100 + f)
            offs.append(len(vals))
    return ids, torch.tensor(offs, dtype=torch.long), torch.tensor(vals, dtype=torch.long)


def _oracle_for(ids, offs, vals, bm, kb, exprs, k, hk):
    index, bbo = O.bloom_build(ids.numpy(), offs.numpy(), vals.numpy(), bm, kb)
    pd, po = _plans(exprs, hk)
    return index, bbo, O.search_packed(index, bbo, pd, po, k, hk)


@pytest.mark.parametrize("exprs", [["0:0"], ["0:0 AND 1:1"], ["0:0 OR 1:1"], ["NOT 0:0"], ["0:0", "1:1", "0:0 AND 1:1"]])
@pytest.mark.parametrize("bool_mask", [True, False])
def test_ops_search_like_reference_tests(exprs, bool_mask):
    st = torch.ops.st
    ids, offs, vals = _make_features(10, 3)
    bi, bo = st.bloom_index_build(ids.cuda(), offs.cuda(), vals.cuda(), 2.0, 7)
    _, (pd, po) = st.parse_expression_query_batch(exprs, torch.ones(1, dtype=torch.long), 7, True, 5)
    res = st.bloom_index_search_batch(bi, bo, pd.cuda(), po.cuda(), 3, 7, bool_mask)
    assert res.is_cuda and res.size(0) == len(exprs)
    assert res.dtype == (torch.bool if bool_mask else torch.long)
    _, _, want = _oracle_for(ids, offs, vals, 2.0, 7, exprs, 3, 7)
    want = O.unpack_bool(want) if bool_mask else want
    np.testing.assert_array_equal(res.cpu().numpy(), want)
    # CPU tensors go through the same HIP path (copied to the GPU and back)
    res_cpu = st.bloom_index_search_batch(bi.cpu(), bo.cpu(), pd, po, 3, 7, bool_mask)
    assert not res_cpu.is_cuda
    np.testing.assert_array_equal(res_cpu.numpy(), want)


@pytest.mark.parametrize("shape", ["basic", "single_doc", "many_docs"] + [f"k{k}" for k in (1, 3, 7, 10)])
def test_ops_build_like_reference_tests(shape):  # test_bloom_indexer.py:112-150
    st = torch.ops.st
    k, bm = 7, 2.0
    if shape == "basic":
        ids, offs, vals = _make_features(10, 3)
    elif shape == "single_doc":
        ids, offs, vals = torch.tensor([0], dtype=torch.int32), torch.tensor([0, 1]), torch.tensor([42])
        k = 3
    elif shape == "many_docs":
        n = 32 * 64 * 2 + 10
        ids, offs, vals = torch.tensor([0], dtype=torch.int32), torch.arange(n + 1), torch.arange(n)
        k = 3
    else:
        ids, offs, vals = _make_features(5, 2)
        k = int(shape[1:])
    bi, bo = st.bloom_index_build(ids.cuda(), offs.cuda(), vals.cuda(), bm, k)
    assert bi.dtype == torch.long and bi.dim() == 1 and bi.numel() > 0
    assert bo[0].item() == 0 and bo[-1].item() > 0
    want_i, want_b = O.bloom_build(ids.numpy(), offs.numpy(), vals.numpy(), bm, k)
    np.testing.assert_array_equal(bi.cpu().numpy(), want_i)
    np.testing.assert_array_equal(bo.cpu().numpy(), want_b)
    if shape == "many_docs":
        assert bo.numel() > 2
    bi2, bo2 = st.bloom_index_build(ids, offs, vals, bm, k)  # CPU tensors, same HIP path
    assert torch.equal(bi2, bi.cpu()) and torch.equal(bo2, bo.cpu())


def test_ops_readme_example():
    """README.md:118-196 with CPU tensors, as the README writes it."""
    st = torch.ops.st
    ids = torch.tensor([1, 2], dtype=torch.int32)
    vals = torch.tensor([100, 200, 201, 100, 101, 200, 102, 202, 100, 200, 203], dtype=torch.long)
    offs = torch.tensor([0, 1, 3, 5, 6, 7, 8, 9, 11], dtype=torch.long)
    bi, bo = st.bloom_index_build(ids, offs, vals, 5.0, 3)
    queries = ["1:100", "1:100 AND NOT 2:201", "1:102 OR 2:203"]
    _, (pd, po) = st.parse_expression_query_batch(queries, torch.full((3,), 3, dtype=torch.long), 7, True, 5)
    mask = st.bloom_index_search_batch(bi.cuda(), bo.cuda(), pd.cuda(), po.cuda(), 3, 7, True)
    hits = [m.nonzero().flatten().tolist() for m in mask[:, :4].cpu()]
    assert hits == [[0, 1, 3], [1, 3], [2, 3]]
    assert mask.shape == (3, 2048)


def test_ops_column_info():  # test_bloom_index_search.py:216-241
    st = torch.ops.st
    offsets = torch.tensor([0, 100, 200, 63, 64], dtype=torch.long)
    lengths = torch.tensor([100, 50, 80, 0, 1], dtype=torch.long)
    counts, starts, firsts = st.generate_column_info_for_clusters(offsets.cuda(), lengths.cuda())
    assert counts.is_cuda and counts.dtype == torch.int32 and starts.dtype == torch.int32
    assert firsts.dtype == torch.int8
    want_s = (offsets // 64).tolist()
    want_f = (offsets % 64).tolist()
    want_c = [(l + f + 63) // 64 if l > 0 else 0 for l, f in zip(lengths.tolist(), want_f)]
    assert counts.cpu().tolist() == want_c and starts.cpu().tolist() == want_s and firsts.cpu().tolist() == want_f


@pytest.mark.parametrize("cfg,docs", [("cfg1", 30000), ("cfg2", 40000), ("cfg3", 12000), ("cfg4", 30000),
                                      ("cfg5", 30000)])
def test_config_shapes_vs_oracle(cfg, docs):
    """The benchmark configurations' corpus and query distributions
    (silvertorch_amd.synthetic) at reduced doc counts: the
    same feature counts, value distributions, k / hash_k / B_MULTIPLIER and
    query shapes (cfg3: bundles wider than the LDS tile, k = 4, boolean trees
    with NOT, whose 1,024 plans are large enough for the multi-threaded
    host compile; cfg4, a build-only configuration: uniform values over 10M
    and 1-8 values per feature, searched with flat queries of 1-4 terms drawn
    from its value distribution), build and search bit-exact against the
    oracle."""
    from silvertorch_amd import synthetic as S

    cspec, qspec = S.CONFIGS[cfg]
    if qspec is None:
        qspec = S.QuerySpec(64, "flat", 1, 4)
    corp = S.make_corpus(cspec, seed=0, num_docs=docs)
    queries = S.make_queries(cspec, qspec, seed=0)
    if cfg == "cfg4":  # terms of docs in the corpus, so that queries match
        rng = np.random.default_rng(4)
        d = rng.integers(0, docs, 32)
        queries += [f"{f + 1}:{int(corp.feature_values[corp.feature_offsets[x * 4 + f]])}"
                    for x, f in zip(d, rng.integers(0, 4, 32))]
    H.note(f"[config] {cfg} docs={docs} queries={len(queries)} k={cspec.k} bm={cspec.b_multiplier}")
    index, bbo = H.build(corp.feature_ids, corp.feature_offsets, corp.feature_values, cspec.b_multiplier, cspec.k)
    want_index, want_bbo = O.bloom_build(corp.feature_ids, corp.feature_offsets, corp.feature_values,
                                         cspec.b_multiplier, cspec.k)
    np.testing.assert_array_equal(bbo, want_bbo)
    np.testing.assert_array_equal(index, want_index)
    pd, po = _plans(queries, cspec.hash_k)
    want = O.search_packed(index, bbo, pd, po, cspec.k, cspec.hash_k)
    np.testing.assert_array_equal(H.search(index, bbo, pd, po, cspec.k, cspec.hash_k), want)
    if cfg != "cfg3":
        got_b = H.search(index, bbo, pd, po, cspec.k, cspec.hash_k, bool_mask=True, bind="host")
        np.testing.assert_array_equal(got_b, O.unpack_bool(want))
    ids, ro, packed = H.search_ids(index, bbo, pd, po, cspec.k, cspec.hash_k, docs)
    np.testing.assert_array_equal(packed, want)
    want_ids, want_ro = O.compact(want, docs)
    np.testing.assert_array_equal(ro, want_ro)
    np.testing.assert_array_equal(ids, want_ids)


def test_mixed_bundle_kinds_in_one_launch():
    """One search launch over bundles of every kind: more distinct widths than
    width slots (bundles without a slot), bundles wider than the LDS tile,
    and staged slotted bundles whose flat programs run as a literal stream."""
    rng = np.random.default_rng(77)
    nb = 150
    n = nb * 2048
    cnt = np.ones(n, dtype=np.int64)
    for b in range(nb):  # one heavy doc per bundle sets the width
        cnt[b * 2048 + int(rng.integers(0, 2048))] = 1 + (b % 90) if b % 37 else 400
    offs = np.concatenate([[0], np.cumsum(cnt)]).astype(np.int64)
    vals = rng.integers(0, 3000, int(offs[-1])).astype(np.int64)
    ids = np.array([3], dtype=np.int32)
    index, bbo = H.build(ids, offs, vals, 1.5, 1)
    widths = np.diff(bbo)
    assert len(set(widths.tolist())) > 64 and widths.max() > 512
    queries = []
    for _ in range(200):
        t = int(rng.integers(1, 6))
        queries.append(" OR ".join(" AND ".join(f"3:{int(rng.integers(0, 3000))}" for _ in range(int(rng.integers(1, 3))))
                                   for _ in range(t)))
    pd, po = _plans(queries, 5)
    H.note(f"[mixed] bundles={nb} widths={len(set(widths.tolist()))} max={widths.max()} queries={len(queries)}")
    want = O.search_packed(index, bbo, pd, po, 1, 5)
    np.testing.assert_array_equal(H.search(index, bbo, pd, po, 1, 5), want)
    np.testing.assert_array_equal(H.search(index, bbo, pd, po, 1, 5, bool_mask=True, bind="device"),
                                  O.unpack_bool(want))


@pytest.mark.parametrize("bind", ["host", "device", "none"])
def test_search_copies_its_plan_from_pinned_memory(bind):
    """st_search_plan_upload_source: the search call's first kernel copies
    the plan blob from pinned host memory into a device buffer that starts
    as garbage (0xEE); the output equals the oracle's, packed and bool."""
    c = G.case("random3")
    H.note(f"[upload source] bind={bind}")
    want = O.search_packed(c["index"], c["bundle_b_offsets"], c["plans_data"], c["plans_offsets"], c["k"], c["hash_k"])
    for bool_mask in (False, True):
        got = H.search(c["index"], c["bundle_b_offsets"], c["plans_data"], c["plans_offsets"], c["k"], c["hash_k"],
                       bool_mask, bind=bind, upload=True)
        np.testing.assert_array_equal(got, O.unpack_bool(want) if bool_mask else want)


def test_upload_signal_words_hold_the_value_after_the_copy():
    """st_search_plan_upload_signal: a plan of 700 queries (a blob over
    64 KB, so several upload workgroups) copied by the search call from
    pinned memory; after the call each group's word holds the value, the
    words past the group count keep their fill, and the output equals the
    oracle's.  The torch ops reuse their pinned plan slots on these words."""
    from silvertorch_amd import capi
    from silvertorch_amd import synthetic as S

    cspec, _ = S.CONFIGS["cfg2"]
    docs = 20_000
    corp = S.make_corpus(cspec, seed=5, num_docs=docs)
    queries = S.make_queries(cspec, S.QuerySpec(700, "flat", 2, 6), seed=5)
    index, bbo = H.build(corp.feature_ids, corp.feature_offsets, corp.feature_values, cspec.b_multiplier, cspec.k)
    pd, po = _plans(queries, cspec.hash_k)
    want = O.search_packed(index, bbo, pd, po, cspec.k, cspec.hash_k)
    L = capi.lib()
    plan = capi.SearchPlan(bytes(pd.tobytes()), po, cspec.k, cspec.hash_k)
    nb = len(bbo) - 1
    plan.prepare_device_binding(nb)
    blob = plan.blob()
    pinned = torch.frombuffer(bytearray(blob), dtype=torch.uint8).pin_memory()
    capi.check(L.st_search_plan_upload_source(plan.handle, pinned.data_ptr()))
    groups = L.st_search_plan_upload_groups(plan.handle)
    H.note(f"[upload signal] blob={len(blob)} bytes groups={groups}")
    assert groups == (len(blob) + 65535) // 65536 and groups >= 2
    words = torch.full((groups + 2,), 7, dtype=torch.long).pin_memory()
    value = 0x0123456789ABCDEF
    capi.check(L.st_search_plan_upload_signal(plan.handle, words.data_ptr(), value))
    blob_d = torch.full((plan.device_bytes,), 0xEE, dtype=torch.uint8, device="cuda")
    idx_d = torch.as_tensor(index).cuda()
    bbo_d = torch.as_tensor(bbo).cuda()
    out = torch.empty((plan.num_queries, nb * 32), dtype=torch.long, device="cuda")
    capi.check(L.st_bloom_index_search_batch(idx_d.data_ptr(), idx_d.numel(), bbo_d.data_ptr(), nb, plan.handle,
                                             blob_d.data_ptr(), 0, out.data_ptr(),
                                             torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert words[:groups].tolist() == [value] * groups
    assert words[groups:].tolist() == [7, 7]
    np.testing.assert_array_equal(out.cpu().numpy(), want)


@pytest.mark.timeout(600)
def test_more_distinct_widths_than_the_census_holds():
    """2100 bundles of 2100 distinct widths (1 .. 2102 rows: staged, column-
    slice and global-memory bundles), more than the device census tracks: no
    width gets a slot, every bundle resolves its own positions.  Packed and
    bool outputs against the oracle for host-bound, device-bound and unbound
    plans (host binding still slots the 64 most frequent widths)."""
    rng = np.random.default_rng(2100)
    nb = 2100
    n = nb * 2048
    cnt = np.zeros(n, dtype=np.int64)
    heavy = np.arange(nb) * 2048 + rng.integers(0, 2048, nb)
    cnt[heavy] = 1 + np.arange(nb)  # width of bundle b: (int)((1 + b) * 1.001)
    offs = np.concatenate([[0], np.cumsum(cnt)]).astype(np.int64)
    vals = rng.integers(0, 5000, int(offs[-1])).astype(np.int64)
    ids = np.array([2], dtype=np.int32)
    index, bbo = H.build(ids, offs, vals, 1.001, 1)
    widths = np.diff(bbo)
    assert len(set(widths.tolist())) == nb and widths.max() > 2048
    queries = [" OR ".join(f"2:{int(v)}" for v in rng.integers(0, 5000, int(rng.integers(1, 4))))
               for _ in range(24)] + ["2:1 AND NOT 2:2", ""]
    pd, po = _plans(queries, 3)
    H.note(f"[census overflow] bundles={nb} distinct widths={len(set(widths.tolist()))}")
    want = O.search_packed(index, bbo, pd, po, 1, 3)
    np.testing.assert_array_equal(H.search(index, bbo, pd, po, 1, 3), want)
    np.testing.assert_array_equal(H.search(index, bbo, pd, po, 1, 3, bool_mask=True, bind="device")[:, :nb * 64],
                                  O.unpack_bool(want)[:, :nb * 64])


@pytest.mark.parametrize("k,neg,many", [(1, False, False), (3, True, False), (4, False, False),
                                        (4, True, True), (7, True, False)])
def test_wide_bundle_slices_vs_oracle(k, neg, many):
    """Bundles wider than the LDS tile and at most 2048 rows (searched in
    column slices by the wide-bundle kernel in packed mode) next to staged
    bundles and bundles past 2048 rows (global-memory path), for several k,
    with and without negated literals, in one or several query batches
    (`many`: more distinct terms than one batch holds).  Packed, bool and
    counted outputs against the oracle, for host-bound, device-bound and
    unbound plans."""
    rng = np.random.default_rng(500 + k)
    heavy = {1: [150, 300, 700, 1024, 1100], 3: [50, 100, 300, 341, 400],
             4: [40, 100, 200, 256, 300], 7: [20, 50, 100, 146, 200]}[k]
    nb, F, vocab = 23, 2, 3000
    n = nb * 2048 - 700  # ragged last bundle
    cnt = rng.integers(1, 4, (n, F)).astype(np.int64)
    for b in range(nb):  # one heavy doc per bundle sets the width
        cnt[b * 2048 + int(rng.integers(0, min(2048, n - b * 2048))), 0] = heavy[b % len(heavy)]
    offs = np.concatenate([[0], np.cumsum(cnt.reshape(-1))]).astype(np.int64)
    vals = rng.integers(0, vocab, int(offs[-1])).astype(np.int64)
    ids = np.array([1, 2], dtype=np.int32)
    index, bbo = H.build(ids, offs, vals, 2.0, k)
    widths = np.diff(bbo)
    assert (widths <= 512).any() and ((widths > 512) & (widths <= 2048)).any() and (widths > 2048).any()

    def term():
        t = f"{int(rng.integers(1, F + 1))}:{int(rng.integers(0, vocab))}"
        return ("NOT " + t) if neg and rng.random() < 0.2 else t

    if many:
        queries = [" OR ".join(term() for _ in range(40)) for _ in range(120)]
    else:
        queries = [" OR ".join(" AND ".join(term() for _ in range(int(rng.integers(1, 3))))
                               for _ in range(int(rng.integers(1, 5)))) for _ in range(300)]
    pd, po = _plans(queries, 7, 64 if many else 5)
    H.note(f"[wide] k={k} neg={neg} many={many} widths={sorted(set(widths.tolist()))}")
    want = O.search_packed(index, bbo, pd, po, k, 7)
    np.testing.assert_array_equal(H.search(index, bbo, pd, po, k, 7), want)
    np.testing.assert_array_equal(H.search(index, bbo, pd, po, k, 7, bool_mask=True, bind="device"),
                                  O.unpack_bool(want))
    _, ro, packed = H.search_ids(index, bbo, pd, po, k, 7, n)
    np.testing.assert_array_equal(packed, want)
    np.testing.assert_array_equal(ro, O.compact(want, n)[1])


def test_plan_ring_slots_survive_failed_calls():
    """A search op that fails after its plan took a slot of the device's
    pinned plan ring (here the bool output of 2^24 empty bundles for 16
    queries, 512 GB, cannot be allocated) frees the slot itself, since no
    upload workgroup will; the int32-ids check of the ids op fails before a
    slot is taken.  After 20 failures of each kind every slot is free and a
    search still runs and gives the same output."""
    import ctypes
    from pathlib import Path

    st = torch.ops.st
    ring = ctypes.CDLL(str(Path(__file__).resolve().parents[1] / "silvertorch_amd" / "_C.so"))
    ring.st_torch_plan_ring_free_slots.restype = ctypes.c_int
    ring.st_torch_plan_ring_free_slots.argtypes = [ctypes.c_int]
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(5)
    n, F = 5000, 2
    cnt = rng.integers(1, 3, (n, F))
    offs = np.concatenate([[0], np.cumsum(cnt.reshape(-1))]).astype(np.int64)
    vals = rng.integers(0, 30, int(offs[-1])).astype(np.int64)
    bi, bo = st.bloom_index_build(torch.tensor([1, 2], dtype=torch.int32, device=dev),
                                  torch.from_numpy(offs).to(dev), torch.from_numpy(vals).to(dev), 5.0, 3)
    queries = [f"1:{i} OR 2:{i + 1}" for i in range(16)]
    _, (pd, po) = st.parse_expression_query_batch(queries, torch.ones(1, dtype=torch.long), 7, True, 5)
    want = st.bloom_index_search_batch(bi, bo, pd, po, 3, 7, False)
    torch.cuda.synchronize()
    assert ring.st_torch_plan_ring_free_slots(0) == 16
    empty_index = torch.empty(0, dtype=torch.long, device=dev)
    many_bundles = torch.zeros((1 << 24) + 1, dtype=torch.long, device=dev)
    H.note("[ring] 20 calls failing after the plan upload was prepared")
    for _ in range(20):
        with pytest.raises(RuntimeError):
            st.bloom_index_search_batch(empty_index, many_bundles, pd, po, 3, 7, True)
    H.note("[ring] 20 calls failing the int32-ids check")
    for _ in range(20):
        with pytest.raises(RuntimeError, match="int32 ids cannot hold"):
            st.bloom_index_search_batch_ids(empty_index, many_bundles[:(1 << 20) + 1], pd, po, 3, 7, 1 << 31)
    torch.cuda.synchronize()
    assert ring.st_torch_plan_ring_free_slots(0) == 16, "a failed call kept its pinned plan slot"
    got = st.bloom_index_search_batch(bi, bo, pd, po, 3, 7, False)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    del many_bundles
    torch.cuda.empty_cache()
