"""Pins the CPU oracle before it is trusted as the parity checker.

Every oracle function is checked against data the oracle did not produce:
sklearn's independent MurmurHash3 vectors, the reference's own CPU ops
(compiled from its sources into oracle/_ref, fixtures in tests/golden/), the
README known answers (README.md:163-196, :255-268), brute force and
closed-form invariants.  The last test plants mistakes in a copy of the
oracle logic and shows the checks catch them.
"""

import numpy as np
import pytest

from oracle import oracle as O
from oracle import parser_oracle as P
from tests import _fixtures as G


def test_murmur_matches_independent_vectors():
    for x, y, seed, want in G.murmur_vectors():
        assert O.murmur3_pair(x, y, seed) == want
        assert P.murmur3_pair(x, y, seed) == want


def test_build_positions_brute_force():
    rng = np.random.default_rng(3)
    for _ in range(300):
        fid, val = int(rng.integers(-50, 50)), int(rng.integers(-(1 << 40), 1 << 40))
        k = int(rng.integers(1, 12))
        b = int(rng.integers(k, 3 * k + 40))
        want, seed = [], 0
        while len(want) < k:  # first k distinct residues over seeds 0, 1, ...
            p = P.murmur3_pair(fid, val, seed) % b
            seed += 1
            if p not in want:
                want.append(p)
        assert O.build_positions(fid, val, b, k) == want


@pytest.mark.parametrize("name", G.case_names())
def test_oracle_build_matches_reference(name):
    c = G.case(name)
    index, bbo = O.bloom_build(c["ids"], c["offsets"], c["values"], c["b_multiplier"], c["build_k"])
    np.testing.assert_array_equal(bbo, c["bundle_b_offsets"])
    np.testing.assert_array_equal(index, c["index"])


@pytest.mark.parametrize("name", G.case_names())
def test_oracle_search_matches_reference(name):
    c = G.case(name)
    packed = O.search_packed(c["index"], c["bundle_b_offsets"], c["plans_data"], c["plans_offsets"], c["k"], c["hash_k"])
    np.testing.assert_array_equal(packed, c["packed"])


def test_readme_known_answers():
    c = G.case("readme")
    index, bbo = O.bloom_build(c["ids"], c["offsets"], c["values"], 5.0, 3)
    _, data, offs = P.parse_batch(c["queries"], 7)
    packed = O.search_packed(index, bbo, np.frombuffer(data, np.int8), np.array(offs), 3, 7)
    ids, ro = O.compact(packed, 4)
    got = [ids[ro[q]:ro[q + 1]].tolist() for q in range(len(ro) - 1)]
    assert got == [[0, 1, 3], [1, 3], [2, 3], [0, 1, 3], [2]]
    assert O.unpack_bool(packed).shape == (5, 2048)  # README.md:260


def _nonzero_csr(packed, num_docs):
    """CSR of mask[:, :num_docs].nonzero() with the mask unpacked MSB-first."""
    q, c = packed.shape
    bits = np.unpackbits(packed.astype(">i8").view(np.uint8).reshape(q, c * 8), axis=1)
    rows, cols = np.nonzero(bits[:, :num_docs])
    ro = np.zeros(q + 1, dtype=np.int64)
    np.add.at(ro, rows + 1, 1)
    return cols.astype(np.int64), np.cumsum(ro)


def test_compact_matches_numpy_nonzero():
    rng = np.random.default_rng(21)
    for q, c in [(0, 0), (3, 0), (0, 5), (4, 33), (7, 64), (5, 1)]:
        for density in (0.0, 0.03, 0.5, 1.0):
            packed = np.packbits(rng.random((q, c * 64)) < density, axis=1).view(">i8").astype(np.int64) \
                if q and c else np.zeros((q, c), dtype=np.int64)
            for nd in sorted({0, 1, 37, max(c * 64 - 5, 0), c * 64, c * 64 + 100}):
                ids, ro = O.compact(packed, nd)
                want_ids, want_ro = _nonzero_csr(packed, nd)
                np.testing.assert_array_equal(ro, want_ro)
                np.testing.assert_array_equal(ids, want_ids)


def test_filtered_topk_matches_brute_force():
    """The oracle's filtered top-k against a numpy restatement on tiny inputs:
    fp64 scores of filter-passing docs, order (score desc, id asc), -1/-inf
    padding; includes exact ties (repeated embeddings) and empty filters."""
    rng = np.random.default_rng(31)
    for n, dim, q, topk in [(1, 4, 1, 1), (70, 8, 3, 5), (130, 16, 4, 20), (200, 8, 2, 300)]:
        emb = rng.integers(-3, 4, (n, dim)).astype(np.float32)  # small ints: many exact ties
        qv = rng.integers(-3, 4, (q, dim)).astype(np.float32)
        cols = (n + 63) // 64
        bits = rng.random((q, cols * 64)) < 0.6
        bits[0, :] = False if q > 1 else bits[0, :]
        packed = np.packbits(bits, axis=1).view(">i8").astype(np.int64)
        ids, scores = O.filtered_topk(emb, qv, packed, topk)
        for qi in range(q):
            passing = [d for d in range(n) if bits[qi, d]]
            sc = {d: float(np.dot(emb[d].astype(np.float64), qv[qi].astype(np.float64))) for d in passing}
            order = sorted(passing, key=lambda d: (-sc[d], d))[:topk]
            want_ids = order + [-1] * (topk - len(order))
            want_sc = [sc[d] for d in order] + [-np.inf] * (topk - len(order))
            assert ids[qi].tolist() == want_ids
            np.testing.assert_array_equal(scores[qi], np.array(want_sc, dtype=np.float32))


def test_parser_oracle_matches_reference_bytes():
    g = G.parser_golden()
    for b in g["batches"]:
        m, data, offs = P.parse_batch(g["expressions"], b["hash_k"], True, b["max_sub_queries"])
        assert m == b["max_stack"]
        assert data.hex() == b["data_hex"]
        assert offs == b["offsets"]
    m, data, offs = P.parse_batch(g["expressions"], 7, False, 5)
    assert (m, len(data), len(offs)) == tuple(g["no_plan"].values())


def test_parser_oracle_errors_match_reference():
    for expr, msg in G.parser_golden()["errors"].items():
        if msg is None:
            P.parse_batch([expr], 7)
        else:
            with pytest.raises(P.ParseError) as ei:
                P.parse_batch([expr], 7)
            assert str(ei.value) == msg


def test_parser_precedence_rules():
    # test_expression_query_parser.py:98-117
    same = [("NOT 1:10 AND 2:20", "(NOT 1:10) AND 2:20"), ("1:10 OR 2:20 AND 3:30", "1:10 OR (2:20 AND 3:30)")]
    for a, b in same:
        assert P.parse_batch([a], 7) == P.parse_batch([b], 7)
    assert P.parse_batch(["(1:10 OR 2:20) AND 3:30"], 7) != P.parse_batch(["1:10 OR 2:20 AND 3:30"], 7)
    assert P.parse_batch(["42:100"], 7)[0] == 1


def test_cfg1_digest():
    from silvertorch_amd import synthetic as S

    d = G.digests()["cfg1"]
    cspec, qspec = S.CONFIGS["cfg1"]
    corp = S.make_corpus(cspec, seed=0)
    assert G.sha(corp.feature_offsets) == d["inputs"]["offsets"]
    assert G.sha(corp.feature_values) == d["inputs"]["values"]
    index, bbo = O.bloom_build(corp.feature_ids, corp.feature_offsets, corp.feature_values, cspec.b_multiplier, cspec.k)
    assert G.sha(index) == d["index"] and G.sha(bbo) == d["bundle_b_offsets"]
    queries = S.make_queries(cspec, qspec, seed=0)
    _, data, offs = P.parse_batch(queries, cspec.hash_k)
    pd, po = np.frombuffer(data, np.int8), np.array(offs, dtype=np.int64)
    assert G.sha(pd) == d["plans_data"] and G.sha(po) == d["plans_offsets"]
    packed = O.search_packed(index, bbo, pd, po, cspec.k, cspec.hash_k)
    assert G.sha(packed) == d["packed"]
    _, ro = O.compact(packed, cspec.num_docs)
    assert np.diff(ro).tolist() == d["match_counts"]


def test_wide_bundles_int16_wrap_digest():
    ids, offs, vals, w = G.wide_corpus()
    index, bbo = O.bloom_build(ids, offs, vals, w["b_multiplier"], w["k"])
    assert bbo.tolist() == w["bundle_b_offsets"]
    assert G.sha(index) == w["index"]
    _, data, po = P.parse_batch(w["queries"], 7)
    packed = O.search_packed(index, bbo, np.frombuffer(data, np.int8), np.array(po), w["k"], 7)
    assert G.sha(packed) == w["packed"]


def test_build_invariants():
    rng = np.random.default_rng(11)
    n, F, k = 5000, 2, 4
    cnt = rng.integers(0, 3, (n, F))
    offs = np.concatenate([[0], np.cumsum(cnt.reshape(-1))]).astype(np.int64)
    vals = rng.integers(0, 1 << 40, int(offs[-1])).astype(np.int64)
    ids = np.array([3, 9], dtype=np.int32)
    index, bbo = O.bloom_build(ids, offs, vals, 2.5, k)
    # closed form of the widths
    per_doc = cnt.sum(1)
    for i in range(len(bbo) - 1):
        m = per_doc[i * 2048:(i + 1) * 2048].max()
        assert bbo[i + 1] - bbo[i] == int(float(m * k) * 2.5)
    # a doc's bits are the union of its terms' positions (no false negatives,
    # nothing extra)
    words = index.view(np.uint64)
    for d in rng.choice(n, 60, replace=False):
        bnd, col, bit = d // 2048, (d % 2048) // 64, np.uint64(1) << np.uint64(63 - d % 64)
        b = int(bbo[bnd + 1] - bbo[bnd])
        want = set()
        for f in range(F):
            for j in range(offs[d * F + f], offs[d * F + f + 1]):
                want |= set(O.build_positions(int(ids[f]), int(vals[j]), b, k))
        have = {p for p in range(b) if words[(bbo[bnd] + p) * 32 + col] & bit}
        assert have == want


def test_search_identities():
    c = G.case("random0")
    base = ["1:1", "1:2", "4:5"]
    exprs = [f"NOT ({base[0]} AND {base[1]})", f"NOT {base[0]} OR NOT {base[1]}", "", f"{base[2]} OR NOT {base[2]}"]
    _, data, offs = P.parse_batch(exprs, c["hash_k"])
    packed = O.search_packed(c["index"], c["bundle_b_offsets"], np.frombuffer(data, np.int8), np.array(offs), c["k"], c["hash_k"])
    np.testing.assert_array_equal(packed[0], packed[1])  # De Morgan
    assert (packed[2] == -1).all() and (packed[3] == -1).all()  # EMPTY, x | ~x


def test_planted_mistakes_are_caught():
    """Variants of the oracle logic with a plausible bug must fail the pins."""
    x, y, seed, want = G.murmur_vectors()[10]
    # (1) swapped key halves, (2) seed off by one
    assert P.murmur3_pair(y, x, seed) != want
    assert P.murmur3_pair(x, y, seed + 1) != want
    # (3) LSB-first doc order in the words, (4) transposed [column][row] layout
    c = G.case("readme")
    index, _ = O.bloom_build(c["ids"], c["offsets"], c["values"], 5.0, 3)
    w = index.view(np.uint64)
    rev = np.array([int(f"{int(v):064b}"[::-1], 2) for v in w], dtype=np.uint64)
    assert not np.array_equal(rev.view(np.int64), c["index"])
    rows = len(index) // 32
    assert not np.array_equal(index.reshape(rows, 32).T.reshape(-1), c["index"])
    # (5) evaluating with the int32 cast of the CUDA path instead of int16
    ids, offs, vals, wd = G.wide_corpus()
    idx, bbo = O.bloom_build(ids, offs, vals, wd["b_multiplier"], wd["k"])
    h = P.murmur3_pair(5, int(vals[4200]), 0)
    b1 = int(bbo[2] - bbo[1])
    assert np.int16(np.int64(h % b1).astype(np.int16)) != h % b1 or h % b1 < 32768


@pytest.mark.parametrize("name", G.partial_case_names())
def test_oracle_partial_response_matches_reference(name):
    """Cluster-restricted search (bloom_index_search.cpp:246-395): the oracle
    reproduces the reference CPU op's three outputs exactly."""
    c = G.partial_case(name)
    k, hk = (int(v) for v in c["params"])
    got = O.partial_response(c["index"], c["bundle_b_offsets"], c["plans_data"], c["plans_offsets"], k, hk,
                             c["cluster_offsets"], c["cluster_lengths"], c.get("plan_index"))
    for g, w in zip(got, (c["cumsum"], c["first"], c["mask"])):
        assert g.dtype == w.dtype
        np.testing.assert_array_equal(g, w)


def test_oracle_partial_multiple_matches_reference():
    """_multiple (bloom_index_search.cpp:420-487) is the single op per chunk;
    the reference's fuse flag does not change its outputs."""
    m = G.partial_multiple()
    for fuse in (0, 1):
        for ch, want in zip(m["chunks"], m["outputs"][fuse]):
            got = O.partial_response(ch["index"], ch["bundle_b_offsets"], m["plans_data"], m["plans_offsets"],
                                     3, 7, ch["cluster_offsets"], ch["cluster_lengths"])
            for g, w in zip(got, want):
                np.testing.assert_array_equal(g, w)


def test_partial_response_columns_are_search_columns():
    """Every returned column word is the full search's word for that plan
    and column; cumsum / offsets follow the integer rules (C++ truncating
    division, int8 offsets) on negative and unaligned starts."""
    c = G.partial_case("varied_plan_index")
    k, hk = (int(v) for v in c["params"])
    full = O.search_packed(c["index"], c["bundle_b_offsets"], c["plans_data"], c["plans_offsets"], k, hk)
    co, cl, pi = c["cluster_offsets"], c["cluster_lengths"], c["plan_index"]
    cumsum, first, mask = O.partial_response(c["index"], c["bundle_b_offsets"], c["plans_data"],
                                             c["plans_offsets"], k, hk, co, cl, pi)
    pos = 0
    for q in range(co.shape[0]):
        for j in range(co.shape[1]):
            s, ln = int(co[q, j]), int(cl[q, j])
            off = int(np.fmod(s, 64))
            assert first[q * co.shape[1] + j] == off
            n = (ln + off + 63) // 64 if ln > 0 else 0
            first_col = int(s / 64) if s >= 0 else -((-s) // 64)
            np.testing.assert_array_equal(mask[pos:pos + n], full[pi[q], first_col:first_col + n])
            pos += n
            assert cumsum[q * co.shape[1] + j] == pos
    assert pos == mask.size
    # out-of-range plan indices and columns are errors, not reads past the end
    with pytest.raises(ValueError, match="plan index"):
        O.partial_response(c["index"], c["bundle_b_offsets"], c["plans_data"], c["plans_offsets"], k, hk,
                           co, cl, np.full(co.shape[0], 99, dtype=np.int64))
    bad = co.copy()
    bad[0, 0] = int(c["bundle_b_offsets"].size - 1) * 2048
    with pytest.raises(ValueError, match="outside the index"):
        O.partial_response(c["index"], c["bundle_b_offsets"], c["plans_data"], c["plans_offsets"], k, hk,
                           bad, np.maximum(cl, 1), pi)


@pytest.mark.parametrize("name", G.KMEAN_CASES)
def test_kmean_oracle_matches_reference(name):
    """fused_kmean_ann oracle vs the reference CPU op's fixtures: every score
    and index bit for bit (filtered cases: the reference was given the
    bit-reversed words of the MSB-first mask; bfloat16 cases: the reference's
    float32 scores of the same values, rounded to bfloat16 by the independent
    torch conversion)."""
    import torch

    c = G.kmean_case(name)
    sc, ix = O.fused_kmean_ann(c["cluster_offsets"], c["cluster_ids"], c["cluster_length"],
                               c["embeddings"], c["queries"], c["max_size"],
                               filter_mask=c.get("mask_msb"), invalid_index=c["invalid"],
                               divisor=c["divisor"], filter_index=c.get("filter_index"),
                               scale=c.get("scale"), bf16=c["bf16"])
    np.testing.assert_array_equal(ix, c["indices"])
    if c["bf16"]:
        valid = c["indices"] != c["invalid"]
        want = torch.from_numpy(c["scores"]).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        np.testing.assert_array_equal(sc[valid], want[valid])
        assert (sc[~valid] == 0xFF7F).all()
        assert "BFloat16" in str(c["ref_error"])
    else:
        assert sc.dtype == c["scores"].dtype
        np.testing.assert_array_equal(sc.view(np.uint8), c["scores"].view(np.uint8))


def test_kmean_halfway_fixture_catches_single_rounding():
    """The f16_halfway fixture separates the reference's float64 -> float32 ->
    float16 chain (fused_kmean_ann.cpp:214) from one direct float64 -> float16
    rounding: a planted single rounding of the exact sums differs from the
    fixture, the double rounding equals it."""
    c = G.kmean_case("f16_halfway")
    e = c["embeddings"].astype(np.float64)
    q = c["queries"].astype(np.float64)
    exact = q @ e.T  # the sums are exact in float64 here
    n = e.shape[0]
    with np.errstate(over="ignore"):
        double = exact.astype(np.float32).astype(np.float16)
        single = exact.astype(np.float16)
    np.testing.assert_array_equal(double.view(np.uint16), c["scores"][:, :n].view(np.uint16))
    assert not np.array_equal(single.view(np.uint16), c["scores"][:, :n].view(np.uint16))
    assert c["scores"][0, 1].view(np.uint16) == 0x3C00 and single[0, 1].view(np.uint16) == 0x3C01


def test_kmean_oracle_partial_wrappers_match_reference():
    """The partial-mask wrappers of the reference CPU op score every doc of the
    selected clusters (the masks are ignored): the unfiltered oracle equals
    them."""
    p = G.kmean_group("partial")
    sc, ix = O.fused_kmean_ann(p["cluster_offsets"], p["cluster_ids"], p["cluster_length"],
                               p["embeddings"], p["queries"], 70)
    np.testing.assert_array_equal(ix, p["indices"])
    np.testing.assert_array_equal(sc, p["scores"])
    m = G.kmean_group("multiple")
    for c, size in enumerate((33, 50)):
        sc, ix = O.fused_kmean_ann(m[f"{c}/cluster_offsets"], m[f"{c}/cluster_ids"],
                                   m[f"{c}/cluster_length"], m[f"{c}/embeddings"], m["queries"], size)
        np.testing.assert_array_equal(ix, m[f"{c}/indices"])
        np.testing.assert_array_equal(sc, m[f"{c}/scores"])


def test_kmean_oracle_filter_identity():
    """Filtering = the unfiltered rows restricted, in order, to the docs whose
    MSB-first mask bit is set (and docs past the mask's words pass); a planted
    LSB-first reading is caught."""
    rng = np.random.default_rng(5)
    sizes = rng.integers(1, 90, 7)
    offs = np.concatenate([[0], np.cumsum(sizes)])
    emb = rng.standard_normal((int(offs[-1]), 16)).astype(np.float32)
    q = rng.standard_normal((3, 16)).astype(np.float32)
    cids = rng.integers(0, 7, (3, 3))
    mask = rng.integers(-2**63, 2**63 - 1, (3, int(offs[-1]) // 64), dtype=np.int64)
    big = 1000
    full_s, full_i = O.fused_kmean_ann(offs, cids, sizes[cids], emb, q, big)
    f_s, f_i = O.fused_kmean_ann(offs, cids, sizes[cids], emb, q, big, filter_mask=mask)
    for b in range(3):
        keep = []
        for j, d in enumerate(full_i[b].tolist()):
            if d < 0:
                break
            w = d >> 6
            if w >= mask.shape[1] or (int(mask[b, w].view(np.uint64)) >> (63 - (d & 63))) & 1:
                keep.append(j)
        np.testing.assert_array_equal(f_i[b][:len(keep)], full_i[b][keep])
        np.testing.assert_array_equal(f_s[b][:len(keep)], full_s[b][keep])
        assert (f_i[b][len(keep):] == -1).all()
    lsb = mask.view(np.uint64)
    rev = np.zeros_like(lsb)
    for i in range(64):
        rev |= ((lsb >> np.uint64(i)) & np.uint64(1)) << np.uint64(63 - i)
    planted, _ = O.fused_kmean_ann(offs, cids, sizes[cids], emb, q, big, filter_mask=rev.view(np.int64))
    assert not np.array_equal(planted, f_s)


@pytest.mark.parametrize("name", G.fresh_case_names())
def test_fresh_oracle_matches_reference(name):
    """take_top_k_and_gather_from_main_and_fresh oracle vs the reference CPU
    op's fixtures (distinct scores per row): top scores, merged indices,
    is_from_fresh and every gathered tensor, bit for bit."""
    c = G.fresh_case(name)

    def arr(path, a):
        return G.bf16_bits_to_f32(a) if path in c["bf16"] else a

    ms, fs = arr("main_scores", c["main_scores"]), arr("fresh_scores", c["fresh_scores"])
    keys = c["keys"]
    ts, ti, ff, g = O.fresh_topk_gather(ms, fs, c["main_indices"], c["fresh_indices"], c["k"],
                                        [arr(f"main_data/{k}", c["main_data"][k]) for k in keys],
                                        [arr(f"fresh_data/{k}", c["fresh_data"][k]) for k in keys])
    np.testing.assert_array_equal(ti, c["top_indices"])
    np.testing.assert_array_equal(ff, c["is_from_fresh"])
    np.testing.assert_array_equal(np.asarray(ts).view(np.uint8) if "top_scores" not in c["bf16"] else ts,
                                  c["top_scores"].view(np.uint8) if "top_scores" not in c["bf16"]
                                  else G.bf16_bits_to_f32(c["top_scores"]))
    for i, k in enumerate(keys):
        want = c["gathered"][k]
        got = g[i]
        if f"gathered/{k}" in c["bf16"]:
            want = G.bf16_bits_to_f32(want)
        assert got.shape == want.shape and got.dtype == want.dtype, (k, got.shape, want.shape)
        np.testing.assert_array_equal(got.view(np.uint8), want.view(np.uint8))


def test_fresh_oracle_ties_nan_and_zero_signs():
    """Cases the fixtures leave open (at::topk does not order equal scores):
    the oracle ranks NaN first, treats -0.0 and +0.0 as equal and breaks ties
    by the lower merged index; a brute-force rank count agrees, and a planted
    mistake (ties by the higher index) is caught."""
    rng = np.random.default_rng(5)
    ms = rng.integers(0, 4, (6, 50)).astype(np.float32)
    fs = rng.integers(0, 4, (6, 20)).astype(np.float32)
    ms[0, 3] = np.nan
    fs[1, 0] = -0.0
    ms[1, :] = 0.0
    ts, ti, ff, _ = O.fresh_topk_gather(ms, fs, None, None, 40, [], [])
    merged = np.concatenate([fs, ms], axis=1)
    for r in range(6):
        def beats(a, b):
            xa, xb = merged[r, a], merged[r, b]
            if np.isnan(xa) != np.isnan(xb):
                return bool(np.isnan(xa))
            if xa != xb and not np.isnan(xa):
                return bool(xa > xb)
            return a < b
        rank = [sum(beats(b, a) for b in range(70) if b != a) for a in range(70)]
        want = sorted(range(70), key=lambda a: rank[a])[:40]
        assert ti[r].tolist() == want
    assert np.isnan(ts[0, 0]) and ti[0, 0] == 20 + 3
    assert ff.tolist() == (ti < 20).tolist()
    planted = np.array([sorted(range(70), key=lambda a: (-merged[r, a], -a))[:40] for r in range(2, 6)])
    assert not np.array_equal(planted, ti[2:])
