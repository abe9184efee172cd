"""Full-size parity of the benchmark configurations against the reference's
own CPU ops: the corpora are regenerated with the seeded numpy generator
(silvertorch_amd.synthetic, seed 0), built and searched on the GPU through
torch.ops.st, and every output compared with the digests the reference CPU
build and search (bloom_indexer.cpp:26-113, bloom_index_search.cpp:173-243)
wrote for the same inputs (tests/golden/ref_full_digests.json, written by
tests/golden/make_golden.py full):

* cfg2 (the headline: 10M docs x 256 queries) and cfg5 (20M docs x 512
  queries): input digests (the generator itself), bundle_b_offsets,
  bloom_index, plan bytes, the packed search output, per-query match counts;
  the bool output equals the packed words bit for bit; the CSR row offsets of
  the ids op are the running sums of the reference's match counts, and its
  ids, strictly ascending per row, each on a set bit of the reference-equal
  packed output, are therefore exactly the set bits (also through
  bloom_mask_to_ids on the packed output);
* cfg3 (50M docs x 1,024 boolean trees with NOT, every bundle wider than
  the LDS tile): input digests, bundle_b_offsets, the 10.7 GB bloom_index,
  plan bytes, the 6.4 GB packed output and the per-query match counts, with
  device-bound and host-bound plans;
* cfg4 (100M docs, build only): input digests, bundle_b_offsets and the
  5.9 GB bloom_index;
* cfg5's fused search + filtered top-k on all 20M docs (every query's
  padding, filter and order; 16 sampled queries against an fp32 torch
  reference of the same values), and on a doc prefix against the oracle's
  fp64 top-k, under the stated tolerance (ids equal except swaps between
  scores within 1e-3 relative; scores within 1e-3 of the fp64 score of the
  returned id).
"""

from __future__ import annotations

import json
import time
from functools import lru_cache
from pathlib import Path

import numpy as np
import pytest
import torch

from silvertorch_amd import synthetic as S
from tests import gpu_helpers as H

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


@lru_cache(None)
def _digests() -> dict:
    return json.loads((GOLDEN / "ref_full_digests.json").read_text())


@pytest.fixture(scope="module", autouse=True)
def _ops():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    import silvertorch_amd.ops._load_ops  # noqa: F401


def _corpus_on_device(cfg: str, t0: float):
    cspec, _ = S.CONFIGS[cfg]
    d = _digests()[cfg]
    H.note(f"[full] {cfg}: generating {cspec.num_docs} docs")
    corp = S.make_corpus(cspec, seed=0, progress=lambda m: H.note(f"[full] {cfg}: {m} ({time.time() - t0:.0f}s)"))
    assert corp.feature_values.size == d["num_values"], "the generator drew another corpus"
    assert S.digest(corp.feature_offsets) == d["inputs"]["offsets"], "feature_offsets differ from the reference's"
    assert S.digest(corp.feature_values) == d["inputs"]["values"], "feature_values differ from the reference's"
    H.note(f"[full] {cfg}: corpus of {corp.feature_values.size} values equals the reference's inputs "
           f"({time.time() - t0:.0f}s)")
    dev = torch.device("cuda:0")
    ids = torch.from_numpy(corp.feature_ids).to(dev)
    offs = torch.from_numpy(corp.feature_offsets).to(dev)
    vals = torch.from_numpy(corp.feature_values).to(dev)
    del corp
    return cspec, ids, offs, vals


def _check_build(cfg: str, bi: torch.Tensor, bo: torch.Tensor, t0: float) -> None:
    d = _digests()[cfg]
    bo_h = bo.cpu().numpy()
    assert bo.numel() - 1 == d["bundles"] and int(bo_h[-1]) == d["bundle_b_offsets_last"]
    assert bo_h[:4].tolist() == d["bundle_b_offsets_head"]
    assert S.digest(bo_h) == d["bundle_b_offsets"], "bundle_b_offsets differ from the reference build"
    assert bi.numel() == d["index_len"]
    assert S.digest(bi.cpu().numpy()) == d["index"], "bloom_index differs from the reference build"
    H.note(f"[full] {cfg}: bundle_b_offsets and the {bi.numel() * 8 / 1e9:.2f} GB bloom_index equal the "
           f"reference's ({time.time() - t0:.0f}s)")


def _bool_equals_packed(boolm: torch.Tensor, packed: torch.Tensor) -> bool:
    """bool[Q, 64 C] == the packed words (doc 64 c + i at bit 63 - i of word
    c), on the device, 16 queries at a time."""
    Q, C = packed.shape
    w = torch.tensor([128, 64, 32, 16, 8, 4, 2, 1], dtype=torch.uint8, device=packed.device)
    for q0 in range(0, Q, 16):
        q1 = min(Q, q0 + 16)
        b = boolm[q0:q1].view(torch.uint8).view(q1 - q0, C, 8, 8)
        be = (b * w).sum(-1, dtype=torch.uint8)  # big-endian bytes of each word
        want = packed[q0:q1].contiguous().view(torch.uint8).view(q1 - q0, C, 8).flip(-1)
        if not torch.equal(be, want):
            return False
    return True


@pytest.mark.timeout(900)
@pytest.mark.parametrize("cfg", ["cfg2", "cfg5"])
def test_full_size_build_and_search_vs_reference(cfg):
    t0 = time.time()
    cspec, ids, offs, vals = _corpus_on_device(cfg, t0)
    _, qspec = S.CONFIGS[cfg]
    st = torch.ops.st
    d = _digests()[cfg]
    bi, bo = st.bloom_index_build(ids, offs, vals, cspec.b_multiplier, cspec.k)
    torch.cuda.synchronize()
    del ids, offs, vals
    _check_build(cfg, bi, bo, t0)

    queries = S.make_queries(cspec, qspec, seed=0)
    import hashlib

    assert hashlib.sha256("\n".join(queries).encode()).hexdigest() == d["queries_sha256"]
    _, (pd, po) = st.parse_expression_query_batch(queries, torch.ones(1, dtype=torch.long), cspec.hash_k, True, 5)
    assert S.digest(pd.numpy()) == d["plans_data"] and S.digest(po.numpy()) == d["plans_offsets"], \
        "plan bytes differ from the reference parser's"
    packed = st.bloom_index_search_batch(bi, bo, pd, po, cspec.k, cspec.hash_k, False)
    torch.cuda.synchronize()
    assert list(packed.shape) == d["packed_shape"]
    got = packed.cpu().numpy()
    counts = S.match_counts(got, cspec.num_docs)
    bad = [q for q, (a, b) in enumerate(zip(counts, d["match_counts"])) if a != b]
    assert not bad, f"match counts differ from the reference's for queries {bad[:10]}"
    assert S.digest(got) == d["packed"], "packed search output differs from the reference's"
    del got
    H.note(f"[full] {cfg}: packed output {list(packed.shape)} of {len(queries)} queries equals the reference's "
           f"({time.time() - t0:.0f}s)")

    boolm = st.bloom_index_search_batch(bi, bo, pd, po, cspec.k, cspec.hash_k, True)
    assert boolm.dtype == torch.bool and boolm.shape == (packed.shape[0], packed.shape[1] * 64)
    assert _bool_equals_packed(boolm, packed), "bool output differs from the packed words"
    del boolm
    ids_out, ro = st.bloom_index_search_batch_ids(bi, bo, pd, po, cspec.k, cspec.hash_k, cspec.num_docs)
    want_ro = np.concatenate([[0], np.cumsum(d["match_counts"])])
    np.testing.assert_array_equal(ro.cpu().numpy(), want_ro)
    assert ids_out.numel() == want_ro[-1]
    _check_ids_against_mask(ids_out, ro, packed, cspec.num_docs)
    ids_m, ro_m = st.bloom_mask_to_ids(packed, cspec.num_docs)
    assert torch.equal(ro_m, ro) and torch.equal(ids_m, ids_out), "mask -> ids differs from the fused ids op"
    H.note(f"[full] {cfg}: bool output, CSR row offsets and every id agree ({time.time() - t0:.0f}s)")


def _check_ids_against_mask(ids, ro, packed, num_docs):
    """Pins CSR ids exactly, given row offsets equal to the reference's match
    counts: within each row the ids ascend strictly, lie below num_docs and
    name set bits of the packed output (doc d of a row at bit 63 - d % 64 of
    word d // 64), so the row's ids are all of its set bits."""
    n = ids.numel()
    if n == 0:
        return
    counts = ro[1:] - ro[:-1]
    rows = torch.repeat_interleave(torch.arange(counts.numel(), device=ids.device), counts)
    d = ids.long()
    assert int(d.min()) >= 0 and int(d.max()) < num_docs, "an id outside [0, num_docs)"
    words = packed[rows, d // 64]
    del rows
    assert bool(((words >> (63 - d % 64)) & 1).bool().all()), "an id names a clear bit"
    del words
    starts = torch.zeros(n, dtype=torch.bool, device=ids.device)
    starts[ro[:-1][counts > 0]] = True
    assert bool(((d[1:] > d[:-1]) | starts[1:]).all()), "ids of a row not strictly ascending"


@pytest.mark.timeout(1500)
def test_full_size_cfg3_build_and_search_vs_reference():
    """cfg3 at full size: 50M docs x 16 features, k = 4, B_MULTIPLIER 10 (bundle
    widths 1,600-1,920 rows: every bundle is wider than the search kernel's
    LDS tile, so the column-slice wide-bundle phase evaluates it), 1,024
    boolean trees with NOT.  Inputs, bundle_b_offsets, the 10.7 GB
    bloom_index, plan bytes, the 6.4 GB packed output and every per-query
    match count against the reference CPU ops' digests
    (bloom_indexer.cpp:26-113, bloom_index_search.cpp:173-243); the search
    runs through the op (device width binding), and once more from a plan
    bound on the host through the C ABI, whose output must be the same."""
    t0 = time.time()
    cspec, ids, offs, vals = _corpus_on_device("cfg3", t0)
    _, qspec = S.CONFIGS["cfg3"]
    st = torch.ops.st
    d = _digests()["cfg3"]
    bi, bo = st.bloom_index_build(ids, offs, vals, cspec.b_multiplier, cspec.k)
    torch.cuda.synchronize()
    del ids, offs, vals
    _check_build("cfg3", bi, bo, t0)

    queries = S.make_queries(cspec, qspec, seed=0)
    import hashlib

    assert hashlib.sha256("\n".join(queries).encode()).hexdigest() == d["queries_sha256"]
    _, (pd, po) = st.parse_expression_query_batch(queries, torch.ones(1, dtype=torch.long), cspec.hash_k, True, 5)
    assert S.digest(pd.numpy()) == d["plans_data"] and S.digest(po.numpy()) == d["plans_offsets"], \
        "plan bytes differ from the reference parser's"
    packed = st.bloom_index_search_batch(bi, bo, pd, po, cspec.k, cspec.hash_k, False)
    torch.cuda.synchronize()
    assert list(packed.shape) == d["packed_shape"]
    got = packed.cpu().numpy()
    counts = S.match_counts(got, cspec.num_docs)
    bad = [q for q, (a, b) in enumerate(zip(counts, d["match_counts"])) if a != b]
    assert not bad, f"match counts differ from the reference's for queries {bad[:10]}"
    assert S.digest(got) == d["packed"], "packed search output differs from the reference's"
    del got
    H.note(f"[full] cfg3: packed output {list(packed.shape)} of {len(queries)} trees equals the reference's "
           f"({time.time() - t0:.0f}s)")

    from silvertorch_amd import capi

    plan = capi.SearchPlan(pd.numpy().tobytes(), po.numpy(), cspec.k, cspec.hash_k)
    plan.bind_widths(bo.cpu().numpy())
    blob = torch.frombuffer(bytearray(plan.blob()), dtype=torch.uint8).to(bi.device)
    host_bound = torch.empty_like(packed)
    nb = bo.numel() - 1
    capi.check(capi.lib().st_bloom_index_search_batch(
        bi.data_ptr(), bi.numel(), bo.data_ptr(), nb, plan.handle, blob.data_ptr(), 0, host_bound.data_ptr(),
        torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert torch.equal(host_bound, packed), "the host-bound plan's output differs from the op's"
    H.note(f"[full] cfg3: host-bound plan through the C ABI gives the same output ({time.time() - t0:.0f}s)")


@pytest.mark.timeout(900)
def test_full_size_cfg4_build_vs_reference():
    t0 = time.time()
    cspec, ids, offs, vals = _corpus_on_device("cfg4", t0)
    bi, bo = torch.ops.st.bloom_index_build(ids, offs, vals, cspec.b_multiplier, cspec.k)
    torch.cuda.synchronize()
    del ids, offs, vals
    _check_build("cfg4", bi, bo, t0)


@pytest.mark.timeout(900)
def test_full_size_cfg5_search_topk():
    """bloom_index_search_topk on all 20M docs of cfg5 (the corpus whose
    search output equals the reference's, test above), its 512 three-term
    filters, bf16[128] doc embeddings N(0, 1/128) and queries N(0, 1) drawn
    on the device (seeded torch), top-100.  For 16 queries spread over the
    batch the result is checked against an fp32 torch reference of the same
    bf16 values on the same filter (scores of every passing doc, -inf
    elsewhere, torch.topk): ids equal except swaps between scores within
    1e-3 relative, returned scores within 1e-3 of the fp64 score of the
    returned id, scores non-increasing and equal scores in ascending id
    order; for every query the ids pass its filter, are distinct, and the
    -1 padding appears exactly when fewer than 100 docs pass."""
    t0 = time.time()
    cspec, ids, offs, vals = _corpus_on_device("cfg5", t0)
    _, qspec = S.CONFIGS["cfg5"]
    st = torch.ops.st
    bi, bo = st.bloom_index_build(ids, offs, vals, cspec.b_multiplier, cspec.k)
    del ids, offs, vals
    queries = S.make_queries(cspec, qspec, seed=0)
    _, (pd, po) = st.parse_expression_query_batch(queries, torch.ones(1, dtype=torch.long), cspec.hash_k, True, 5)
    n, dim, topk = cspec.num_docs, 128, 100
    emb, qv = S.make_embeddings_device(n, dim, len(queries), seed=0)
    H.note(f"[full] cfg5 top-k: {n} docs x {len(queries)} queries, bf16[{dim}], top-{topk} "
           f"({time.time() - t0:.0f}s)")
    got_ids, got_sc = st.bloom_index_search_topk(bi, bo, pd, po, cspec.k, cspec.hash_k, emb, qv, n, topk)
    packed = st.bloom_index_search_batch(bi, bo, pd, po, cspec.k, cspec.hash_k, False)
    torch.cuda.synchronize()
    assert S.digest(packed.cpu().numpy()) == _digests()["cfg5"]["packed"], "the filter differs from the reference's"
    counts = torch.tensor(_digests()["cfg5"]["match_counts"])
    # every query: padding exactly past the passing docs, ids pass the filter, distinct
    have = (got_ids >= 0).sum(1).cpu()
    assert torch.equal(have, torch.clamp(counts, max=topk)), "padding does not match the passing doc counts"
    valid = got_ids >= 0
    d = torch.where(valid, got_ids, torch.zeros_like(got_ids))
    rows = torch.arange(len(queries), device=d.device)[:, None].expand_as(d)
    bits = (packed[rows, d // 64] >> (63 - d % 64)) & 1
    assert bool((bits.bool() | ~valid).all()), "a returned id fails its filter"
    srt = torch.sort(torch.where(valid, got_ids, torch.full_like(got_ids, -1)), dim=1).values
    assert bool(((srt[:, 1:] != srt[:, :-1]) | (srt[:, 1:] < 0)).all()), "duplicate ids"
    sc = got_sc.cpu().numpy()
    gi = got_ids.cpu().numpy()
    for q in range(len(queries)):
        m = int(have[q])
        assert np.all(np.diff(sc[q, :m]) <= 0), "scores not non-increasing"
        eq = np.diff(sc[q, :m]) == 0
        assert np.all(np.diff(gi[q, :m])[eq] > 0), "equal scores not in ascending id order"
    H.note(f"[full] cfg5 top-k: padding, filter, distinctness and order hold for all {len(queries)} queries "
           f"({time.time() - t0:.0f}s)")
    # fp32 reference for sampled queries
    sample = list(range(0, len(queries), len(queries) // 16))[:16]
    qf = qv[sample].float()
    ref = torch.empty((len(sample), n), dtype=torch.float32, device=qv.device)
    for r0 in range(0, n, 1 << 21):
        r1 = min(n, r0 + (1 << 21))
        ref[:, r0:r1] = (emb[r0:r1].float() @ qf.T).T
    docs = torch.arange(n, device=qv.device)
    for i, q in enumerate(sample):
        passing = ((packed[q, docs // 64] >> (63 - docs % 64)) & 1).bool()
        ref[i] = torch.where(passing, ref[i], torch.full_like(ref[i], -float("inf")))
    want_sc, want_ids = torch.topk(ref, topk, dim=1)
    want_sc, want_ids = want_sc.cpu().numpy(), want_ids.cpu().numpy()
    emb_rows = emb[got_ids[sample].clamp(min=0)].float().cpu().numpy().astype(np.float64)
    qf64 = qf.cpu().numpy().astype(np.float64)
    for i, q in enumerate(sample):
        m = int(have[q])
        exact = emb_rows[i, :m] @ qf64[i]
        np.testing.assert_allclose(sc[q, :m], exact, rtol=1e-3, atol=1e-6)
        for j in range(m):
            if gi[q, j] != want_ids[i, j]:
                assert abs(exact[j] - want_sc[i, j]) <= 1e-3 * max(abs(want_sc[i, j]), 1e-6), \
                    (q, j, gi[q, j], want_ids[i, j], exact[j], want_sc[i, j])
    H.note(f"[full] cfg5 top-k: {len(sample)} sampled queries agree with the fp32 reference "
           f"({time.time() - t0:.0f}s)")


@pytest.mark.timeout(600)
def test_cfg5_search_topk_prefix_vs_oracle():
    """bloom_index_search_topk on cfg5's corpus (its first 131,072 docs), its
    512 three-term AND/OR filters and bf16[128] embeddings (docs N(0, 1/128),
    queries N(0, 1), seeded numpy), top-100, against the oracle."""
    from tests.test_gpu_topk import _check

    cspec, qspec = S.CONFIGS["cfg5"]
    n, dim, topk = 131072, 128, 100
    corp = S.make_corpus(cspec, seed=0, num_docs=n)
    queries = S.make_queries(cspec, qspec, seed=0)
    emb, qv = S.make_embeddings(n, dim, len(queries), seed=0)
    H.note(f"[full] cfg5 top-k: {n} docs x {len(queries)} queries, bf16[{dim}], top-{topk}")
    st = torch.ops.st
    dev = torch.device("cuda:0")
    bi, bo = st.bloom_index_build(torch.from_numpy(corp.feature_ids).to(dev),
                                  torch.from_numpy(corp.feature_offsets).to(dev),
                                  torch.from_numpy(corp.feature_values).to(dev), cspec.b_multiplier, cspec.k)
    _, (pd, po) = st.parse_expression_query_batch(queries, torch.ones(1, dtype=torch.long), cspec.hash_k, True, 5)
    ids, sc = st.bloom_index_search_topk(bi, bo, pd, po, cspec.k, cspec.hash_k, emb.to(dev), qv.to(dev), n, topk)
    packed = st.bloom_index_search_batch(bi, bo, pd, po, cspec.k, cspec.hash_k, False).cpu().numpy()
    passing = sum(S.match_counts(packed, n))
    H.note(f"[full] cfg5 top-k: {passing} passing doc-query pairs; checking against the oracle")
    _check(ids.cpu().numpy(), sc.cpu().numpy(), emb.float().numpy(), qv.float().numpy(), packed, n, topk)
