"""GPU parity of the compaction of matching ids (CSR ids + row offsets)
against the C oracle's compaction, itself pinned to numpy's nonzero on the
unpacked mask (tests/test_oracle_golden.py).  Bit-exact integer output."""

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


def _random_mask(rng, q, c, density):
    if q == 0 or c == 0:
        return np.zeros((q, c), dtype=np.int64)
    bits = rng.random((q, c * 64)) < density
    return np.packbits(bits, axis=1).view(">i8").astype(np.int64)


@pytest.mark.parametrize("shape", [(0, 0), (3, 0), (0, 32), (1, 1), (4, 33), (7, 64), (13, 97), (64, 32 * 40)])
@pytest.mark.parametrize("int64_ids", [False, True])
def test_compact_random_masks(shape, int64_ids):
    rng = np.random.default_rng(sum(shape) + int64_ids)
    q, c = shape
    for density in (0.0, 0.02, 0.4, 1.0):
        packed = _random_mask(rng, q, c, density)
        for nd in sorted({0, 1, 31, 32, 33, max(c * 64 - 7, 0), c * 64, c * 64 + 9}):
            H.note(f"[compact] shape={shape} density={density} num_docs={nd} int64={int64_ids}")
            ids, ro = H.compact(packed, nd, int64_ids)
            want_ids, want_ro = O.compact(packed, nd)
            np.testing.assert_array_equal(ro, want_ro)
            np.testing.assert_array_equal(ids.astype(np.int64), want_ids)
            assert ids.dtype == (np.int64 if int64_ids else np.int32)


def test_compact_more_tiles_than_the_folded_prefix_takes():
    """1,100 queries x 1,920 chunks = 2.11 M chunk counts, more than the
    1,024 scan tiles of 2,048 whose prefix the apply pass sums itself, so the
    tile sums get their own scan pass.  The mask is built on the device from
    planted ids (a few per row, some past num_docs, one row empty, one row
    with a whole chunk set); the expected output is those ids in order."""
    q, nch = 1100, 1920
    c = 32 * nch
    nd = c * 64 - 1000
    rng = np.random.default_rng(11)
    rows, ids = [], []
    for r in range(q):
        if r == 5:
            chosen = np.arange(64 * 32 * 7, 64 * 32 * 8)  # chunk 7 full
        elif r == 6:
            chosen = np.zeros(0, np.int64)
        else:
            chosen = rng.choice(c * 64, size=int(rng.integers(1, 40)), replace=False)
            if r % 97 == 0:
                chosen = np.concatenate([chosen, np.arange(nd - 3, nd + 5)])
        chosen = np.unique(chosen.astype(np.int64))
        rows.append(np.full(chosen.size, r, np.int64))
        ids.append(chosen)
    rows, ids = np.concatenate(rows), np.concatenate(ids)
    flat = torch.zeros(q * c, dtype=torch.long, device="cuda")
    word = torch.as_tensor(rows * c + (ids >> 6)).cuda()
    # distinct bits of one word sum to their OR (bit 63 is -2^63 in int64)
    bit = torch.as_tensor(np.left_shift(np.uint64(1), (63 - (ids & 63)).astype(np.uint64)).view(np.int64)).cuda()
    flat.index_add_(0, word, bit)
    packed = flat.view(q, c)
    H.note(f"[compact] planted ids q={q} c={c} num_docs={nd}")
    got_ids, got_ro = H.compact(packed, nd)
    keep = ids < nd
    want_ids = ids[keep]
    want_ro = np.concatenate([[0], np.cumsum(np.bincount(rows[keep], minlength=q))])
    np.testing.assert_array_equal(got_ro, want_ro)
    np.testing.assert_array_equal(got_ids.astype(np.int64), want_ids)


def test_compact_cfg1_search_output():
    """The cfg1 search output (README-scale corpus, 32 queries) end to end."""
    from silvertorch_amd import synthetic as S
    cspec, qspec = S.CONFIGS["cfg1"]
    corp = S.make_corpus(cspec, seed=0)
    queries = S.make_queries(cspec, qspec, seed=0)
    index, bbo = H.build(corp.feature_ids, corp.feature_offsets, corp.feature_values, cspec.b_multiplier, cspec.k)
    _, data, offs = P.parse_batch(queries, cspec.hash_k)
    pd, po = np.frombuffer(data, np.int8).copy(), np.array(offs, np.int64)
    packed = H.search(index, bbo, pd, po, cspec.k, cspec.hash_k)
    H.note("[compact] cfg1")
    ids, ro = H.compact(packed, cspec.num_docs)
    want_ids, want_ro = O.compact(O.search_packed(index, bbo, pd, po, cspec.k, cspec.hash_k), cspec.num_docs)
    np.testing.assert_array_equal(ro, want_ro)
    np.testing.assert_array_equal(ids, want_ids)


@pytest.mark.parametrize("seed", range(3))
def test_fused_search_counts_vs_oracle(seed):
    """Search with per-(query, bundle) counts in the same pass, then ids:
    equal to the oracle's search followed by the oracle's compaction, for doc
    counts that end inside a bundle and inside a half-word."""
    rng = np.random.default_rng(100 + seed)
    n = int(rng.integers(3000, 9000))
    F = 3
    cnt = rng.integers(0, 4, (n, F))
    offs = np.concatenate([[0], np.cumsum(cnt.reshape(-1))]).astype(np.int64)
    vals = rng.integers(0, 40, int(offs[-1])).astype(np.int64)
    ids_f = np.array([1, 2, 3], dtype=np.int32)
    index, bbo = H.build(ids_f, offs, vals, 3.0, 3)
    terms = [f"{int(rng.integers(1, 4))}:{int(rng.integers(0, 40))}" for _ in range(40)]
    queries = [f"{terms[i]} OR {terms[i + 1]} AND NOT {terms[i + 2]}" for i in range(0, 36)] + ["", "NOT " + terms[0]]
    _, data, po = P.parse_batch(queries, 7)
    pd, po = np.frombuffer(data, np.int8).copy(), np.array(po, np.int64)
    want_packed = O.search_packed(index, bbo, pd, po, 3, 7)
    for nd in (n, n - 17, 0, (len(bbo) - 1) * 2048):
        H.note(f"[fused ids] seed={seed} num_docs={nd}")
        ids, ro, packed = H.search_ids(index, bbo, pd, po, 3, 7, nd)
        np.testing.assert_array_equal(packed, want_packed)
        want_ids, want_ro = O.compact(want_packed, nd)
        np.testing.assert_array_equal(ro, want_ro)
        np.testing.assert_array_equal(ids.astype(np.int64), want_ids)


def test_ops_ids_readme_known_answers():
    """README.md:255-268: ids of the five README queries over four docs,
    through the fused search-to-ids op and through mask -> ids."""
    st = torch.ops.st
    c = G.case("readme")
    bi, bo = st.bloom_index_build(torch.from_numpy(c["ids"]).cuda(), torch.from_numpy(c["offsets"]).cuda(),
                                  torch.from_numpy(c["values"]).cuda(), 5.0, 3)
    _, (pd, po) = st.parse_expression_query_batch(list(c["queries"]), torch.ones(1, dtype=torch.long), 7, True, 5)
    want = [[0, 1, 3], [1, 3], [2, 3], [0, 1, 3], [2]]
    H.note("[compact] readme via ops")
    ids, ro = st.bloom_index_search_batch_ids(bi, bo, pd, po, 3, 7, 4)
    ro = ro.cpu().tolist()
    assert ids.dtype == torch.int32 and ids.is_cuda
    assert [ids[ro[q]:ro[q + 1]].cpu().tolist() for q in range(5)] == want
    packed = st.bloom_index_search_batch(bi, bo, pd, po, 3, 7, False)
    ids64, ro64 = st.bloom_mask_to_ids(packed, 4, True)
    assert ids64.dtype == torch.long and ro64.cpu().tolist() == ro
    # CPU tensors: computed on the GPU, returned on the host
    ids_c, ro_c = st.bloom_mask_to_ids(packed.cpu(), 4)
    assert not ids_c.is_cuda and ro_c.tolist() == ro and ids_c.tolist() == ids.cpu().tolist()
    with pytest.raises(RuntimeError, match="num_docs must be non-negative"):
        st.bloom_mask_to_ids(packed, -1)
    with pytest.raises(RuntimeError, match="2-D int64"):
        st.bloom_mask_to_ids(packed.view(-1), 4)
