"""GPU parity of fused_kmean_ann (the clustered scoring step after the search)
and its partial-mask wrappers: the reference CPU op's fixtures bit for bit,
random shapes against the oracle, the search's packed mask as the filter, and
a direct C-ABI call.  Reference: fused_kmean_ann.cpp:85-311,
test_fused_kmean_ann.py."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import silvertorch_amd.ops._load_ops  # noqa: F401
from oracle import oracle as O
from oracle import parser_oracle as P
from silvertorch_amd import capi
from tests import _fixtures as G
from tests import gpu_helpers as H

pytestmark = pytest.mark.gpu
st = torch.ops.st

def _t(a: np.ndarray, bf16: bool = False, dev="cuda"):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if bf16:
        t = t.view(torch.int16).view(torch.bfloat16)
    return t.to(dev)

def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.cpu()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()

def _run(c, dev="cuda", **over):
    kw = dict(invalid_index_value=c["invalid"], divisor_for_int8=c["divisor"])
    if "mask_msb" in c:
        kw["filtering_bit_mask"] = _t(c["mask_msb"], dev=dev)
    if "filter_index" in c:
        kw["filtering_bit_index"] = _t(c["filter_index"], dev=dev)
    if "scale" in c:
        kw["per_embedding_scale"] = _t(c["scale"], dev=dev)
    kw.update(over)
    return st.fused_kmean_ann(_t(c["cluster_offsets"], dev=dev), _t(c["cluster_ids"], dev=dev),
                              _t(c["cluster_length"], dev=dev), _t(c["embeddings"], c["bf16"], dev),
                              _t(c["queries"], c["bf16"], dev), c["max_size"], **kw)

@pytest.mark.parametrize("name", G.KMEAN_CASES)
def test_matches_reference_fixtures(name):
    c = G.kmean_case(name)
    H.note(f"[kmean] fixture {name}")
    sc, ix = _run(c)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(ix.cpu().numpy(), c["indices"])
    got = _bits(sc)
    if c["bf16"]:
        valid = c["indices"] != c["invalid"]
        want = O.bf16_round(c["scores"])
        np.testing.assert_array_equal(got[valid], want[valid])
        assert (got[~valid] == 0xFF7F).all()
    else:
        assert sc.cpu().numpy().dtype == c["scores"].dtype
        np.testing.assert_array_equal(got.view(np.uint8), c["scores"].view(np.uint8))

def test_cpu_key_matches_cuda_key():
    c = G.kmean_case("i8_scale")
    a_s, a_i = _run(c)
    b_s, b_i = _run(c, dev="cpu")
    assert b_s.device.type == "cpu"
    assert torch.equal(a_s.cpu(), b_s) and torch.equal(a_i.cpu(), b_i)

def test_partial_mask_wrappers_match_reference():
    p = G.kmean_group("partial")
    dummy = torch.zeros(1, dtype=torch.long, device="cuda")
    sc, ix = st.fused_kmean_ann_with_partial_masks(
        _t(p["cluster_offsets"]), _t(p["cluster_ids"]), _t(p["cluster_length"]), _t(p["embeddings"]),
        _t(p["queries"]), 70, dummy, dummy.to(torch.int8), dummy)
    np.testing.assert_array_equal(ix.cpu().numpy(), p["indices"])
    np.testing.assert_array_equal(sc.cpu().numpy(), p["scores"])
    m = G.kmean_group("multiple")
    ms = st.fused_kmean_ann_with_partial_masks_multiple(
        _t(m["queries"]), [_t(m[f"{c}/cluster_offsets"]) for c in range(2)],
        [_t(m[f"{c}/cluster_ids"]) for c in range(2)], [_t(m[f"{c}/cluster_length"]) for c in range(2)],
        [_t(m[f"{c}/embeddings"]) for c in range(2)], [33, 50], [dummy] * 2, [dummy.to(torch.int8)] * 2,
        [dummy] * 2, fuse=True)
    for c in range(2):
        np.testing.assert_array_equal(ms[1][c].cpu().numpy(), m[f"{c}/indices"])
        np.testing.assert_array_equal(ms[0][c].cpu().numpy(), m[f"{c}/scores"])

def _random_case(rng, dim, dtype, batch, probes, max_size, filtered=False, cluster_max=700):
    nclus = int(rng.integers(3, 12))
    sizes = rng.integers(0, cluster_max, nclus)
    offs = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    n = int(offs[-1])
    if dtype == "int8":
        emb = rng.integers(-128, 128, (n, dim)).astype(np.int8)
        q = rng.integers(-128, 128, (batch, dim)).astype(np.int8)
    else:
        emb = rng.standard_normal((n, dim)).astype(np.float32)
        q = rng.standard_normal((batch, dim)).astype(np.float32)
        if dtype == "float16":
            emb, q = emb.astype(np.float16), q.astype(np.float16)
        if dtype == "bfloat16":
            emb, q = O.bf16_round(emb), O.bf16_round(q)
    cids = rng.integers(0, nclus, (batch, probes)).astype(np.int64)
    mask = rng.integers(-2**63, 2**63 - 1, (batch, max(1, n // 64)), dtype=np.int64) if filtered else None
    return dict(cluster_offsets=offs, cluster_ids=cids, cluster_length=sizes[cids].astype(np.int64),
                embeddings=emb, queries=q, max_size=max_size, mask=mask, bf16=dtype == "bfloat16")

# dims 40 (bf16) and 20 (f32): 80-byte rows, a partial last 64-byte staging
# slice; maxlen 12000: clusters longer than one 4,096-doc pass-bit chunk;
# seed 2571: a float64 sum that float32 rounds onto a float16 half-way point
@pytest.mark.parametrize("dim,dtype,filtered,divisor,maxlen,seed", [
    (128, "float32", False, -1, 2500, None), (1280, "float32", True, -1, 2500, None),
    (17, "float32", True, -1, 2500, None), (64, "float16", True, -1, 2500, None),
    (256, "bfloat16", False, -1, 2500, None), (96, "bfloat16", True, -1, 2500, None),
    (32, "int8", False, -1, 2500, None), (128, "int8", True, 13, 2500, None),
    (64, "float16", True, -1, 2500, 2571), (40, "bfloat16", True, -1, 2500, None),
    (20, "float32", False, -1, 2500, None), (64, "bfloat16", True, -1, 12000, None),
    (48, "float32", False, -1, 12000, None)])
def test_random_vs_oracle(dim, dtype, filtered, divisor, maxlen, seed):
    rng = np.random.default_rng(dim + len(dtype) if seed is None else seed)
    long_clusters = maxlen > 2500
    c = _random_case(rng, dim, dtype, int(rng.integers(1, 4 if long_clusters else 24)), int(rng.integers(1, 6)),
                     int(rng.integers(maxlen // 2 if long_clusters else 1, maxlen)), filtered,
                     cluster_max=9000 if long_clusters else 700)
    H.note(f"[kmean] random dim={dim} {dtype} filtered={filtered} docs={c['cluster_offsets'][-1]}")
    kw = dict(divisor_for_int8=divisor)
    if filtered:
        kw["filtering_bit_mask"] = _t(c["mask"])
    sc, ix = st.fused_kmean_ann(_t(c["cluster_offsets"]), _t(c["cluster_ids"]), _t(c["cluster_length"]),
                                _t(c["embeddings"], c["bf16"]), _t(c["queries"], c["bf16"]),
                                c["max_size"], **kw)
    want_s, want_i = O.fused_kmean_ann(c["cluster_offsets"], c["cluster_ids"], c["cluster_length"],
                                       c["embeddings"], c["queries"], c["max_size"], filter_mask=c["mask"],
                                       divisor=divisor, bf16=c["bf16"])
    np.testing.assert_array_equal(ix.cpu().numpy(), want_i)
    np.testing.assert_array_equal(_bits(sc).view(np.uint8), want_s.view(np.uint8))

# Calls of 2,048 (row, probe) pairs or more take the balanced form (ids
# listed per pair, then scoring spread over the chip by groups of 64 slots:
# kmean_list_kernel, kmean_score_kernel); smaller ones a workgroup per pair
# (kmean_ann_kernel).  Rows are independent, so a large call must equal the
# same rows called in slices of fewer pairs; three rows are also checked
# against the oracle.  dim 1280 float32 exceeds the balanced form's LDS and
# takes the workgroup form at both sizes.
@pytest.mark.parametrize("dim,dtype,filtered,findex,divisor,width", [
    (128, "bfloat16", True, False, -1, 6000), (17, "float32", True, True, -1, 3000),
    (64, "float16", False, False, -1, 900), (32, "int8", True, False, -1, 5000),
    (96, "int8", False, False, 7, 5000), (40, "bfloat16", True, True, -1, 200),
    (1024, "float32", True, False, -1, 4000), (1280, "float32", False, False, -1, 2000)])
def test_balanced_form_matches_slices_and_oracle(dim, dtype, filtered, findex, divisor, width):
    rng = np.random.default_rng(dim * 7 + len(dtype) + width)
    B, P_ = 512, 8
    nclus = 24
    sizes = rng.integers(0, 1500 if dim >= 1024 else 3000, nclus)
    sizes[3] = 0
    offs = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    n = int(offs[-1])
    if dtype == "int8":
        emb = rng.integers(-128, 128, (n, dim)).astype(np.int8)
        q = rng.integers(-128, 128, (B, dim)).astype(np.int8)
    else:
        emb = rng.standard_normal((n, dim)).astype(np.float32)
        q = rng.standard_normal((B, dim)).astype(np.float32)
        if dtype == "float16":
            emb, q = emb.astype(np.float16), q.astype(np.float16)
        if dtype == "bfloat16":
            emb, q = O.bf16_round(emb), O.bf16_round(q)
    bf16 = dtype == "bfloat16"
    cids = rng.integers(-1, nclus + 1, (B, P_)).astype(np.int64)  # ids outside the offsets select nothing
    clen = np.where((cids >= 0) & (cids < nclus), sizes[np.clip(cids, 0, nclus - 1)], 5).astype(np.int64)
    clen[rng.random((B, P_)) < 0.1] //= 3  # a prefix of the cluster
    mask = fidx = None
    if filtered:
        mrows = 37 if findex else B
        mask = rng.integers(-2**63, 2**63 - 1, (mrows, n // 64 + 1), dtype=np.int64)
        mask &= rng.integers(-2**63, 2**63 - 1, mask.shape, dtype=np.int64)  # density 1/4
        if findex:
            fidx = rng.integers(-2, mrows + 2, B).astype(np.int64)  # some rows name no mask row
    e_t, q_t = _t(emb, bf16), _t(q, bf16)
    o_t = _t(offs)

    def call(r0, r1):
        kw = dict(divisor_for_int8=divisor, invalid_index_value=-3)
        if filtered:
            kw["filtering_bit_mask"] = _t(mask if findex else mask[r0:r1])
            if findex:
                kw["filtering_bit_index"] = _t(fidx[r0:r1])
        return st.fused_kmean_ann(o_t, _t(cids[r0:r1]), _t(clen[r0:r1]), e_t, q_t[r0:r1], width, **kw)

    H.note(f"[kmean balanced] dim={dim} {dtype} filtered={filtered} index={findex} width={width} docs={n}")
    sc, ix = call(0, B)
    for r0 in range(0, B, 128):  # 1,024 pairs per call: workgroup kernel
        s2, i2 = call(r0, r0 + 128)
        assert torch.equal(ix[r0:r0 + 128], i2), f"indices of rows {r0}.. differ between the kernels"
        assert np.array_equal(_bits(sc[r0:r0 + 128]), _bits(s2)), f"scores of rows {r0}.. differ"
    for b in (0, 201, B - 1):
        m = None
        if filtered:
            m = mask[fidx[b]:fidx[b] + 1] if findex and 0 <= fidx[b] < mask.shape[0] else (
                np.zeros((1, mask.shape[1]), np.int64) if findex else mask[b:b + 1])
        ws, wi = O.fused_kmean_ann(offs, np.clip(cids[b:b + 1], 0, nclus - 1), np.where(
            (cids[b:b + 1] >= 0) & (cids[b:b + 1] < nclus), clen[b:b + 1], 0), emb, q[b:b + 1], width,
            filter_mask=m, invalid_index=-3, divisor=divisor, bf16=bf16)
        np.testing.assert_array_equal(ix[b:b + 1].cpu().numpy(), wi)
        np.testing.assert_array_equal(_bits(sc[b:b + 1]).view(np.uint8), ws.view(np.uint8))


def test_search_mask_as_filter():
    """The packed output of bloom_index_search_batch filters the scoring, doc d
    at bit 63 - d % 64, as the reference CUDA op reads it."""
    rng = np.random.default_rng(9)
    n, F = 9000, 2
    cnt = rng.integers(1, 3, (n, F))
    offs = np.concatenate([[0], np.cumsum(cnt.reshape(-1))]).astype(np.int64)
    vals = rng.integers(0, 40, int(offs[-1])).astype(np.int64)
    ids = np.array([1, 2], np.int32)
    bi, bo = st.bloom_index_build(_t(ids), _t(offs), _t(vals), 3.0, 3)
    queries = ["1:3 OR 2:5", "1:7", "NOT 2:1", "1:2 AND 2:2"]
    _, data, po = P.parse_batch(queries, 7, True, 5)
    pd = torch.from_numpy(np.frombuffer(data, dtype=np.int8).copy())
    packed = st.bloom_index_search_batch(bi, bo, pd.cuda(), torch.tensor(po).cuda(), 3, 7, False)
    coffs = np.concatenate([[0], np.sort(rng.choice(n, 13, replace=False)), [n]]).astype(np.int64)
    sizes = np.diff(coffs)  # 14 clusters covering the docs
    emb = rng.standard_normal((n, 48)).astype(np.float32)
    qv = rng.standard_normal((4, 48)).astype(np.float32)
    cids = rng.integers(0, len(sizes), (4, 5)).astype(np.int64)
    sc, ix = st.fused_kmean_ann(_t(coffs), _t(cids), _t(sizes[cids].astype(np.int64)), _t(emb), _t(qv),
                                4000, filtering_bit_mask=packed)
    want_s, want_i = O.fused_kmean_ann(coffs, cids, sizes[cids], emb, qv, 4000,
                                       filter_mask=packed.cpu().numpy())
    np.testing.assert_array_equal(ix.cpu().numpy(), want_i)
    np.testing.assert_array_equal(sc.cpu().numpy(), want_s)
    # every returned doc passes its query's search
    m = O.unpack_bool(packed.cpu().numpy())
    for b in range(4):
        got = ix[b].cpu().numpy()
        got = got[got >= 0]
        assert m[b, got].all()

def test_edge_cases():
    rng = np.random.default_rng(4)
    emb = _t(rng.standard_normal((50, 16)).astype(np.float32))
    q = _t(rng.standard_normal((2, 16)).astype(np.float32))
    offs = _t(np.array([0, 20, 50], np.int64))
    # no probes: all padding
    sc, ix = st.fused_kmean_ann(offs, _t(np.zeros((2, 0), np.int64)), _t(np.zeros((2, 0), np.int64)),
                                emb, q, 5, invalid_index_value=-7)
    assert sc.shape == (2, 32) and (ix.cpu() == -7).all()
    assert (sc.cpu() == -torch.finfo(torch.float32).max).all()
    # a cluster id outside the offsets selects nothing; width 0 gives empty rows
    sc, ix = st.fused_kmean_ann(offs, _t(np.array([[5, 1], [-1, 0]], np.int64)),
                                _t(np.array([[3, 4], [2, 3]], np.int64)), emb, q, 40)
    np.testing.assert_array_equal(ix.cpu().numpy()[0, :5], [20, 21, 22, 23, -1])
    np.testing.assert_array_equal(ix.cpu().numpy()[1, :4], [0, 1, 2, -1])
    sc, ix = st.fused_kmean_ann(offs, _t(np.array([[1]], np.int64))[:, :1].expand(2, 1).contiguous(),
                                _t(np.array([[3], [3]], np.int64)), emb, q, 0)
    assert sc.shape == (2, 0) and ix.shape == (2, 0)
    # a filtering_bit_index row outside the mask passes no doc; a valid one
    # filters as that row of the mask does
    mask = _t(np.array([[-1, -1]], np.int64))
    sc, ix = st.fused_kmean_ann(offs, _t(np.array([[1], [1]], np.int64)), _t(np.array([[30], [30]], np.int64)),
                                emb, q, 40, filtering_bit_mask=mask,
                                filtering_bit_index=_t(np.array([3, 0], np.int64)))
    assert (ix.cpu()[0] == -1).all()
    np.testing.assert_array_equal(ix.cpu().numpy()[1, :31], list(range(20, 50)) + [-1])
    sc, ix = st.fused_kmean_ann(offs, _t(np.array([[1], [1]], np.int64)), _t(np.array([[30], [30]], np.int64)),
                                emb, q, 40, filtering_bit_mask=mask,
                                filtering_bit_index=_t(np.array([-1, 0], np.int64)))
    assert (ix.cpu()[0] == -1).all() and ix.cpu()[1, 0] == 20
    with pytest.raises(RuntimeError):  # two queries, one mask row, no index
        st.fused_kmean_ann(offs, _t(np.array([[1], [1]], np.int64)), _t(np.array([[3], [3]], np.int64)),
                           emb, q, 40, filtering_bit_mask=mask)
    with pytest.raises(RuntimeError):
        st.fused_kmean_ann(offs, _t(np.zeros((2, 1), np.int64)), _t(np.zeros((3, 1), np.int64)), emb, q, 5)
    with pytest.raises(RuntimeError):
        st.fused_kmean_ann(offs, _t(np.zeros((2, 1), np.int64)), _t(np.zeros((2, 1), np.int64)),
                           emb.double(), q.double(), 5)

def test_c_abi_direct():
    """st_fused_kmean_ann through ctypes on device buffers equals the op."""
    c = G.kmean_case("i8_div")
    L = capi.lib()
    offs, cids, clen = _t(c["cluster_offsets"]), _t(c["cluster_ids"]), _t(c["cluster_length"])
    emb, q = _t(c["embeddings"]), _t(c["queries"])
    B, P_ = cids.shape
    width = (c["max_size"] + 31) // 32 * 32
    assert L.st_kmean_ann_score_dtype(3, c["divisor"], 0) == 1
    sc = torch.empty((B, width), dtype=torch.float16, device="cuda")
    ix = torch.empty((B, width), dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    ws = torch.empty(L.st_fused_kmean_ann_workspace_bytes(B, P_), dtype=torch.uint8, device="cuda")
    capi.check(L.st_fused_kmean_ann(offs.data_ptr(), offs.numel(), cids.data_ptr(), clen.data_ptr(), B, P_,
                                    emb.data_ptr(), emb.shape[0], emb.shape[1], 3, q.data_ptr(), width,
                                    None, 0, 0, None, None, c["divisor"], c["invalid"], ws.data_ptr(),
                                    sc.data_ptr(), ix.data_ptr(), stream))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(ix.cpu().numpy(), c["indices"])
    np.testing.assert_array_equal(_bits(sc), c["scores"].view(np.uint16))
    # a dim outside [1, 1280] is rejected before any launch
    rc = L.st_fused_kmean_ann(offs.data_ptr(), offs.numel(), cids.data_ptr(), clen.data_ptr(), B, P_,
                              emb.data_ptr(), emb.shape[0], 2048, 3, q.data_ptr(), width, None, 0, 0, None,
                              None, c["divisor"], c["invalid"], ws.data_ptr(), sc.data_ptr(), ix.data_ptr(),
                              stream)
    assert rc != 0 and b"dim" in L.st_last_error()
