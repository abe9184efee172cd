"""Writes the golden fixtures under tests/golden/ (run in the build container).

Sources of truth, neither of which is this repository's code:
  * MurmurHash3_x64_128 vectors from scikit-learn's independent public-domain
    source (sklearn/utils/src/MurmurHash3.cpp), compiled into a temporary
    directory: murmur_x64_128.json.  Keys are LE(x)||LE(y), 16 bytes; the
    fixture stores h1 ^ h2 of the 128-bit output.
  * The reference's own CPU ops (bloom_index_build, bloom_index_search_batch,
    parse_expression_query_batch), compiled from its sources by
    ``make -C oracle ref`` into oracle/_ref/libst_ref.so:
      ref_parser.json   plan bytes / offsets / max stack per expression batch,
                        and which expressions raise;
      ref_cases.npz     small build + search cases stored in full;
      ref_digests.json  sha256 digests of larger cases (cfg1 and a case with
                        bundles wider than 32767 rows) plus generator params;
      ref_partial.npz   cluster-restricted search outputs (partial response,
                        single and multiple-chunk ops) on small cases.

      ref_kmean.npz     fused_kmean_ann(_with_partial_masks(_multiple)) of the
                        reference's CPU op (fused_kmean_ann.cpp) on small
                        cases: every embedding dtype, int8 divisor and
                        per-embedding scale, truncated rows, filtered rows.
      ref_fresh.npz     take_top_k_and_gather_from_main_and_fresh of the
                        reference's CPU op (fresh_index_post_processing.cpp)
                        on cases with distinct scores per row (at::topk
                        leaves the order of equal scores open).

Usage:  python tests/golden/make_golden.py [partial|kmean|fresh]   (only that file)
        python tests/golden/make_golden.py full [cfg2 cfg5 cfg4 ...]
                (ref_full_digests.json: full-size configurations, minutes)
The reference library registers torch.ops.st.*, so this script never imports
silvertorch_amd.
"""

from __future__ import annotations

import ctypes
import hashlib
import json
import subprocess
import sys
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))



def _sklearn_murmur_source() -> Path:
    import sklearn

    return Path(sklearn.__file__).parent / "utils" / "src" / "MurmurHash3.cpp"


def murmur_vectors() -> dict:
    src = _sklearn_murmur_source()
    with tempfile.TemporaryDirectory() as td:
        so = Path(td) / "libmm.so"
        subprocess.run(["g++", "-O2", "-shared", "-fPIC", str(src), "-I", str(src.parent), "-o", str(so)], check=True)
        L = ctypes.CDLL(str(so))
        fn = L.MurmurHash3_x64_128  # (const void* key, int len, uint32_t seed, void* out)
        fn.restype = None
        rng = np.random.default_rng(2024)
        rows = []
        specials = [(0, 0, 0), (1, 100, 0), (2, 200, 6), ((1 << 64) - 1, (1 << 63), 3),
                    (1, (1 << 64) - 200, 1), (42, 100, 4294967295)]
        for _ in range(200):
            x, y = (int(v) for v in rng.integers(0, 1 << 63, 2, dtype=np.int64))
            if rng.random() < 0.5:
                x = int(rng.integers(-5, 20)) & ((1 << 64) - 1)
            seed = int(rng.integers(0, 64))
            specials.append((x, y, seed))
        for x, y, seed in specials:
            key = (ctypes.c_uint64 * 2)(x, y)
            out = (ctypes.c_uint64 * 2)()
            fn(key, 16, ctypes.c_uint32(seed), out)
            rows.append([str(x), str(y), str(seed), str(out[0] ^ out[1])])
    return {"source": "sklearn/utils/src/MurmurHash3.cpp MurmurHash3_x64_128, h1^h2", "vectors": rows}


def main() -> None:
    import torch

    ref = ROOT / "oracle" / "_ref" / "libst_ref.so"
    if not ref.exists():
        subprocess.run(["make", "-C", str(ROOT / "oracle"), "ref"], check=True)
    torch.ops.load_library(str(ref))
    st = torch.ops.st
    from silvertorch_amd import synthetic as S

    (HERE / "murmur_x64_128.json").write_text(json.dumps(murmur_vectors(), indent=0))

    # ---------------- parser
    exprs = ["1:100", "1:100 AND NOT 2:201", "1:102 OR 2:203", "", "-1:-200", "NOT NOT 1:10",
             "(1:100 & 2:200) | !(3:300 & 4:400:0.8)", "1:10 | 2:20 | 3:30 | 4:40 | 5:50",
             "(1:10 | 2:20 | 3:30 | 4:40) & 5:50", "1:10 OR 2:20 AND NOT 3:30", "42:100:0.5",
             "1:1:2", "((((1:1))))", "1:1 & 2:2 & 3:3 & 4:4 & 5:5 & 6:6 & 7:7 | 8:8", "  7:7  ",
             "NOT (1:1 OR 2:2 OR 3:3) AND NOT 4:4", "9223372036854775807:-9223372036854775808"]
    batches = []
    for hk in (1, 3, 7):
        for ms in (1, 2, 3, 5, 0):
            m, (pd, po) = st.parse_expression_query_batch(exprs, torch.ones(1, dtype=torch.long), hk, True, ms)
            batches.append({"hash_k": hk, "max_sub_queries": ms, "max_stack": int(m),
                            "data_hex": pd.numpy().tobytes().hex(), "offsets": po.tolist()})
    m, (pd, po) = st.parse_expression_query_batch(exprs, torch.ones(1, dtype=torch.long), 7, False, 5)
    no_plan = {"max_stack": int(m), "data_len": int(pd.numel()), "offsets_len": int(po.numel())}
    errors = {}
    for e in ["42", "(1:10 AND 2:20", "1:10 XOR 2:20", "1:10 AND", "1:10 2:20", "1:10 $", "1.5:3", "1:", "1:2:",
              "()", "AND 1:1", "1:1 OR", "NOT", "1:1)", "1:-", "--1:1"]:
        try:
            st.parse_expression_query_batch([e], torch.ones(1, dtype=torch.long), 7, True, 5)
            errors[e] = None
        except RuntimeError as ex:
            errors[e] = str(ex).splitlines()[0]
    (HERE / "ref_parser.json").write_text(json.dumps(
        {"expressions": exprs, "batches": batches, "no_plan": no_plan, "errors": errors}, indent=0))

    # ---------------- small build + search cases (stored in full)
    cases = {}
    readme_ids = np.array([1, 2], dtype=np.int32)
    readme_vals = np.array([100, 200, 201, 100, 101, 200, 102, 202, 100, 200, 203], dtype=np.int64)
    readme_offs = np.array([0, 1, 3, 5, 6, 7, 8, 9, 11], dtype=np.int64)
    rng = np.random.default_rng(7)

    def add_case(name, ids, offs, vals, bm, kb, queries, ks, hk, ms=5, parse_hk=None):
        parse_hk = hk if parse_hk is None else parse_hk
        bi, bo = st.bloom_index_build(torch.from_numpy(ids), torch.from_numpy(offs), torch.from_numpy(vals), bm, kb)
        _, (pd, po) = st.parse_expression_query_batch(queries, torch.ones(1, dtype=torch.long), parse_hk, True, ms)
        packed = st.bloom_index_search_batch(bi, bo, pd, po, ks, hk, False)
        boolm = st.bloom_index_search_batch(bi, bo, pd, po, ks, hk, True)
        assert np.array_equal(np.packbits(boolm.numpy(), axis=1).view(">u8").astype(np.int64).reshape(packed.shape),
                              packed.numpy())
        cases[f"{name}/ids"] = ids
        cases[f"{name}/offsets"] = offs
        cases[f"{name}/values"] = vals
        cases[f"{name}/params"] = np.array([bm, kb, ks, hk, ms, parse_hk], dtype=np.float64)
        cases[f"{name}/queries"] = np.array(queries, dtype=object).astype(str)
        cases[f"{name}/plans_data"] = pd.numpy()
        cases[f"{name}/plans_offsets"] = po.numpy()
        cases[f"{name}/index"] = bi.numpy()
        cases[f"{name}/bundle_b_offsets"] = bo.numpy()
        cases[f"{name}/packed"] = packed.numpy()

    readme_q = ["1:100", "1:100 AND NOT 2:201", "1:102 OR 2:203", "1:100 AND 2:200", "1:102"]
    add_case("readme", readme_ids, readme_offs, readme_vals, 5.0, 3, readme_q, 3, 7)

    def make_features(n, F):  # test_bloom_index_search.py:41-53 fixture shape
        ids = np.arange(F, dtype=np.int32)
        vals = np.array([d * 100 + f for d in range(n) for f in range(F)], dtype=np.int64)
        offs = np.arange(n * F + 1, dtype=np.int64)
        return ids, offs, vals

    ids, offs, vals = make_features(10, 3)
    add_case("features10x3", ids, offs, vals, 2.0, 7, ["0:0", "1:1", "0:0 AND 1:1", "0:0 OR 1:1", "NOT 0:0", ""], 3, 7)
    n = 32 * 64 * 2 + 10  # test_bloom_indexer.py:123-145 multi-bundle shape
    add_case("multibundle", np.array([0], dtype=np.int32), np.arange(n + 1, dtype=np.int64),
             np.arange(n, dtype=np.int64), 2.0, 3, ["0:5", "0:4100 OR 0:4101", "NOT 0:7", "0:1 AND 0:2"], 3, 3)

    for i, (kb, ks, hk, bm) in enumerate([(3, 3, 7, 5.0), (7, 3, 7, 2.0), (1, 1, 1, 1.5), (10, 10, 10, 3.0),
                                          (4, 4, 2, 2.0), (3, 0, 7, 5.0), (3, 3, 0, 5.0), (5, 8, 8, 4.0)]):
        ndoc = int(rng.integers(1, 7000))
        F = int(rng.integers(1, 5))
        cnt = rng.integers(0, 5, (ndoc, F))
        offs = np.concatenate([[0], np.cumsum(cnt.reshape(-1))]).astype(np.int64)
        vals = rng.integers(-3, 40, int(offs[-1])).astype(np.int64)
        ids = (np.arange(F, dtype=np.int32) * 7 - 3).astype(np.int32)
        qs = []
        for _ in range(12):
            t = int(rng.integers(1, 7))
            parts = []
            for j in range(t):
                term = f"{int(ids[rng.integers(0, F)])}:{int(rng.integers(-3, 40))}"
                if rng.random() < 0.25:
                    term = "NOT " + term
                if rng.random() < 0.15:
                    term = f"({term} OR {int(ids[rng.integers(0, F)])}:{int(rng.integers(-3, 40))})"
                parts.append(term)
                if j < t - 1:
                    parts.append(str(rng.choice(["AND", "OR"])))
            qs.append(" ".join(parts))
        qs.append("")
        # hash_k 0 at search time: plans parsed with hash_k 7 (the reference
        # parser divides by hash_k), searched with hash_k 0.
        add_case(f"random{i}", ids, offs, vals, bm, kb, qs, ks, hk, int(rng.integers(1, 6)),
                 parse_hk=hk if hk > 0 else 7)
    np.savez_compressed(HERE / "ref_cases.npz", **cases)

    # ---------------- digests of larger cases
    digests = {}

    def h(a: np.ndarray) -> str:
        return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()

    cspec, qspec = S.CONFIGS["cfg1"]
    corp = S.make_corpus(cspec, seed=0)
    queries = S.make_queries(cspec, qspec, seed=0)
    bi, bo = st.bloom_index_build(torch.from_numpy(corp.feature_ids), torch.from_numpy(corp.feature_offsets),
                                  torch.from_numpy(corp.feature_values), cspec.b_multiplier, cspec.k)
    _, (pd, po) = st.parse_expression_query_batch(queries, torch.ones(1, dtype=torch.long), cspec.hash_k, True, 5)
    packed = st.bloom_index_search_batch(bi, bo, pd, po, cspec.k, cspec.hash_k, False).numpy()
    digests["cfg1"] = {
        "inputs": {"offsets": h(corp.feature_offsets), "values": h(corp.feature_values)},
        "queries_sha256": hashlib.sha256("\n".join(queries).encode()).hexdigest(),
        "plans_data": h(pd.numpy()), "plans_offsets": h(po.numpy()),
        "index": h(bi.numpy()), "bundle_b_offsets": h(bo.numpy()), "packed": h(packed),
        "index_len": int(bi.numel()), "bundle_b_offsets_head": bo.numpy()[:4].tolist(),
        "packed_row0_head": packed[0, :8].tolist(),
        "match_counts": [int(np.unpackbits(packed[q].astype(">i8").view(np.uint8))[:cspec.num_docs].sum())
                         for q in range(packed.shape[0])],
    }

    # Two bundles: bundle 0 exactly 32768 rows wide, bundle 1 wider than
    # 32767 rows, so the reference's int16 position cast wraps into bundle 0.
    wide = {"k": 4, "b_multiplier": 2.0, "doc0_terms": 4096, "doc2048_terms": 5000}
    n = 2048 + 16
    cnt = np.ones(n, dtype=np.int64)
    cnt[0] = wide["doc0_terms"]
    cnt[2048] = wide["doc2048_terms"]
    offs = np.concatenate([[0], np.cumsum(cnt)]).astype(np.int64)
    vals = (np.arange(int(offs[-1]), dtype=np.int64) * 7919) % 100003
    ids = np.array([5], dtype=np.int32)
    bi, bo = st.bloom_index_build(torch.from_numpy(ids), torch.from_numpy(offs), torch.from_numpy(vals),
                                  wide["b_multiplier"], wide["k"])
    qs = [f"5:{int(v)}" for v in vals[[0, 5, 4095, 4097, 6000, 9000, 9100]]] + \
         ["5:1 OR 5:2", "NOT 5:3", f"5:{int(vals[4200])} AND NOT 5:{int(vals[10])}"]
    _, (pd, po) = st.parse_expression_query_batch(qs, torch.ones(1, dtype=torch.long), 7, True, 5)
    packed = st.bloom_index_search_batch(bi, bo, pd, po, 4, 7, False).numpy()
    wide.update({"queries": qs, "bundle_b_offsets": bo.tolist(), "index": h(bi.numpy()), "packed": h(packed),
                 "value_rule": "values[i] = (i * 7919) % 100003; doc 0 and doc 2048 carry the wide counts"})
    digests["wide_bundles"] = wide
    (HERE / "ref_digests.json").write_text(json.dumps(digests, indent=1))
    print("golden fixtures written to", HERE)


def partial_fixtures() -> None:
    """ref_partial.npz: bloom_index_search_batch_return_partial_response(_multiple)
    of the reference's CPU op (bloom_index_search.cpp:246-487) on small cases:
    the reference test's shape (test_bloom_index_search.py:301-423), clusters
    at unaligned doc offsets crossing bundle boundaries with empty clusters and
    a query_plan_index, and a three-chunk _multiple call."""
    import torch

    ref = ROOT / "oracle" / "_ref" / "libst_ref.so"
    if not ref.exists():
        subprocess.run(["make", "-C", str(ROOT / "oracle"), "ref"], check=True)
    torch.ops.load_library(str(ref))
    st = torch.ops.st
    out = {}
    rng = np.random.default_rng(11)

    def corpus(n, F, vocab):
        cnt = rng.integers(0, 4, (n, F))
        offs = np.concatenate([[0], np.cumsum(cnt.reshape(-1))]).astype(np.int64)
        vals = rng.integers(0, vocab, int(offs[-1])).astype(np.int64)
        return np.arange(1, F + 1, dtype=np.int32), offs, vals

    def add(name, ids, offs, vals, queries, co, cl, pi, k=3, hash_k=7, bm=3.0):
        bi, bo = st.bloom_index_build(torch.from_numpy(ids), torch.from_numpy(offs), torch.from_numpy(vals), bm, k)
        _, (pd, po) = st.parse_expression_query_batch(queries, torch.ones(1, dtype=torch.long), hash_k, True, 5)
        res = st.bloom_index_search_batch_return_partial_response(
            bi, bo, pd, po, torch.from_numpy(co), torch.from_numpy(cl), k, hash_k,
            None if pi is None else torch.from_numpy(pi))
        for key, v in (("index", bi.numpy()), ("bundle_b_offsets", bo.numpy()), ("plans_data", pd.numpy()),
                       ("plans_offsets", po.numpy()), ("cluster_offsets", co), ("cluster_lengths", cl),
                       ("params", np.array([k, hash_k], dtype=np.int64)),
                       ("cumsum", res[0].numpy()), ("first", res[1].numpy()), ("mask", res[2].numpy())):
            out[f"{name}/{key}"] = v
        if pi is not None:
            out[f"{name}/plan_index"] = pi

    # the reference test's shape: 256 docs x 3 features, "0:0" twice, 2 clusters
    n, F = 256, 3
    ids = np.arange(F, dtype=np.int32)
    vals = np.array([d * 100 + f for d in range(n) for f in range(F)], dtype=np.int64)
    offs = np.arange(n * F + 1, dtype=np.int64)
    add("basic", ids, offs, vals, ["0:0"] * 2, np.array([[0, 128]] * 2, dtype=np.int64),
        np.array([[128, 128]] * 2, dtype=np.int64), None, hash_k=7, bm=5.0)

    ids, offs, vals = corpus(6000, 2, 300)
    qs = ["1:5", "1:7 AND 2:9", "1:3 OR NOT 2:4", "", "NOT (1:1 OR 2:2) AND 1:8", "2:11 OR 2:12 OR 1:13"]
    total = 6000
    co = rng.integers(0, total - 1, (5, 3)).astype(np.int64)
    cl = np.minimum(rng.integers(0, 900, (5, 3)), total - co).astype(np.int64)
    cl[1, 2] = 0
    cl[3, 0] = -5
    co[2, 1] = 2040  # crosses the first bundle boundary
    cl[2, 1] = 30
    add("varied_plan_index", ids, offs, vals, qs, co, cl, np.array([3, 0, 5, 1, 1], dtype=np.int64))
    add("varied_rows", ids, offs, vals, qs, np.concatenate([co, co[:1]]), np.concatenate([cl, cl[:1]]), None)

    # _multiple over three chunks, one plan batch
    chunks = []
    for n in (3000, 700, 4500):
        ids, offs, vals = corpus(n, 2, 200)
        bi, bo = st.bloom_index_build(torch.from_numpy(ids), torch.from_numpy(offs), torch.from_numpy(vals), 3.0, 3)
        co = rng.integers(0, n - 1, (3, 2)).astype(np.int64)
        cl = np.minimum(rng.integers(1, 500, (3, 2)), n - co).astype(np.int64)
        chunks.append((bi, bo, co, cl))
    qs = ["1:5 OR 2:6", "NOT 1:7", "2:8 AND 1:9"]
    _, (pd, po) = st.parse_expression_query_batch(qs, torch.ones(1, dtype=torch.long), 7, True, 5)
    for fuse in (False, True):
        r = st.bloom_index_search_batch_return_partial_response_multiple(
            [c[0] for c in chunks], [c[1] for c in chunks], pd, po,
            [torch.from_numpy(c[2]) for c in chunks], [torch.from_numpy(c[3]) for c in chunks], 3, 7, None, fuse)
        for i in range(len(chunks)):
            out[f"multiple_fuse{int(fuse)}/{i}/cumsum"] = r[0][i].numpy()
            out[f"multiple_fuse{int(fuse)}/{i}/first"] = r[1][i].numpy()
            out[f"multiple_fuse{int(fuse)}/{i}/mask"] = r[2][i].numpy()
    for i, (bi, bo, co, cl) in enumerate(chunks):
        out[f"multiple/{i}/index"] = bi.numpy()
        out[f"multiple/{i}/bundle_b_offsets"] = bo.numpy()
        out[f"multiple/{i}/cluster_offsets"] = co
        out[f"multiple/{i}/cluster_lengths"] = cl
    out["multiple/plans_data"] = pd.numpy()
    out["multiple/plans_offsets"] = po.numpy()
    np.savez_compressed(HERE / "ref_partial.npz", **out)
    print("partial-response fixtures written to", HERE / "ref_partial.npz")


def kmean_fixtures() -> None:
    """ref_kmean.npz: fused_kmean_ann of the reference's CPU op
    (fused_kmean_ann.cpp:85-227) and its partial-mask wrappers (:229-311).
    Filtered cases: the reference CPU op reads doc d's filter bit as bit d % 64
    (LSB first) while the search output and the reference CUDA op put doc d
    at bit 63 - d % 64; those cases give the CPU op the bit-reversed words of
    an MSB-first mask, so the stored output is the MSB-first semantics."""
    import torch

    ref = ROOT / "oracle" / "_ref" / "libst_ref.so"
    if not ref.exists():
        subprocess.run(["make", "-C", str(ROOT / "oracle"), "ref"], check=True)
    torch.ops.load_library(str(ref))
    st = torch.ops.st
    out = {}
    rng = np.random.default_rng(21)

    def rev64(words: np.ndarray) -> np.ndarray:
        w = words.view(np.uint64).copy()
        r = np.zeros_like(w)
        for i in range(64):
            r |= ((w >> np.uint64(i)) & np.uint64(1)) << np.uint64(63 - i)
        return r.view(np.int64)

    def emb(n, dim, dtype):
        if dtype == "int8":
            return torch.from_numpy(rng.integers(-128, 128, (n, dim)).astype(np.int8))
        t = torch.from_numpy(rng.standard_normal((n, dim)).astype(np.float32))
        return t.to({"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}[dtype])

    def save_tensor(key, t):
        if t.dtype == torch.bfloat16:
            out[key] = t.view(torch.int16).numpy().view(np.uint16)
            out[key + "@bf16"] = np.array(1)
        else:
            out[key] = t.numpy()

    def add(name, sizes, dim, dtype, batch, probes, max_size, divisor=-1, scale=False,
            filtered=False, findex=False, invalid=-1):
        sizes = np.asarray(sizes, np.int64)
        offs = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
        n = int(offs[-1])
        e, q = emb(n, dim, dtype), emb(batch, dim, dtype)
        cids = rng.integers(0, len(sizes), (batch, probes)).astype(np.int64)
        clen = sizes[cids]
        kw = dict(invalid_index_value=invalid, divisor_for_int8=divisor)
        mask = fi = None
        if scale:
            sc = torch.from_numpy((rng.random(n) * 4 + 0.5).astype(np.float32)).to(torch.float16)
            kw["per_embedding_scale"] = sc
            save_tensor(f"{name}/scale", sc)
        if filtered:
            rows = batch if not findex else 3
            mask = rng.integers(-2**63, 2**63 - 1, (rows, (n + 63) // 64 - 1 if n > 128 else (n + 63) // 64),
                                dtype=np.int64)
            kw["filtering_bit_mask"] = torch.from_numpy(rev64(mask))
            out[f"{name}/mask_msb"] = mask
            if findex:
                fi = rng.integers(0, rows, batch).astype(np.int64)
                kw["filtering_bit_index"] = torch.from_numpy(fi)
                out[f"{name}/filter_index"] = fi
        if dtype == "bfloat16":
            # the reference CPU op raises for bfloat16 (its -FLT_MAX padding
            # overflows BFloat16); its float32 scores on the same (exactly
            # widened) values are stored, the test rounds them to bfloat16
            try:
                st.fused_kmean_ann(torch.from_numpy(offs), torch.from_numpy(cids), torch.from_numpy(clen),
                                   e, q, max_size, **kw)
                raise SystemExit("the reference CPU op accepted bfloat16 embeddings")
            except RuntimeError as err:
                out[f"{name}/ref_error"] = np.array(str(err).splitlines()[0])
            sc_, ix_ = st.fused_kmean_ann(torch.from_numpy(offs), torch.from_numpy(cids),
                                          torch.from_numpy(clen), e.float(), q.float(), max_size, **kw)
        else:
            sc_, ix_ = st.fused_kmean_ann(torch.from_numpy(offs), torch.from_numpy(cids),
                                          torch.from_numpy(clen), e, q, max_size, **kw)
        out[f"{name}/cluster_offsets"] = offs
        out[f"{name}/cluster_ids"] = cids
        out[f"{name}/cluster_length"] = clen
        save_tensor(f"{name}/embeddings", e)
        save_tensor(f"{name}/queries", q)
        out[f"{name}/params"] = np.array([max_size, divisor, invalid], np.int64)
        save_tensor(f"{name}/scores", sc_)
        out[f"{name}/indices"] = ix_.numpy()

    add("readme", [3, 5, 7], 64, "float32", 2, 2, 12)  # the op's documented example shape
    add("f32_trunc", rng.integers(1, 70, 9), 16, "float32", 4, 3, 40)
    add("f16", rng.integers(1, 70, 9), 64, "float16", 3, 3, 200)
    add("bf16", rng.integers(1, 70, 9), 128, "bfloat16", 3, 2, 150)
    add("i8_raw", rng.integers(1, 70, 9), 32, "int8", 3, 3, 200)
    add("i8_div", rng.integers(1, 70, 9), 32, "int8", 3, 3, 200, divisor=7)
    add("i8_scale", rng.integers(1, 70, 9), 48, "int8", 3, 3, 200, scale=True)
    add("f32_odd_dim", rng.integers(1, 40, 6), 17, "float32", 2, 4, 64, invalid=-99)
    add("f32_filter", rng.integers(20, 90, 8), 32, "float32", 4, 3, 250, filtered=True)
    add("bf16_filter_index", rng.integers(20, 90, 8), 32, "bfloat16", 5, 3, 250, filtered=True,
        findex=True)

    # partial-mask wrappers: the CPU op ignores the masks (and filtering_bit_index)
    sizes = rng.integers(1, 40, 6).astype(np.int64)
    offs = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    e, q = emb(int(offs[-1]), 32, "float32"), emb(3, 32, "float32")
    cids = rng.integers(0, 6, (3, 2)).astype(np.int64)
    dummy = torch.zeros(1, dtype=torch.long)
    s1, i1 = st.fused_kmean_ann_with_partial_masks(torch.from_numpy(offs), torch.from_numpy(cids),
                                                   torch.from_numpy(sizes[cids]), e, q, 70, dummy,
                                                   dummy.to(torch.int8), dummy)
    out["partial/cluster_offsets"] = offs
    out["partial/cluster_ids"] = cids
    out["partial/cluster_length"] = sizes[cids]
    out["partial/embeddings"] = e.numpy()
    out["partial/queries"] = q.numpy()
    out["partial/scores"] = s1.numpy()
    out["partial/indices"] = i1.numpy()
    lo, ll, le, lm = [], [], [], []
    for c in range(2):
        sz = rng.integers(1, 30, 5).astype(np.int64)
        of = np.concatenate([[0], np.cumsum(sz)]).astype(np.int64)
        ci = rng.integers(0, 5, (3, 2)).astype(np.int64)
        lo.append(torch.from_numpy(of)); ll.append(torch.from_numpy(ci)); le.append(torch.from_numpy(sz[ci]))
        lm.append(emb(int(of[-1]), 32, "float32"))
        out[f"multiple/{c}/cluster_offsets"] = of
        out[f"multiple/{c}/cluster_ids"] = ci
        out[f"multiple/{c}/cluster_length"] = sz[ci]
        out[f"multiple/{c}/embeddings"] = lm[-1].numpy()
    ms = st.fused_kmean_ann_with_partial_masks_multiple(q, lo, ll, le, lm, [33, 50], [dummy] * 2,
                                                        [dummy.to(torch.int8)] * 2, [dummy] * 2)
    out["multiple/queries"] = q.numpy()
    for c in range(2):
        out[f"multiple/{c}/scores"] = ms[0][c].numpy()
        out[f"multiple/{c}/indices"] = ms[1][c].numpy()

    # float16 rounding: the reference rounds float64 -> float32 -> float16
    # (fused_kmean_ann.cpp:214).  Query (1, 1, 2^-10); each doc's exact sum:
    # 1 + 2^-11 (a half-way point, ties to 1.0), 1 + 2^-11 + 2^-34 (float32
    # rounds it onto the half-way point -> 1.0; one float64 -> float16
    # rounding gives 1 + 2^-10), 1 + 2^-11 + 2^-22 (above it), 1 + 3*2^-11
    # (ties to even upwards), the negation of the second, 2^-24 and 3*2^-24
    # (subnormal; halved by the second query's 0.5 they become ties), 65519
    # and 65520 (largest finite / infinity).
    t = 2.0 ** -11
    rows = [[1, t, 0], [1, t, 2.0 ** -24], [1, t, 2.0 ** -12], [1 + 2 * t, t, 0], [-1, -t, -(2.0 ** -24)],
            [2.0 ** -24, 0, 0], [3 * 2.0 ** -24, 0, 0], [65504, 15, 0], [65504, 16, 0]]
    e = torch.tensor(rows, dtype=torch.float64).to(torch.float16)
    assert torch.equal(e.double(), torch.tensor(rows, dtype=torch.float64)), "rows must be exact in float16"
    q = torch.tensor([[1.0, 1.0, 2.0 ** -10], [0.5, 1.0, 2.0 ** -10]], dtype=torch.float16)
    offs = np.array([0, len(rows)], np.int64)
    cids = np.zeros((2, 1), np.int64)
    clen = np.full((2, 1), len(rows), np.int64)
    sc_, ix_ = st.fused_kmean_ann(torch.from_numpy(offs), torch.from_numpy(cids), torch.from_numpy(clen),
                                  e, q, 32)
    name = "f16_halfway"
    out[f"{name}/cluster_offsets"] = offs
    out[f"{name}/cluster_ids"] = cids
    out[f"{name}/cluster_length"] = clen
    out[f"{name}/embeddings"] = e.numpy()
    out[f"{name}/queries"] = q.numpy()
    out[f"{name}/params"] = np.array([32, -1, -1], np.int64)
    out[f"{name}/scores"] = sc_.numpy()
    out[f"{name}/indices"] = ix_.numpy()
    np.savez_compressed(HERE / "ref_kmean.npz", **out)
    print("fused_kmean_ann fixtures written to", HERE / "ref_kmean.npz")


def fresh_fixtures() -> None:
    """ref_fresh.npz: take_top_k_and_gather_from_main_and_fresh of the
    reference's CPU op (fresh_index_post_processing.cpp:231-270).  Scores are
    distinct within each merged row (a permutation of exactly representable
    values), so the reference's top-k order is fully determined.  Indices
    include values outside the data rows (read as row 0).  Per case: inputs,
    k, the data tensors, and the four outputs; bfloat16 tensors are stored as
    uint16 bits with a '@bf16' marker."""
    import torch

    ref = ROOT / "oracle" / "_ref" / "libst_ref.so"
    if not ref.exists():
        subprocess.run(["make", "-C", str(ROOT / "oracle"), "ref"], check=True)
    torch.ops.load_library(str(ref))
    st = torch.ops.st
    out = {}
    rng = np.random.default_rng(77)

    def save(key, t):
        if t.dtype == torch.bfloat16:
            out[key] = t.view(torch.int16).numpy().view(np.uint16)
            out[key + "@bf16"] = np.array(1)
        else:
            out[key] = t.numpy()

    def distinct_scores(R, n, dtype):
        # permutations of values exact in every score dtype used here
        if dtype in (torch.float16, torch.bfloat16):
            base = np.arange(n, dtype=np.float64) - n // 2      # |v| <= 256 for bf16 cases
        elif not dtype.is_floating_point:
            base = np.arange(n, dtype=np.float64) - (0 if dtype == torch.uint8 else n // 2)
        else:
            base = (np.arange(n, dtype=np.float64) - n / 3) * 0.37
        rows = np.stack([rng.permutation(base) for _ in range(R)]) if n else np.zeros((R, 0))
        return torch.from_numpy(rows).to(dtype)

    def add(name, R, nf, nm, k, score_dtype, index_dtype, datas, main_rows, fresh_rows):
        merged = distinct_scores(R, nf + nm, score_dtype)
        fresh_s, main_s = merged[:, :nf].contiguous(), merged[:, nf:].contiguous()
        # source rows mostly valid, some negative or past the data (read as row 0)
        mi = torch.from_numpy(rng.integers(-2, main_rows + 2, (R, nm))).to(index_dtype)
        fi = torch.from_numpy(rng.integers(-2, fresh_rows + 2, (R, nf))).to(index_dtype)
        keys, mds, fds = [], [], []
        for key, (dtype, dim) in datas.items():
            shape_m = (main_rows,) if dim == 0 else (main_rows, dim)
            shape_f = (fresh_rows,) if dim == 0 else (fresh_rows, dim)
            if dtype.is_floating_point:
                md = torch.from_numpy(rng.standard_normal(shape_m)).to(dtype)
                fd = torch.from_numpy(rng.standard_normal(shape_f)).to(dtype)
            else:
                hi = 100 if dtype in (torch.int8, torch.uint8) else 1 << 20
                md = torch.from_numpy(rng.integers(0, hi, shape_m)).to(dtype)
                fd = torch.from_numpy(rng.integers(0, hi, shape_f)).to(dtype)
            keys.append(key)
            mds.append(md)
            fds.append(fd)
        ts, ti, ff, g = st.take_top_k_and_gather_from_main_and_fresh(main_s, fresh_s, mi, fi, k, keys, mds, fds, 2)
        save(f"{name}/main_scores", main_s)
        save(f"{name}/fresh_scores", fresh_s)
        out[f"{name}/main_indices"] = mi.numpy()
        out[f"{name}/fresh_indices"] = fi.numpy()
        out[f"{name}/k"] = np.array(k)
        out[f"{name}/keys"] = np.array(keys)
        for key, md, fd in zip(keys, mds, fds):
            save(f"{name}/main_data/{key}", md)
            save(f"{name}/fresh_data/{key}", fd)
            save(f"{name}/gathered/{key}", g[key])
        save(f"{name}/top_scores", ts)
        out[f"{name}/top_indices"] = ti.numpy()
        out[f"{name}/is_from_fresh"] = ff.numpy()

    # the reference test's own inputs (test_fresh_index_post_processing.py:38-100)
    main_scores = torch.tensor([[0.90, 0.10, 0.70, 0.80, 0.40], [0.15, 0.28, 0.85, 0.05, 0.38]], dtype=torch.float16)
    fresh_scores = torch.tensor([[0.95, 0.20, 0.30, 0.60], [0.62, 0.99, 0.48, 0.31]], dtype=torch.float16)
    vecs = [[float(i), float(i) + 0.5, float(i) - 0.5, float(i) * 2.0] for i in range(7)]
    for index_dtype in (torch.int32, torch.int64):
        for k in (3, 7, 20):
            name = f"readme_{str(index_dtype)[6:]}_k{k}"
            mi = torch.tensor([[2, 5, 4, 3, 0], [6, 2, 3, 1, 0]], dtype=index_dtype)
            fi = torch.tensor([[1, 0, 2, 3], [4, 1, 3, 0]], dtype=index_dtype)
            mds = [torch.tensor([10, 20, 30, 40, 50, 60, 70]), torch.tensor(vecs, dtype=torch.bfloat16)]
            fds = [torch.tensor([100, 200, 300, 400, 500]), torch.tensor(vecs[:5], dtype=torch.bfloat16)]
            keys = ["item_ids", "embeddings"]
            ts, ti, ff, g = st.take_top_k_and_gather_from_main_and_fresh(main_scores, fresh_scores, mi, fi, k,
                                                                         keys, mds, fds, 2)
            save(f"{name}/main_scores", main_scores)
            save(f"{name}/fresh_scores", fresh_scores)
            out[f"{name}/main_indices"] = mi.numpy()
            out[f"{name}/fresh_indices"] = fi.numpy()
            out[f"{name}/k"] = np.array(k)
            out[f"{name}/keys"] = np.array(keys)
            for key, md, fd in zip(keys, mds, fds):
                save(f"{name}/main_data/{key}", md)
                save(f"{name}/fresh_data/{key}", fd)
                save(f"{name}/gathered/{key}", g[key])
            save(f"{name}/top_scores", ts)
            out[f"{name}/top_indices"] = ti.numpy()
            out[f"{name}/is_from_fresh"] = ff.numpy()

    add("f32_mixed", 7, 33, 300, 50, torch.float32, torch.int64,
        {"ids": (torch.int64, 0), "emb": (torch.float32, 5), "tag": (torch.uint8, 0)}, 40, 9)
    add("f64_main_only", 3, 0, 100, 10, torch.float64, torch.int32,
        {"ids": (torch.int32, 0), "w": (torch.float16, 3)}, 17, 4)
    add("f16_fresh_only", 4, 120, 0, 16, torch.float16, torch.int64,
        {"v": (torch.int16, 2)}, 5, 60)
    add("bf16_k_clamped", 5, 200, 300, 1000, torch.bfloat16, torch.int32,
        {"e": (torch.bfloat16, 8), "d": (torch.float64, 0)}, 500, 200)
    add("i32_scores", 4, 20, 10, 7, torch.int32, torch.int64, {"x": (torch.int8, 0)}, 3, 30)
    add("i64_scores_k0", 2, 5, 6, 0, torch.int64, torch.int64, {"x": (torch.int64, 0)}, 6, 5)
    add("f32_long_rows", 3, 1500, 12000, 300, torch.float32, torch.int64, {"ids": (torch.int32, 0)}, 2000, 300)
    add("f32_k_global", 2, 3000, 7000, 9000, torch.float32, torch.int32,
        {"ids": (torch.int32, 0)}, 1000, 500)
    add("u8_scores", 3, 40, 60, 25, torch.uint8, torch.int64, {"x": (torch.float32, 0)}, 60, 40)
    np.savez_compressed(HERE / "ref_fresh.npz", **out)
    print("take_top_k_and_gather_from_main_and_fresh fixtures written to", HERE / "ref_fresh.npz")


def full_digests(names: list[str]) -> None:
    """ref_full_digests.json: the benchmark configurations at full size,
    built and searched by the reference's CPU ops on the numpy-generated
    corpora (silvertorch_amd.synthetic.make_corpus / make_queries, seed 0):
    digests (synthetic.digest) of the inputs, bundle_b_offsets, bloom_index,
    the plan bytes and the packed search output, and the per-query match
    counts.  cfg4 is a build-only configuration."""
    import torch

    from silvertorch_amd import synthetic as S

    ref = ROOT / "oracle" / "_ref" / "libst_ref.so"
    if not ref.exists():
        subprocess.run(["make", "-C", str(ROOT / "oracle"), "ref"], check=True)
    torch.ops.load_library(str(ref))
    st = torch.ops.st
    path = HERE / "ref_full_digests.json"
    out = json.loads(path.read_text()) if path.exists() else {}
    for name in names:
        import time

        t0 = time.time()
        cspec, qspec = S.CONFIGS[name]
        corp = S.make_corpus(cspec, seed=0)
        rec = {"seed": 0, "num_docs": cspec.num_docs, "num_values": int(corp.feature_values.size),
               "inputs": {"offsets": S.digest(corp.feature_offsets), "values": S.digest(corp.feature_values)}}
        print(f"{name}: corpus {time.time() - t0:.0f}s", flush=True)
        bi, bo = st.bloom_index_build(torch.from_numpy(corp.feature_ids), torch.from_numpy(corp.feature_offsets),
                                      torch.from_numpy(corp.feature_values), cspec.b_multiplier, cspec.k)
        del corp
        print(f"{name}: reference build {time.time() - t0:.0f}s", flush=True)
        rec.update(index=S.digest(bi.numpy()), index_len=int(bi.numel()),
                   bundle_b_offsets=S.digest(bo.numpy()), bundles=int(bo.numel() - 1),
                   bundle_b_offsets_head=bo[:4].tolist(), bundle_b_offsets_last=int(bo[-1]))
        if qspec is not None:
            queries = S.make_queries(cspec, qspec, seed=0)
            _, (pd, po) = st.parse_expression_query_batch(queries, torch.ones(1, dtype=torch.long),
                                                          cspec.hash_k, True, 5)
            packed = st.bloom_index_search_batch(bi, bo, pd, po, cspec.k, cspec.hash_k, False).numpy()
            print(f"{name}: reference search {time.time() - t0:.0f}s", flush=True)
            rec.update(queries_sha256=hashlib.sha256("\n".join(queries).encode()).hexdigest(),
                       plans_data=S.digest(pd.numpy()), plans_offsets=S.digest(po.numpy()),
                       packed=S.digest(packed), packed_shape=list(packed.shape),
                       match_counts=S.match_counts(packed, cspec.num_docs))
            del packed
        out[name] = rec
        del bi, bo
        path.write_text(json.dumps(out, indent=1))
        print(f"{name} written to {path} ({time.time() - t0:.0f}s)", flush=True)


if __name__ == "__main__":
    if sys.argv[1:] == ["partial"]:
        partial_fixtures()
    elif sys.argv[1:] == ["kmean"]:
        kmean_fixtures()
    elif sys.argv[1:] == ["fresh"]:
        fresh_fixtures()
    elif sys.argv[1:2] == ["full"]:
        full_digests(sys.argv[2:] or ["cfg2", "cfg5", "cfg4"])
    else:
        main()
        partial_fixtures()
        kmean_fixtures()
        fresh_fixtures()
