"""ctypes front end of the C oracle (bloom_oracle.c) -- TEST INFRASTRUCTURE ONLY.

Each wrapper names the reference code it restates; see bloom_oracle.c for the
full citation list and for how each function is pinned.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"

_lib = None

_i64p = ctypes.POINTER(ctypes.c_int64)


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        L.or_murmur3_pair.restype = ctypes.c_uint64
        L.or_murmur3_pair.argtypes = [ctypes.c_uint64] * 3
        L.or_build_positions.restype = ctypes.c_int
        L.or_build_positions.argtypes = [ctypes.c_int64] * 4 + [ctypes.POINTER(ctypes.c_int32)]
        L.or_bundle_b_offsets.restype = None
        L.or_bundle_b_offsets.argtypes = [_i64p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_double, _i64p]
        L.or_bloom_build.restype = ctypes.c_int
        L.or_bloom_build.argtypes = [ctypes.POINTER(ctypes.c_int32), _i64p, _i64p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _i64p, _i64p]
        L.or_search_batch.restype = ctypes.c_int
        L.or_search_batch.argtypes = [_i64p, ctypes.c_int64, _i64p, ctypes.c_int64, ctypes.POINTER(ctypes.c_int8), ctypes.c_int64, _i64p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _i64p]
        L.or_partial_response.restype = ctypes.c_int
        L.or_partial_response.argtypes = [_i64p, ctypes.c_int64, _i64p, ctypes.c_int64, ctypes.POINTER(ctypes.c_int8),
                                          ctypes.c_int64, _i64p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                          _i64p, _i64p, ctypes.c_int64, ctypes.c_int64, _i64p,
                                          ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int8), _i64p,
                                          ctypes.c_int64, _i64p]
        L.or_unpack_bool.restype = None
        L.or_unpack_bool.argtypes = [_i64p, ctypes.c_int64, ctypes.c_int64, ctypes.POINTER(ctypes.c_uint8)]
        L.or_compact.restype = None
        L.or_compact.argtypes = [_i64p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _i64p, _i64p]
        L.or_filtered_topk.restype = ctypes.c_int
        L.or_filtered_topk.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_int64, ctypes.c_int64, ctypes.POINTER(ctypes.c_float), ctypes.c_int64, _i64p, ctypes.c_int64, ctypes.c_int64, _i64p, ctypes.POINTER(ctypes.c_float)]
        _lib = L
    return _lib


def _p(a: np.ndarray, ct):
    return a.ctypes.data_as(ctypes.POINTER(ct))


def murmur3_pair(x: int, y: int, seed: int) -> int:
    """murmur_hash3_2x64 (bloom_index_util.cuh:59-106)."""
    m = (1 << 64) - 1
    return int(lib().or_murmur3_pair(x & m, y & m, seed & m))


def build_positions(fid: int, value: int, b: int, k: int) -> list[int]:
    """assign_one_bits_position (bloom_index_util.cuh:183-207)."""
    out = np.zeros(max(k, 1), dtype=np.int32)
    rc = lib().or_build_positions(fid, value, b, k, _p(out, ctypes.c_int32))
    if rc != 0:
        raise ValueError("no k distinct positions exist for this b")
    return out[:k].tolist()


def bundle_b_offsets(offsets: np.ndarray, num_features: int, k: int, b_multiplier: float) -> np.ndarray:
    """Per-bundle width pass (bloom_indexer.cpp:43-70)."""
    offsets = np.ascontiguousarray(offsets, dtype=np.int64)
    n = (offsets.size - 1) // num_features
    nb = (n + 2047) // 2048
    out = np.zeros(nb + 1, dtype=np.int64)
    lib().or_bundle_b_offsets(_p(offsets, ctypes.c_int64), n, num_features, k, b_multiplier, _p(out, ctypes.c_int64))
    return out


def bloom_build(feature_ids, offsets, values, b_multiplier: float, k: int):
    """bloom_index_build_cpu (bloom_indexer.cpp:26-113) -> (index, bundle_b_offsets)."""
    ids = np.ascontiguousarray(feature_ids, dtype=np.int32)
    offsets = np.ascontiguousarray(offsets, dtype=np.int64)
    values = np.ascontiguousarray(values, dtype=np.int64)
    F = ids.size
    n = (offsets.size - 1) // F
    bbo = bundle_b_offsets(offsets, F, k, b_multiplier)
    index = np.zeros(max(int(bbo[-1]) * 32, 1), dtype=np.int64)
    if values.size == 0:
        values = np.zeros(1, dtype=np.int64)
    rc = lib().or_bloom_build(_p(ids, ctypes.c_int32), _p(offsets, ctypes.c_int64), _p(values, ctypes.c_int64),
                              F, n, k, _p(bbo, ctypes.c_int64), _p(index, ctypes.c_int64))
    if rc != 0:
        raise ValueError("oracle build rejected its arguments")
    return index[: int(bbo[-1]) * 32], bbo


def search_packed(index, bbo, plans_data, plans_offsets, k: int, hash_k: int) -> np.ndarray:
    """bloom_index_search_batch_cpu with return_bool_mask=False
    (bloom_index_search.cpp:27-243) -> int64[Q, nb*32]."""
    index = np.ascontiguousarray(index, dtype=np.int64)
    bbo = np.ascontiguousarray(bbo, dtype=np.int64)
    pdata = np.ascontiguousarray(plans_data, dtype=np.int8)
    poffs = np.ascontiguousarray(plans_offsets, dtype=np.int64)
    q = poffs.size // 8
    nb = bbo.size - 1
    out = np.zeros((q, nb * 32), dtype=np.int64)
    idx = index if index.size else np.zeros(1, dtype=np.int64)
    pd = pdata if pdata.size else np.zeros(1, dtype=np.int8)
    po = poffs if poffs.size else np.zeros(1, dtype=np.int64)
    rc = lib().or_search_batch(_p(idx, ctypes.c_int64), index.size, _p(bbo, ctypes.c_int64), nb,
                               _p(pd, ctypes.c_int8), pdata.size, _p(po, ctypes.c_int64), q, k, hash_k,
                               _p(out, ctypes.c_int64))
    if rc != 0:
        raise ValueError(f"oracle search rejected plan {-rc - 1}")
    return out


PARTIAL_ERRORS = {-1: "plan index out of range", -2: "cluster columns outside the index",
                  -3: "int32 column total overflows", -5: "malformed plan"}


def partial_response(index, bbo, plans_data, plans_offsets, k: int, hash_k: int,
                     cluster_offsets, cluster_lengths, plan_index=None):
    """bloom_index_search_batch_return_partial_response_cpu
    (bloom_index_search.cpp:246-395) -> (column_counts_cumsum int32[R*C],
    first_item_offsets_in_column int8[R*C], column_mask_response int64[...])."""
    index = np.ascontiguousarray(index, dtype=np.int64)
    bbo = np.ascontiguousarray(bbo, dtype=np.int64)
    pdata = np.ascontiguousarray(plans_data, dtype=np.int8)
    poffs = np.ascontiguousarray(plans_offsets, dtype=np.int64)
    co = np.ascontiguousarray(cluster_offsets, dtype=np.int64)
    cl = np.ascontiguousarray(cluster_lengths, dtype=np.int64)
    if co.ndim != 2 or co.shape != cl.shape:
        raise ValueError(f"cluster arrays must be 2-D of one shape: {co.shape} vs {cl.shape}")
    rows, clusters = co.shape
    pi = None if plan_index is None else np.ascontiguousarray(plan_index, dtype=np.int64)
    cumsum = np.zeros(max(rows * clusters, 1), dtype=np.int32)
    first = np.zeros(max(rows * clusters, 1), dtype=np.int8)
    total = np.zeros(1, dtype=np.int64)
    idx = index if index.size else np.zeros(1, dtype=np.int64)
    pd = pdata if pdata.size else np.zeros(1, dtype=np.int8)
    po = poffs if poffs.size else np.zeros(1, dtype=np.int64)
    co_ = co if co.size else np.zeros(1, dtype=np.int64)
    cl_ = cl if cl.size else np.zeros(1, dtype=np.int64)

    def run(mask, cap):
        return lib().or_partial_response(
            _p(idx, ctypes.c_int64), index.size, _p(bbo, ctypes.c_int64), bbo.size - 1,
            _p(pd, ctypes.c_int8), pdata.size, _p(po, ctypes.c_int64), poffs.size // 8, k, hash_k,
            _p(co_, ctypes.c_int64), _p(cl_, ctypes.c_int64), rows, clusters,
            None if pi is None else _p(pi, ctypes.c_int64), _p(cumsum, ctypes.c_int32),
            _p(first, ctypes.c_int8), _p(mask, ctypes.c_int64), cap, _p(total, ctypes.c_int64))

    probe = np.zeros(1, dtype=np.int64)
    rc = run(probe, 0)
    if rc not in (0, -4):
        raise ValueError(f"oracle partial response: {PARTIAL_ERRORS.get(rc, rc)}")
    mask = np.zeros(max(int(total[0]), 1), dtype=np.int64)
    rc = run(mask, mask.size)
    if rc != 0:
        raise ValueError(f"oracle partial response: {PARTIAL_ERRORS.get(rc, rc)}")
    n = rows * clusters
    return cumsum[:n], first[:n], mask[: int(total[0])]


def unpack_bool(packed: np.ndarray) -> np.ndarray:
    """bool mask layout of bloom_index_search.cpp:231-236."""
    packed = np.ascontiguousarray(packed, dtype=np.int64)
    rows, cols = packed.shape
    out = np.zeros((rows, cols * 64), dtype=np.uint8)
    if packed.size:
        lib().or_unpack_bool(_p(packed, ctypes.c_int64), rows, cols, _p(out, ctypes.c_uint8))
    return out.astype(bool)


def compact(packed: np.ndarray, num_docs: int):
    """Matching ids below num_docs per query (README.md:191) -> (ids, row_offsets)."""
    packed = np.ascontiguousarray(packed, dtype=np.int64)
    rows, cols = packed.shape
    ro = np.zeros(rows + 1, dtype=np.int64)
    src = packed if packed.size else np.zeros(1, dtype=np.int64)
    lib().or_compact(_p(src, ctypes.c_int64), rows, cols, num_docs, _p(ro, ctypes.c_int64), None)
    ids = np.zeros(max(int(ro[-1]), 1), dtype=np.int64)
    lib().or_compact(_p(src, ctypes.c_int64), rows, cols, num_docs, _p(ro, ctypes.c_int64), _p(ids, ctypes.c_int64))
    return ids[: int(ro[-1])], ro


def filtered_topk(emb: np.ndarray, qv: np.ndarray, packed: np.ndarray, topk: int):
    """Top-k by (fp64 score desc, id asc) over filter-passing docs."""
    emb = np.ascontiguousarray(emb, dtype=np.float32)
    qv = np.ascontiguousarray(qv, dtype=np.float32)
    packed = np.ascontiguousarray(packed, dtype=np.int64)
    n, dim = emb.shape
    q = qv.shape[0]
    if packed.ndim != 2 or packed.shape[0] != q or packed.shape[1] * 64 < n or qv.shape[1] != dim:
        raise ValueError(f"shapes do not match: emb {emb.shape}, qv {qv.shape}, packed {packed.shape}")
    ids = np.zeros((q, topk), dtype=np.int64)
    scores = np.zeros((q, topk), dtype=np.float32)
    rc = lib().or_filtered_topk(_p(emb, ctypes.c_float), n, dim, _p(qv, ctypes.c_float), q,
                                _p(packed, ctypes.c_int64), packed.shape[1], topk,
                                _p(ids, ctypes.c_int64), _p(scores, ctypes.c_float))
    if rc != 0:
        raise MemoryError("oracle top-k allocation failed")
    return ids, scores


def bf16_round(f32: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns (uint16), round to nearest even, as
    c10::BFloat16's conversion does (finite inputs)."""
    u = np.ascontiguousarray(f32, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def fused_kmean_ann(cluster_offsets, cluster_ids, cluster_length, embeddings, queries,
                    max_size: int, filter_mask=None, invalid_index: int = -1, divisor: int = -1,
                    filter_index=None, scale=None, bf16: bool = False):
    """Restates the reference CPU op fused_kmean_ann (fused_kmean_ann.cpp:85-227):
    per query row, over the probes in order, the docs of each selected cluster
    (cluster_offsets[cid] + i, i < cluster_length) that pass the row's filter
    take consecutive slots until the row width (max_size rounded up to 32,
    :104-107) is full; the rest is padding.  Float scores: the float64 dot
    product summed in dimension order (:45-55), then converted to the score
    dtype; int8: the exact integer sum, divided as float32 by divisor_for_int8
    or the per-embedding float16 scale and stored as float16 when either is
    given (:30-41, :196-206).  One deliberate difference: the filter bit of doc
    d is bit 63 - d % 64 of word d / 64 (the search output's layout and the
    reference CUDA op's reading), where the CPU op reads bit d % 64.  bfloat16
    embeddings arrive as uint16 bit patterns with bf16=True; their padding is
    0xFF7F (the CUDA op's, simple_index_mm.cuh:123; the CPU op raises).
    Returns (scores, indices int32), both [B, width]."""
    cluster_offsets = np.asarray(cluster_offsets, np.int64)
    cluster_ids = np.asarray(cluster_ids, np.int64)
    cluster_length = np.asarray(cluster_length, np.int64)
    B, P = cluster_ids.shape
    width = (max_size + 31) // 32 * 32
    is_i8 = embeddings.dtype == np.int8
    if bf16:
        e64 = bf16_to_f32(embeddings).astype(np.float64)
        q64 = bf16_to_f32(queries).astype(np.float64)
    elif not is_i8:
        e64 = embeddings.astype(np.float64)
        q64 = queries.astype(np.float64)
    if is_i8:
        half = divisor != -1 or scale is not None
        scores = np.full((B, width), np.float16(-65504.0) if half else np.iinfo(np.int32).min,
                         dtype=np.float16 if half else np.int32)
    elif bf16:
        scores = np.full((B, width), 0xFF7F, dtype=np.uint16)
    elif embeddings.dtype == np.float16:
        scores = np.full((B, width), -65504.0, dtype=np.float16)
    else:
        scores = np.full((B, width), -np.finfo(np.float32).max, dtype=np.float32)
    indices = np.full((B, width), invalid_index, dtype=np.int32)
    for b in range(B):
        write = 0
        frow = int(filter_index[b]) if filter_index is not None else b
        for p in range(P):
            cid, clen = int(cluster_ids[b, p]), int(cluster_length[b, p])
            start = int(cluster_offsets[cid])
            for i in range(clen):
                if write >= width:
                    break
                doc = start + i
                if filter_mask is not None:
                    word = doc >> 6
                    if word < filter_mask.shape[1]:
                        w = int(np.asarray(filter_mask[frow, word]).view(np.uint64))
                        if not (w >> (63 - (doc & 63))) & 1:
                            continue
                if is_i8:
                    raw = int(np.dot(embeddings[doc].astype(np.int64), queries[b].astype(np.int64)))
                    if scale is not None:
                        scores[b, write] = np.float16(np.float32(raw) / np.float32(scale[doc]))
                    elif divisor != -1:
                        scores[b, write] = np.float16(np.float32(raw) / np.float32(divisor))
                    else:
                        scores[b, write] = raw
                else:
                    s = float(np.cumsum(e64[doc] * q64[b])[-1])  # sequential float64 sum
                    if bf16:
                        scores[b, write] = bf16_round(np.array([s], np.float32))[0]
                    else:
                        scores[b, write] = scores.dtype.type(np.float32(s))
                indices[b, write] = doc
                write += 1
    return scores, indices


def _score_rank_columns(scores: np.ndarray):
    """(is_nan, value) per score: NaN ranks above every number (the
    comparator of at::topk's CPU kernel) and -0.0 equals +0.0."""
    s = np.asarray(scores)
    if s.dtype.kind == "f":
        f = s.astype(np.float64)
        nan = np.isnan(f)
        return nan.astype(np.int64), np.where(nan, 0.0, f) + 0.0  # -0.0 + 0.0 == +0.0
    return np.zeros(s.shape, np.int64), s.astype(np.int64)


def fresh_topk_gather(main_scores, fresh_scores, main_indices, fresh_indices, k: int,
                      main_data: list, fresh_data: list):
    """Restates take_top_k_and_gather_from_main_and_fresh_cpu
    (fresh_index_post_processing.cpp:231-270) and its gather (:44-163):
    merged = cat(fresh, main) per row; the min(k, Nf + Nm) best, largest
    first; is_from_fresh = merged index < Nf; data row through fresh_indices
    [r, t] (t < Nf) or main_indices[r, t - Nf], a row outside the data read
    as row 0.  at::topk leaves the order of equal scores open; this
    restatement puts the lower merged index first (the order the HIP kernel
    promises).  Scores must share one dtype (bf16 as float32 values).
    Returns (top_scores, top_indices int64, is_from_fresh bool, [gathered])."""
    main_scores = np.asarray(main_scores)
    fresh_scores = np.asarray(fresh_scores)
    R, Nm = main_scores.shape
    Nf = fresh_scores.shape[1]
    merged = np.concatenate([fresh_scores, main_scores], axis=1)
    kc = min(k, Nf + Nm)
    is_nan, vals = _score_rank_columns(merged)
    cols = np.arange(Nf + Nm)
    top_idx = np.zeros((R, kc), np.int64)
    for r in range(R):
        # NaN first, then larger value, then lower merged index
        top_idx[r] = np.lexsort((cols, -vals[r], -is_nan[r]))[:kc]
    top_scores = np.take_along_axis(merged, top_idx, axis=1)
    is_fresh = top_idx < Nf
    gathered = []
    for md, fd in zip(main_data, fresh_data):
        md, fd = np.asarray(md), np.asarray(fd)
        rows = []
        for r in range(R):
            for j in range(kc):
                t = int(top_idx[r, j])
                if t < Nf:
                    src, data = int(fresh_indices[r, t]), fd
                else:
                    src, data = int(main_indices[r, t - Nf]), md
                if src < 0 or src >= data.shape[0]:
                    src = 0
                rows.append(data[src])
        shape = (R * kc,) + md.shape[1:]
        gathered.append(np.array(rows, dtype=md.dtype).reshape(shape) if rows else np.zeros(shape, md.dtype))
    return top_scores, top_idx, is_fresh, gathered
