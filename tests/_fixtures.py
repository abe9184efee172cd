"""Loaders for the committed golden fixtures (tests/golden/)."""

from __future__ import annotations

import hashlib
import json
import struct
from functools import lru_cache
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"


@lru_cache(None)
def murmur_vectors() -> list[tuple[int, int, int, int]]:
    d = json.loads((GOLDEN / "murmur_x64_128.json").read_text())
    return [tuple(int(v) for v in row) for row in d["vectors"]]


@lru_cache(None)
def parser_golden() -> dict:
    return json.loads((GOLDEN / "ref_parser.json").read_text())


@lru_cache(None)
def digests() -> dict:
    return json.loads((GOLDEN / "ref_digests.json").read_text())


@lru_cache(None)
def _cases_npz():
    return dict(np.load(GOLDEN / "ref_cases.npz", allow_pickle=False))


def case_names() -> list[str]:
    return sorted({k.split("/")[0] for k in _cases_npz()})


def case(name: str) -> dict:
    z = _cases_npz()
    c = {k.split("/", 1)[1]: v for k, v in z.items() if k.startswith(name + "/")}
    bm, kb, ks, hk, ms, phk = c["params"].tolist()
    c.update(b_multiplier=bm, build_k=int(kb), k=int(ks), hash_k=int(hk), max_sub=int(ms), parse_hash_k=int(phk))
    c["queries"] = [str(q) for q in c["queries"]]
    return c


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def wide_corpus():
    w = digests()["wide_bundles"]
    n = 2048 + 16
    cnt = np.ones(n, dtype=np.int64)
    cnt[0] = w["doc0_terms"]
    cnt[2048] = w["doc2048_terms"]
    offs = np.concatenate([[0], np.cumsum(cnt)]).astype(np.int64)
    vals = (np.arange(int(offs[-1]), dtype=np.int64) * 7919) % 100003
    return np.array([5], dtype=np.int32), offs, vals, w


def encode_plan(ops, offsets, hashes, params=()):
    """Encodes one plan in the reference's layout (bloom_index_util.cpp:81-124)."""
    buf, offs = bytearray(), []
    for raw in (bytes(ops), struct.pack(f"<{len(offsets)}i", *offsets),
                struct.pack(f"<{len(params)}i", *params), struct.pack(f"<{len(hashes)}Q", *hashes)):
        start = len(buf)
        buf += raw + b"\0" * ((-len(raw)) % 8)
        offs += [start, start + len(raw)]
    return bytes(buf), offs


@lru_cache(None)
def _partial_npz():
    return dict(np.load(GOLDEN / "ref_partial.npz", allow_pickle=False))


def partial_case_names() -> list[str]:
    return sorted({k.split("/")[0] for k in _partial_npz()
                   if not k.startswith("multiple")})


def partial_case(name: str) -> dict:
    z = _partial_npz()
    return {k.split("/", 1)[1]: v for k, v in z.items() if k.startswith(name + "/")}


def partial_multiple() -> dict:
    """Chunks of the _multiple fixture: list of dicts plus the shared plans and
    the reference outputs for fuse = False / True."""
    z = _partial_npz()
    n = len({k.split("/")[1] for k in z if k.startswith("multiple/") and k.split("/")[1].isdigit()})
    chunks = [{f: z[f"multiple/{i}/{f}"] for f in ("index", "bundle_b_offsets", "cluster_offsets",
                                                   "cluster_lengths")} for i in range(n)]
    outs = {fuse: [tuple(z[f"multiple_fuse{fuse}/{i}/{f}"] for f in ("cumsum", "first", "mask"))
                   for i in range(n)] for fuse in (0, 1)}
    return {"chunks": chunks, "plans_data": z["multiple/plans_data"],
            "plans_offsets": z["multiple/plans_offsets"], "outputs": outs}


@lru_cache(None)
def _kmean_npz():
    return dict(np.load(GOLDEN / "ref_kmean.npz", allow_pickle=False))


KMEAN_CASES = ["readme", "f32_trunc", "f16", "f16_halfway", "bf16", "i8_raw", "i8_div", "i8_scale", "f32_odd_dim",
               "f32_filter", "bf16_filter_index"]


def kmean_case(name: str) -> dict:
    """One fused_kmean_ann fixture of the reference CPU op (see
    tests/golden/make_golden.py): inputs, parameters and expected outputs.
    bfloat16 cases: 'bf16' is set, embeddings/queries are uint16 bit patterns
    and 'scores' holds the reference's float32 scores of the exactly widened
    values (the reference CPU op raises for bfloat16)."""
    z = _kmean_npz()
    pre = name + "/"
    c = {k[len(pre):]: v for k, v in z.items() if k.startswith(pre)}
    c["bf16"] = "embeddings@bf16" in c
    max_size, divisor, invalid = (int(v) for v in c["params"])
    c.update(max_size=max_size, divisor=divisor, invalid=invalid)
    return c


def kmean_group(prefix: str) -> dict:
    z = _kmean_npz()
    return {k[len(prefix) + 1:]: v for k, v in z.items() if k.startswith(prefix + "/")}


@lru_cache(None)
def _fresh_npz():
    return dict(np.load(GOLDEN / "ref_fresh.npz", allow_pickle=False))


def fresh_case_names() -> list[str]:
    return sorted({k.split("/")[0] for k in _fresh_npz()})


def fresh_case(name: str) -> dict:
    """One take_top_k_and_gather_from_main_and_fresh fixture of the reference
    CPU op (tests/golden/make_golden.py fresh_fixtures): arrays by field, with
    'main_data' / 'fresh_data' / 'gathered' dicts by key.  bfloat16 arrays are
    uint16 bit patterns listed in 'bf16' (the set of field paths)."""
    z = _fresh_npz()
    pre = name + "/"
    c: dict = {"main_data": {}, "fresh_data": {}, "gathered": {}, "bf16": set()}
    for k, v in z.items():
        if not k.startswith(pre):
            continue
        path = k[len(pre):]
        if path.endswith("@bf16"):
            c["bf16"].add(path[:-5])
            continue
        parts = path.split("/")
        if len(parts) == 2:
            c[parts[0]][parts[1]] = v
        else:
            c[path] = v
    c["k"] = int(c["k"])
    c["keys"] = [str(s) for s in c["keys"]]
    return c


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)
