"""CPU tests of the product's host side and of the C ABI boundary.

* the C-ABI library loads and exports every function include/*.h declares;
* the product parser (C++, behind the C ABI and torch.ops.st) emits the
  reference's plan bytes (tests/golden/ref_parser.json) and raises with the
  reference's messages;
* the plan compiler accepts every reference-produced plan and rejects the
  malformed ones where the reference CPU search fails or reads out of bounds
  (bloom_index_search.cpp:72-171);
* the torch.ops.st schemas match the reference's (bloom_indexer.cpp:117-124,
  bloom_index_search.cpp:549-558, expression_query_parser.cpp:457-464).
No compute kernel is launched here.
"""

import re
import struct
from pathlib import Path

import numpy as np
import pytest

from oracle import parser_oracle as P
from silvertorch_amd import capi
from tests import _fixtures as G

ROOT = Path(__file__).resolve().parents[1]


def declared_functions() -> list[str]:
    text = "\n".join(p.read_text() for p in (ROOT / "include").glob("*.h"))
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(st_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = capi.lib()
    names = declared_functions()
    assert len(names) >= 19
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(capi.SIGNATURES)
    assert b"gfx950" in lib.st_version()


def test_host_murmur_matches_independent_vectors():
    lib = capi.lib()
    for x, y, seed, want in G.murmur_vectors():
        assert lib.st_murmur_hash3_2x64(x, y, seed) == want


def test_parser_matches_reference_bytes():
    g = G.parser_golden()
    for b in g["batches"]:
        m, data, offs = capi.parse_expression_query_batch(g["expressions"], b["hash_k"], True, b["max_sub_queries"])
        assert m == b["max_stack"]
        assert data.hex() == b["data_hex"]
        assert offs == b["offsets"]
    m, data, offs = capi.parse_expression_query_batch(g["expressions"], 7, False, 5)
    assert (m, len(data), len(offs)) == tuple(g["no_plan"].values())


def test_parser_errors_match_reference():
    for expr, msg in G.parser_golden()["errors"].items():
        if msg is None:
            capi.parse_expression_query_batch([expr], 7)
            continue
        with pytest.raises(capi.StError) as ei:
            capi.parse_expression_query_batch([expr], 7)
        assert str(ei.value) == msg


def test_parser_int64_limits():
    """Feature ids and values span int64; one past either end is an error that
    names the token (the reference's std::stoll throws out_of_range there,
    expression_query_parser.cpp:342-343)."""
    lo, hi = -(1 << 63), (1 << 63) - 1
    exprs = [f"{hi}:{lo}", f"{lo}:{hi}", "-0:0"]
    assert capi.parse_expression_query_batch(exprs, 3, True, 5) == P.parse_batch(exprs, 3, True, 5)
    for expr, what, tok, pos in [(f"{hi + 1}:1", "feature id", str(hi + 1), 0),
                                 (f"1:{lo - 1}", "feature value", str(lo - 1), 2),
                                 (f"2:2 AND 99999999999999999999:1", "feature id", "99999999999999999999", 8)]:
        with pytest.raises(capi.StError) as ei:
            capi.parse_expression_query_batch([expr], 7)
        assert str(ei.value) == f"{what} '{tok}' at position {pos} does not fit a signed 64-bit integer"


def test_parser_parallel_batch_matches_oracle():
    """A batch large enough for the host pool gives the oracle's bytes and the
    first failing expression's error."""
    rng = np.random.default_rng(7)
    exprs = [_random_expr(rng) for _ in range(300)]
    assert capi.parse_expression_query_batch(exprs, 5, True, 4) == P.parse_batch(exprs, 5, True, 4)
    bad = list(exprs)
    bad[200] = "1:1 XOR 2:2"
    bad[250] = "$"
    with pytest.raises(capi.StError) as ei:
        capi.parse_expression_query_batch(bad, 5)
    assert str(ei.value) == "Unknown keyword 'XOR' at position 4"


def _random_expr(rng, depth=0):
    if depth > 2 or rng.random() < 0.35:
        t = f"{int(rng.integers(-3, 20))}:{int(rng.integers(-50, 50))}"
        if rng.random() < 0.2:
            t += ":0.5" if rng.random() < 0.5 else ":3"
        return t
    n = int(rng.integers(1, 7))
    sep = [" AND ", " OR ", " & ", " | "][int(rng.integers(0, 4))]
    body = sep.join(_random_expr(rng, depth + 1) for _ in range(n))
    if rng.random() < 0.5:
        body = f"({body})"
    if rng.random() < 0.2:
        body = ("NOT " if rng.random() < 0.5 else "!") + body
    return body


def test_parser_matches_oracle_on_random_expressions():
    rng = np.random.default_rng(99)
    for _ in range(60):
        exprs = [_random_expr(rng) for _ in range(int(rng.integers(1, 8)))]
        hk = int(rng.integers(1, 9))
        ms = int(rng.integers(-1, 7))
        assert capi.parse_expression_query_batch(exprs, hk, True, ms) == P.parse_batch(exprs, hk, True, ms)


_plan = G.encode_plan


def test_plan_compiler_accepts_reference_plans():
    for name in G.case_names():
        c = G.case(name)
        plan = capi.SearchPlan(c["plans_data"].tobytes(), c["plans_offsets"], c["k"], c["hash_k"])
        assert plan.num_queries == len(c["plans_offsets"]) // 8
        assert len(plan.blob()) > 0


@pytest.mark.parametrize("ops,offsets,nh,msg", [
    ([9], [0, 0], 0, "unknown operator: 9"),
    ([4, 4, 3], [0, 1, 2, 4], 14, "NOT query should have 1 parameter, but got 2"),
    ([4, 1], [0, 1, 4], 7, "pops 3 values from a shorter stack"),
    ([], [0], 0, "has no operators"),
    ([4, 4, 1], [0, 1, 2, 4], 7, "needs hashes [7, 14)"),
    ([4, 1], [0, 1], 7, "has no child count"),
])
def test_plan_compiler_rejects_malformed_plans(ops, offsets, nh, msg):
    data, offs = _plan(ops, offsets, list(range(nh)))
    with pytest.raises(capi.StError, match=re.escape(msg)):
        capi.SearchPlan(data, offs, 3, 7)


def test_plan_compiler_limits():
    data, offs = _plan([4], [0, 1], list(range(11)))
    with pytest.raises(capi.StError, match="at most 10"):
        capi.SearchPlan(data, offs, 11, 11)
    capi.SearchPlan(data, offs, 11, 10)  # k_eff = min(k, hash_k) = 10
    capi.SearchPlan(data, offs, 0, 7)  # every term is all ones
    with pytest.raises(capi.StError, match="outside plans_data"):
        capi.SearchPlan(data, [0, 1, 8, 12, 16, 16, 16, 10_000], 3, 7)


def test_plan_compiler_nesting_and_identity_operators():
    # Nesting has no limit (the compiler walks trees with explicit stacks, as
    # the reference's std::stack evaluation has none): 100000 nested NOTs
    # around one term, and a 20000-deep left chain (((t0 AND t1) OR t2) AND
    # t3) ... of distinct terms (more than a batch's position area holds: a
    # generic batch).
    n = 100_000
    data, offs = _plan([4] + [3] * n, list(range(n + 2)), list(range(7)))
    assert capi.SearchPlan(data, offs, 3, 7).num_queries == 1
    n = 20_000
    ops, cnt = [4], [0, 1]
    for i in range(1, n):
        ops += [4, 1 if i % 2 else 2]
        cnt += [cnt[-1] + 1, cnt[-1] + 3]
    data, offs = _plan(ops, cnt, list(range(7 * n)))
    assert capi.SearchPlan(data, offs, 3, 7).num_queries == 1
    # A negative child count pops nothing, as the reference's pop loop does
    # not run: AND/OR push their identity.
    data, offs = _plan([4, 1], [0, 1, -2], list(range(7)))
    assert capi.SearchPlan(data, offs, 3, 7).num_queries == 1


_BIG_PLAN_SCRIPT = r"""
import hashlib, sys
import numpy as np
from silvertorch_amd import capi, synthetic as S
cspec, qspec = S.CONFIGS["cfg3"]
queries = S.make_queries(cspec, qspec, seed=1)
_, data, offs = capi.parse_expression_query_batch(queries, cspec.hash_k, True, 5)
assert len(data) >= 192 * 1024, len(data)  # large enough for the parallel compile
plan = capi.SearchPlan(data, offs, cspec.k, cspec.hash_k)
w = 1600 + 40 * (np.arange(300) % 9)
plan.bind_widths(np.concatenate([[0], np.cumsum(w)]))
print(hashlib.sha256(plan.blob()).hexdigest())
"""


def test_plan_compiler_threads_give_identical_plans():
    """Large plans are compiled query by query on several host threads; the
    bound plan must not depend on their number or timing."""
    import os
    import subprocess
    import sys

    digests = set()
    for threads in ("1", "3", "8", "8"):
        env = dict(os.environ, ST_PLAN_THREADS=threads, PYTHONPATH=str(ROOT))
        out = subprocess.run([sys.executable, "-c", _BIG_PLAN_SCRIPT], env=env, cwd=ROOT,
                             capture_output=True, text=True, timeout=300)
        assert out.returncode == 0, out.stderr
        digests.add(out.stdout.strip())
    assert len(digests) == 1


def test_plan_compiler_reports_first_failing_query_of_a_large_plan():
    """With the parallel compile, the error raised is the one of the first
    malformed query, as in a query-by-query compile."""
    from silvertorch_amd import synthetic as S

    cspec, qspec = S.CONFIGS["cfg3"]
    queries = S.make_queries(cspec, qspec, seed=2)
    _, data, offs = capi.parse_expression_query_batch(queries, cspec.hash_k, True, 5)
    assert len(data) >= 192 * 1024
    data = bytearray(data)
    for q in (900, 700):  # an unknown operator code as the first op of each
        data[offs[8 * q]] = 9
    with pytest.raises(capi.StError, match="unknown operator: 9"):
        capi.SearchPlan(bytes(data), offs, cspec.k, cspec.hash_k)
    data[offs[8 * 700]] = 9
    bad = list(offs)
    bad[8 * 650 + 7] = len(data) + 8  # query 650's hash range runs past the data
    with pytest.raises(capi.StError, match="query plan 650"):
        capi.SearchPlan(bytes(data), bad, cspec.k, cspec.hash_k)


def test_torch_ops_schemas_and_cpu_parser():
    import torch

    import silvertorch_amd.ops._load_ops  # noqa: F401

    st = torch.ops.st
    schemas = {s.name: str(s) for s in torch._C._jit_get_all_schemas() if s.name.startswith("st::")}
    assert set(schemas) >= {"st::bloom_index_build", "st::bloom_index_search_batch",
                            "st::parse_expression_query_batch", "st::generate_column_info_for_clusters"}
    assert "bool fast_build=False" in schemas["st::bloom_index_build"]
    assert "bool return_bool_mask=True" in schemas["st::bloom_index_search_batch"]
    assert "int max_sub_queries=5" in schemas["st::parse_expression_query_batch"]
    g = G.parser_golden()
    m, (pd, po) = st.parse_expression_query_batch(g["expressions"], torch.ones(1, dtype=torch.long), 7, True, 5)
    want = next(b for b in g["batches"] if b["hash_k"] == 7 and b["max_sub_queries"] == 5)
    assert m == want["max_stack"]
    assert pd.dtype == torch.int8 and po.dtype == torch.int64
    assert pd.numpy().tobytes().hex() == want["data_hex"]
    with pytest.raises(RuntimeError, match="Unknown keyword"):
        st.parse_expression_query_batch(["1:1 XOR 2:2"], torch.ones(1, dtype=torch.long), 7)


def test_cpu_tensor_calls_fail_loudly_without_gpu():
    import torch

    import silvertorch_amd.ops._load_ops  # noqa: F401

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible; CPU-tensor calls run on it")
    c = G.case("readme")
    with pytest.raises(RuntimeError, match="no GPU is visible"):
        torch.ops.st.bloom_index_build(torch.from_numpy(c["ids"]), torch.from_numpy(c["offsets"]),
                                       torch.from_numpy(c["values"]), 5.0, 3)
    # argument errors come first, as in the reference CPU op (bloom_indexer.cpp:33-36)
    with pytest.raises(RuntimeError, match="b_multiplier must be greater than 1.0"):
        torch.ops.st.bloom_index_build(torch.from_numpy(c["ids"]), torch.from_numpy(c["offsets"]),
                                       torch.from_numpy(c["values"]), 1.0, 3)
    with pytest.raises(RuntimeError, match="unknown operator"):
        data, offs = _plan([9], [0, 0], [])
        torch.ops.st.bloom_index_search_batch(torch.from_numpy(c["index"]), torch.from_numpy(c["bundle_b_offsets"]),
                                              torch.frombuffer(bytearray(data), dtype=torch.int8),
                                              torch.tensor(offs, dtype=torch.long), 3, 7, False)


def test_partial_response_argument_errors_before_device_work():
    """The cluster-restricted op checks its arguments as the reference does
    (bloom_index_search.cpp:256-311) before any device work."""
    import torch

    import silvertorch_amd.ops._load_ops  # noqa: F401

    st = torch.ops.st
    idx = torch.zeros(64, dtype=torch.long)
    bbo = torch.tensor([0, 2], dtype=torch.long)
    pd = torch.zeros(8, dtype=torch.int8)
    po = torch.zeros(8, dtype=torch.long)
    co = torch.zeros((1, 1), dtype=torch.long)
    with pytest.raises(RuntimeError, match="selected_cluster_offsets dim must be 2"):
        st.bloom_index_search_batch_return_partial_response(idx, bbo, pd, po, co[0], co, 3, 7)
    with pytest.raises(RuntimeError, match="selected_cluster_lengths dtype must be Long"):
        st.bloom_index_search_batch_return_partial_response(idx, bbo, pd, po, co, co.int(), 3, 7)
    with pytest.raises(RuntimeError, match="must have same shape"):
        st.bloom_index_search_batch_return_partial_response(idx, bbo, pd, po, co, torch.zeros((1, 2), dtype=torch.long), 3, 7)
    with pytest.raises(RuntimeError, match="query_plan_index dim must be 1"):
        st.bloom_index_search_batch_return_partial_response(idx, bbo, pd, po, co, co, 3, 7, co)
    with pytest.raises(RuntimeError, match="list_bloom_index should not be empty"):
        st.bloom_index_search_batch_return_partial_response_multiple([], [], pd, po, [], [], 3, 7)
