"""GPU parity of take_top_k_and_gather_from_main_and_fresh
(fresh_index_post_processing.cpp:231-270 of the reference):

* the op through torch.ops.st on GPU tensors (and on CPU tensors, which run
  on the GPU) against the fixtures the reference CPU op wrote
  (tests/golden/ref_fresh.npz, distinct scores per row), bit for bit: top
  scores, merged indices, is_from_fresh, every gathered tensor; one case
  keeps more than 8192 entries (the kept list in global memory);
* the C ABI (st_fresh_topk / st_fresh_gather) against the oracle on
  tie-heavy rows, NaN and signed zeros, every score type, both index types,
  long rows and large k (the order of equal scores, which at::topk leaves
  open, is the lower merged index first);
* the reference's argument errors.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from silvertorch_amd import capi
from tests import _fixtures as G
from tests import gpu_helpers as H

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _ops():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    import silvertorch_amd.ops._load_ops  # noqa: F401


def _t(c, path, a):
    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.view(torch.bfloat16) if path in c["bf16"] else t


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    return t.numpy().view(np.uint8)


def _run_fixture(name, device):
    c = G.fresh_case(name)
    keys = c["keys"]
    args = [_t(c, "main_scores", c["main_scores"]), _t(c, "fresh_scores", c["fresh_scores"]),
            torch.from_numpy(c["main_indices"]), torch.from_numpy(c["fresh_indices"])]
    md = [_t(c, f"main_data/{k}", c["main_data"][k]) for k in keys]
    fd = [_t(c, f"fresh_data/{k}", c["fresh_data"][k]) for k in keys]
    if device == "cuda":
        args = [a.cuda() for a in args]
        md = [a.cuda() for a in md]
        fd = [a.cuda() for a in fd]
    H.note(f"[fresh] case={name} device={device} rows={args[0].shape[0]} k={c['k']}")
    ts, ti, ff, g = torch.ops.st.take_top_k_and_gather_from_main_and_fresh(*args, c["k"], keys, md, fd, 2)
    assert ts.device.type == device and ti.dtype == torch.int64 and ff.dtype == torch.bool
    np.testing.assert_array_equal(ti.cpu().numpy(), c["top_indices"])
    np.testing.assert_array_equal(ff.cpu().numpy(), c["is_from_fresh"])
    np.testing.assert_array_equal(_bits(ts), c["top_scores"].view(np.uint8))
    assert sorted(g.keys()) == sorted(keys)
    for k in keys:
        want = c["gathered"][k]
        assert tuple(g[k].shape) == want.shape, (k, tuple(g[k].shape), want.shape)
        np.testing.assert_array_equal(_bits(g[k]), want.view(np.uint8), err_msg=k)


@pytest.mark.parametrize("name", G.fresh_case_names())
def test_op_matches_reference_fixtures(name):
    _run_fixture(name, "cuda")


@pytest.mark.parametrize("name", ["readme_int64_k7", "bf16_k_clamped", "f32_k_global"])
def test_op_on_cpu_tensors_matches_reference_fixtures(name):
    _run_fixture(name, "cpu")


_NP = {"float32": np.float32, "float16": np.float16, "float64": np.float64, "int64": np.int64, "int32": np.int32,
       "int16": np.int16, "int8": np.int8, "uint8": np.uint8}


def _capi_topk(ms, fs, k, stype):
    """st_fresh_topk through the C ABI on device copies of ms / fs."""
    L = capi.lib()
    R, Nm = ms.shape
    Nf = fs.shape[1]
    tdt = {"bfloat16": torch.bfloat16}.get(stype) or getattr(torch, stype)
    ms_d, fs_d = ms.to(tdt).cuda().contiguous(), fs.to(tdt).cuda().contiguous()
    ts = torch.empty((R, k), dtype=tdt, device="cuda")
    ti = torch.empty((R, k), dtype=torch.int64, device="cuda")
    ff = torch.empty((R, k), dtype=torch.uint8, device="cuda")
    ws = torch.empty(max(1, L.st_fresh_topk_workspace_bytes(R, k)), dtype=torch.uint8, device="cuda")
    capi.check(L.st_fresh_topk(ms_d.data_ptr() if Nm else None, fs_d.data_ptr() if Nf else None,
                               capi.FRESH_SCORE_TYPES[stype], R, Nm, Nf, k, ws.data_ptr(), ts.data_ptr(),
                               ti.data_ptr(), ff.data_ptr(), H._stream()))
    torch.cuda.synchronize()
    return ts.cpu(), ti.cpu().numpy(), ff.cpu().numpy().astype(bool)


@pytest.mark.parametrize("stype", ["float32", "float16", "bfloat16", "float64", "int64", "int32", "int16",
                                   "int8", "uint8"])
@pytest.mark.parametrize("rows,nf,nm,k,levels", [
    (5, 30, 70, 25, 6),          # heavy ties
    (3, 0, 500, 500, 4),         # main only, k = the whole row
    (4, 1001, 2999, 1000, 30),   # 1,024 kept: sorted runs merged; parts not multiples of 4
    (4, 1000, 3000, 1000, 12),   # the same with 16-byte score loads (4-byte types)
    (4, 2000, 0, 64, 50),        # fresh only
    (2, 3000, 9000, 9000, 40),   # kept list in global memory, ties
    (3, 6000, 10384, 4096, 30),  # the largest row and k of the register selection
    (2, 8000, 8385, 3000, 20),   # one entry more: the streaming merge, kept list in LDS
    (9, 1, 1, 1, 2),
])
def test_capi_topk_ties_vs_oracle(stype, rows, nf, nm, k, levels):
    rng = np.random.default_rng(rows * 1000 + nf + nm + k)
    lo = 0 if stype == "uint8" else -levels // 2
    ms = torch.from_numpy(rng.integers(lo, lo + levels, (rows, nm)).astype(np.float64))
    fs = torch.from_numpy(rng.integers(lo, lo + levels, (rows, nf)).astype(np.float64))
    if stype.startswith("float") or stype == "bfloat16":
        ms = ms / 4
        fs = fs / 4
    H.note(f"[fresh capi] {stype} rows={rows} nf={nf} nm={nm} k={k}")
    ts, ti, ff = _capi_topk(ms, fs, k, stype)
    tdt = {"bfloat16": torch.bfloat16}.get(stype) or getattr(torch, stype)
    ms_v, fs_v = ms.to(tdt), fs.to(tdt)
    to_np = (lambda t: t.float().numpy()) if stype == "bfloat16" else (lambda t: t.numpy())
    ws, wi, wf, _ = O.fresh_topk_gather(to_np(ms_v), to_np(fs_v), None, None, k, [], [])
    np.testing.assert_array_equal(ti, wi)
    np.testing.assert_array_equal(ff, wf)
    np.testing.assert_array_equal(to_np(ts), ws)


def test_capi_topk_nan_and_signed_zeros():
    ms = torch.tensor([[0.5, float("nan"), -0.0, 1.0, float("-inf"), 0.0, float("nan")]], dtype=torch.float32)
    fs = torch.tensor([[0.0, float("inf"), -1.0]], dtype=torch.float32)
    for stype in ("float32", "float16", "bfloat16", "float64"):
        ts, ti, ff = _capi_topk(ms, fs, 10, stype)
        ws, wi, wf, _ = O.fresh_topk_gather(ms.numpy(), fs.numpy(), None, None, 10, [], [])
        np.testing.assert_array_equal(ti, wi, err_msg=stype)
        assert ti[0].tolist() == [4, 9, 1, 6, 3, 0, 5, 8, 2, 7], (stype, ti)
        np.testing.assert_array_equal(ff, wf)


@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
def test_op_gather_dtypes_and_clamping_vs_oracle(index_dtype):
    rng = np.random.default_rng(11)
    R, nf, nm, k = 6, 40, 90, 70
    ms = torch.from_numpy(rng.standard_normal((R, nm)).astype(np.float32))
    fs = torch.from_numpy(rng.standard_normal((R, nf)).astype(np.float32))
    mi = torch.from_numpy(rng.integers(-3, 33, (R, nm))).to(index_dtype)
    fi = torch.from_numpy(rng.integers(-3, 13, (R, nf))).to(index_dtype)
    datas = {"u8": torch.from_numpy(rng.integers(0, 255, (30,)).astype(np.uint8)),
             "f64": torch.from_numpy(rng.standard_normal((30, 3))),
             "bf": torch.from_numpy(rng.standard_normal((30, 7)).astype(np.float32)).to(torch.bfloat16),
             "i16": torch.from_numpy(rng.integers(-999, 999, (30, 2)).astype(np.int16)),
             "empty_main": torch.zeros((0, 4), dtype=torch.float32)}
    fresh = {"u8": datas["u8"][:10], "f64": datas["f64"][:10], "bf": datas["bf"][:10], "i16": datas["i16"][:10],
             "empty_main": torch.ones((10, 4), dtype=torch.float32)}
    keys = list(datas)
    ts, ti, ff, g = torch.ops.st.take_top_k_and_gather_from_main_and_fresh(
        ms.cuda(), fs.cuda(), mi.cuda(), fi.cuda(), k, keys, [datas[x].cuda() for x in keys],
        [fresh[x].cuda() for x in keys], 1)
    conv = lambda t: t.float().numpy() if t.dtype == torch.bfloat16 else t.numpy()  # noqa: E731
    _, wi, _, wg = O.fresh_topk_gather(ms.numpy(), fs.numpy(), mi.numpy(), fi.numpy(), k,
                                       [conv(datas[x]) if x != "empty_main" else np.zeros((1, 4), np.float32)
                                        for x in keys], [conv(fresh[x]) for x in keys])
    np.testing.assert_array_equal(ti.cpu().numpy(), wi)
    for x, w in zip(keys, wg):
        got = g[x].cpu()
        if x == "empty_main":  # an empty data tensor gives zeros (the reference reads out of bounds)
            assert got.shape == (R * k, 4)
            from_main = ~(ti.cpu().numpy().reshape(-1) < nf)
            assert (got.numpy()[from_main] == 0).all()
            np.testing.assert_array_equal(got.numpy()[~from_main], w[~from_main])
            continue
        np.testing.assert_array_equal(conv(got), w, err_msg=x)


def test_op_gather_many_keys_wide_rows_and_unaligned_data_vs_oracle():
    """Ten keys, rows of 2,400 bytes (150 16-byte units), rows whose data
    pointer is only 2-byte aligned (2-byte units), 1-byte rows, a dim-0
    tensor, int64 ids."""
    rng = np.random.default_rng(23)
    R, nf, nm, k = 5, 30, 70, 40
    ms = torch.from_numpy(rng.standard_normal((R, nm)).astype(np.float32))
    fs = torch.from_numpy(rng.standard_normal((R, nf)).astype(np.float32))
    mi = torch.from_numpy(rng.integers(-2, 25, (R, nm)))
    fi = torch.from_numpy(rng.integers(-2, 9, (R, nf)))

    def unaligned_bf16(rows, dim):  # contiguous, data pointer 2 bytes past a 16-byte boundary
        base = torch.from_numpy(rng.standard_normal(rows * dim + 1).astype(np.float32)).to(torch.bfloat16).cuda()
        return base[1:].view(rows, dim)

    main = {"wide": torch.from_numpy(rng.standard_normal((24, 600)).astype(np.float32)).cuda(),
            "bf_odd": unaligned_bf16(24, 7),
            "u8": torch.from_numpy(rng.integers(0, 255, (24,)).astype(np.uint8)).cuda(),
            "ids": torch.from_numpy(rng.integers(0, 2**40, (24,))).cuda(),
            "zero": torch.zeros((24, 0), dtype=torch.float32).cuda()}
    fresh = {"wide": torch.from_numpy(rng.standard_normal((8, 600)).astype(np.float32)).cuda(),
             "bf_odd": unaligned_bf16(8, 7),
             "u8": torch.from_numpy(rng.integers(0, 255, (8,)).astype(np.uint8)).cuda(),
             "ids": torch.from_numpy(rng.integers(0, 2**40, (8,))).cuda(),
             "zero": torch.zeros((8, 0), dtype=torch.float32).cuda()}
    for j in range(5):
        main[f"i32_{j}"] = torch.from_numpy(rng.integers(-99, 99, (24, j + 1)).astype(np.int32)).cuda()
        fresh[f"i32_{j}"] = torch.from_numpy(rng.integers(-99, 99, (8, j + 1)).astype(np.int32)).cuda()
    keys = list(main)
    assert len(keys) == 10 and main["bf_odd"].data_ptr() % 16 == 2
    _, ti, _, g = torch.ops.st.take_top_k_and_gather_from_main_and_fresh(
        ms.cuda(), fs.cuda(), mi.cuda(), fi.cuda(), k, keys, [main[x] for x in keys],
        [fresh[x] for x in keys], 1)
    conv = lambda t: t.float().cpu().numpy() if t.dtype == torch.bfloat16 else t.cpu().numpy()  # noqa: E731
    _, wi, _, wg = O.fresh_topk_gather(ms.numpy(), fs.numpy(), mi.numpy(), fi.numpy(), k,
                                       [conv(main[x]) for x in keys], [conv(fresh[x]) for x in keys])
    np.testing.assert_array_equal(ti.cpu().numpy(), wi)
    for x, w in zip(keys, wg):
        got = conv(g[x])
        assert got.shape == tuple(w.shape), x
        np.testing.assert_array_equal(got, w, err_msg=x)


def test_op_argument_errors():
    st = torch.ops.st
    ms = torch.rand(2, 5, device="cuda")
    fs = torch.rand(2, 3, device="cuda")
    mi = torch.zeros(2, 5, dtype=torch.long, device="cuda")
    fi = torch.zeros(2, 3, dtype=torch.long, device="cuda")
    d = torch.arange(5, device="cuda")
    with pytest.raises(RuntimeError, match="keys and list_main_data should have the same size"):
        st.take_top_k_and_gather_from_main_and_fresh(ms, fs, mi, fi, 3, ["a", "b"], [d], [d])
    with pytest.raises(RuntimeError, match="keys and list_fresh_data should have the same size"):
        st.take_top_k_and_gather_from_main_and_fresh(ms, fs, mi, fi, 3, ["a"], [d], [d, d])
    with pytest.raises(RuntimeError, match="should have the same dim"):
        st.take_top_k_and_gather_from_main_and_fresh(ms, fs, mi, fi, 3, ["a"], [d], [d.view(5, 1)])
    with pytest.raises(RuntimeError, match="same number of element in the last dim"):
        st.take_top_k_and_gather_from_main_and_fresh(ms, fs, mi, fi, 3, ["a"], [d.view(5, 1)],
                                                     [torch.zeros(5, 2, dtype=d.dtype, device="cuda")])
    with pytest.raises(RuntimeError, match="should have the same scalar_type"):
        st.take_top_k_and_gather_from_main_and_fresh(ms, fs, mi, fi, 3, ["a"], [d], [d.float()])
    with pytest.raises(RuntimeError, match=r"The main data dim must be in \[1, 2\]"):
        st.take_top_k_and_gather_from_main_and_fresh(ms, fs, mi, fi, 3, ["a"], [d.view(1, 5, 1)],
                                                     [d.view(1, 5, 1)])
    with pytest.raises(RuntimeError, match="not implemented for 'Bool'"):
        b = torch.zeros(5, dtype=torch.bool, device="cuda")
        st.take_top_k_and_gather_from_main_and_fresh(ms, fs, mi, fi, 3, ["a"], [b], [b])
    with pytest.raises(RuntimeError, match="k out of range"):
        st.take_top_k_and_gather_from_main_and_fresh(ms, fs, mi, fi, -1, [], [], [])
    with pytest.raises(RuntimeError, match="expected scalar type"):
        st.take_top_k_and_gather_from_main_and_fresh(ms, fs, mi, fi.int(), 3, ["a"], [d], [d])
    # promotion of mixed score dtypes, as at::cat does
    ts, ti, _, _ = st.take_top_k_and_gather_from_main_and_fresh(ms.half(), fs, mi, fi, 8, [], [], [])
    assert ts.dtype == torch.float32 and ti.shape == (2, 8)
