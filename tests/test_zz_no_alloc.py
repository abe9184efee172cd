"""st_fused_kmean_ann_noalloc (the entry point that allocates nothing: its
per-(row, probe) counts live in the library's fixed device array) against
st_fused_kmean_ann with a caller workspace, through the C ABI: bit-identical
scores and indices on two calls in a row, the second smaller, filtered and
unfiltered; calls past the array's capacity are rejected; calls on two
streams do not race on the array."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from silvertorch_amd import capi
from tests import gpu_helpers as H

pytestmark = pytest.mark.gpu

MAX_PAIRS = 1 << 20


def _case(rng, batch, probes, dim, filtered):
    nclus = 40
    sizes = rng.integers(0, 3000, nclus)
    offs = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    n = int(offs[-1])
    emb = O.bf16_round(rng.standard_normal((n, dim)).astype(np.float32))
    q = O.bf16_round(rng.standard_normal((batch, dim)).astype(np.float32))
    cids = rng.integers(0, nclus, (batch, probes)).astype(np.int64)
    mask = rng.integers(-2**63, 2**63 - 1, (batch, n // 64 + 1), dtype=np.int64) if filtered else None
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return dict(offs=d(offs), cids=d(cids), clen=d(sizes[cids].astype(np.int64)), emb=d(emb), q=d(q),
                mask=d(mask) if filtered else None, n=n, batch=batch, probes=probes, dim=dim)


def _call(c, width, noalloc):
    L = capi.lib()
    B, P = c["batch"], c["probes"]
    sc = torch.full((B, width), 7, dtype=torch.int16, device="cuda")
    ix = torch.full((B, width), 7, dtype=torch.int32, device="cuda")
    m = c["mask"]
    args = [c["offs"].data_ptr(), c["offs"].numel(), c["cids"].data_ptr(), c["clen"].data_ptr(), B, P,
            c["emb"].data_ptr(), c["n"], c["dim"], 2, c["q"].data_ptr(), width,
            m.data_ptr() if m is not None else None, m.shape[0] if m is not None else 0,
            m.shape[1] if m is not None else 0, None, None, -1, -1]
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        rc = L.st_fused_kmean_ann_noalloc(*args, sc.data_ptr(), ix.data_ptr(), stream)
    else:
        ws = torch.empty(max(L.st_fused_kmean_ann_workspace_bytes(B, P), 1), dtype=torch.uint8, device="cuda")
        rc = L.st_fused_kmean_ann(*args, ws.data_ptr(), sc.data_ptr(), ix.data_ptr(), stream)
    capi.check(rc)
    torch.cuda.synchronize()
    return sc.cpu().numpy(), ix.cpu().numpy()


@pytest.mark.parametrize("filtered", [False, True])
def test_noalloc_matches_workspace_entry_point(filtered):
    rng = np.random.default_rng(31 + filtered)
    # each call smaller than the one before; the first (4,096 pairs) takes the
    # balanced form, whose group prefix also lives in the scratch array
    for batch, probes, width in ((512, 8, 3000), (48, 6, 6400), (5, 3, 96)):
        c = _case(rng, batch, probes, 64, filtered)
        H.note(f"[noalloc] filtered={filtered} batch={batch} probes={probes} width={width} docs={c['n']}")
        want_s, want_i = _call(c, width, noalloc=False)
        got_s, got_i = _call(c, width, noalloc=True)
        np.testing.assert_array_equal(got_i, want_i)
        np.testing.assert_array_equal(got_s, want_s)
        assert (want_i[:, 0] >= 0).any()


def test_noalloc_rejects_more_pairs_than_its_scratch():
    L = capi.lib()
    dummy = torch.zeros(64, dtype=torch.int64, device="cuda")
    p = dummy.data_ptr()
    stream = torch.cuda.current_stream().cuda_stream
    rc = L.st_fused_kmean_ann_noalloc(p, 2, p, p, MAX_PAIRS // 4 + 1, 4, p, 1, 8, 0, p, 32, None, 0, 0, None,
                                      None, -1, -1, p, p, stream)
    assert rc != 0 and b"exceeds" in L.st_last_error()
    # no probes: no counts needed, any batch is accepted (all padding)
    sc = torch.empty((2, 32), dtype=torch.float32, device="cuda")
    ix = torch.empty((2, 32), dtype=torch.int32, device="cuda")
    q = torch.zeros((2, 8), dtype=torch.float32, device="cuda")
    capi.check(L.st_fused_kmean_ann_noalloc(p, 2, None, None, 2, 0, p, 1, 8, 0, q.data_ptr(), 32, None, 0, 0,
                                            None, None, -1, -9, sc.data_ptr(), ix.data_ptr(), stream))
    torch.cuda.synchronize()
    assert (ix.cpu() == -9).all()


def test_noalloc_calls_on_two_streams_do_not_race():
    """Two calls on two streams, issued back to back without any ordering by
    the caller: the second waits for the first (the shared scratch array),
    so both equal the workspace entry point's results."""
    rng = np.random.default_rng(77)
    a = _case(rng, 512, 8, 64, True)
    b = _case(rng, 300, 7, 64, False)
    want_a = _call(a, 3000, noalloc=False)
    want_b = _call(b, 2000, noalloc=False)
    L = capi.lib()
    outs = []
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    H.note("[noalloc] two streams")
    bufs = [(torch.full((c["batch"], w), 7, dtype=torch.int16, device="cuda"),
             torch.full((c["batch"], w), 7, dtype=torch.int32, device="cuda")) for c, w in ((a, 3000), (b, 2000))]
    torch.cuda.synchronize()  # the outputs' fills are done before either stream writes them
    for (c, width, s), (sc, ix) in zip(((a, 3000, s1), (b, 2000, s2)), bufs):
        B, P = c["batch"], c["probes"]
        m = c["mask"]
        capi.check(L.st_fused_kmean_ann_noalloc(
            c["offs"].data_ptr(), c["offs"].numel(), c["cids"].data_ptr(), c["clen"].data_ptr(), B, P,
            c["emb"].data_ptr(), c["n"], c["dim"], 2, c["q"].data_ptr(), width,
            m.data_ptr() if m is not None else None, m.shape[0] if m is not None else 0,
            m.shape[1] if m is not None else 0, None, None, -1, -1, sc.data_ptr(), ix.data_ptr(),
            s.cuda_stream))
        outs.append((sc, ix))
    torch.cuda.synchronize()
    for (sc, ix), (ws, wi) in zip(outs, (want_a, want_b)):
        np.testing.assert_array_equal(ix.cpu().numpy(), wi)
        np.testing.assert_array_equal(sc.cpu().numpy(), ws)
