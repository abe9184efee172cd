"""Drives the C ABI (include/silvertorch_hip.h) with torch device tensors."""

from __future__ import annotations

import sys

import numpy as np
import torch

from silvertorch_amd import capi


def note(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def build(ids, offsets, values, b_multiplier: float, k: int):
    """C-ABI build -> (index, bundle_b_offsets) as numpy arrays."""
    L = capi.lib()
    ids_d = torch.as_tensor(np.ascontiguousarray(ids, dtype=np.int32)).cuda()
    off_d = torch.as_tensor(np.ascontiguousarray(offsets, dtype=np.int64)).cuda()
    val_d = torch.as_tensor(np.ascontiguousarray(values, dtype=np.int64)).cuda()
    F = ids_d.numel()
    n = (off_d.numel() - 1) // F
    nb = (n + 2047) // 2048
    bbo = torch.empty(nb + 1, dtype=torch.long, device="cuda")
    stats = torch.empty(6, dtype=torch.long, device="cuda")
    capi.check(L.st_bloom_build_bundle_offsets(off_d.data_ptr(), n, F, k, b_multiplier, bbo.data_ptr(),
                                               stats.data_ptr(), _stream()))
    s = stats.cpu().tolist()
    assert s[2] == 0 and 0 <= s[3] <= s[4] <= val_d.numel(), s
    index = torch.empty(s[0] * 32, dtype=torch.long, device="cuda")
    capi.check(L.st_bloom_index_build(ids_d.data_ptr(), off_d.data_ptr(),
                                      val_d.data_ptr() if val_d.numel() else None, F, n, val_d.numel(), k,
                                      bbo.data_ptr(), s[1], index.data_ptr() if index.numel() else None,
                                      index.numel(), _stream()))
    torch.cuda.synchronize()
    return index.cpu().numpy(), bbo.cpu().numpy()


def search(index, bbo, plans_data, plans_offsets, k: int, hash_k: int, bool_mask: bool = False,
           bind: str | None = None, upload: bool = False):
    """C-ABI search; index / bbo may be numpy arrays or cuda tensors.  bind:
    "host" (st_search_plan_bind_widths), "device"
    (st_search_plan_prepare_device_binding) or "none"; with bind=None all
    three run and must agree."""
    if bind is None:
        a = search(index, bbo, plans_data, plans_offsets, k, hash_k, bool_mask, "host")
        for mode in ("device", "none"):
            b = search(index, bbo, plans_data, plans_offsets, k, hash_k, bool_mask, mode)
            np.testing.assert_array_equal(a, b, err_msg=f"host-bound and {mode} plans disagree")
        return a
    L = capi.lib()
    idx_d = index if isinstance(index, torch.Tensor) else torch.as_tensor(np.ascontiguousarray(index, np.int64)).cuda()
    bbo_d = bbo if isinstance(bbo, torch.Tensor) else torch.as_tensor(np.ascontiguousarray(bbo, np.int64)).cuda()
    plan = capi.SearchPlan(bytes(np.asarray(plans_data, dtype=np.int8).tobytes()), plans_offsets, k, hash_k)
    nb = bbo_d.numel() - 1
    if bind == "host":
        plan.bind_widths(bbo_d.cpu().numpy())
    elif bind == "device":
        plan.prepare_device_binding(nb)
    blob = plan.blob()
    blob_d = None
    pinned = None
    if blob and upload:  # the search call copies the blob from pinned memory itself
        pinned = torch.frombuffer(bytearray(blob), dtype=torch.uint8).pin_memory()
        capi.check(L.st_search_plan_upload_source(plan.handle, pinned.data_ptr()))
        blob_d = torch.full((plan.device_bytes,), 0xEE, dtype=torch.uint8, device="cuda")
    elif blob:
        blob_d = torch.zeros(plan.device_bytes, dtype=torch.uint8, device="cuda")
        blob_d[:len(blob)] = torch.frombuffer(bytearray(blob), dtype=torch.uint8).cuda()
    q = plan.num_queries
    if bool_mask:
        out = torch.empty((q, nb * 2048), dtype=torch.bool, device="cuda")
    else:
        out = torch.empty((q, nb * 32), dtype=torch.long, device="cuda")
    capi.check(L.st_bloom_index_search_batch(idx_d.data_ptr() if idx_d.numel() else None, idx_d.numel(),
                                             bbo_d.data_ptr(), nb, plan.handle,
                                             blob_d.data_ptr() if blob_d is not None else None,
                                             int(bool_mask), out.data_ptr() if out.numel() else None, _stream()))
    torch.cuda.synchronize()
    return out.cpu().numpy()


def compact(packed, num_docs: int, int64_ids: bool = False):
    """C-ABI compaction of a packed mask -> (ids, row_offsets) as numpy arrays."""
    L = capi.lib()
    p = packed if isinstance(packed, torch.Tensor) else torch.as_tensor(np.ascontiguousarray(packed, np.int64)).cuda()
    q, c = p.shape
    ro = torch.empty(q + 1, dtype=torch.long, device="cuda")
    ws = torch.empty(max(L.st_bloom_compact_workspace_bytes(q, c), 1), dtype=torch.uint8, device="cuda")
    capi.check(L.st_bloom_compact_offsets(p.data_ptr() if p.numel() else None, q, c, num_docs,
                                          ws.data_ptr(), ro.data_ptr(), _stream()))
    total = int(ro[q].item())
    ids = torch.empty(total, dtype=torch.long if int64_ids else torch.int32, device="cuda")
    capi.check(L.st_bloom_compact_ids(p.data_ptr() if p.numel() else None, q, c, num_docs, ws.data_ptr(),
                                      ids.data_ptr() if total else None, int(int64_ids), _stream()))
    torch.cuda.synchronize()
    return ids.cpu().numpy(), ro.cpu().numpy()


def search_ids(index, bbo, plans_data, plans_offsets, k: int, hash_k: int, num_docs: int,
               int64_ids: bool = False):
    """Fused search + count (st_bloom_index_search_batch_counts), then the id
    writes -> (ids, row_offsets, packed) as numpy arrays."""
    L = capi.lib()
    idx_d = torch.as_tensor(np.ascontiguousarray(index, np.int64)).cuda()
    bbo_d = torch.as_tensor(np.ascontiguousarray(bbo, np.int64)).cuda()
    plan = capi.SearchPlan(bytes(np.asarray(plans_data, dtype=np.int8).tobytes()), plans_offsets, k, hash_k)
    plan.bind_widths(bbo_d.cpu().numpy())
    blob = plan.blob()
    blob_d = torch.frombuffer(bytearray(blob), dtype=torch.uint8).cuda() if blob else None
    q, nb = plan.num_queries, bbo_d.numel() - 1
    packed = torch.empty((q, nb * 32), dtype=torch.long, device="cuda")
    ro = torch.empty(q + 1, dtype=torch.long, device="cuda")
    ws = torch.empty(max(L.st_bloom_compact_workspace_bytes(q, nb * 32), 1), dtype=torch.uint8, device="cuda")
    capi.check(L.st_bloom_index_search_batch_counts(
        idx_d.data_ptr() if idx_d.numel() else None, idx_d.numel(), bbo_d.data_ptr(), nb, plan.handle,
        blob_d.data_ptr() if blob_d is not None else None, num_docs,
        packed.data_ptr() if packed.numel() else None, ws.data_ptr(), ro.data_ptr(), _stream()))
    total = int(ro[q].item())
    ids = torch.empty(total, dtype=torch.long if int64_ids else torch.int32, device="cuda")
    if total:
        capi.check(L.st_bloom_compact_ids(packed.data_ptr(), q, nb * 32, num_docs, ws.data_ptr(),
                                          ids.data_ptr(), int(int64_ids), _stream()))
    torch.cuda.synchronize()
    return ids.cpu().numpy(), ro.cpu().numpy(), packed.cpu().numpy()
