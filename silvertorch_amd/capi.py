"""ctypes binding of the C ABI (include/silvertorch_hip.h).

This is the binding a non-torch caller would write; the parity tests use it
to drive the HIP library directly with device pointers.  Loading fails loudly
when the library has not been built.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libsilvertorch_hip.so"

_i64 = ctypes.c_int64
_i64p = ctypes.POINTER(ctypes.c_int64)
_vp = ctypes.c_void_p

# name -> (restype, argtypes); mirrors include/silvertorch_hip.h
SIGNATURES = {
    "st_last_error": (ctypes.c_char_p, []),
    "st_version": (ctypes.c_char_p, []),
    "st_murmur_hash3_2x64": (ctypes.c_uint64, [ctypes.c_uint64] * 3),
    "st_bloom_build_bundle_offsets": (ctypes.c_int, [_vp, _i64, _i64, _i64, ctypes.c_double, _vp, _vp, _vp]),
    "st_bloom_index_build": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp]),
    "st_search_plan_create": (ctypes.c_int, [_vp, _i64, _vp, _i64, _i64, _i64, ctypes.POINTER(_vp)]),
    "st_search_plan_bind_widths": (ctypes.c_int, [_vp, _vp, _i64]),
    "st_search_plan_prepare_device_binding": (ctypes.c_int, [_vp, _i64]),
    "st_search_plan_device_bytes": (_i64, [_vp]),
    "st_search_plan_upload_source": (ctypes.c_int, [_vp, _vp]),
    "st_search_plan_upload_signal": (ctypes.c_int, [_vp, _vp, ctypes.c_uint64]),
    "st_search_plan_upload_groups": (_i64, [_vp]),
    "st_search_plan_num_queries": (_i64, [_vp]),
    "st_search_plan_blob_bytes": (_i64, [_vp]),
    "st_search_plan_blob": (_vp, [_vp]),
    "st_search_plan_destroy": (None, [_vp]),
    "st_bloom_index_search_batch": (ctypes.c_int, [_vp, _i64, _vp, _i64, _vp, _vp, ctypes.c_int, _vp, _vp]),
    "st_parse_expression_query_batch": (ctypes.c_int, [ctypes.POINTER(ctypes.c_char_p), _i64, _i64, ctypes.c_int, _i64, ctypes.POINTER(_vp)]),
    "st_parsed_plans_max_stack": (_i64, [_vp]),
    "st_parsed_plans_data_bytes": (_i64, [_vp]),
    "st_parsed_plans_data": (_vp, [_vp]),
    "st_parsed_plans_offsets_len": (_i64, [_vp]),
    "st_parsed_plans_offsets": (_vp, [_vp]),
    "st_parsed_plans_destroy": (None, [_vp]),
    "st_generate_column_info_for_clusters": (ctypes.c_int, [_vp, _vp, _i64, _vp, _vp, _vp, _vp]),
    "st_bloom_compact_workspace_bytes": (_i64, [_i64, _i64]),
    "st_bloom_compact_offsets": (ctypes.c_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp]),
    "st_bloom_compact_ids": (ctypes.c_int, [_vp, _i64, _i64, _i64, _vp, _vp, ctypes.c_int, _vp]),
    "st_filtered_topk_workspace_bytes": (_i64, [_i64]),
    "st_filtered_topk": (ctypes.c_int, [_vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _vp, _vp, _vp, _vp]),
    "st_kmean_ann_score_dtype": (ctypes.c_int, [ctypes.c_int, _i64, ctypes.c_int]),
    "st_fused_kmean_ann_workspace_bytes": (_i64, [_i64, _i64]),
    "st_fused_kmean_ann": (ctypes.c_int, [_vp, _i64, _vp, _vp, _i64, _i64, _vp, _i64, _i64, ctypes.c_int,
                                          _vp, _i64, _vp, _i64, _i64, _vp, _vp, _i64, _i64, _vp, _vp, _vp,
                                          _vp]),
    "st_fused_kmean_ann_noalloc": (ctypes.c_int, [_vp, _i64, _vp, _vp, _i64, _i64, _vp, _i64, _i64, ctypes.c_int,
                                                  _vp, _i64, _vp, _i64, _i64, _vp, _vp, _i64, _i64, _vp, _vp,
                                                  _vp]),
    "st_bloom_index_search_batch_counts": (ctypes.c_int, [_vp, _i64, _vp, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _vp]),
    "st_search_plan_partial_items": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _vp, _i64, _vp, _vp, _vp,
                                                    _i64p, _i64p]),
    "st_bloom_index_search_partial": (ctypes.c_int, [_vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _vp]),
    "st_fresh_topk_workspace_bytes": (_i64, [_i64, _i64]),
    "st_fresh_topk": (ctypes.c_int, [_vp, _vp, ctypes.c_int, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp]),
    "st_fresh_gather": (ctypes.c_int, [_vp, _i64, _i64, _vp, _vp, ctypes.c_int, _i64, _i64, _i64, _i64, _vp, _i64,
                                       _vp, _i64, _i64, ctypes.c_int, _vp, _vp]),
}

# score type codes of st_fresh_topk (ST_SCORE_*)
FRESH_SCORE_TYPES = {"float32": 0, "float16": 1, "bfloat16": 2, "float64": 3, "int64": 4, "int32": 5,
                     "int16": 6, "int8": 7, "uint8": 8}

# struct st_partial_item (include/silvertorch_hip.h)
PARTIAL_ITEM_BYTES = 32

_lib = None


class StError(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m silvertorch_amd._build` "
                "(silvertorch_amd has no CPU fallback)")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        raise StError(lib().st_last_error().decode(errors="replace"))


def parse_expression_query_batch(expressions, hash_k: int, return_query_plan: bool = True,
                                 max_sub_queries: int = 5):
    """-> (max_stack, plans_data bytes, plans_offsets list[int])."""
    L = lib()
    arr = (ctypes.c_char_p * max(len(expressions), 1))(*[e.encode() for e in expressions])
    out = _vp()
    check(L.st_parse_expression_query_batch(arr, len(expressions), hash_k, int(return_query_plan),
                                            max_sub_queries, ctypes.byref(out)))
    try:
        n = L.st_parsed_plans_data_bytes(out)
        m = L.st_parsed_plans_offsets_len(out)
        data = ctypes.string_at(L.st_parsed_plans_data(out), n) if n else b""
        offs = list((ctypes.c_int64 * m).from_address(L.st_parsed_plans_offsets(out))) if m else []
        return int(L.st_parsed_plans_max_stack(out)), data, offs
    finally:
        L.st_parsed_plans_destroy(out)


class SearchPlan:
    """Owns an st_search_plan compiled from host plan arrays."""

    def __init__(self, plans_data: bytes, plans_offsets, k: int, hash_k: int):
        import numpy as np

        self._data = np.frombuffer(bytes(plans_data), dtype=np.int8).copy()
        self._offs = np.ascontiguousarray(plans_offsets, dtype=np.int64)
        self.handle = _vp()
        check(lib().st_search_plan_create(
            self._data.ctypes.data if self._data.size else None, self._data.size,
            self._offs.ctypes.data if self._offs.size else None, self._offs.size,
            k, hash_k, ctypes.byref(self.handle)))

    def bind_widths(self, bundle_b_offsets) -> None:
        import numpy as np

        self._bbo = np.ascontiguousarray(bundle_b_offsets, dtype=np.int64)
        check(lib().st_search_plan_bind_widths(self.handle, self._bbo.ctypes.data, self._bbo.size - 1))

    def prepare_device_binding(self, num_bundles: int) -> None:
        check(lib().st_search_plan_prepare_device_binding(self.handle, num_bundles))

    @property
    def device_bytes(self) -> int:
        return int(lib().st_search_plan_device_bytes(self.handle))

    @property
    def num_queries(self) -> int:
        return int(lib().st_search_plan_num_queries(self.handle))

    def blob(self) -> bytes:
        n = lib().st_search_plan_blob_bytes(self.handle)
        return ctypes.string_at(lib().st_search_plan_blob(self.handle), n) if n else b""

    def __del__(self):
        h = getattr(self, "handle", None)
        if h and _lib is not None:
            _lib.st_search_plan_destroy(h)
        self.handle = None
