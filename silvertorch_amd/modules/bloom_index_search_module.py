"""Bloom index search as an nn.Module (reference:
silvertorch/modules/bloom_index_search_module.py:22-72)."""

from __future__ import annotations

import torch
import torch.nn as nn

import silvertorch_amd.ops._load_ops  # noqa: F401  (registers torch.ops.st)


class BloomIndexSearchModule(nn.Module):
    """Holds a bloom index and its bundle offsets as buffers (so they follow
    ``.to(device)`` and ``state_dict``; a saved index loads into a new module)
    and searches it with encoded query plans.

    Args:
        k: row positions per term in the search (``k`` of
            ``bloom_index_search_batch``).
        hash_k: hashes carried per term by the plans.
    """

    def __init__(self, k: int, hash_k: int) -> None:
        super().__init__()
        self.k = k
        self.hash_k = hash_k
        self.register_buffer("bloom_index", torch.empty(0, dtype=torch.int64))
        self.register_buffer("bloom_bundle_b_offsets", torch.empty(0, dtype=torch.int64))

    def set_bloom_index(self, bloom_index: torch.Tensor) -> None:
        self.bloom_index = bloom_index

    def set_bloom_bundle_b_offsets(self, bloom_bundle_b_offsets: torch.Tensor) -> None:
        self.bloom_bundle_b_offsets = bloom_bundle_b_offsets

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                              unexpected_keys, error_msgs):
        # The index buffers take the saved index's size, so a persisted index
        # loads into a freshly constructed module (whose buffers are empty);
        # they stay on the module's device.
        for name in ("bloom_index", "bloom_bundle_b_offsets"):
            saved = state_dict.get(prefix + name)
            cur = getattr(self, name)
            if isinstance(saved, torch.Tensor) and saved.shape != cur.shape:
                setattr(self, name, torch.empty(saved.shape, dtype=cur.dtype, device=cur.device))
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys,
                                      unexpected_keys, error_msgs)

    def forward(self, bloom_query_plans_data: torch.Tensor, bloom_query_plans_offsets: torch.Tensor,
                return_bool_mask: bool = True) -> torch.Tensor:
        """Searches every plan over every doc column: bool[Q, 2048 nb] when
        ``return_bool_mask``, else the packed int64[Q, 32 nb] words."""
        return torch.ops.st.bloom_index_search_batch(
            self.bloom_index, self.bloom_bundle_b_offsets, bloom_query_plans_data,
            bloom_query_plans_offsets, self.k, self.hash_k, return_bool_mask)
