"""Builder of BloomIndexSearchModule (reference:
silvertorch/modules/bloom_index_search_module_builder.py:22-116)."""

from __future__ import annotations

import torch

import silvertorch_amd.ops._load_ops  # noqa: F401  (registers torch.ops.st)
from silvertorch_amd.modules.bloom_index_search_module import BloomIndexSearchModule


class BloomIndexSearchModuleBuilder:
    """Makes a BloomIndexSearchModule either from feature data (the index is
    built with ``bloom_index_build``) or from a prebuilt index and its bundle
    offsets.  Setters return the builder, so calls chain.

    As in the reference builder, the index built from feature data uses
    ``hash_k`` as the build's bits-per-term count and ``b_multiplier`` 2.0
    unless set.
    """

    def __init__(self, k: int, hash_k: int) -> None:
        self._k = k
        self._hash_k = hash_k
        self._bloom_index: torch.Tensor | None = None
        self._bloom_bundle_b_offsets: torch.Tensor | None = None
        self._features: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None
        self._b_multiplier = 2.0
        self._device: torch.device | None = None

    def set_bloom_index(self, bloom_index: torch.Tensor) -> "BloomIndexSearchModuleBuilder":
        self._bloom_index = bloom_index
        return self

    def set_bloom_bundle_b_offsets(self, bloom_bundle_b_offsets: torch.Tensor) -> "BloomIndexSearchModuleBuilder":
        self._bloom_bundle_b_offsets = bloom_bundle_b_offsets
        return self

    def set_feature_data(self, feature_ids: torch.Tensor, feature_offsets: torch.Tensor,
                         feature_values: torch.Tensor) -> "BloomIndexSearchModuleBuilder":
        self._features = (feature_ids, feature_offsets, feature_values)
        return self

    def set_b_multiplier(self, b_multiplier: float) -> "BloomIndexSearchModuleBuilder":
        self._b_multiplier = b_multiplier
        return self

    def set_device(self, device: torch.device) -> "BloomIndexSearchModuleBuilder":
        self._device = device
        return self

    def build(self) -> BloomIndexSearchModule:
        if self._features is not None:
            ids, offsets, values = self._features
            index, bundle_offsets = torch.ops.st.bloom_index_build(
                ids, offsets, values, self._b_multiplier, self._hash_k)
        elif self._bloom_index is not None:
            if self._bloom_bundle_b_offsets is None:
                raise ValueError("bloom_bundle_b_offsets must be set when using a pre-built bloom_index")
            index, bundle_offsets = self._bloom_index, self._bloom_bundle_b_offsets
        else:
            raise ValueError("Either feature data (via set_feature_data) or bloom_index "
                             "(via set_bloom_index) must be set before building")
        module = BloomIndexSearchModule(k=self._k, hash_k=self._hash_k)
        module.set_bloom_index(index)
        module.set_bloom_bundle_b_offsets(bundle_offsets)
        return module.to(self._device) if self._device is not None else module
