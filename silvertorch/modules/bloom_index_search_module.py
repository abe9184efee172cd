"""``silvertorch.modules.bloom_index_search_module``: silvertorch_amd.modules.bloom_index_search_module."""

from silvertorch_amd.modules.bloom_index_search_module import BloomIndexSearchModule  # noqa: F401

__all__ = ["BloomIndexSearchModule"]
