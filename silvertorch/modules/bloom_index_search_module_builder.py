"""``silvertorch.modules.bloom_index_search_module_builder``: silvertorch_amd.modules.bloom_index_search_module_builder."""

from silvertorch_amd.modules.bloom_index_search_module_builder import BloomIndexSearchModuleBuilder  # noqa: F401

__all__ = ["BloomIndexSearchModuleBuilder"]
