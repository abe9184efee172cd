"""Builder of FilterQueryParserModule (reference:
silvertorch/modules/filter_query_parser_module_builder.py:20-46)."""

from __future__ import annotations

from silvertorch_amd.modules.filter_query_parser_module import FilterQueryParserModule


class FilterQueryParserModuleBuilder:
    """Makes a FilterQueryParserModule, returned in eval mode."""

    def __init__(self, hash_k: int, max_sub_queries: int = 5) -> None:
        self._hash_k = hash_k
        self._max_sub_queries = max_sub_queries

    def build(self) -> FilterQueryParserModule:
        module = FilterQueryParserModule(hash_k=self._hash_k, max_sub_queries=self._max_sub_queries)
        module.eval()
        return module
