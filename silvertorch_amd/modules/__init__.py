"""nn.Module surface of the bloom retrieval path, mirroring the reference's
silvertorch.modules (bloom_index_search_module.py, filter_query_parser_module.py
and their builders) over this build's torch.ops.st operators."""

from silvertorch_amd.modules.bloom_index_search_module import BloomIndexSearchModule  # noqa: F401
from silvertorch_amd.modules.bloom_index_search_module_builder import (  # noqa: F401
    BloomIndexSearchModuleBuilder,
)
from silvertorch_amd.modules.filter_query_parser_module import FilterQueryParserModule  # noqa: F401
from silvertorch_amd.modules.filter_query_parser_module_builder import (  # noqa: F401
    FilterQueryParserModuleBuilder,
)

__all__ = [
    "BloomIndexSearchModule",
    "BloomIndexSearchModuleBuilder",
    "FilterQueryParserModule",
    "FilterQueryParserModuleBuilder",
]
