"""``silvertorch.modules``: the silvertorch_amd.modules classes under the
reference's import path."""

from silvertorch_amd.modules import (  # noqa: F401
    BloomIndexSearchModule,
    BloomIndexSearchModuleBuilder,
    FilterQueryParserModule,
    FilterQueryParserModuleBuilder,
)

__all__ = [
    "BloomIndexSearchModule",
    "BloomIndexSearchModuleBuilder",
    "FilterQueryParserModule",
    "FilterQueryParserModuleBuilder",
]
