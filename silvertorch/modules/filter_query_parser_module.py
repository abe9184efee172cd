"""``silvertorch.modules.filter_query_parser_module``: silvertorch_amd.modules.filter_query_parser_module."""

from silvertorch_amd.modules.filter_query_parser_module import FilterQueryParserModule  # noqa: F401

__all__ = ["FilterQueryParserModule"]
