"""``silvertorch.modules.filter_query_parser_module_builder``: silvertorch_amd.modules.filter_query_parser_module_builder."""

from silvertorch_amd.modules.filter_query_parser_module_builder import FilterQueryParserModuleBuilder  # noqa: F401

__all__ = ["FilterQueryParserModuleBuilder"]
