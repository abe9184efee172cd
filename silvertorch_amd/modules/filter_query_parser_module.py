"""Expression parser as an nn.Module (reference:
silvertorch/modules/filter_query_parser_module.py:22-63)."""

from __future__ import annotations

import torch
import torch.nn as nn

import silvertorch_amd.ops._load_ops  # noqa: F401  (registers torch.ops.st)


class FilterQueryParserModule(nn.Module):
    """Parses filter expressions into the encoded plans that
    BloomIndexSearchModule consumes.

    Args:
        hash_k: hashes carried per term.
        max_sub_queries: longest operand run kept in one AND / OR before the
            parser nests it.
    """

    def __init__(self, hash_k: int, max_sub_queries: int = 5) -> None:
        super().__init__()
        self.hash_k = hash_k
        self.max_sub_queries = max_sub_queries

    def forward(self, expressions: list[str], silvertorch_ks: torch.Tensor) -> tuple[int, list[torch.Tensor]]:
        """-> (max stack depth, [plans_data int8, plans_offsets int64])."""
        return torch.ops.st.parse_expression_query_batch(
            expressions, silvertorch_ks, self.hash_k, True, self.max_sub_queries)
