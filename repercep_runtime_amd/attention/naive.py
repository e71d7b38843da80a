"""SDPA floor op (src/repercep/attention/naive.py:19-44 of the reference)."""

from __future__ import annotations

from typing import TYPE_CHECKING

if TYPE_CHECKING:
    import torch

    from repercep_runtime_amd.attention.types import AttentionShape
    from repercep_runtime_amd.hardware import DType


class NaiveAttention:
    """``torch.nn.functional.scaled_dot_product_attention`` as an AttentionOp."""

    name = "naive-sdpa"
    available = True

    def supports(self, shape: AttentionShape, dtype: DType) -> bool:
        return True

    def __call__(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, *,
                 causal: bool = False, scale: float | None = None) -> torch.Tensor:
        from torch.nn.functional import scaled_dot_product_attention

        return scaled_dot_product_attention(query, key, value, is_causal=causal, scale=scale)
