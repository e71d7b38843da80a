"""The ``AttentionOp`` Protocol (src/repercep/attention/protocol.py:14-54 of the reference).

Structural and runtime-checkable: any object with ``name``, ``available``,
``supports(shape, dtype)`` and ``__call__(query, key, value, *, causal,
scale)`` is an AttentionOp, so ops of this package drop into the reference's
registry and callers unchanged.
"""

from __future__ import annotations

from typing import TYPE_CHECKING, Protocol, runtime_checkable

if TYPE_CHECKING:
    import torch

    from repercep_runtime_amd.attention.types import AttentionShape
    from repercep_runtime_amd.hardware import DType


@runtime_checkable
class AttentionOp(Protocol):
    name: str

    @property
    def available(self) -> bool: ...

    def supports(self, shape: AttentionShape, dtype: DType) -> bool: ...

    def __call__(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, *,
                 causal: bool = False, scale: float | None = None) -> torch.Tensor:
        """(batch, heads, seq, head_dim) in; (batch, heads, seq_len_q, head_dim) out."""
        ...
