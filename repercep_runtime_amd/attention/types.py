"""Attention problem descriptors (src/repercep/attention/types.py:9-40 of the reference)."""

from __future__ import annotations

from dataclasses import dataclass

from repercep_runtime_amd.hardware import _StrEnum


class AttentionKind(_StrEnum):
    FULL = "full"
    CAUSAL = "causal"
    NEIGHBORHOOD = "neighborhood"


@dataclass(frozen=True, slots=True)
class AttentionShape:
    """One attention call; layout convention (batch, heads, seq, head_dim)."""

    batch: int
    heads: int
    seq_len_q: int
    seq_len_kv: int
    head_dim: int
    kind: AttentionKind = AttentionKind.FULL

    @property
    def is_self_attention(self) -> bool:
        return self.seq_len_q == self.seq_len_kv
