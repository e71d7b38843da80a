"""Attention ops of the MI355X FP8 path (mirrors src/repercep/attention/__init__.py)."""

from __future__ import annotations

from repercep_runtime_amd.attention import diffusers_backend as _diffusers_backend  # noqa: F401
from repercep_runtime_amd.attention.fp8_hip import FP8HipAttention
from repercep_runtime_amd.attention.fp8_scaled_mm import FP8HipScaledMMAttention
from repercep_runtime_amd.attention.naive import NaiveAttention
from repercep_runtime_amd.attention.protocol import AttentionOp
from repercep_runtime_amd.attention.registry import select_attention_op
from repercep_runtime_amd.attention.types import AttentionKind, AttentionShape

__all__ = [
    "AttentionKind",
    "AttentionOp",
    "AttentionShape",
    "FP8HipAttention",
    "FP8HipScaledMMAttention",
    "NaiveAttention",
    "select_attention_op",
]
