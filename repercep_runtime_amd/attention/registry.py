"""Attention op selection (src/repercep/attention/registry.py:37-39, 65-132 of the reference).

``REPERCEP_FP8_ATTENTION`` keeps its meaning and is read at import time as in
the reference: one of 1/true/on/triton/scaled_mm/te/transformer_engine
enables FP8.  On AMD the candidates follow the reference's order and
sub-values: the fused ``FP8HipAttention`` (in place of FP8TritonAttention)
unless the value is scaled_mm/te/transformer_engine, then the unfused
``FP8HipScaledMMAttention`` (in place of FP8ScaledMMAttention) unless it is
triton/te/transformer_engine, then the ``NaiveAttention`` floor.  Other
vendors get the floor.
"""

from __future__ import annotations

import os
from typing import TYPE_CHECKING

from repercep_runtime_amd.attention.fp8_hip import FP8HipAttention
from repercep_runtime_amd.attention.fp8_scaled_mm import FP8HipScaledMMAttention
from repercep_runtime_amd.attention.naive import NaiveAttention
from repercep_runtime_amd.hardware import DeviceArch, DType, Vendor

if TYPE_CHECKING:
    from repercep_runtime_amd.attention.protocol import AttentionOp
    from repercep_runtime_amd.attention.types import AttentionShape

_FP8_ENV = os.environ.get("REPERCEP_FP8_ATTENTION", "").lower()
_FP8_TRUTHY = ("1", "true", "on", "triton", "scaled_mm", "te", "transformer_engine")
_FP8_ENABLED = _FP8_ENV in _FP8_TRUTHY


def select_attention_op(arch: DeviceArch, shape: AttentionShape, dtype: DType) -> AttentionOp:
    """First op, in preference order, whose ``supports(shape, dtype)`` is True."""
    candidates: list[AttentionOp] = []
    if arch.vendor is Vendor.AMD and _FP8_ENABLED:
        if _FP8_ENV not in ("scaled_mm", "te", "transformer_engine"):
            candidates.append(FP8HipAttention())
        if _FP8_ENV not in ("triton", "te", "transformer_engine"):
            candidates.append(FP8HipScaledMMAttention())
    candidates.append(NaiveAttention())
    for op in candidates:
        if op.supports(shape, dtype):
            return op
    return NaiveAttention()
