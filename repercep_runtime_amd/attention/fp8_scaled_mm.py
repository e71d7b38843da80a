"""The unfused FP8 attention on MI355X as an ``AttentionOp``.

The drop-in for the reference's ``FP8ScaledMMAttention``
(src/repercep/attention/fp8_scaled_mm.py:58-221): row-wise FP8 quantization
of Q and K, a row-scaled FP8 GEMM into bf16 scores, a bf16 softmax, row-wise
P and V^T codes, and a second row-scaled FP8 GEMM -- each step a gfx950
kernel of librepercep_fp8.so (``ops.fp8_scaled_mm_attention``) where the
reference calls ``torch._scaled_grouped_mm`` (hipBLASLt) and torch ops.  It
materialises the (B*H, Sq, Skv) scores, so ``supports()`` keeps the
reference's 4 GiB cap on them; the fused ``FP8HipAttention`` is the path for
long sequences.

Same members and error behaviour as the reference's op: ``available`` is
False and ``__call__`` raises RuntimeError when the library cannot load.
``supports()`` follows :87-105: BF16/FP16 (the reference also lists its FP8
dtypes, which no caller passes to an op that quantizes itself), head dims
{64, 96, 128, 192, 256}, FULL and CAUSAL, both sequence lengths multiples
of 16 and at least 16.
"""

from __future__ import annotations

from typing import TYPE_CHECKING

from repercep_runtime_amd.attention.types import AttentionKind, AttentionShape
from repercep_runtime_amd.hardware import DType

if TYPE_CHECKING:
    import torch

_MIN_DIM = 16
_SUPPORTED_HEAD_DIMS = frozenset({64, 96, 128, 192, 256})
_SUPPORTED_KINDS = frozenset({AttentionKind.FULL, AttentionKind.CAUSAL})
_MAX_SCORES_BYTES = 4 * 1024 ** 3


class FP8HipScaledMMAttention:
    """Unfused FP8 attention (row-wise scales, two FP8 GEMMs) on gfx950."""

    name = "fp8-hip-scaled-mm"

    def __init__(self) -> None:
        self._fn = None
        self._import_error: str | None = None
        try:
            from repercep_runtime_amd import _capi
            from repercep_runtime_amd.ops import fp8_scaled_mm_attention

            _capi.lib()
            self._fn = fp8_scaled_mm_attention
        except Exception as exc:  # library missing or not loadable
            self._import_error = f"{type(exc).__name__}: {exc}"

    @property
    def available(self) -> bool:
        return self._fn is not None

    def supports(self, shape: AttentionShape, dtype: DType) -> bool:
        scores_bytes = shape.batch * shape.heads * shape.seq_len_q * shape.seq_len_kv * 2
        return (
            self._fn is not None
            and dtype in (DType.BF16, DType.FP16)
            and shape.head_dim in _SUPPORTED_HEAD_DIMS
            and shape.kind in _SUPPORTED_KINDS
            and shape.seq_len_q >= _MIN_DIM
            and shape.seq_len_kv >= _MIN_DIM
            and shape.seq_len_q % _MIN_DIM == 0
            and shape.seq_len_kv % _MIN_DIM == 0
            and scores_bytes <= _MAX_SCORES_BYTES
        )

    def __call__(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, *,
                 causal: bool = False, scale: float | None = None) -> torch.Tensor:
        if self._fn is None:
            raise RuntimeError(
                "FP8 HIP scaled-mm attention is not available "
                f"(load error: {self._import_error}). "
                "Pin attention_backend='naive-sdpa' on hardware without it."
            )
        return self._fn(query, key, value, causal=causal, scale=scale)
