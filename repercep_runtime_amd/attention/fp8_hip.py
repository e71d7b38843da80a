"""FP8 flash attention on MI355X as an ``AttentionOp``.

The drop-in for the reference's ``FP8TritonAttention``
(src/repercep/attention/fp8_triton.py:42-110): same members, same error
behaviour (``available`` False when the kernel cannot be loaded,
``__call__`` raising RuntimeError then), backed by the hand-written gfx950
kernels in librepercep_fp8.so instead of the gfx942 Triton kernel.

``supports()`` differences, all widenings of what the hardware path can do:
* cross-attention (seq_len_kv != seq_len_q) is accepted -- the reference
  gates it out (fp8_triton.py:90-91) although its kernel body handles it;
* head dims: the reference's set (32, 64, 128, 256);
* dtypes BF16 and FP16, as the reference's (fp8_triton.py:85).
"""

from __future__ import annotations

from typing import TYPE_CHECKING

from repercep_runtime_amd.attention.types import AttentionKind, AttentionShape
from repercep_runtime_amd.hardware import DType

if TYPE_CHECKING:
    import torch

_MIN_SEQ_LEN = 128
_SUPPORTED_KINDS = frozenset({AttentionKind.FULL, AttentionKind.CAUSAL})


class FP8HipAttention:
    """Fused FP8 flash attention (gfx950 HIP kernels via the C ABI)."""

    name = "fp8-hip-flash"

    def __init__(self) -> None:
        self._fn = None
        self._import_error: str | None = None
        try:
            from repercep_runtime_amd import _capi
            from repercep_runtime_amd.ops import SUPPORTED_HEAD_DIMS, fp8_flash_attention

            _capi.lib()
            self._fn = fp8_flash_attention
            self._head_dims = SUPPORTED_HEAD_DIMS
        except Exception as exc:  # library missing or not loadable
            self._import_error = f"{type(exc).__name__}: {exc}"

    @property
    def available(self) -> bool:
        return self._fn is not None

    def supports(self, shape: AttentionShape, dtype: DType) -> bool:
        return (
            self._fn is not None
            and dtype in (DType.BF16, DType.FP16)
            and shape.head_dim in self._head_dims
            and shape.kind in _SUPPORTED_KINDS
            and shape.seq_len_q >= 1
            and shape.seq_len_kv >= _MIN_SEQ_LEN
        )

    def __call__(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, *,
                 causal: bool = False, scale: float | None = None) -> torch.Tensor:
        if self._fn is None:
            raise RuntimeError(
                "FP8 HIP attention is not available "
                f"(load error: {self._import_error}). "
                "Fall back to attention_backend='naive-sdpa'."
            )
        return self._fn(query, key, value, causal=causal, scale=scale)
