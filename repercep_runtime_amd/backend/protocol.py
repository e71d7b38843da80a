"""The ``Backend`` Protocol (src/repercep/backend/protocol.py:16-52 of the reference)."""

from __future__ import annotations

from typing import TYPE_CHECKING, Protocol, runtime_checkable

if TYPE_CHECKING:
    import torch

    from repercep_runtime_amd.attention.protocol import AttentionOp
    from repercep_runtime_amd.attention.types import AttentionShape
    from repercep_runtime_amd.hardware import BackendCapabilities, DeviceSpec, DType, Vendor


@runtime_checkable
class Backend(Protocol):
    vendor: Vendor
    name: str

    def is_available(self) -> bool: ...

    def devices(self) -> tuple[DeviceSpec, ...]: ...

    def capabilities(self) -> BackendCapabilities: ...

    def torch_device(self, index: int = 0) -> torch.device: ...

    def default_dtype(self) -> DType: ...

    def attention_op(self, shape: AttentionShape, dtype: DType) -> AttentionOp: ...
