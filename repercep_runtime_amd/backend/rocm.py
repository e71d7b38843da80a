"""ROCm backend (src/repercep/backend/rocm.py:31-99 of the reference) with MI355X.

The reference maps only gfx942/gfx90a and hard-codes MI300X in
``attention_op`` (rocm.py:31-34, :98-99).  Here gfx950 maps to ``MI355X``
and ``attention_op`` selects for the architecture of device 0.
"""

from __future__ import annotations

from typing import TYPE_CHECKING

from repercep_runtime_amd.attention.registry import select_attention_op
from repercep_runtime_amd.hardware import (
    MI250X,
    MI300X,
    MI355X,
    BackendCapabilities,
    DeviceArch,
    DeviceSpec,
    DType,
    Vendor,
)

if TYPE_CHECKING:
    import torch

    from repercep_runtime_amd.attention.protocol import AttentionOp
    from repercep_runtime_amd.attention.types import AttentionShape

_GFX_TO_ARCH: dict[str, DeviceArch] = {
    "gfx950": MI355X,
    "gfx942": MI300X,
    "gfx90a": MI250X,
}


class ROCmBackend:
    vendor: Vendor = Vendor.AMD
    name: str = "rocm"

    def is_available(self) -> bool:
        try:
            import torch
        except ImportError:
            return False
        return bool(torch.version.hip) and torch.cuda.is_available()

    def devices(self) -> tuple[DeviceSpec, ...]:
        import torch

        specs: list[DeviceSpec] = []
        for i in range(torch.cuda.device_count()):
            props = torch.cuda.get_device_properties(i)
            gfx = props.gcnArchName.split(":")[0]
            arch = _GFX_TO_ARCH.get(gfx, DeviceArch(Vendor.AMD, gfx, "unknown"))
            specs.append(DeviceSpec(index=i, arch=arch, name=props.name,
                                    total_memory_bytes=props.total_memory,
                                    multi_processor_count=props.multi_processor_count))
        return tuple(specs)

    def arch(self) -> DeviceArch:
        devs = self.devices() if self.is_available() else ()
        return devs[0].arch if devs else MI355X

    def capabilities(self) -> BackendCapabilities:
        from repercep_runtime_amd import _capi

        ops = (("fp8-hip-flash", "fp8-hip-scaled-mm", "naive-sdpa") if _capi.available()
               else ("naive-sdpa",))
        return BackendCapabilities(
            dtypes=frozenset({DType.FP32, DType.FP16, DType.BF16, DType.FP8_E4M3,
                              DType.FP8_E5M2, DType.INT8}),
            supports_flash_attention=False,
            supports_fp8=True,
            supports_torch_compile=True,
            attention_ops=ops,
        )

    def torch_device(self, index: int = 0) -> torch.device:
        import torch

        return torch.device("cuda", index)

    def default_dtype(self) -> DType:
        return DType.BF16

    def attention_op(self, shape: AttentionShape, dtype: DType) -> AttentionOp:
        return select_attention_op(self.arch(), shape, dtype)
