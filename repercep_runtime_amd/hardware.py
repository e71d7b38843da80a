"""Hardware domain types, mirroring src/repercep/hardware.py of the reference.

``Vendor``, ``DType``, ``DeviceArch``, ``DeviceSpec`` and
``BackendCapabilities`` keep the reference's names and values
(hardware.py:14-95).  The reference uses ``enum.StrEnum`` (Python >= 3.11);
these are ``str``-mixin enums with the same values and ``str()`` output, so
they compare and print the same on Python 3.10.  ``MI355X`` (gfx950, CDNA4)
is the architecture the reference's table lacks.
"""

from __future__ import annotations

import enum
from dataclasses import dataclass


class _StrEnum(str, enum.Enum):
    def __str__(self) -> str:
        return str(self.value)


class Vendor(_StrEnum):
    AMD = "amd"
    NVIDIA = "nvidia"
    INTEL = "intel"


class DType(_StrEnum):
    FP32 = "fp32"
    FP16 = "fp16"
    BF16 = "bf16"
    FP8_E4M3 = "fp8_e4m3"
    FP8_E5M2 = "fp8_e5m2"
    INT8 = "int8"


@dataclass(frozen=True, slots=True)
class DeviceArch:
    vendor: Vendor
    gfx_id: str
    family: str

    def __str__(self) -> str:
        return f"{self.vendor.value}:{self.gfx_id}"


MI355X = DeviceArch(Vendor.AMD, "gfx950", "CDNA4")
MI300X = DeviceArch(Vendor.AMD, "gfx942", "CDNA3")
MI250X = DeviceArch(Vendor.AMD, "gfx90a", "CDNA2")


@dataclass(frozen=True, slots=True)
class DeviceSpec:
    index: int
    arch: DeviceArch
    name: str
    total_memory_bytes: int
    multi_processor_count: int

    @property
    def total_memory_gib(self) -> float:
        return self.total_memory_bytes / (1024**3)


@dataclass(frozen=True, slots=True)
class BackendCapabilities:
    dtypes: frozenset[DType]
    supports_flash_attention: bool
    supports_fp8: bool
    supports_torch_compile: bool
    attention_ops: tuple[str, ...]
