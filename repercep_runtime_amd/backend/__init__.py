"""Backend seam (mirrors src/repercep/backend of the reference; ROCm only here)."""

from repercep_runtime_amd.backend.protocol import Backend
from repercep_runtime_amd.backend.rocm import ROCmBackend

__all__ = ["Backend", "ROCmBackend"]
