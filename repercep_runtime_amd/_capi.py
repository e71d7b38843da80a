"""ctypes binding of librepercep_fp8.so (declarations in include/repercep_fp8.h).

The library is the product: there is no Python or CPU fallback.  When the
shared object is missing or cannot be loaded every entry point raises
``HipLibraryError`` with the reason, so a GPU host without the built library
fails loudly instead of silently computing something else.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "librepercep_fp8.so"

RP_OK = 0
RP_SCALE_PER_BH = 0
RP_SCALE_PER_TENSOR = 1
RP_LAYOUT_BHSD = 0
RP_LAYOUT_BHDS = 1
RP_OUT_BF16 = 0
RP_OUT_F32 = 1
RP_OUT_F16 = 2
RP_DTYPE_BF16 = 0
RP_DTYPE_F16 = 1
RP_MASK_NONE = 0
RP_MASK_CAUSAL = 1
RP_MASK_SHARED_PREFIX = 2
RP_ROPE_NONE = 0
RP_ROPE_HALF = 1
RP_ROPE_INTERLEAVED = 2
RP_QKV_NOALLOC_SCRATCH_BYTES = 1 << 20
RP_B_NK = 0
RP_B_KN = 1
RP_GEMM_BALANCED_WORKSPACE_BYTES = 256

#: Every function include/repercep_fp8.h declares.
EXPORTS = (
    "rp_abi_version", "rp_status_string", "rp_last_error",
    "rp_fp8_quant_workspace_bytes", "rp_fp8_scale", "rp_fp8_quantize",
    "rp_fp8_scale_quantize", "rp_fp8_quant_qkv_workspace_bytes", "rp_fp8_scale_quantize_qkv",
    "rp_fp8_scale_quantize_qkv_noalloc",
    "rp_fp8_attn_fwd",
    "rp_fp8_attn_workspace_bytes",
    "rp_fp8_attn_blocks_per_workgroup", "rp_fp8_attn_resident_kv",
    "rp_fp8_attn_fwd_split", "rp_fp8_attn_balanced_plan",
    "rp_fp8_attn_fwd_wsplit", "rp_fp8_attn_wsplit_plan",
    "rp_fp8_attn_balanced_workspace_bytes", "rp_fp8_attn_fwd_balanced",
    "rp_fp8_attn_q16_supported", "rp_fp8_attn_fwd_q16",
    "rp_fp8_rmsnorm_quant_workspace_bytes",
    "rp_fp8_rmsnorm_scale_quantize", "rp_fp8_rmsnorm_quant_qkv_workspace_bytes",
    "rp_fp8_rmsnorm_scale_quantize_qkv", "rp_fp8_gemm", "rp_fp8_linear",
    "rp_fp8_linear_balanced", "rp_fp8_transpose",
    "rp_fp8_gemm_rowwise", "rp_fp8_rowwise_quantize", "rp_transpose16",
    "rp_fp8_softmax_rowwise_quantize",
    "rp_selftest_e4m3", "rp_selftest_scale",
)


class HipLibraryError(RuntimeError):
    """The gfx950 library is missing, failed to load, or a call failed."""


_lib: ctypes.CDLL | None = None
_load_error: str | None = None

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_f32 = ctypes.c_float
_sz = ctypes.c_size_t


def _declare(L: ctypes.CDLL) -> None:
    L.rp_abi_version.restype = _int
    L.rp_abi_version.argtypes = []
    L.rp_status_string.restype = ctypes.c_char_p
    L.rp_status_string.argtypes = [_int]
    L.rp_last_error.restype = ctypes.c_char_p
    L.rp_last_error.argtypes = []
    L.rp_fp8_quant_workspace_bytes.restype = _sz
    L.rp_fp8_quant_workspace_bytes.argtypes = [_i64, _i64, _i64, _i64, _int]
    L.rp_fp8_scale.restype = _int
    L.rp_fp8_scale.argtypes = [_vp, _int, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int, _vp,
                               _vp, _sz, _vp]
    L.rp_fp8_quantize.restype = _int
    L.rp_fp8_quantize.argtypes = [_vp, _int, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int,
                                  _vp, _vp, _int, _i64, _vp]
    L.rp_fp8_scale_quantize.restype = _int
    L.rp_fp8_scale_quantize.argtypes = [_vp, _int, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                        _int, _vp, _vp, _int, _i64, _vp, _sz, _vp]
    L.rp_fp8_quant_qkv_workspace_bytes.restype = _sz
    L.rp_fp8_quant_qkv_workspace_bytes.argtypes = [_i64] * 5 + [_int]
    L.rp_fp8_scale_quantize_qkv.restype = _int
    L.rp_fp8_scale_quantize_qkv.argtypes = ([_vp, _vp, _vp, _int] + [_i64] * 14
                                            + [_int, _vp, _vp, _vp, _vp, _i64, _vp, _sz, _vp])
    L.rp_fp8_scale_quantize_qkv_noalloc.restype = _int
    L.rp_fp8_scale_quantize_qkv_noalloc.argtypes = ([_vp, _vp, _vp, _int] + [_i64] * 14
                                                    + [_int, _vp, _vp, _vp, _vp, _i64, _vp])
    L.rp_fp8_attn_fwd.restype = _int
    L.rp_fp8_attn_fwd.argtypes = [_vp, _vp, _vp, _i64, _vp, _vp, _vp, _int, _f32, _vp, _int,
                                  _i64, _i64, _i64, _int, _int, _int, _int, _int, _int, _int,
                                  _int, _vp]
    L.rp_fp8_attn_blocks_per_workgroup.restype = _int
    L.rp_fp8_attn_blocks_per_workgroup.argtypes = [_int] * 7
    L.rp_fp8_attn_resident_kv.restype = _int
    L.rp_fp8_attn_resident_kv.argtypes = [_int] * 7
    L.rp_fp8_attn_workspace_bytes.restype = _sz
    L.rp_fp8_attn_workspace_bytes.argtypes = [_int, _int, _int, _int, _int]
    L.rp_fp8_attn_fwd_split.restype = _int
    L.rp_fp8_attn_fwd_split.argtypes = (list(L.rp_fp8_attn_fwd.argtypes[:-1])
                                        + [_int, _vp, _sz, _vp])
    L.rp_fp8_attn_fwd_wsplit.restype = _int
    L.rp_fp8_attn_fwd_wsplit.argtypes = (list(L.rp_fp8_attn_fwd.argtypes[:-1]) + [_int, _vp])
    L.rp_fp8_attn_wsplit_plan.restype = _int
    L.rp_fp8_attn_wsplit_plan.argtypes = [_int, _int, ctypes.POINTER(_int), ctypes.POINTER(_int)]
    L.rp_fp8_attn_balanced_plan.restype = _int
    L.rp_fp8_attn_balanced_plan.argtypes = [_int] * 7 + [ctypes.POINTER(_int)] * 2
    L.rp_fp8_attn_balanced_workspace_bytes.restype = _sz
    L.rp_fp8_attn_balanced_workspace_bytes.argtypes = [_int] * 6 + [_vp]
    L.rp_fp8_attn_fwd_balanced.restype = _int
    L.rp_fp8_attn_fwd_balanced.argtypes = (list(L.rp_fp8_attn_fwd.argtypes[:-1])
                                           + [_vp, _sz, _vp])
    L.rp_fp8_attn_q16_supported.restype = _int
    L.rp_fp8_attn_q16_supported.argtypes = [_int] * 7 + [_vp]
    L.rp_fp8_attn_fwd_q16.restype = _int
    L.rp_fp8_attn_fwd_q16.argtypes = ([_vp, _int, _i64, _i64, _i64]
                                      + list(L.rp_fp8_attn_fwd.argtypes[1:-1])
                                      + [_int, _vp, _sz, _vp])
    L.rp_fp8_rmsnorm_quant_workspace_bytes.restype = _sz
    L.rp_fp8_rmsnorm_quant_workspace_bytes.argtypes = [_i64, _i64, _i64, _i64, _int]
    L.rp_fp8_rmsnorm_scale_quantize.restype = _int
    L.rp_fp8_rmsnorm_scale_quantize.argtypes = [_vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                                _vp, _f32, _vp, _vp, _int, _int, _vp, _vp, _vp,
                                                _sz, _vp]
    L.rp_fp8_rmsnorm_quant_qkv_workspace_bytes.restype = _sz
    L.rp_fp8_rmsnorm_quant_qkv_workspace_bytes.argtypes = [_i64] * 5 + [_int]
    L.rp_fp8_rmsnorm_scale_quantize_qkv.restype = _int
    L.rp_fp8_rmsnorm_scale_quantize_qkv.argtypes = ([_vp] * 3 + [_i64] * 14 + [_vp, _vp, _f32]
                                                    + [_vp] * 4 + [_int, _int] + [_vp] * 4
                                                    + [_i64, _vp, _sz, _vp])
    L.rp_fp8_gemm.restype = _int
    L.rp_fp8_gemm.argtypes = [_vp, _vp, _int, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _f32,
                              _f32, _vp, _vp, _vp]
    L.rp_fp8_linear.restype = _int
    L.rp_fp8_linear.argtypes = [_vp, _vp, _int, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                                _f32, _f32, _vp, _vp, _vp]
    L.rp_fp8_linear_balanced.restype = _int
    L.rp_fp8_linear_balanced.argtypes = (list(L.rp_fp8_linear.argtypes[:-1]) + [_vp, _sz, _vp])
    L.rp_fp8_gemm_rowwise.restype = _int
    L.rp_fp8_gemm_rowwise.argtypes = ([_vp, _vp, _int, _vp] + [_i64] * 6 + [_vp, _vp]
                                      + [_i64] * 6 + [_vp])
    L.rp_fp8_rowwise_quantize.restype = _int
    L.rp_fp8_rowwise_quantize.argtypes = [_vp, _int, _i64, _i64, _i64, _vp, _vp, _i64, _vp]
    L.rp_transpose16.restype = _int
    L.rp_transpose16.argtypes = [_vp, _vp] + [_i64] * 7 + [_vp]
    L.rp_fp8_softmax_rowwise_quantize.restype = _int
    L.rp_fp8_softmax_rowwise_quantize.argtypes = [_vp, _i64, _i64, _i64, _i64, _int, _f32, _vp,
                                                  _vp, _i64, _vp]
    L.rp_fp8_transpose.restype = _int
    L.rp_fp8_transpose.argtypes = [_vp, _vp, _i64, _i64, _i64, _i64, _vp]
    L.rp_selftest_e4m3.restype = _int
    L.rp_selftest_e4m3.argtypes = [_vp, _vp, _i64, _vp]
    L.rp_selftest_scale.restype = _int
    L.rp_selftest_scale.argtypes = [_vp, _int, _vp, _vp, _i64, _vp]


def lib() -> ctypes.CDLL:
    """The loaded library; raises HipLibraryError if it is not available."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    path = Path(os.environ.get("REPERCEP_FP8_LIB", str(LIB_PATH)))
    if not path.exists():
        _load_error = (f"{path} is missing: build it with "
                       f"`python -c 'import __graft_entry__ as g; g.build()'`")
        raise HipLibraryError(_load_error)
    try:
        L = ctypes.CDLL(str(path))
    except OSError as exc:
        _load_error = f"cannot load {path}: {exc}"
        raise HipLibraryError(_load_error) from exc
    _declare(L)
    _lib = L
    return L


def available() -> bool:
    try:
        lib()
    except HipLibraryError:
        return False
    return True


def load_error() -> str | None:
    return _load_error


def check(status: int, what: str) -> None:
    """Raise HipLibraryError for a non-zero status, with the library's message."""
    if status != RP_OK:
        L = lib()
        msg = (L.rp_last_error() or b"").decode(errors="replace")
        kind = (L.rp_status_string(status) or b"").decode(errors="replace")
        raise HipLibraryError(f"{what}: {kind} ({status}): {msg}")
