"""ctypes binding of the C oracle (oracle/c/fp8_oracle.c).  Test infrastructure only.

Every function here follows the same reference lines as its C counterpart;
see the C file's header for the citations.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

from oracle.build_oracle import LIB, build

_lib: ctypes.CDLL | None = None

_u8p = ctypes.POINTER(ctypes.c_uint8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64 = ctypes.c_int64


def lib() -> ctypes.CDLL:
    """Load (building on first use if needed) the oracle shared library."""
    global _lib
    if _lib is not None:
        return _lib
    path = Path(LIB)
    if not path.exists():
        build()
    L = ctypes.CDLL(str(path))
    L.or_e4m3fn_encode.restype = ctypes.c_uint8
    L.or_e4m3fn_encode.argtypes = [ctypes.c_float]
    L.or_e4m3fn_decode.restype = ctypes.c_float
    L.or_e4m3fn_decode.argtypes = [ctypes.c_uint8]
    L.or_e4m3fn_encode_array.argtypes = [_f32p, _i64, _u8p]
    L.or_amax_bf16.restype = ctypes.c_uint16
    L.or_amax_bf16.argtypes = [_u16p, _i64]
    L.or_amax_bf16_rows.restype = ctypes.c_uint16
    L.or_amax_bf16_rows.argtypes = [_u16p, _i64, _i64, _i64]
    L.or_dequant_from_amax.restype = ctypes.c_float
    L.or_dequant_from_amax.argtypes = [ctypes.c_uint16]
    L.or_qmul_from_dequant.restype = ctypes.c_float
    L.or_qmul_from_dequant.argtypes = [ctypes.c_float]
    L.or_quantize_bf16.argtypes = [_u16p, _i64, ctypes.c_float, _u8p]
    L.or_quantize_bf16_rows.argtypes = [_u16p, _i64, _i64, _i64, ctypes.c_float, _u8p]
    L.or_attn_rows.argtypes = [
        _u8p, _u8p, _u8p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
        ctypes.c_float, ctypes.c_float, ctypes.c_float, ctypes.c_float,
        ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
        _i32p, ctypes.c_int, _f32p,
    ]
    L.or_gemm_rows.argtypes = [
        _u8p, _u8p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
        ctypes.c_float, ctypes.c_float, _i32p, ctypes.c_int, _u16p,
    ]
    L.or_rmsnorm_bf16_rows.argtypes = [_u16p, _i64, ctypes.c_int, ctypes.c_float, _u16p]
    L.or_num_threads.restype = ctypes.c_int
    _lib = L
    return L


def _ptr(a: np.ndarray, typ):  # type: ignore[no-untyped-def]
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(typ)


def encode_e4m3fn(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint8)
    lib().or_e4m3fn_encode_array(_ptr(x, _f32p), x.size, _ptr(out, _u8p))
    return out


def amax_bf16(bits: np.ndarray) -> int:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    return int(lib().or_amax_bf16(_ptr(bits, _u16p), bits.size))


def dequant_from_amax(amax_bits: int) -> np.float32:
    return np.float32(lib().or_dequant_from_amax(ctypes.c_uint16(amax_bits)))


def quantize_bf16(bits: np.ndarray, dequant: float) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, dtype=np.uint8)
    lib().or_quantize_bf16(_ptr(bits, _u16p), bits.size, ctypes.c_float(dequant), _ptr(out, _u8p))
    return out


def quantize_groups(bits: np.ndarray, n_groups: int) -> tuple[np.ndarray, np.ndarray]:
    """Per-group amax scale + codes for a bf16 array whose leading elements
    split evenly into ``n_groups`` contiguous groups (per-(B,H) when the array
    is (B,H,S,D) contiguous and n_groups = B*H; per-tensor when 1)."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    flat = bits.reshape(n_groups, -1)
    scales = np.empty(n_groups, dtype=np.float32)
    codes = np.empty(flat.shape, dtype=np.uint8)
    for g in range(n_groups):
        scales[g] = dequant_from_amax(amax_bf16(flat[g]))
        codes[g] = quantize_bf16(flat[g], float(scales[g]))
    return scales, codes.reshape(bits.shape)


def rmsnorm_bf16(bits: np.ndarray, eps: float) -> np.ndarray:
    """RMSNorm over the last axis (unit weight, no rotation) of bf16 bit
    patterns, as bf16 bit patterns: ``oracle.prologue.rmsnorm_rope`` in C."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    D = bits.shape[-1]
    assert D % 16 == 0 and D <= 512
    out = np.empty(bits.shape, dtype=np.uint16)
    lib().or_rmsnorm_bf16_rows(_ptr(bits, _u16p), bits.size // D, D, ctypes.c_float(eps),
                               _ptr(out, _u16p))
    return out


def attn_rows(
    q8: np.ndarray, k8: np.ndarray, v8: np.ndarray,
    q_scale: float, k_scale: float, v_scale: float, sm_scale: float,
    rows: np.ndarray, *, block_n: int = 128, mask: int = 0, prefix: int = 0,
    suffix: int = 1, pquant: bool = True,
) -> np.ndarray:
    """Tile-exact FP8 attention emulation for one (b, h) slice; fp32 (len(rows), D)."""
    q8 = np.ascontiguousarray(q8, dtype=np.uint8)
    k8 = np.ascontiguousarray(k8, dtype=np.uint8)
    v8 = np.ascontiguousarray(v8, dtype=np.uint8)
    rows = np.ascontiguousarray(rows, dtype=np.int32)
    Sq, D = q8.shape
    Skv = k8.shape[0]
    assert v8.shape == (Skv, D) and D <= 512 and block_n <= 1024
    out = np.empty((rows.size, D), dtype=np.float32)
    lib().or_attn_rows(
        _ptr(q8, _u8p), _ptr(k8, _u8p), _ptr(v8, _u8p), Sq, Skv, D,
        ctypes.c_float(q_scale), ctypes.c_float(k_scale), ctypes.c_float(v_scale),
        ctypes.c_float(sm_scale), block_n, mask, prefix, suffix, int(pquant),
        _ptr(rows, _i32p), rows.size, _ptr(out, _f32p),
    )
    return out


def gemm_rows(a8: np.ndarray, bt8: np.ndarray, a_scale: float, b_scale: float,
              rows: np.ndarray) -> np.ndarray:
    """Rows of bf16(fp32(A8 @ B8) * a_scale*b_scale) as bf16 bit patterns; bt8 is (N, K)."""
    a8 = np.ascontiguousarray(a8, dtype=np.uint8)
    bt8 = np.ascontiguousarray(bt8, dtype=np.uint8)
    rows = np.ascontiguousarray(rows, dtype=np.int32)
    M, K = a8.shape
    N = bt8.shape[0]
    assert bt8.shape[1] == K and K <= 16384
    out = np.empty((rows.size, N), dtype=np.uint16)
    lib().or_gemm_rows(_ptr(a8, _u8p), _ptr(bt8, _u8p), M, N, K, ctypes.c_float(a_scale),
                       ctypes.c_float(b_scale), _ptr(rows, _i32p), rows.size, _ptr(out, _u16p))
    return out


def num_threads() -> int:
    return int(lib().or_num_threads())
