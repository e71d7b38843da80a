"""Quantizer oracle -- TEST INFRASTRUCTURE ONLY.

``per_group_dequant`` / ``quantize`` restate the reference's OCP quantizer
(kernels/triton_kernels/fp8_flash_attn_hopper.py:374-398, the e4m3fn sibling
of the gfx942 fnuz code at kernels/triton_kernels/fp8_flash_attn.py:425-448)
with the same torch CPU operations, so they inherit torch's dtype flow:

* ``x.abs().amax()`` of a bf16 tensor is bf16, ``clamp(min=1e-6)`` clamps in
  bf16, and ``amax / (0.95*448)`` divides in fp32 and rounds back to bf16
  before ``.to(float32)``: the dequant scale carries bf16 precision.
* fp16 input follows the same dtype flow in fp16, with one difference of
  evaluation: on the GPU, torch's true-divide kernel computes
  ``tensor / cpu_scalar`` as ``tensor * (1 / scalar)`` with the reciprocal
  rounded to fp32 (ATen's BinaryDivTrueKernel), while its CPU kernel
  divides.  For bf16 both forms give the same scale for every amax value;
  for fp16 they differ on two values, so the fp16 scale is written out as
  the GPU evaluates it: fp16(max(amax, fp16(1e-6)) * RN(1/425.6)).
* ``1.0 / dequant`` is a correctly rounded fp32 reciprocal; the product with
  ``x.float()`` is one fp32 multiply; ``.to(float8_e4m3fn)`` rounds to
  nearest even.

The granularity is per (batch, head) -- the reference's -- or per tensor
(one group), the BASELINE wording; callers label which one they use.

``encode_e4m3fn`` / ``decode_e4m3fn`` are numpy implementations written from
the format definition (bias 7, 3 mantissa bits, S.1111.111 = NaN, max 448).

Parity: pinned.  tests/test_oracle_quant.py checks the encoder against torch's
cast over every sign/exponent/top-mantissa pattern with all rounding-relevant
low bits, the scale formula over every bf16 and fp16 amax value (both
evaluation forms), the C restatement against this module bit for bit, and
closed-form cases (zero groups, power-of-two scale invariance, clamp, NaN/Inf
propagation).  tests/test_gpu_quant.py checks the fp16 and bf16 scales
against the reference expression evaluated by torch on the GPU, for every
amax value.
"""

from __future__ import annotations

import numpy as np
import torch

FP8_E4M3FN_MAX = 448.0
FP8_E4M3FNUZ_MAX = 240.0


def per_group_dequant(x: torch.Tensor, granularity: str = "bh",
                      fp8_max: float = FP8_E4M3FN_MAX) -> torch.Tensor:
    """Dequant scale per group: (B*H,) for "bh", (1,) for "tensor".

    Follows fp8_flash_attn_hopper.py:381-385 (``_per_bh_scale``).
    """
    if granularity == "bh":
        B, H = x.shape[0], x.shape[1]
        flat = x.abs().reshape(B * H, -1)
    elif granularity == "tensor":
        flat = x.abs().reshape(1, -1)
    else:
        raise ValueError(f"unknown granularity {granularity!r}")
    amax = flat.amax(dim=1).clamp(min=1e-6)
    if x.dtype == torch.float16:
        # the GPU's evaluation of `amax / (0.95 * fp8_max)`: multiply by the
        # fp32 reciprocal of the scalar, round to fp16
        inv = (torch.tensor(1.0, dtype=torch.float32)
               / torch.tensor(0.95 * fp8_max, dtype=torch.float32)).to(amax.device)
        return (amax.to(torch.float32) * inv).to(torch.float16).to(torch.float32)
    return (amax / (0.95 * fp8_max)).to(torch.float32)


def quantize(x: torch.Tensor, dequant: torch.Tensor, granularity: str = "bh",
             fp8_dtype: torch.dtype = torch.float8_e4m3fn,
             fp8_max: float = FP8_E4M3FN_MAX) -> torch.Tensor:
    """e4m3 codes of ``x`` under the given dequant scales.

    Follows fp8_flash_attn_hopper.py:394-398 (``_quantize``).
    """
    if granularity == "bh":
        shape = (x.shape[0], x.shape[1]) + (1,) * (x.dim() - 2)
    else:
        shape = (1,) * x.dim()
    q_mul = (1.0 / dequant).reshape(shape)
    scaled = (x.to(torch.float32) * q_mul).clamp(-fp8_max, fp8_max)
    return scaled.to(fp8_dtype)


def quantize_codes(x: torch.Tensor, granularity: str = "bh") -> tuple[np.ndarray, np.ndarray]:
    """(dequant scales fp32, uint8 codes) for a bf16 or fp16 tensor, OCP e4m3fn."""
    dq = per_group_dequant(x, granularity)
    codes = quantize(x, dq, granularity).view(torch.uint8)
    return dq.numpy(), codes.numpy()


# ------------------------------------------------------------------ encoder
def encode_e4m3fn(x: np.ndarray) -> np.ndarray:
    """fp32 -> e4m3fn codes, round to nearest even, NaN for |x| that does
    not round to a finite e4m3 value (no saturation)."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    sign = ((u >> 24) & 0x80).astype(np.uint8)
    a = u & np.uint32(0x7FFFFFFF)
    mag = a.view(np.float32)
    out = np.zeros(x.shape, dtype=np.uint32)
    sub = mag < np.float32(2.0 ** -6)
    # subnormal quantum 2^-9; np.rint rounds half to even
    out[sub] = np.rint(mag[sub] * np.float32(512.0)).astype(np.uint32)
    nrm = ~sub
    an = a[nrm]
    exp32 = an >> 23
    mant = an & np.uint32(0x7FFFFF)
    keep = mant >> 20
    rest = mant & np.uint32(0xFFFFF)
    up = (rest > 0x80000) | ((rest == 0x80000) & ((keep & 1) == 1))
    with np.errstate(over="ignore"):
        out[nrm] = ((exp32.astype(np.int64) - 127 + 7) * 8 + keep + up).clip(0, 0x7F).astype(np.uint32)
    nan = (a > np.uint32(0x7F800000)) | (mag >= np.float32(480.0)) | (out >= 0x7F)
    out[nan] = 0x7F
    return (out.astype(np.uint8) | sign)


def decode_table() -> np.ndarray:
    """float32 value of each of the 256 e4m3fn codes (NaN for 0x7f/0xff)."""
    c = np.arange(256, dtype=np.uint32)
    e = (c >> 3) & 0xF
    m = (c & 7).astype(np.float64)
    mag = np.where(e == 0, m / 512.0, (1.0 + m / 8.0) * np.exp2(e.astype(np.float64) - 7.0))
    mag = np.where((e == 15) & ((c & 7) == 7), np.nan, mag)
    return np.where(c & 0x80, -mag, mag).astype(np.float32)


DECODE = decode_table()


def decode_e4m3fn(codes: np.ndarray) -> np.ndarray:
    return DECODE[np.asarray(codes, dtype=np.uint8)]


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    """Raw bf16 bit patterns of a CPU bf16 tensor as uint16."""
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)
