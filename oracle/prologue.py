"""Fused QK-norm prologue oracle -- TEST INFRASTRUCTURE ONLY.

``rmsnorm_rope`` restates the normalisation the Cosmos/Wan attention
processors apply to Q and K before the FP8 path (reference
docs/walkthroughs/02-architecture.md:114-123: ``attn.norm_q`` / ``norm_k``,
diffusers' RMSNorm, then ``apply_rotary_emb(use_real=True)``), with the
fp32 operation order the gfx950 prologue commits to:

    ss  = x_0^2 + ... + x_7^2 per 8-element chunk, in order; then the chunk
          sums pairwise over chunk indices c and c ^ o, o = D/16, ..., 1
    r   = 1 / sqrt(ss * (1/D) + eps)              (IEEE sqrt, IEEE divide)
    n   = bf16(x * r); with a weight, n = bf16(n * w)
    y   = bf16(n * cos + rot(n) * sin)            three separate roundings

Every step is one correctly rounded fp32 operation, as numpy performs them.
Only the summation order is a choice: torch sums in its own order, so
torch's RMSNorm and this one can differ by one bf16 step where the fp32
value sits within a few fp32 ulps of a bf16 rounding boundary.
``quantize_prologue`` then applies the reference quantizer (``oracle.quant``)
to y.

Parity: pinned.  tests/test_oracle_prologue.py checks y against an fp64
RMSNorm (within one bf16 step everywhere), against torch's CPU restatement
(equal except for rare boundary cases, never more than one step), closed
forms (zero rows, constant rows, unit and power-of-two weights), and the
rotation with cos = 1, sin = 0 (identity) and cos = 0, sin = 1 (the pairing
and its signs, for both layouts).
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import quant

F32 = np.float32
ROPE_NONE, ROPE_HALF, ROPE_INTERLEAVED = 0, 1, 2


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> nearest-even bf16 value, as fp32 (NaN stays NaN)."""
    x = np.asarray(x, dtype=F32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(F32)
    return np.where(np.isnan(x), x, out).astype(F32)


def bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(F32)


def f32_to_bits(x: np.ndarray) -> np.ndarray:
    """bf16-exact fp32 values -> their bf16 bit patterns."""
    return (np.asarray(x, dtype=F32).view(np.uint32) >> 16).astype(np.uint16)


def rmsnorm_rope(x_bits: np.ndarray, eps: float, weight_bits: np.ndarray | None = None,
                 cos: np.ndarray | None = None, sin: np.ndarray | None = None,
                 rope: int = ROPE_NONE, mutation: str | None = None) -> np.ndarray:
    """y (bf16-exact fp32) for x bf16 bits of shape (..., S, D); cos/sin (S, D) fp32."""
    x = bits_to_f32(x_bits)
    D = x.shape[-1]
    chunks = x.reshape(x.shape[:-1] + (D // 8, 8))
    sq = (chunks * chunks).astype(F32)   # exact: a bf16 square has <= 16 bits
    ss = sq[..., 0]
    for i in range(1, 8):
        ss = (ss + sq[..., i]).astype(F32)
    o = D // 16
    while o >= 1:
        idx = np.arange(D // 8) ^ o
        ss = (ss + ss[..., idx]).astype(F32)
        o //= 2
    ss = ss[..., 0]
    mean = (ss * F32(1.0 / D)).astype(F32)
    r = (F32(1.0) / np.sqrt((mean + F32(eps)).astype(F32))).astype(F32)
    n = bf16_round(x * r[..., None])
    if weight_bits is not None:
        n = bf16_round(n * bits_to_f32(weight_bits))
    if rope == ROPE_NONE:
        return n
    if rope == ROPE_HALF:
        h = D // 2
        rot = np.concatenate([-n[..., h:], n[..., :h]], axis=-1)
    else:
        pairs = n.reshape(n.shape[:-1] + (D // 2, 2))
        rot = np.stack([-pairs[..., 1], pairs[..., 0]], axis=-1).reshape(n.shape)
    if mutation == "rope_sign":
        rot = -rot
    a = (n * cos).astype(F32)
    b = (rot * sin).astype(F32)
    if mutation == "rope_fma":   # n*cos + rot*sin contracted: one rounding fewer
        return bf16_round((a.astype(np.float64) + rot.astype(np.float64) * sin).astype(F32))
    return bf16_round((a + b).astype(F32))


def quantize_prologue(x: torch.Tensor, eps: float, weight: torch.Tensor | None = None,
                      cos: np.ndarray | None = None, sin: np.ndarray | None = None,
                      rope: int = ROPE_NONE, granularity: str = "bh"
                      ) -> tuple[np.ndarray, np.ndarray]:
    """(dequant scales, codes) of the fused prologue for a (B, H, S, D) bf16 tensor."""
    wb = None if weight is None else quant.bf16_bits(weight)
    y = rmsnorm_rope(quant.bf16_bits(x), eps, wb, cos, sin, rope)
    yt = torch.from_numpy(f32_to_bits(y).view(np.int16)).view(torch.bfloat16)
    return quant.quantize_codes(yt, granularity)
