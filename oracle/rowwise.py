"""Row-wise FP8 quantizer and unfused FP8 attention oracle -- TEST INFRASTRUCTURE ONLY.

``rowwise_quantize`` restates ``_rowwise_quantize`` of the reference's unfused
FP8 attention (src/repercep/attention/fp8_scaled_mm.py:107-133) with the same
torch CPU operations, in the OCP e4m3fn format: FP8_MAX 448 and
``torch.float8_e4m3fn`` where the gfx942 code has 240 and e4m3fnuz -- the
adaptation the OCP siblings of the per-(b,h) quantizer make
(kernels/triton_kernels/fp8_flash_attn_hopper.py:374-398).  Its dtype flow:

* ``x.abs().amax(dim=-1).clamp(min=1e-6)`` stays in the input dtype;
* ``target / amax`` is ``amax.reciprocal() * target`` (torch's
  ``Tensor.__rdiv__``): the reciprocal and the product each round to the input
  dtype, so the multiplier carries 8 (bf16) or 11 (fp16) bits;
* ``amax / target`` is the per-(b,h) dequant scale; for fp16 it is written out
  as the GPU evaluates a tensor-by-CPU-scalar division (a multiply by the
  fp32 reciprocal), as ``oracle.quant`` does;
* ``(x.float() * quant_mul).clamp(-448, 448).to(float8_e4m3fn)`` rounds to
  nearest even.

``scaled_mm_attention`` restates ``FP8ScaledMMAttention.__call__`` (:135-221):
row-wise Q and K, ``torch._scaled_grouped_mm`` as the exact product scaled
per row and column (``grouped_scaled_mm``: fp32(fp32(acc) * s_a[m]) * s_b[n],
rounded to bf16 once), ``scores * scale`` in bf16, the causal mask,
``torch.softmax`` in bf16, row-wise P, V transposed and quantized per row of
V^T, and the second grouped product.

Parity: ``rowwise_quantize`` is pinned (tests/test_oracle_rowwise.py) by
hand-derived codes of one row, the closed form of a row's largest element
(always code 0x7D = 416: x_max * qmul lies within 1% of 425.6), scale
invariance under powers of two, per-row independence, the e4m3 rounding bound
of every element, zero and NaN rows, and planted mistakes (the per-(b,h)
multiplier, an fp32 multiplier, the 448 target, the wrong axis, no clamp)
that each fail one of them.  ``scaled_mm_attention`` is pinned against an
fp64 softmax attention of the unquantized inputs within FP8 noise and by its
parts (``grouped_scaled_mm`` against an integer product, exact).  The bit
patterns of hipBLASLt's grouped-GEMM epilogue and of torch's GPU softmax are
parity unpinned: outputs are compared within tolerance.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from oracle.quant import DECODE

FP8_MAX = 448.0


def rowwise_quantize(x: torch.Tensor, fp8_max: float = FP8_MAX, *, mutation: str | None = None
                     ) -> tuple[torch.Tensor, torch.Tensor]:
    """(codes uint8 x.shape, dequant fp32 x.shape[:-1]) for a CPU bf16/fp16 tensor.

    ``mutation`` plants a mistake for the pin tests: "perbh_mul" (x * fp32(1 /
    dequant), the per-(b,h) quantizer's multiplier), "fp32_mul" (the
    multiplier left in fp32), "target448", "axis0" (amax over the first axis),
    "no_clamp".
    """
    target = (1.0 if mutation == "target448" else 0.95) * fp8_max
    axis = 0 if mutation == "axis0" else -1
    amax = x.abs().amax(dim=axis, keepdim=True).clamp(min=1e-6)
    if x.dtype == torch.float16:
        inv = torch.tensor(1.0, dtype=torch.float32) / torch.tensor(target, dtype=torch.float32)
        dequant = (amax.to(torch.float32) * inv).to(torch.float16)
    else:
        dequant = amax / target
    if mutation == "perbh_mul":
        quant_mul = 1.0 / dequant.to(torch.float32)
    elif mutation == "fp32_mul":
        quant_mul = target / amax.to(torch.float32)
    else:
        quant_mul = target / amax          # amax.reciprocal() * target, in x's dtype
    scaled = x.to(torch.float32) * quant_mul.to(torch.float32)
    if mutation != "no_clamp":
        scaled = scaled.clamp(-fp8_max, fp8_max)
    codes = scaled.to(torch.float8_e4m3fn).view(torch.uint8)
    return codes, dequant.to(torch.float32).squeeze(axis)


def grouped_scaled_mm(a8: np.ndarray, bt8: np.ndarray, sa: np.ndarray, sb: np.ndarray
                      ) -> torch.Tensor:
    """bf16 (Z, M, N) = bf16(fp32(fp32(A8 . B8) * sa[m]) * sb[n]) for A8 (Z, M, K),
    B^T (Z, N, K) codes and scales (Z, M), (Z, N): the exact product, rounded to
    fp32 once, scaled by the row's then the column's scale."""
    A = DECODE[a8].astype(np.float64)
    Bt = DECODE[bt8].astype(np.float64)
    acc = np.einsum("zmk,znk->zmn", A, Bt).astype(np.float32)
    t = (acc * sa.astype(np.float32)[:, :, None]).astype(np.float32)
    t = (t * sb.astype(np.float32)[:, None, :]).astype(np.float32)
    return torch.from_numpy(t).to(torch.bfloat16)


def softmax_probs(scores_raw: torch.Tensor, scale: float, causal: bool) -> torch.Tensor:
    """P of fp8_scaled_mm.py:159-166: bf16 scores times the temperature, the
    causal mask (key j visible to query i iff j <= i), torch.softmax in bf16."""
    scores = scores_raw * scale
    if causal:
        sq, skv = scores.shape[-2:]
        mask = torch.ones(sq, skv, dtype=torch.bool).triu(1)
        scores = scores.masked_fill(mask, float("-inf"))
    return torch.softmax(scores, dim=-1)


def scaled_mm_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
                        causal: bool = False, scale: float | None = None) -> torch.Tensor:
    """(B, H, Sq, D) output of FP8ScaledMMAttention.__call__ (fp8_scaled_mm.py:135-221),
    OCP e4m3fn, for CPU (B, H, S, D) inputs."""
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    b, h, sq, d = q.shape
    skv = k.shape[2]
    bh = b * h
    cdt = torch.bfloat16
    qb = q.to(cdt).reshape(bh, sq, d)
    kb = k.to(cdt).reshape(bh, skv, d)
    vb = v.to(cdt).reshape(bh, skv, d)
    q8, qs = rowwise_quantize(qb)
    k8, ks = rowwise_quantize(kb)
    scores_raw = grouped_scaled_mm(q8.numpy(), k8.numpy(), qs.numpy(), ks.numpy())
    p = softmax_probs(scores_raw, scale, causal)
    p8, ps = rowwise_quantize(p)
    vt = vb.transpose(-1, -2).contiguous()
    vt8, vs = rowwise_quantize(vt)
    out = grouped_scaled_mm(p8.numpy(), vt8.numpy(), ps.numpy(), vs.numpy())
    return out.reshape(b, h, sq, d).to(q.dtype)
