"""GEMM oracle -- TEST INFRASTRUCTURE ONLY.

Restates kernels/hip/fp8_attn/fp8_gemm.hip:79-156: C = bf16(fp32(A8 @ B8) *
(a_scale * b_scale)), the scale product formed once in fp32 (:148) and
applied to the fp32 accumulator before a round-to-nearest-even bf16 cast
(:152).  The products of two e4m3 values are exact; the sum is accumulated
exactly (float64) and rounded to fp32 once, standing in for the MFMA's fp32
accumulator whose internal order is not observable.

Parity: pinned by the reference's known-answer tests
(tests/test_mfma_fragment_layout.py:262-315: all-ones -> K, small integers in
[-2, 2] exact) restated in tests/test_oracle_gemm.py, plus the C restatement
checked against this module.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle.quant import DECODE


def emulate(a8: np.ndarray, bt8: np.ndarray, a_scale: float, b_scale: float) -> torch.Tensor:
    """bf16 (M, N) = bf16(fp32(A8 @ B8) * a_scale*b_scale); bt8 is B8 transposed, (N, K)."""
    A = DECODE[a8].astype(np.float64)
    Bt = DECODE[bt8].astype(np.float64)
    acc = (A @ Bt.T).astype(np.float32)
    scale = np.float32(a_scale) * np.float32(b_scale)
    return torch.from_numpy(acc * scale).to(torch.bfloat16)
