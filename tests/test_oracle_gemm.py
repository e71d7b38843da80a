"""Pins of the GEMM oracle (CPU only).

The oracle restates kernels/hip/fp8_attn/fp8_gemm.hip:79-156,
C = bf16(fp32(A8 @ B8) * (a_scale * b_scale)), in numpy (oracle/gemm.py) and
C (oracle/c/fp8_oracle.c).  The reference's own known-answer tests
(tests/test_mfma_fragment_layout.py:262-315) are restated here against the
oracle: all-ones operands sum to K, and small-integer operands give the
exact integer product.  The epilogue scale and the agreement of the two
restatements are pinned beside them.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gemm, native, quant


def _codes(x: np.ndarray) -> np.ndarray:
    return quant.encode_e4m3fn(np.asarray(x, dtype=np.float32))


def _bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def _both(a8: np.ndarray, bt8: np.ndarray, sa: float, sb: float) -> tuple[np.ndarray, np.ndarray]:
    ref = gemm.emulate(a8, bt8, sa, sb).float().numpy()
    rows = np.arange(a8.shape[0])
    c = _bf16_to_f32(native.gemm_rows(a8, bt8, sa, sb, rows))
    return ref, c


@pytest.mark.parametrize("K", [64, 128, 256])
def test_all_ones_sum_to_k(K: int) -> None:
    """test_mfma_fragment_layout.py:262-285: A = B = 1 -> every C == K."""
    a8 = _codes(np.ones((16, K)))
    bt8 = _codes(np.ones((16, K)))
    for out in _both(a8, bt8, 1.0, 1.0):
        assert (out == K).all()


def test_small_integers_exact() -> None:
    """test_mfma_fragment_layout.py:288-315: integers in [-2, 2] give the exact product."""
    g = torch.Generator().manual_seed(0)
    a = torch.randint(-2, 3, (32, 64), generator=g).float()
    b = torch.randint(-2, 3, (64, 32), generator=g).float()
    want = (a @ b).to(torch.bfloat16).float().numpy()
    a8 = _codes(a.numpy())
    bt8 = _codes(b.t().contiguous().numpy())
    for out in _both(a8, bt8, 1.0, 1.0):
        assert np.array_equal(out, want)


def test_scales_multiply_the_accumulator() -> None:
    a8 = _codes(np.ones((4, 128)))
    bt8 = _codes(np.ones((8, 128)))
    for out in _both(a8, bt8, 0.5, 3.0):
        assert (out == 192.0).all()


def test_random_codes_numpy_and_c_agree_and_match_fp32_matmul() -> None:
    rng = np.random.default_rng(3)
    a = rng.standard_normal((48, 512)).astype(np.float32) * 50
    b = rng.standard_normal((40, 512)).astype(np.float32) * 50
    a8, bt8 = _codes(a), _codes(b)
    ref, c = _both(a8, bt8, 0.01, 0.02)
    assert np.array_equal(ref, c)
    # an independent library product of the decoded operands, fp32
    A = torch.from_numpy(quant.decode_e4m3fn(a8))
    Bt = torch.from_numpy(quant.decode_e4m3fn(bt8))
    lib = ((A @ Bt.t()) * (np.float32(0.01) * np.float32(0.02))).numpy()
    assert np.allclose(ref, lib, rtol=2 ** -7, atol=1e-3)


def test_oracle_reproduces_golden_vectors() -> None:
    """Both restatements reproduce the committed known-answer vectors (the
    reference test's exact regime) bit for bit."""
    from tests._helpers import golden_gemm_cases

    cases = golden_gemm_cases()
    assert len(cases) == 4
    for name, a8, b8, sa, sb, c_bits in cases:
        bt8 = np.ascontiguousarray(b8.T)
        emu = gemm.emulate(a8, bt8, sa, sb).view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(emu, c_bits), name
        rows = native.gemm_rows(a8, bt8, sa, sb, np.arange(a8.shape[0]))
        assert np.array_equal(rows, c_bits), name
