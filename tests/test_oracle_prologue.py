"""Pins of the fused QK-norm prologue oracle (oracle/prologue.py).

The normalisation is checked against fp64 and against torch's own RMSNorm
restatement (they may differ by one bf16 step where torch sums the squares in
another order); the weight multiply and the rotary step, which have no order
freedom, are checked bit for bit against torch restatements of diffusers'
RMSNorm weight step and apply_rotary_emb(use_real=True) with both unbind
layouts.  Planted mistakes (rotation sign, a contracted rotation) fail.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import prologue as P
from oracle import quant


def _x(seed: int, shape, scale: float = 1.0) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


def _tables(S: int, D: int, seed: int = 7) -> tuple[np.ndarray, np.ndarray]:
    rng = np.random.default_rng(seed)
    ang = rng.uniform(-40.0, 40.0, size=(S, D)).astype(np.float32)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def _ulp(v: np.ndarray) -> np.ndarray:
    a = np.maximum(np.abs(v.astype(np.float64)), 2.0 ** -126)
    return 2.0 ** (np.floor(np.log2(a)) - 7)


@pytest.mark.parametrize("D,scale", [(128, 1.0), (64, 1.0), (128, 1e-3), (128, 300.0)])
def test_rmsnorm_within_one_bf16_step_of_fp64(D: int, scale: float) -> None:
    x = _x(D, (2, 3, 257, D), scale)
    y = P.rmsnorm_rope(quant.bf16_bits(x), 1e-6)
    xd = x.double().numpy()
    exact = xd / np.sqrt((xd ** 2).mean(-1, keepdims=True) + 1e-6)
    err = np.abs(y - exact)
    assert (err <= _ulp(exact) * 0.5 + 1e-300).mean() > 0.999   # mostly the nearest bf16
    assert (err <= _ulp(exact) * 1.0 + 1e-300).all()


def test_rmsnorm_matches_torch_but_for_rare_boundary_cases() -> None:
    x = _x(3, (1, 4, 4096, 128))
    y = P.rmsnorm_rope(quant.bf16_bits(x), 1e-6)
    xf = x.float()
    ref = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
    ref = ref.float().numpy()
    diff = np.abs(y - ref)
    assert (diff == 0).mean() > 0.999
    assert (diff <= _ulp(ref)).all()


def test_closed_forms() -> None:
    D = 64
    zero = np.zeros((3, D), dtype=np.uint16)
    assert np.array_equal(P.rmsnorm_rope(zero, 1e-6), np.zeros((3, D), np.float32))
    const = quant.bf16_bits(torch.full((2, D), 3.0, dtype=torch.bfloat16))
    y = P.rmsnorm_rope(const, 0.0)
    assert np.array_equal(y, np.ones((2, D), np.float32))             # 3 / sqrt(9) = 1
    alt = torch.tensor([[2.0, -2.0] * (D // 2)], dtype=torch.bfloat16)
    assert np.array_equal(P.rmsnorm_rope(quant.bf16_bits(alt), 0.0),
                          np.array([[1.0, -1.0] * (D // 2)], np.float32))
    x = _x(5, (5, D))
    base = P.rmsnorm_rope(quant.bf16_bits(x), 1e-6)
    ones = quant.bf16_bits(torch.ones(D, dtype=torch.bfloat16))
    twos = quant.bf16_bits(torch.full((D,), 2.0, dtype=torch.bfloat16))
    assert np.array_equal(P.rmsnorm_rope(quant.bf16_bits(x), 1e-6, ones), base)
    assert np.array_equal(P.rmsnorm_rope(quant.bf16_bits(x), 1e-6, twos), 2 * base)


def test_weight_step_is_torch_bf16_multiply() -> None:
    x = _x(11, (3, 100, 128))
    w = _x(12, (128,), 0.5)
    n = torch.from_numpy(P.f32_to_bits(P.rmsnorm_rope(quant.bf16_bits(x), 1e-6))
                         .view(np.int16)).view(torch.bfloat16)
    y = P.rmsnorm_rope(quant.bf16_bits(x), 1e-6, quant.bf16_bits(w))
    assert np.array_equal(y, (n * w).float().numpy())


def _torch_rope(n: torch.Tensor, cos: np.ndarray, sin: np.ndarray, unbind_dim: int) -> np.ndarray:
    """diffusers apply_rotary_emb(use_real=True) restated in torch ops."""
    if unbind_dim == -1:
        re, im = n.reshape(*n.shape[:-1], -1, 2).unbind(-1)
        rot = torch.stack([-im, re], dim=-1).flatten(-2)
    else:
        re, im = n.reshape(*n.shape[:-1], 2, -1).unbind(-2)
        rot = torch.cat([-im, re], dim=-1)
    c, s = torch.from_numpy(cos), torch.from_numpy(sin)
    return (n.float() * c + rot.float() * s).to(torch.bfloat16).float().numpy()


@pytest.mark.parametrize("mode,unbind", [(P.ROPE_HALF, -2), (P.ROPE_INTERLEAVED, -1)])
@pytest.mark.parametrize("D", [64, 128])
def test_rope_step_is_apply_rotary_emb(mode: int, unbind: int, D: int) -> None:
    S = 300
    x = _x(20 + D, (2, 2, S, D))
    w = _x(21, (D,), 0.7)
    cos, sin = _tables(S, D)
    wb = quant.bf16_bits(w)
    n = torch.from_numpy(P.f32_to_bits(P.rmsnorm_rope(quant.bf16_bits(x), 1e-6, wb))
                         .view(np.int16)).view(torch.bfloat16)
    y = P.rmsnorm_rope(quant.bf16_bits(x), 1e-6, wb, cos, sin, mode)
    assert np.array_equal(y, _torch_rope(n, cos, sin, unbind))
    # identity and pure rotation: the pairing and its signs
    one, zero = np.ones((S, D), np.float32), np.zeros((S, D), np.float32)
    assert np.array_equal(P.rmsnorm_rope(quant.bf16_bits(x), 1e-6, wb, one, zero, mode),
                          n.float().numpy())
    rot = P.rmsnorm_rope(quant.bf16_bits(x), 1e-6, wb, zero, one, mode)
    nn = n.float().numpy()
    if mode == P.ROPE_HALF:
        assert np.array_equal(rot[..., :D // 2], -nn[..., D // 2:])
        assert np.array_equal(rot[..., D // 2:], nn[..., :D // 2])
    else:
        assert np.array_equal(rot[..., 0::2], -nn[..., 1::2])
        assert np.array_equal(rot[..., 1::2], nn[..., 0::2])


@pytest.mark.parametrize("mutation", ["rope_sign", "rope_fma"])
def test_planted_rope_mistakes_fail_the_pin(mutation: str) -> None:
    S, D = 300, 128
    x = _x(40, (1, 2, S, D))
    cos, sin = _tables(S, D)
    n = torch.from_numpy(P.f32_to_bits(P.rmsnorm_rope(quant.bf16_bits(x), 1e-6))
                         .view(np.int16)).view(torch.bfloat16)
    bad = P.rmsnorm_rope(quant.bf16_bits(x), 1e-6, None, cos, sin, P.ROPE_HALF,
                         mutation=mutation)
    assert not np.array_equal(bad, _torch_rope(n, cos, sin, -2))


def test_quantize_prologue_is_the_quantizer_of_y() -> None:
    x = _x(50, (1, 3, 200, 64), 4.0)
    dq, codes = P.quantize_prologue(x, 1e-6)
    y = P.rmsnorm_rope(quant.bf16_bits(x), 1e-6)
    yt = torch.from_numpy(P.f32_to_bits(y).view(np.int16)).view(torch.bfloat16)
    dq2, codes2 = quant.quantize_codes(yt, "bh")
    assert np.array_equal(dq, dq2) and np.array_equal(codes, codes2)
    # RMS-normalised rows have |y| <= sqrt(D): amax = 8 at most for D = 64
    assert float(np.max(np.abs(y))) <= 8.0


@pytest.mark.parametrize("D", [64, 128, 256])
def test_c_rmsnorm_equals_numpy_restatement(D: int) -> None:
    """oracle/c or_rmsnorm_bf16_rows (used for full-size per-tensor scales) is
    the numpy restatement bit for bit, on rows that stress the summation
    order: mixed magnitudes inside a row, zero rows (r = 1/sqrt(eps)), rows
    whose squares overflow (r = 0) or underflow, and a single large entry."""
    from oracle import native

    x = _x(D + 11, (3, 5, 130, D)).float()
    x[0, 0, :, : D // 2] *= 1e3                      # order-sensitive sums
    x[0, 1, 3] = 0.0
    x[0, 2, 4] = 1e30
    x[1, 0, 5] *= 1e-25
    x[1, 1, 6] = 0.0
    x[1, 1, 6, 7] = 5.0
    bits = quant.bf16_bits(x.to(torch.bfloat16))
    for eps in (1e-6, 0.0, 1e-2):
        ref = P.f32_to_bits(P.rmsnorm_rope(bits, eps))
        got = native.rmsnorm_bf16(bits, eps)
        assert np.array_equal(got, ref), (D, eps, int((got != ref).sum()))


def test_c_rmsnorm_planted_order_change_is_caught() -> None:
    """A different summation order (plain left-to-right over the row) changes
    some bf16 results on order-sensitive rows, so the pin above can tell."""
    from oracle import native

    x = _x(5, (1, 1, 4096, 128)).float()
    x[..., ::3] *= 1e3
    bits = quant.bf16_bits(x.to(torch.bfloat16))
    got = P.bits_to_f32(native.rmsnorm_bf16(bits, 1e-6))
    xf = P.bits_to_f32(bits)
    ss = np.zeros(xf.shape[:-1], dtype=np.float32)
    for d in range(128):
        ss = (ss + xf[..., d] * xf[..., d]).astype(np.float32)
    r = (np.float32(1.0) / np.sqrt((ss * np.float32(1 / 128) + np.float32(1e-6))
                                   .astype(np.float32))).astype(np.float32)
    naive = P.bf16_round(xf * r[..., None])
    assert not np.array_equal(got, naive)
