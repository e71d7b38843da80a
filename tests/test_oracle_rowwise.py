"""Pins of the row-wise quantizer and unfused FP8 attention oracle (oracle/rowwise.py).

Reference: src/repercep/attention/fp8_scaled_mm.py:107-133 (``_rowwise_quantize``)
and :135-221 (``FP8ScaledMMAttention.__call__``), in the OCP e4m3fn format.
The pins are hand-derived codes, the closed form of a row's largest element,
invariants (powers of two, row independence), the e4m3 rounding bound, and
special rows; each planted mistake of ``rowwise_quantize`` fails one of them.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import rowwise
from oracle.quant import decode_e4m3fn

MUTATIONS = ("perbh_mul", "fp32_mul", "target448", "axis0")


def _rows(seed: int, n: int = 64, cols: int = 128, dtype=torch.bfloat16) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    # fp16 rows keep amax above 425.6 / 65504, where fp16(1/amax) * 425.6 is finite
    lo, hi = (-4, 4) if dtype == torch.bfloat16 else (-2, 3)
    mag = torch.logspace(lo, hi, n).reshape(n, 1)
    return (torch.randn(n, cols, generator=g) * mag).to(dtype)


# ------------------------------------------------------------------ pins
def pin_known_answers(fn) -> bool:
    """Codes derived by hand.  Row 0, bf16: amax 1, 1/amax = 1, qmul =
    bf16(425.6) = 426; 0.7890625 * 426 = 336.14 rounds up to 352 (0x7B), where
    the per-(b,h) multiplier 1/bf16(1/425.6) = 425.56 gives 335.8 -> 320.
    Row 1: amax 1.75, bf16(1/1.75) = 0.5703125, qmul = bf16(242.725) = 243;
    1.25 * 243 = 303.75 -> 288 (0x79), where the fp32 multiplier 243.2 gives the
    tie 304 -> 320.  Dequant scales: bf16(1/425.6) and bf16(1.75/425.6)."""
    x = torch.tensor([[1.0, 0.7890625, -0.5, 0.0, 0.125, 0.0, 0.0, 0.0],
                      [1.75, 1.25, -1.75, 0.875, 0.0, 0.0, 0.0, 0.0]], dtype=torch.bfloat16)
    codes, dq = fn(x)
    want = np.array([[0x7D, 0x7B, 0xF5, 0x00, 0x65, 0, 0, 0],
                     [0x7D, 0x79, 0xFD, 0x75, 0x00, 0, 0, 0]], dtype=np.uint8)
    return (np.array_equal(codes.numpy(), want)
            and dq.tolist() == [0.002349853515625, 0.004119873046875])


def pin_row_max_is_416(fn) -> bool:
    """x_max * qmul = amax * dtype(dtype(1/amax) * 425.6) lies within two
    dtype roundings (< 1%) of 425.6, between the e4m3 midpoints 400 and 432:
    every row's largest element is code 0x7D (416), with its sign."""
    for dtype in (torch.bfloat16, torch.float16):
        x = _rows(3, dtype=dtype)
        codes, _ = fn(x)
        idx = x.float().abs().argmax(dim=-1)
        c = codes.numpy()[np.arange(x.shape[0]), idx.numpy()]
        if not np.all((c & 0x7F) == 0x7D):
            return False
    return True


def pin_power_of_two_invariance(fn) -> bool:
    """Scaling a row by 2^k leaves its codes unchanged and scales its dequant
    by 2^k (while the amax stays clear of the 1e-6 clamp and of overflow)."""
    x = _rows(5, n=16, dtype=torch.bfloat16)[4:12]
    c0, d0 = fn(x)
    for k in (-6, -1, 3, 9):
        ck, dk = fn((x.float() * 2.0 ** k).to(torch.bfloat16))
        if not (torch.equal(ck, c0) and torch.equal(dk, d0 * 2.0 ** k)):
            return False
    return True


def pin_rows_independent(fn) -> bool:
    """A row's codes and scale depend on that row alone."""
    x = _rows(7, n=32)
    c, d = fn(x)
    perm = torch.randperm(32, generator=torch.Generator().manual_seed(1))
    cp, dp = fn(x[perm])
    y = x.clone()
    y[5] *= 64
    cy, dy = fn(y)
    keep = torch.arange(32) != 5
    return (torch.equal(cp, c[perm]) and torch.equal(dp, d[perm])
            and torch.equal(cy[keep], c[keep]) and torch.equal(dy[keep], d[keep]))


def pin_rounding_bound(fn) -> bool:
    """Every code is the nearest e4m3 value of x * qmul, qmul = 425.6 / amax
    within 1%: decoding, dividing by 425.6 / amax and comparing with x leaves
    at most half an e4m3 step (2^-4 relative, 2^-10 absolute in codes) plus the
    multiplier's 1%."""
    x = _rows(9, n=48, cols=64)
    codes, _ = fn(x)
    xf = x.float().numpy()
    amax = np.abs(xf).max(axis=-1, keepdims=True)
    qm = 425.6 / amax
    got = decode_e4m3fn(codes.numpy()) / qm
    tol = (2.0 ** -4 + 0.011) * np.abs(xf) + 2.0 ** -10 / qm + 1e-30
    return bool(np.all(np.abs(got - xf) <= tol))


PINS = (pin_known_answers, pin_row_max_is_416, pin_power_of_two_invariance,
        pin_rows_independent, pin_rounding_bound)


@pytest.mark.parametrize("pin", PINS, ids=[p.__name__ for p in PINS])
def test_oracle_satisfies_pin(pin) -> None:
    assert pin(rowwise.rowwise_quantize)


@pytest.mark.parametrize("mutation", MUTATIONS)
def test_planted_mistake_fails_a_pin(mutation: str) -> None:
    fn = lambda x: rowwise.rowwise_quantize(x, mutation=mutation)   # noqa: E731
    failed = [p.__name__ for p in PINS if not p(fn)]
    assert failed, f"mutation {mutation!r} passes every pin"


def test_fp16_known_answer() -> None:
    """fp16 flow: qmul = fp16(fp16(1/1) * 425.6) = 425.5 (fp16 spacing 0.25), so
    0.7890625 * 425.5 = 335.74 -> 320 (0x7A), unlike bf16's 0x7B; dequant
    fp16(1 * fp32(1/425.6)) = 1232 * 2^-19."""
    x = torch.tensor([[1.0, 0.7890625, 0.0, -0.25, 0.0, 0.0, 0.0, 0.0]], dtype=torch.float16)
    codes, dq = rowwise.rowwise_quantize(x)
    # -0.25 * 425.5 = -106.375 -> -104 (0xED)
    assert codes.numpy().tolist() == [[0x7D, 0x7A, 0x00, 0xED, 0, 0, 0, 0]]
    assert dq.item() == 1232 * 2.0 ** -19


def test_fp16_small_rows_saturate_like_the_reference() -> None:
    """fp16 rows with amax below 425.6 / 65504: the multiplier fp16(fp16(1/amax)
    * 425.6) overflows to inf, so every nonzero element becomes +-448 (0x7E)
    and zeros NaN (0 * inf) -- what the reference's fp16 flow does."""
    x = torch.tensor([[1e-3, -5e-4, 0.0, 2e-4, 0.0, 0.0, 0.0, 0.0]], dtype=torch.float16)
    codes, dq = rowwise.rowwise_quantize(x)
    c = codes.numpy()[0]
    assert c[[0, 1, 3]].tolist() == [0x7E, 0xFE, 0x7E]
    assert ((c[[2, 4, 5, 6, 7]] & 0x7F) == 0x7F).all()      # NaN, sign unspecified
    assert 0 < dq.item() < 1e-5


def test_special_rows() -> None:
    """Zero row: amax clamps to bf16(1e-6), codes 0.  NaN anywhere: NaN amax,
    every code NaN.  An infinite element: amax inf, qmul 0, finite elements
    code +-0 and the infinite one NaN (inf * 0).  A NaN code's sign is not
    specified (x86 and the GPU give opposite signs for 0 * inf)."""
    x = torch.zeros(3, 8, dtype=torch.bfloat16)
    x[1] = torch.linspace(-1, 1, 8)
    x[1, 2] = float("nan")
    x[2] = torch.linspace(-1, 1, 8)
    x[2, 7] = float("inf")
    codes, dq = rowwise.rowwise_quantize(x)
    c = codes.numpy()
    assert (c[0] == 0).all()
    assert dq[0].item() == torch.tensor(
        torch.tensor(1e-6, dtype=torch.bfloat16).item() / 425.6).to(torch.bfloat16).item()
    assert ((c[1] & 0x7F) == 0x7F).all() and math.isnan(dq[1].item())
    assert ((c[2, :7] & 0x7F) == 0).all() and (c[2, 7] & 0x7F) == 0x7F
    assert math.isinf(dq[2].item())


# ------------------------------------------------------ unfused attention
def test_grouped_scaled_mm_exact_on_integers() -> None:
    """Integer codes and power-of-two scales: every sum and product is exact,
    so the result is the integer product scaled, rounded to bf16 once."""
    g = torch.Generator().manual_seed(2)
    a = torch.randint(-3, 4, (2, 24, 64), generator=g).float()
    b = torch.randint(-3, 4, (2, 16, 64), generator=g).float()
    sa = 2.0 ** torch.randint(-4, 4, (2, 24), generator=g).float()
    sb = 2.0 ** torch.randint(-4, 4, (2, 16), generator=g).float()
    got = rowwise.grouped_scaled_mm(a.to(torch.float8_e4m3fn).view(torch.uint8).numpy(),
                                    b.to(torch.float8_e4m3fn).view(torch.uint8).numpy(),
                                    sa.numpy(), sb.numpy())
    want = ((a @ b.transpose(1, 2)) * sa[:, :, None] * sb[:, None, :]).to(torch.bfloat16)
    assert torch.equal(got, want)


def _exact_attention(q, k, v, causal: bool, scale: float) -> np.ndarray:
    qd, kd, vd = (t.double().numpy() for t in (q, k, v))
    s = np.einsum("bhqd,bhkd->bhqk", qd, kd) * scale
    if causal:
        sq, skv = s.shape[-2:]
        s = np.where(np.tril(np.ones((sq, skv), dtype=bool)), s, -np.inf)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("bhqk,bhkd->bhqd", p, vd)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("qk_div", [8.0, 1.0])
def test_unfused_attention_within_fp8_noise_of_exact(causal: bool, qk_div: float) -> None:
    """The reference's acceptance regime (tests/test_attention_fp8.py:77-101:
    Q, K = randn/8, mean relative error vs SDPA < 0.30) and unscaled Q, K:
    the oracle is within a few percent of the fp64 softmax attention; with
    unscaled Q, K a dropped temperature or mask lands far outside that."""
    g = torch.Generator().manual_seed(11)
    q = (torch.randn(1, 2, 128, 64, generator=g) / qk_div).to(torch.bfloat16)
    k = (torch.randn(1, 2, 128, 64, generator=g) / qk_div).to(torch.bfloat16)
    v = torch.randn(1, 2, 128, 64, generator=g).to(torch.bfloat16)
    scale = 64 ** -0.5
    exact = _exact_attention(q, k, v, causal, scale)
    out = rowwise.scaled_mm_attention(q, k, v, causal=causal).float().numpy()
    rel = np.abs(out - exact).mean() / np.abs(exact).mean()
    assert rel < 0.06, rel
    if qk_div == 1.0:
        sharp = _exact_attention(q, k, v, causal, 1.0)       # a dropped temperature
        assert np.abs(sharp - exact).mean() / np.abs(exact).mean() > 4 * rel
        if causal:
            full = _exact_attention(q, k, v, False, scale)   # a dropped mask
            assert np.abs(full - exact).mean() / np.abs(exact).mean() > 4 * rel
