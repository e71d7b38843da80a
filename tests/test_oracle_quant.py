"""Pins of the quantizer oracle (CPU only).

The oracle restates _per_bh_scale / _quantize of
kernels/triton_kernels/fp8_flash_attn_hopper.py:374-398 twice: with the same
torch CPU operations (oracle/quant.py) and in plain C (oracle/c/fp8_oracle.c,
the checker the GPU tests use at full size).  These tests pin both against
torch's own e4m3fn cast, against each other, and against closed forms that a
plausible mistake would break:

* the e4m3fn encoders against ``Tensor.to(torch.float8_e4m3fn)`` over every
  sign / exponent / 12 top mantissa bits combination with the low 11 bits set
  to the patterns that decide round-to-nearest-even (zero, one, just below,
  at and just above the half, all ones) -- a truncating or round-half-up
  encoder fails here;
* the scale formula over all 65536 bf16 amax values against the torch
  restatement -- an fp32 (not bf16) divide, a missing clamp or a 448 divisor
  fails here;
* closed forms: the group's largest element always lands on code 0x7D (416),
  all-zero groups, NaN/Inf propagation, -0.0, power-of-two invariance.

The ``*_catches_planted_mistake`` tests plant each of those mistakes in a copy
of the oracle and check that a pin fails.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import native, quant

F8 = torch.float8_e4m3fn


def _structured_fp32() -> np.ndarray:
    """Every sign x exponent x top-12 mantissa bits, with 6 low-bit patterns."""
    sign = np.array([0, 1], dtype=np.uint32) << 31
    exp = np.arange(256, dtype=np.uint32) << 23
    hi = np.arange(1 << 12, dtype=np.uint32) << 11
    lo = np.array([0, 1, 0x3FF, 0x400, 0x401, 0x7FF], dtype=np.uint32)
    u = (sign[:, None, None, None] | exp[None, :, None, None] | hi[None, None, :, None]
         | lo[None, None, None, :]).ravel()
    return u.view(np.float32)


def _torch_codes(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x).to(F8).view(torch.uint8).numpy()


def _same_codes(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Equal codes, treating any two NaN codes (0x7F / 0xFF) as equal."""
    nan_a = (a & 0x7F) == 0x7F
    nan_b = (b & 0x7F) == 0x7F
    return (a == b) | (nan_a & nan_b)


@pytest.fixture(scope="module")
def structured() -> tuple[np.ndarray, np.ndarray]:
    x = _structured_fp32()
    return x, _torch_codes(x)


def test_numpy_encoder_matches_torch_cast(structured: tuple[np.ndarray, np.ndarray]) -> None:
    x, ref = structured
    got = quant.encode_e4m3fn(x)
    bad = ~_same_codes(got, ref)
    assert not bad.any(), f"{bad.sum()} mismatches, first x={x[bad][:4]}"


def test_c_encoder_matches_torch_cast(structured: tuple[np.ndarray, np.ndarray]) -> None:
    x, ref = structured
    got = native.encode_e4m3fn(x)
    bad = ~_same_codes(got, ref)
    assert not bad.any(), f"{bad.sum()} mismatches, first x={x[bad][:4]}"


def test_encoder_known_codes() -> None:
    """Hand-derived codes from the format (bias 7, 3 mantissa bits)."""
    cases = [
        (0.0, 0x00), (-0.0, 0x80), (1.0, 0x38), (-1.0, 0xB8), (448.0, 0x7E), (-448.0, 0xFE),
        (2.0 ** -6, 0x08),          # smallest normal
        (2.0 ** -9, 0x01),          # smallest subnormal
        (2.0 ** -10, 0x00),         # tie between 0 and 2^-9 -> even (0)
        (3 * 2.0 ** -10, 0x02),     # tie between 1 and 2 quanta -> even (2)
        (1.0625, 0x38),             # tie between 1.0 and 1.125 -> even mantissa (1.0)
        (1.1875, 0x3A),             # tie between 1.125 and 1.25 -> even (1.25)
        (464.0, 0x7E),              # tie between 448 and (NaN slot 480) -> 448
        (465.0, 0x7F),              # rounds past 448 -> NaN, no saturation
        (416.0, 0x7D), (425.6, 0x7D), (432.0, 0x7E),
    ]
    x = np.array([c[0] for c in cases], dtype=np.float32)
    want = np.array([c[1] for c in cases], dtype=np.uint8)
    assert np.array_equal(quant.encode_e4m3fn(x), want)
    assert np.array_equal(native.encode_e4m3fn(x), want)
    assert np.array_equal(_torch_codes(x), want)


def test_decode_table_round_trips() -> None:
    codes = np.arange(256, dtype=np.uint8)
    vals = quant.decode_e4m3fn(codes)
    finite = ~np.isnan(vals)
    assert finite.sum() == 254                     # 0x7F and 0xFF are the NaNs
    assert np.array_equal(quant.encode_e4m3fn(vals[finite]), codes[finite])
    c_vals = np.array([native.lib().or_e4m3fn_decode(int(c)) for c in codes], dtype=np.float32)
    assert np.array_equal(np.isnan(c_vals), ~finite)
    assert np.array_equal(c_vals[finite], vals[finite])
    assert vals[0x7E] == 448.0 and vals[0x01] == 2.0 ** -9


def _all_bf16() -> torch.Tensor:
    return torch.from_numpy(np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.int16)
                            ).view(torch.bfloat16)


def _torch_dequant_per_value(vals: torch.Tensor) -> np.ndarray:
    """The reference's scale expression applied to each value as its own amax."""
    amax = vals.abs().reshape(-1, 1).amax(dim=1).clamp(min=1e-6)
    return (amax / (0.95 * 448.0)).to(torch.float32).numpy()


def _scales_equal(a: np.ndarray, b: np.ndarray) -> bool:
    a = np.asarray(a, dtype=np.float32)
    b = np.asarray(b, dtype=np.float32)
    return bool(((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))).all())


def test_scale_formula_every_bf16_amax() -> None:
    vals = _all_bf16()
    ref = _torch_dequant_per_value(vals)
    amax_bits = vals.abs().view(torch.int16).numpy().view(np.uint16)
    c = np.array([native.dequant_from_amax(int(b)) for b in amax_bits], dtype=np.float32)
    assert _scales_equal(c, ref)
    # the dequant scale carries bf16 precision: its low 16 bits are zero
    fin = np.isfinite(ref)
    assert not (ref[fin].view(np.uint32) & 0xFFFF).any()


def test_bf16_scale_divide_and_reciprocal_forms_agree() -> None:
    """torch's GPU kernel takes ``amax / 425.6`` as ``amax * RN(1/425.6f)``,
    its CPU kernel divides; for bf16 the rounded scales agree on every amax
    value, so the CPU restatement is the GPU's too."""
    lo = torch.tensor(1e-6).to(torch.bfloat16).item()
    vals = _all_bf16().abs().to(torch.float32)
    vals = torch.where(vals.isnan(), vals, vals.clamp(min=lo))
    a = vals.numpy()
    inv = np.float32(1.0) / np.float32(425.6)
    div = torch.from_numpy((a / np.float32(425.6)).astype(np.float32)).to(torch.bfloat16)
    mul = torch.from_numpy((a * inv).astype(np.float32)).to(torch.bfloat16)
    assert torch.equal(div.view(torch.int16), mul.view(torch.int16))


def _all_f16() -> torch.Tensor:
    """Every non-negative fp16 value from +0 to +inf, then one NaN."""
    bits = np.concatenate([np.arange(0, 0x7C01), [0x7E00]]).astype(np.uint16)
    return torch.from_numpy(bits.view(np.int16)).view(torch.float16)


def test_fp16_scale_every_amax() -> None:
    """The fp16 scale over every amax value against an independent numpy
    restatement of the GPU's evaluation, fp16(max(a, fp16(1e-6)) * RN(1/425.6))."""
    vals = _all_f16()
    n = vals.numel()
    got = quant.per_group_dequant(vals.reshape(1, n, 1, 1)).numpy()
    a = vals.to(torch.float32).numpy()
    lo = np.float32(np.float16(1e-6))
    assert lo == np.float32(17 * 2.0 ** -24)
    a = np.where(np.isnan(a), a, np.maximum(a, lo))
    want = (a * (np.float32(1.0) / np.float32(425.6))).astype(np.float32)
    want = want.astype(np.float16).astype(np.float32)
    assert _scales_equal(got, want)
    # the division form (torch's CPU kernel) departs from it on exactly two
    # amax values: a restatement that divided would fail the GPU pin there
    div = (vals.clamp(min=1e-6) / (0.95 * 448.0)).to(torch.float32).numpy()
    differ = ~((div.view(np.uint32) == want.view(np.uint32)) | (np.isnan(div) & np.isnan(want)))
    assert int(differ.sum()) == 2
    # maxima below ~1.3e-5 underflow to a zero fp16 scale, as the reference's does
    zero = want == 0
    assert zero.any() and a[zero].max() < 1.3e-5 and a[~zero & np.isfinite(a)].min() > 1.2e-5
    assert np.isinf(want[n - 2]) and np.isnan(want[n - 1])     # inf and NaN maxima propagate


def test_own_scale_keeps_bf16_rows_inside_the_clamp() -> None:
    """The attention launches that quantize Q's bf16 rows themselves
    (rp_fp8_attn_fwd_q16) leave out the clamp to +-448: with the group's own
    scale, |x| <= amax gives |fl(x * qm)| <= fl(amax * qm), and over every
    finite bf16 amax that product stays <= 426.67, so the clamp never binds.
    For fp16 the scale can round to a subnormal or to 0, the product passes
    448 on 977 amax values, and those rows keep the clamp."""
    vals = _all_bf16()
    amax = vals.to(torch.float32).abs()
    fin = torch.isfinite(amax)
    amax_b = vals[fin].abs()
    dq = quant.per_group_dequant(amax_b.reshape(1, -1, 1, 1)).numpy()
    qm = (np.float32(1.0) / dq).astype(np.float32)
    prod = (amax_b.to(torch.float32).numpy() * qm).astype(np.float32)
    assert np.isfinite(prod).all()
    assert prod.max() <= 448.0 and abs(float(prod.max()) - 426.6667) < 1e-3
    worst = float(amax_b[int(prod.argmax())].to(torch.float32))
    assert abs(worst - 1.043081e-6) < 1e-12
    f16 = _all_f16()[:-2]                     # every finite non-negative fp16 value
    dq16 = quant.per_group_dequant(f16.reshape(1, -1, 1, 1)).numpy()
    with np.errstate(divide="ignore", invalid="ignore"):
        p16 = (f16.to(torch.float32).numpy() * (np.float32(1.0) / dq16)).astype(np.float32)
    assert int((p16 > 448.0).sum()) == 977


def _bf16_rne(x: np.float32) -> np.float32:
    u = np.array([x], dtype=np.float32).view(np.uint32)[0]
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return np.array([u], dtype=np.uint32).view(np.float32)[0]


def test_scale_closed_forms() -> None:
    f32 = np.float32
    # bf16(1e-6) is 0x3586; the zero group's scale is bf16(that / 425.6f)
    clamp = np.array([0x35860000], dtype=np.uint32).view(np.float32)[0]
    want = _bf16_rne(f32(clamp / f32(425.6)))
    assert native.dequant_from_amax(0) == want
    assert quant.per_group_dequant(torch.zeros(1, 1, 4, 4, dtype=torch.bfloat16))[0].item() == want
    # amax 425.6 -> bf16 425.5 -> 425.5 / 425.6 rounds to bf16 1.0
    x = torch.full((1, 1, 2, 2), 425.6).to(torch.bfloat16)
    assert quant.per_group_dequant(x)[0].item() == 1.0
    assert native.dequant_from_amax(int(quant.bf16_bits(x)[0, 0, 0, 0])) == 1.0


def _rand_groups(seed: int, shape=(2, 3, 67, 64), scale: float = 3.0) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


@pytest.mark.parametrize("granularity", ["bh", "tensor"])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_c_quantizer_matches_torch_restatement(granularity: str, seed: int) -> None:
    x = _rand_groups(seed, scale=10.0 ** (seed - 1))
    dq_ref, codes_ref = quant.quantize_codes(x, granularity)
    n = x.shape[0] * x.shape[1] if granularity == "bh" else 1
    dq, codes = native.quantize_groups(quant.bf16_bits(x), n)
    assert _scales_equal(dq, dq_ref)
    assert np.array_equal(codes, codes_ref.reshape(codes.shape))


def test_group_max_lands_on_416() -> None:
    """|x| = amax maps to amax / bf16(amax / 425.6) in [423.9, 427.3] -> code 0x7D (416)."""
    for seed in range(8):
        x = _rand_groups(seed, shape=(1, 4, 50, 64), scale=10.0 ** (seed - 4))
        dq, codes = quant.quantize_codes(x, "bh")
        for h in range(4):
            xa = x[0, h].float().abs()
            i = int(torch.argmax(xa))
            assert codes[0, h].reshape(-1)[i] & 0x7F == 0x7D


def test_special_groups() -> None:
    x = _rand_groups(5, shape=(1, 5, 16, 16)).float()
    x[0, 0] = 0.0                            # all-zero group
    x[0, 1, 3, 3] = float("nan")             # NaN propagates through amax
    x[0, 2, 1, 1] = float("inf")             # inf amax -> q_mul 0
    x[0, 3] = -0.0
    x = x.to(torch.bfloat16)
    dq, codes = quant.quantize_codes(x, "bh")
    dqc, codesc = native.quantize_groups(quant.bf16_bits(x), 5)
    assert _scales_equal(dqc, dq)
    assert _same_codes(codesc, codes).all()      # NaN sign is not specified
    assert not codes[0, 0].any()
    assert np.isnan(dq[1]) and ((codes[0, 1] & 0x7F) == 0x7F).all()
    assert np.isinf(dq[2])
    c2 = codes[0, 2].reshape(-1)
    assert (c2[1 * 16 + 1] & 0x7F) == 0x7F             # inf * 0 = NaN
    assert not np.delete(c2 & 0x7F, 1 * 16 + 1).any()   # finite * 0 = 0 (sign kept)
    assert (codes[0, 3] == 0x80).all()


def test_power_of_two_invariance() -> None:
    """x * 2^k has the same codes and a 2^k times larger dequant scale."""
    x = _rand_groups(9, shape=(1, 2, 40, 32))
    dq, codes = quant.quantize_codes(x, "bh")
    for k in (-20, -3, 5, 30):
        xk = (x.float() * 2.0 ** k).to(torch.bfloat16)
        dqk, codesk = native.quantize_groups(quant.bf16_bits(xk), 2)
        assert np.array_equal(codesk, codes.reshape(codesk.shape))
        assert np.array_equal(dqk, (dq * np.float32(2.0 ** k)).astype(np.float32))


# ---------------------------------------------------------------- mutations
def _mut_dequant(x: torch.Tensor, mutation: str) -> np.ndarray:
    amax = x.abs().reshape(-1, 1).amax(dim=1)
    if mutation == "fp32_divide":
        return (amax.float().clamp(min=1e-6) / (0.95 * 448.0)).numpy()
    if mutation == "divisor_448":
        return (amax.clamp(min=1e-6) / 448.0).to(torch.float32).numpy()
    if mutation == "no_clamp":
        return (amax / (0.95 * 448.0)).to(torch.float32).numpy()
    raise ValueError(mutation)


def _mut_encode(x: np.ndarray, mutation: str) -> np.ndarray:
    if mutation == "truncate":
        u = x.view(np.uint32) & np.uint32(0xFFF00000)       # drop the rounding
        return quant.encode_e4m3fn(u.view(np.float32))
    if mutation == "half_up":
        u = x.view(np.uint32).copy()
        tie = (u & np.uint32(0xFFFFF)) == 0x80000
        u[tie] += 1                                          # ties go away from zero
        return quant.encode_e4m3fn(u.view(np.float32))
    if mutation == "saturate":
        return quant.encode_e4m3fn(np.clip(x, -448.0, 448.0).astype(np.float32))
    raise ValueError(mutation)


@pytest.mark.parametrize("mutation", ["fp32_divide", "divisor_448", "no_clamp"])
def test_scale_pin_catches_planted_mistake(mutation: str) -> None:
    vals = _all_bf16()
    ref = _torch_dequant_per_value(vals)
    assert not _scales_equal(_mut_dequant(vals, mutation), ref)


@pytest.mark.parametrize("mutation", ["truncate", "half_up", "saturate"])
def test_encoder_pin_catches_planted_mistake(mutation: str,
                                             structured: tuple[np.ndarray, np.ndarray]) -> None:
    x, ref = structured
    assert not _same_codes(_mut_encode(x, mutation), ref).all()


def test_oracle_reproduces_golden_vectors() -> None:
    """Both restatements (numpy and C) reproduce the committed vectors of the
    reference quantizer's torch ops bit for bit: scales and every code."""
    from tests._helpers import golden_quant_cases

    cases = golden_quant_cases()
    assert [c[0] for c in cases] == ["mixed", "randn", "ties"]
    for name, bits, dq_ref, codes_ref in cases:
        B, H = bits.shape[:2]
        x = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)
        dq, codes = quant.quantize_codes(x, "bh")
        assert np.array_equal(dq.view(np.uint32), dq_ref.view(np.uint32)), name
        assert np.array_equal(codes, codes_ref), name
        dq_c, codes_c = native.quantize_groups(bits, B * H)
        assert np.array_equal(dq_c.view(np.uint32), dq_ref.view(np.uint32)), name
        assert np.array_equal(codes_c.reshape(codes_ref.shape), codes_ref), name
