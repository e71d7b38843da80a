"""GPU parity of the fused QK-norm prologue (rp_fp8_rmsnorm_scale_quantize):
scales and codes bit-exact against oracle/prologue.py, which restates the
normalisation with the kernel's summation order and the reference quantizer.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import prologue as P
from repercep_runtime_amd import ops
from repercep_runtime_amd.workloads import C2
from tests._helpers import codes_np

pytestmark = pytest.mark.gpu


def _x(seed: int, shape, scale: float = 1.0) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


def _tables(S: int, D: int) -> tuple[np.ndarray, np.ndarray]:
    """Cosmos-like rotary tables: angle = position * 10000^(-2i/D)."""
    pos = np.arange(S, dtype=np.float64)[:, None]
    inv = 10000.0 ** (-np.arange(0, D, 2, dtype=np.float64) / D)
    ang = np.repeat(pos * inv[None, :], 2, axis=1)[:, :D]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


CASES = [
    # name, shape, D-scale, weight, rope, granularity
    ("plain_d128", (1, 4, 1000, 128), 1.0, False, None, "bh"),
    ("plain_d64", (2, 3, 777, 64), 1.0, False, None, "bh"),
    ("weight_d128", (1, 2, 513, 128), 3.0, True, None, "bh"),
    ("rope_half", (1, 3, 600, 128), 1.0, True, "half", "bh"),
    ("rope_interleaved", (2, 2, 300, 64), 1.0, False, "interleaved", "bh"),
    ("per_tensor", (2, 3, 400, 128), 0.01, True, "half", "tensor"),
    ("tiny_rows", (1, 1, 5, 64), 1.0, True, "half", "bh"),
    # rows of one block step across many heads (S below the 32/16-row step)
    ("per_tensor_short_heads", (2, 5, 3, 64), 1.0, False, "interleaved", "tensor"),
    ("short_heads_d128", (1, 7, 2, 128), 1.0, True, "half", "bh"),
    ("per_tensor_ragged", (3, 3, 37, 128), 1.0, True, None, "tensor"),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_prologue_bit_exact(gpu: torch.device, case: tuple) -> None:
    name, shape, scale, use_w, rope, gran = case
    B, H, S, D = shape
    seed = sum(map(ord, name))
    x = _x(seed, shape, scale)
    x[0, 0, 0] = 0                      # a zero row
    w = _x(seed + 1, (D,), 0.8) if use_w else None
    cs = _tables(S, D) if rope else (None, None)
    mode = {None: P.ROPE_NONE, "half": P.ROPE_HALF, "interleaved": P.ROPE_INTERLEAVED}[rope]
    dq_ref, codes_ref = P.quantize_prologue(x, 1e-6, w, cs[0], cs[1], mode, gran)
    rope_t = None if rope is None else tuple(torch.from_numpy(t).to(gpu) for t in cs)
    dq, codes = ops.rmsnorm_scale_quantize(
        x.to(gpu), None if w is None else w.to(gpu), 1e-6, rope_t, rope or "half", gran)
    assert np.array_equal(dq.cpu().numpy().view(np.uint32), dq_ref.view(np.uint32)), name
    got = codes_np(codes)
    mism = np.flatnonzero(got.reshape(-1) != codes_ref.reshape(-1))
    assert mism.size == 0, f"{name}: {mism.size} codes differ, first at {mism[:5]}"


def test_prologue_reads_permuted_bshd_view(gpu: torch.device) -> None:
    """A (B, S, H, D) buffer viewed as (B, H, S, D), no copy."""
    x_bshd = _x(3, (2, 300, 4, 128))
    xg = x_bshd.to(gpu).permute(0, 2, 1, 3)
    dq, codes = ops.rmsnorm_scale_quantize(xg)
    dq_ref, codes_ref = P.quantize_prologue(x_bshd.permute(0, 2, 1, 3).contiguous(), 1e-6)
    assert np.array_equal(dq.cpu().numpy(), dq_ref)
    assert np.array_equal(codes_np(codes), codes_ref)


def test_prologue_cosmos_full_size_heads(gpu: torch.device) -> None:
    """BASELINE config 2's Q at full size (1, 32, 56320, 128), pre-norm N(0,1):
    three heads compared element for element (per-head groups are independent)."""
    g = torch.Generator(device=gpu).manual_seed(C2.seed)
    q = torch.randn((1, C2.H, C2.Sq, C2.D), generator=g, device=gpu).to(torch.bfloat16)
    dq, codes = ops.rmsnorm_scale_quantize(q)
    for h in (0, 17, 31):
        xh = q[:, h:h + 1].cpu()
        dq_ref, codes_ref = P.quantize_prologue(xh, 1e-6)
        assert dq.cpu().numpy()[h] == dq_ref[0], h
        assert np.array_equal(codes_np(codes[:, h:h + 1]), codes_ref), h


def test_qknorm_attention_matches_unfused(gpu: torch.device) -> None:
    """Attention on pre-norm Q/K through the fused prologue against the same
    kernel on Q/K normalised and rotated by the oracle first: the FP8 operands
    are identical, so the outputs are bit-identical."""
    B, H, S, D = 1, 4, 700, 128
    q, k, v = _x(60, (B, H, S, D)), _x(61, (B, H, S, D)), _x(62, (B, H, S, D))
    wq, wk = _x(63, (D,), 0.9), _x(64, (D,), 1.1)
    cos, sin = _tables(S, D)
    rope = tuple(torch.from_numpy(t).to(gpu) for t in (cos, sin))
    out = ops.fp8_flash_attention_qknorm(
        q.to(gpu), k.to(gpu), v.to(gpu), norm_q_weight=wq.to(gpu), norm_k_weight=wk.to(gpu),
        rope_q=rope, rope_k=rope, out_dtype=torch.float32)

    def prep(x, w):
        y = P.rmsnorm_rope(P.f32_to_bits(x.float().numpy()), 1e-6, P.f32_to_bits(w.float().numpy()),
                           cos, sin, P.ROPE_HALF)
        return torch.from_numpy(P.f32_to_bits(y).view(np.int16)).view(torch.bfloat16)

    ref = ops.fp8_flash_attention(prep(q, wq).to(gpu), prep(k, wk).to(gpu), v.to(gpu),
                                  out_dtype=torch.float32, kv_splits=1)
    assert torch.equal(out, ref)
    assert math.isfinite(float(out.abs().max()))


@pytest.mark.parametrize("gran", ["bh", "tensor"])
def test_unit_weight_is_the_identity_on_extremes(gpu: torch.device, gran: str) -> None:
    """bf16(bf16(x * r) * 1) = bf16(x * r): the weighted and unweighted
    prologues agree bit for bit -- scales, codes and NaN payloads -- on rows
    with NaN, Inf, values whose squares overflow (r = 0), values whose squares
    underflow, and zeros, with and without eps."""
    g = torch.Generator().manual_seed(77)
    x = torch.randn(2, 3, 40, 128, generator=g)
    x[0, 0, 1, 5] = float("nan")
    x[0, 1, 2, 9] = float("inf")
    x[0, 2, 3, 0] = -float("inf")
    x[1, 0, 4] = 1e30                                  # squares overflow: r = 0
    x[1, 0, 5] *= 1e-25                                # squares underflow to 0
    x[1, 1, 6] = 0.0
    x[1, 2, 7, 3] = 3e38
    x = x.to(torch.bfloat16).to(gpu)
    ones = torch.ones(128, dtype=torch.bfloat16, device=gpu)
    for eps in (1e-6, 0.0):
        dq_a, c_a = ops.rmsnorm_scale_quantize(x, None, eps, None, "half", gran)
        dq_b, c_b = ops.rmsnorm_scale_quantize(x, ones, eps, None, "half", gran)
        assert torch.equal(dq_a.view(torch.int32), dq_b.view(torch.int32)), eps
        assert torch.equal(c_a.view(torch.uint8), c_b.view(torch.uint8)), eps
