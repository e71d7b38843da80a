"""GPU parity of the fused QK-norm prologue (rp_fp8_rmsnorm_scale_quantize, and
rp_fp8_rmsnorm_scale_quantize_qkv with V's quantizer in the same launches):
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


QKV_CASES = [
    # name, (B, H, Sq, Skv, D), weights, rope, granularity, permuted (B, S, H, D) inputs
    ("self_d128", (1, 4, 1000, 1000, 128), False, None, "bh", False),
    ("cross_weights_tensor", (2, 3, 700, 300, 128), True, None, "tensor", True),
    ("kv_longer_rope_half_d64", (1, 3, 200, 777, 64), True, "half", "bh", False),
    ("interleaved_tensor_d64", (2, 2, 300, 300, 64), False, "interleaved", "tensor", True),
    ("rope_half_d128_strided", (1, 2, 513, 640, 128), True, "half", "bh", True),
    ("tiny", (1, 1, 5, 3, 64), False, None, "bh", False),
]


@pytest.mark.parametrize("case", QKV_CASES, ids=[c[0] for c in QKV_CASES])
def test_fused_qkv_prologue_bit_exact(gpu: torch.device, case: tuple) -> None:
    """rp_fp8_rmsnorm_scale_quantize_qkv: Q's and K's scales and codes equal
    the prologue oracle's (each with its own weight and tables), V's transposed
    codes equal the plain quantizer oracle's, and all of it -- V^T's zeroed
    padding columns included -- equals the three single-tensor calls."""
    from oracle import native
    from tests._helpers import bf16_bits

    name, (B, H, Sq, Skv, D), use_w, rope, gran, permuted = case
    seed = sum(map(ord, name))

    def make(S, sd, scale):
        if permuted:
            return _x(sd, (B, S, H, D), scale).to(gpu).permute(0, 2, 1, 3)
        return _x(sd, (B, H, S, D), scale).to(gpu)

    q, k, v = make(Sq, seed, 2.0), make(Skv, seed + 1, 1.0), make(Skv, seed + 2, 0.5)
    wq = _x(seed + 3, (D,), 0.8) if use_w else None
    wk = _x(seed + 4, (D,), 1.2) if use_w else None
    tq, tk = (_tables(Sq, D), _tables(Skv, D)) if rope else ((None, None), (None, None))
    to_dev = lambda t: None if t[0] is None else tuple(torch.from_numpy(a).to(gpu) for a in t)  # noqa: E731
    dev_w = lambda w: None if w is None else w.to(gpu)  # noqa: E731
    qs, q8, ks, k8, vs, vt8 = ops.rmsnorm_scale_quantize_qkv(
        q, k, v, norm_q_weight=dev_w(wq), norm_k_weight=dev_w(wk), rope_q=to_dev(tq),
        rope_k=to_dev(tk), rope_layout=rope or "half", granularity=gran)
    mode = {None: P.ROPE_NONE, "half": P.ROPE_HALF, "interleaved": P.ROPE_INTERLEAVED}[rope]
    for x, w, t, s, c in ((q, wq, tq, qs, q8), (k, wk, tk, ks, k8)):
        dq_ref, codes_ref = P.quantize_prologue(x.cpu().contiguous(), 1e-6, w, t[0], t[1], mode,
                                                gran)
        assert np.array_equal(s.cpu().numpy().view(np.uint32), dq_ref.view(np.uint32)), name
        assert np.array_equal(codes_np(c), codes_ref), name
    n = B * H if gran == "bh" else 1
    dv_ref, cv_ref = native.quantize_groups(bf16_bits(v.cpu().contiguous()), n)
    assert np.array_equal(vs.cpu().numpy(), dv_ref), name
    vt = codes_np(vt8)
    assert np.array_equal(np.ascontiguousarray(np.swapaxes(vt[..., :Skv], -1, -2)), cv_ref)
    assert not vt[..., Skv:].any(), "V^T padding columns must be zero"
    # the single-tensor calls, bit for bit
    s1, c1 = ops.rmsnorm_scale_quantize(q, dev_w(wq), 1e-6, to_dev(tq), rope or "half", gran)
    s2, c2 = ops.rmsnorm_scale_quantize(k, dev_w(wk), 1e-6, to_dev(tk), rope or "half", gran)
    s3, c3 = ops.scale_quantize(v, gran, "bhds")
    for a, b in ((qs, s1), (ks, s2), (vs, s3)):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32)), name
    for a, b in ((q8, c1), (k8, c2), (vt8, c3)):
        assert a.shape == b.shape and torch.equal(a.view(torch.uint8), b.view(torch.uint8)), name


def test_fused_qkv_refuses_rope_for_one_tensor(gpu: torch.device) -> None:
    """One rotary layout serves Q and K in the fused call: tables for only one
    of them are refused on the host (fp8_flash_attention_qknorm then runs the
    single-tensor calls)."""
    x = torch.zeros(1, 2, 64, 64, dtype=torch.bfloat16, device=gpu)
    t = tuple(torch.from_numpy(a).to(gpu) for a in _tables(64, 64))
    with pytest.raises(ValueError, match="both q and k"):
        ops.rmsnorm_scale_quantize_qkv(x, x, x, rope_q=t)


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
