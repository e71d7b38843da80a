"""GPU parity of the row-wise FP8 path and the unfused FP8 attention.

Reference: src/repercep/attention/fp8_scaled_mm.py:58-221 (``FP8ScaledMMAttention``,
``_rowwise_quantize`` at :107-133), restated in oracle/rowwise.py.  Row-wise
codes and scales are bit-exact; the row-scaled GEMM is one rounding of the
exact sum; P (a softmax) is compared code by code within one e4m3 step, and
the attention output within BASELINE's tolerance of the oracle and within the
reference's own bound of SDPA.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import rowwise
from oracle.quant import DECODE
from repercep_runtime_amd import ops
from tests._helpers import bf16_bits, bf16_to_f32, err_stats

pytestmark = pytest.mark.gpu


def _codes_equal(got: torch.Tensor, ref: torch.Tensor) -> None:
    """Bit-identical codes, except that a NaN code's sign is not specified."""
    g = got.view(torch.uint8).cpu().numpy()
    r = ref.view(torch.uint8).cpu().numpy()
    nan = (r & 0x7F) == 0x7F
    assert np.array_equal(g[~nan], r[~nan]), f"{int((g[~nan] != r[~nan]).sum())} codes differ"
    assert ((g[nan] & 0x7F) == 0x7F).all()


@pytest.mark.parametrize("rows,cols,dtype", [
    (1000, 128, torch.bfloat16), (777, 64, torch.bfloat16), (300, 96, torch.bfloat16),
    (65, 8, torch.bfloat16), (40, 2048, torch.bfloat16), (9, 4104, torch.bfloat16),
    (513, 128, torch.float16), (33, 3000, torch.float16),
])
def test_rowwise_quantize_bit_exact(gpu: torch.device, rows: int, cols: int,
                                    dtype: torch.dtype) -> None:
    g = torch.Generator().manual_seed(rows * 7 + cols)
    lo, hi = (-6, 6) if dtype == torch.bfloat16 else (-2, 3)
    mag = torch.logspace(lo, hi, rows).reshape(rows, 1)
    x = (torch.randn(rows, cols, generator=g) * mag).to(dtype)
    x[0] = 0                                   # a zero row
    if rows > 4:
        x[1, cols // 2] = float("nan")         # a NaN row
        x[2, 0] = float("inf")                 # an infinite element
        x[3] = x[3].abs().neg()                # all negative
    if dtype == torch.float16 and rows > 5:
        x[4] = x[4] * 1e-3                     # fp16 multiplier overflow: saturation
    dq, codes = ops.rowwise_quantize(x.to(gpu))
    ref_codes, ref_dq = rowwise.rowwise_quantize(x)
    _codes_equal(codes, ref_codes)
    d = dq.cpu().numpy()
    r = ref_dq.numpy()
    assert np.array_equal(np.isnan(d), np.isnan(r))
    assert np.array_equal(d[~np.isnan(r)].view(np.uint32), r[~np.isnan(r)].view(np.uint32))


def test_rowwise_quantize_strided_rows_and_nd(gpu: torch.device) -> None:
    """A row-strided view (every other row of a buffer) and an N-D tensor
    whose rows flatten to one stride."""
    g = torch.Generator().manual_seed(3)
    buf = torch.randn(200, 256, generator=g).to(torch.bfloat16)
    view = buf.to(gpu)[:, :128]
    dq, codes = ops.rowwise_quantize(view)
    ref_codes, ref_dq = rowwise.rowwise_quantize(buf[:, :128].contiguous())
    _codes_equal(codes, ref_codes)
    assert torch.equal(dq.cpu(), ref_dq)
    x = torch.randn(2, 3, 50, 64, generator=g).to(torch.bfloat16)
    dq, codes = ops.rowwise_quantize(x.to(gpu))
    assert dq.shape == (2, 3, 50) and codes.shape == (2, 3, 50, 64)
    ref_codes, ref_dq = rowwise.rowwise_quantize(x)
    _codes_equal(codes, ref_codes)
    assert torch.equal(dq.cpu(), ref_dq)


def test_transpose16_exact(gpu: torch.device) -> None:
    x = torch.randn(3, 130, 70).to(torch.bfloat16)
    t = ops.transpose16(x.to(gpu))
    assert torch.equal(t.cpu(), x.transpose(-1, -2).contiguous())


@pytest.mark.parametrize("zmnk", [(3, 128, 256, 128), (2, 300, 200, 64), (1, 64, 100, 48),
                                  (4, 256, 64, 512),
                                  # tiles wholly inside C: the unchecked store path
                                  (1, 512, 512, 256), (2, 256, 272, 128)])
def test_gemm_rowwise_one_rounding_of_exact(gpu: torch.device, zmnk: tuple) -> None:
    """Every output is the bf16 rounding of a value within
    2^-14 * sum|a||b| * s_m * s_n (the MFMA's sum) plus the two fp32 roundings
    of the scaling of the exact scaled sum; BASELINE metrics vs the oracle."""
    Z, M, N, K = zmnk
    g = torch.Generator().manual_seed(M + N + K)
    a8 = torch.randn(Z, M, K, generator=g).mul(30).to(torch.float8_e4m3fn)
    bt8 = torch.randn(Z, N, K, generator=g).mul(30).to(torch.float8_e4m3fn)
    sa = torch.rand(Z, M, generator=g) * 0.02 + 1e-3
    sb = torch.rand(Z, N, generator=g) * 0.02 + 1e-3
    got = ops.gemm_rowwise(a8.to(gpu), bt8.to(gpu), sa.to(gpu), sb.to(gpu)).cpu()
    ref = rowwise.grouped_scaled_mm(a8.view(torch.uint8).numpy(), bt8.view(torch.uint8).numpy(),
                                    sa.numpy(), sb.numpy())
    A = DECODE[a8.view(torch.uint8).numpy()].astype(np.float64)
    B = DECODE[bt8.view(torch.uint8).numpy()].astype(np.float64)
    s = sa.numpy().astype(np.float64)[:, :, None] * sb.numpy().astype(np.float64)[:, None, :]
    exact = np.einsum("zmk,znk->zmn", A, B) * s
    eps = 2.0 ** -14 * np.einsum("zmk,znk->zmn", np.abs(A), np.abs(B)) * s \
        + 2.0 ** -22 * np.abs(exact)
    gv = bf16_to_f32(bf16_bits(got)).astype(np.float64)
    lo = bf16_to_f32(bf16_bits(torch.from_numpy(exact - eps).float().to(torch.bfloat16)))
    hi = bf16_to_f32(bf16_bits(torch.from_numpy(exact + eps).float().to(torch.bfloat16)))
    bad = (gv < np.minimum(lo, hi)) | (gv > np.maximum(lo, hi))
    st = err_stats(gv, bf16_to_f32(bf16_bits(ref)))
    print(zmnk, st, "outside:", int(bad.sum()), flush=True)
    assert not bad.any()
    assert st["rel_mean"] <= 1e-3


def test_gemm_rowwise_integers_exact(gpu: torch.device) -> None:
    g = torch.Generator().manual_seed(2)
    a = torch.randint(-3, 4, (2, 64, 128), generator=g).float()
    b = torch.randint(-3, 4, (2, 32, 128), generator=g).float()
    sa = 2.0 ** torch.randint(-4, 4, (2, 64), generator=g).float()
    sb = 2.0 ** torch.randint(-4, 4, (2, 32), generator=g).float()
    got = ops.gemm_rowwise(a.to(torch.float8_e4m3fn).to(gpu), b.to(torch.float8_e4m3fn).to(gpu),
                           sa.to(gpu), sb.to(gpu)).cpu()
    want = ((a @ b.transpose(1, 2)) * sa[:, :, None] * sb[:, None, :]).to(torch.bfloat16)
    assert torch.equal(got, want)


@pytest.mark.parametrize("causal", [False, True])
def test_softmax_rowwise_quantize_vs_oracle(gpu: torch.device, causal: bool) -> None:
    """P = softmax(bf16(raw * scale)) in bf16 and its row-wise codes: the sum
    of exponentials runs in another order than torch's, so a P value may sit
    one bf16 step away and its code one e4m3 step; the scales agree within
    one bf16 step and almost every code is identical (every one of these
    seeds' codes with the accurate expf; the bound leaves room for a rare
    P value on the other side of a rounding boundary)."""
    g = torch.Generator().manual_seed(5 + causal)
    raw = (torch.randn(3, 96, 384, generator=g) * 4).to(torch.bfloat16)
    scale = 0.125
    dq, codes = ops.softmax_rowwise_quantize(raw.to(gpu), scale, causal)
    p = rowwise.softmax_probs(raw, scale, causal)
    ref_codes, ref_dq = rowwise.rowwise_quantize(p)
    d, r = dq.cpu().numpy(), ref_dq.numpy()
    assert np.all(np.abs(d - r) <= r * 2.0 ** -7)
    gc = codes.view(torch.uint8).cpu().numpy().astype(np.int32)
    rc = ref_codes.numpy().astype(np.int32)
    assert np.all(np.abs(gc - rc) <= 1)
    same = (gc == rc).mean()
    print(f"softmax codes identical: {same:.6f} (causal={causal})", flush=True)
    assert same > 0.9999
    if causal:      # masked entries quantize to code 0
        q = np.arange(96)[None, :, None]
        j = np.arange(384)[None, None, :]
        assert (gc[np.broadcast_to(j > q, gc.shape)] == 0).all()


@pytest.mark.parametrize("shape,skv,causal,dtype", [
    ((1, 4, 512, 128), None, False, torch.bfloat16),
    ((1, 4, 512, 128), None, True, torch.bfloat16),
    ((2, 3, 256, 64), None, False, torch.float16),
    ((1, 2, 384, 256), None, True, torch.bfloat16),
    ((1, 2, 128, 96), None, False, torch.bfloat16),
    # cross shapes: the causal mask is triu(1) on (Sq, Skv), top-left aligned
    # (fp8_scaled_mm.py:163-166), and the second GEMM runs over Skv
    ((1, 2, 256, 128), 384, False, torch.bfloat16),
    ((1, 2, 256, 128), 384, True, torch.bfloat16),
    ((1, 3, 384, 64), 256, True, torch.float16),
])
def test_scaled_mm_attention_vs_oracle(gpu: torch.device, shape: tuple, skv: int | None,
                                       causal: bool, dtype: torch.dtype) -> None:
    """The whole unfused op against the oracle's restatement of
    FP8ScaledMMAttention.__call__, within BASELINE's tolerance."""
    g = torch.Generator().manual_seed(sum(shape) + (skv or 0))
    kshape = shape if skv is None else (*shape[:2], skv, shape[3])
    q = torch.randn(*shape, generator=g).to(dtype)
    k, v = (torch.randn(*kshape, generator=g).to(dtype) for _ in range(2))
    out = ops.fp8_scaled_mm_attention(q.to(gpu), k.to(gpu), v.to(gpu), causal=causal)
    assert out.dtype == dtype and out.shape == shape
    ref = rowwise.scaled_mm_attention(q, k, v, causal=causal)
    st = err_stats(out.float().cpu().numpy(), ref.float().numpy())
    print(shape, skv, causal, dtype, st, flush=True)
    assert st["max_abs"] <= 2e-2 and st["mean_abs"] <= 2e-3 and st["rel_mean"] <= 1e-2


def test_op_matches_sdpa_like_the_reference(gpu: torch.device) -> None:
    """tests/test_attention_fp8.py:77-101 of the reference: (1, 4, 512, 128),
    Q, K = randn/8, mean relative error against SDPA below 0.30."""
    from repercep_runtime_amd.attention import FP8HipScaledMMAttention, NaiveAttention
    from repercep_runtime_amd.attention.types import AttentionShape
    from repercep_runtime_amd.hardware import DType

    op = FP8HipScaledMMAttention()
    assert op.available and op.name == "fp8-hip-scaled-mm"
    assert op.supports(AttentionShape(1, 4, 512, 512, 128), DType.BF16)
    torch.manual_seed(0)
    q = torch.randn(1, 4, 512, 128, device=gpu, dtype=torch.bfloat16) / 8.0
    k = torch.randn(1, 4, 512, 128, device=gpu, dtype=torch.bfloat16) / 8.0
    v = torch.randn(1, 4, 512, 128, device=gpu, dtype=torch.bfloat16)
    ref = NaiveAttention()(q.float(), k.float(), v.float())
    out = op(q, k, v)
    assert out.shape == ref.shape and torch.isfinite(out).all()
    rel = ((out.float() - ref).abs().mean() / ref.abs().mean()).item()
    print(f"scaled-mm mean rel vs SDPA {rel:.4f}", flush=True)
    assert rel < 0.30
