"""Seeded random shapes through every attention launch and the GEMM.

The other GPU tests pin each launch on hand-picked shapes.  These draw head
count, query and key lengths (ragged everywhere, key ranges from 1 key to
thousands), head dim, mask, scale granularity and output dtype from a fixed
seed, run one launch per case -- one key range, the balanced launch, key
splits, the short-query launch, or the op's own choice (autotuning off: one
range, or the resident-K/V kernel with Q quantized inside it where that
applies) -- and compare sampled rows with the tile-exact oracle under the
bounds tests/test_gpu_attention.py uses: BASELINE's absolute bounds scaled
by the output peak above 1 (for fewer than 256 keys the maximum error may
reach 6e-2 of the peak: with a few keys one flipped P code, an e4m3 step of
6-12% of a dominant key's weight, moves the output by that share of a value;
the same D = 32, 91-key rows differ from the oracle by 0.032-0.036 through
every launch, all bit-identical to each other), a relative mean error of
1e-2 for one range
(the kernel and the oracle differ only by fp32 rounding and the rare P code
it flips), 5e-2 for launches that split the keys (each range quantizes P
against its own running max; the reference runs one range,
kernels/triton_kernels/fp8_flash_attn.py:334-391).  A second set calls
fp8_flash_attention as a caller does, over two batches, fp16 input,
(B, S, H, D) views, causal and shared-prefix masks and a caller's softmax
scale, against the oracle's torch restatement of the quantizer (rows whose
mask leaves them fewer than 256 keys take the few-key bound).  GEMM shapes: every
output a bf16 rounding of a value near the exact sum, as in
tests/test_gpu_gemm.py, with B in the reference's (K, N) layout or
transposed, and the bias and row-scaled epilogues on their own seeded
shapes.
"""

from __future__ import annotations

import math
import random

import numpy as np
import pytest
import torch

from oracle import native
from repercep_runtime_amd import _capi, ops
from tests._helpers import baseline_tolerance, bf16_bits, err_stats
from tests.test_gpu_gemm import _assert_one_rounding_apart

pytestmark = pytest.mark.gpu


def _attention_cases() -> list[tuple]:
    rng = random.Random(20261202)
    cases = []
    for i in range(28):
        D = rng.choice([32, 64, 128, 128, 256])
        short_keys = rng.random() < 0.35
        H = rng.choice([16, 40]) if short_keys else rng.choice([1, 2, 5, 8])
        Sq = rng.randint(4000, 10000) if short_keys else rng.randint(1, 2200)
        Skv = rng.randint(1, 512) if short_keys else rng.randint(1, 2600)
        causal = (not short_keys) and rng.random() < 0.3
        launch = rng.choice(["op", "one", "balanced", "split", "wsplit"])
        if launch == "wsplit" and D not in (64, 128):
            launch = "one"
        splits = rng.choice([2, 3, 5])
        block_m = rng.choice(ops.WSPLIT_BLOCK_MS)
        odt = rng.choice([torch.bfloat16, torch.float32, torch.float16])
        gran = rng.choice(["bh", "tensor"])
        cases.append((f"r{i}_{launch}", H, Sq, Skv, D, causal, launch, splits, block_m, odt,
                      gran))
    return cases


CASES = _attention_cases()


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_random_attention_shape_vs_oracle(gpu: torch.device, case: tuple,
                                          monkeypatch: pytest.MonkeyPatch) -> None:
    name, H, Sq, Skv, D, causal, launch, splits, block_m, odt, gran = case
    monkeypatch.setenv("REPERCEP_FP8_DISABLE_AUTOTUNE", "1")
    g = torch.Generator().manual_seed(sum(map(ord, name)))
    q, k, v = (torch.randn(1, H, S, D, generator=g).to(torch.bfloat16) for S in (Sq, Skv, Skv))
    sm = 1.0 / math.sqrt(D)
    print(f"{name}: H={H} Sq={Sq} Skv={Skv} D={D} causal={causal} {launch} splits={splits} "
          f"block_m={block_m} out={odt} scales per {gran}", flush=True)
    qg, kg, vg = q.to(gpu), k.to(gpu), v.to(gpu)
    if launch == "op":
        out = ops.fp8_flash_attention(qg, kg, vg, causal=causal, granularity=gran,
                                      out_dtype=odt)
        keys_split = False
    else:
        qs, q8, ks, k8, vs, vt8 = ops.scale_quantize_qkv(qg, kg, vg, gran)
        kv_splits = {"one": 1, "balanced": 0, "split": splits, "wsplit": 1}[launch]
        bm = block_m if launch == "wsplit" else ops.BLOCK_M
        out = ops.attention_fp8(q8.view(torch.uint8), k8.view(torch.uint8),
                                vt8.view(torch.uint8), qs, ks, vs, sm, out_dtype=odt,
                                causal=causal, kv_splits=kv_splits, block_m=bm)
        keys_split = launch in ("balanced", "split", "wsplit")
    torch.cuda.synchronize()
    out = out.float().cpu().numpy()
    rng = np.random.default_rng(len(name) + Sq)
    rows = np.unique(np.concatenate([[0, Sq - 1], rng.integers(0, Sq, 40)]))
    n = H if gran == "bh" else 1
    qsc, q8n = native.quantize_groups(bf16_bits(q), n)
    ksc, k8n = native.quantize_groups(bf16_bits(k), n)
    vsc, v8n = native.quantize_groups(bf16_bits(v), n)
    for h in sorted({0, H // 2, H - 1}):
        si = h if gran == "bh" else 0
        ref = native.attn_rows(q8n[0, h], k8n[0, h], v8n[0, h], qsc[si], ksc[si], vsc[si], sm,
                               rows, block_n=ops.BLOCK_N, mask=1 if causal else 0)
        if odt != torch.float32:
            ref = torch.from_numpy(ref).to(odt).float().numpy()
        got = out[0, h][rows]
        st = err_stats(got, ref)
        max_tol, mean_tol = baseline_tolerance(ref)
        if Skv < 256:
            max_tol = max(max_tol, 6e-2 * max(1.0, float(np.abs(ref).max())))
        rel_tol = 5e-2 if keys_split else 1e-2
        print(f"  head {h}: {st} (tol max {max_tol:.3g}, mean {mean_tol:.3g}, "
              f"rel {rel_tol})", flush=True)
        assert np.isfinite(got).all(), f"{name} h={h}: non-finite output"
        assert st["max_abs"] <= max_tol and st["mean_abs"] <= mean_tol, (name, h, st)
        assert st["rel_mean"] <= rel_tol, (name, h, st)


def _op_cases() -> list[tuple]:
    rng = random.Random(4417)
    cases = []
    for i in range(20):
        D = rng.choice([32, 64, 128, 128, 256])
        B = rng.choice([1, 2])
        H = rng.randint(1, 6)
        mask = rng.choice(["none", "none", "causal", "prefix"])
        if mask == "prefix":
            suffix = rng.choice([1, 4, 8, 16])
            Sq = suffix * rng.randint(1, 40)
            prefix = rng.randint(1, 900)
            Skv = prefix + Sq
        else:
            suffix = prefix = None
            Sq, Skv = rng.randint(1, 2000), rng.randint(1, 2600)
        scale = rng.choice([None, None, round(rng.uniform(0.03, 0.3), 4)])
        dtype = rng.choice([torch.bfloat16, torch.float16])
        layout = rng.choice(["bhsd", "bshd"])
        gran = rng.choice(["bh", "tensor"])
        odt = rng.choice([None, torch.float32])
        cases.append((f"o{i}_{mask}", B, H, Sq, Skv, D, mask, prefix, suffix, scale, dtype,
                      layout, gran, odt))
    return cases


OP_CASES = _op_cases()


@pytest.mark.parametrize("case", OP_CASES, ids=[c[0] for c in OP_CASES])
def test_random_op_call_vs_oracle(gpu: torch.device, case: tuple,
                                  monkeypatch: pytest.MonkeyPatch) -> None:
    """fp8_flash_attention as a caller runs it on seeded inputs the cases
    above leave out: two batches, fp16 input, (B, S, H, D) memory viewed as
    (B, H, S, D), causal and shared-prefix masks, a caller's softmax scale;
    the oracle quantizes with the reference's torch expressions (fp16 scale
    included) and replays one key range."""
    from oracle import quant
    (name, B, H, Sq, Skv, D, mask, prefix, suffix, scale, dtype, layout, gran,
     odt) = case
    monkeypatch.setenv("REPERCEP_FP8_DISABLE_AUTOTUNE", "1")
    g = torch.Generator().manual_seed(sum(map(ord, name)) + 7)

    def make(S: int) -> torch.Tensor:
        if layout == "bshd":
            return torch.randn(B, S, H, D, generator=g).to(dtype).permute(0, 2, 1, 3)
        return torch.randn(B, H, S, D, generator=g).to(dtype)

    q, k, v = make(Sq), make(Skv), make(Skv)
    print(f"{name}: B={B} H={H} Sq={Sq} Skv={Skv} D={D} mask={mask} prefix={prefix} "
          f"suffix={suffix} scale={scale} {dtype} {layout} scales per {gran} out={odt}",
          flush=True)
    kw = {"prefix_len": prefix, "suffix_len": suffix} if mask == "prefix" else {}
    out = ops.fp8_flash_attention(q.to(gpu), k.to(gpu), v.to(gpu), causal=mask == "causal",
                                  scale=scale, granularity=gran, out_dtype=odt, **kw)
    torch.cuda.synchronize()
    assert out.dtype == (odt or dtype) and out.shape == (B, H, Sq, D)
    out = out.float().cpu().numpy()
    sm = scale if scale is not None else 1.0 / math.sqrt(D)
    qs, q8 = quant.quantize_codes(q.contiguous(), gran)
    ks, k8 = quant.quantize_codes(k.contiguous(), gran)
    vs, v8 = quant.quantize_codes(v.contiguous(), gran)
    mcode = {"none": 0, "causal": 1, "prefix": 2}[mask]
    rng = np.random.default_rng(len(name) + Sq)
    rows = np.unique(np.concatenate([[0, Sq - 1], rng.integers(0, Sq, 32)]))
    for b in range(B):
        for h in sorted({0, H - 1}):
            si = b * H + h if gran == "bh" else 0
            ref = native.attn_rows(q8[b, h], k8[b, h], v8[b, h], qs[si], ks[si], vs[si], sm,
                                   rows, block_n=ops.BLOCK_N, mask=mcode, prefix=prefix or 0,
                                   suffix=suffix or 1)
            if (odt or dtype) != torch.float32:
                ref = torch.from_numpy(ref).to(odt or dtype).float().numpy()
            got = out[b, h][rows]
            st = err_stats(got, ref)
            max_tol, mean_tol = baseline_tolerance(ref)
            if Skv < 256 or mask != "none":   # rows that see fewer than 256 keys
                max_tol = max(max_tol, 6e-2 * max(1.0, float(np.abs(ref).max())))
            print(f"  b={b} h={h}: {st} (tol max {max_tol:.3g}, mean {mean_tol:.3g})",
                  flush=True)
            assert np.isfinite(got).all(), f"{name} b={b} h={h}: non-finite output"
            assert st["max_abs"] <= max_tol and st["mean_abs"] <= mean_tol, (name, b, h, st)
            assert st["rel_mean"] <= 1e-2, (name, b, h, st)


def _gemm_cases() -> list[tuple]:
    rng = random.Random(7)
    return [(f"g{i}", rng.randint(1, 2600), 16 * rng.randint(1, 150), 64 * rng.randint(1, 36),
             rng.random() < 0.5) for i in range(16)]


GEMM_CASES = _gemm_cases()


@pytest.mark.parametrize("case", GEMM_CASES, ids=[c[0] for c in GEMM_CASES])
def test_random_gemm_shape_is_one_rounding_of_the_exact_sum(gpu: torch.device,
                                                             case: tuple) -> None:
    name, M, N, K, kn = case
    print(f"{name}: M={M} N={N} K={K} B {'(K, N)' if kn else '(N, K)'}", flush=True)
    g = torch.Generator().manual_seed(sum(map(ord, name)) + K)
    a8 = (torch.randn(M, K, generator=g) * 0.5).to(torch.float8_e4m3fn).view(torch.uint8)
    bt8 = (torch.randn(N, K, generator=g) * 0.5).to(torch.float8_e4m3fn).view(torch.uint8)
    sa, sb = 0.37, 1.9
    if kn:
        c = ops.fp8_gemm(a8.to(gpu), bt8.t().contiguous().to(gpu), sa, sb)
    else:
        c = ops.fp8_gemm(a8.to(gpu), bt8.to(gpu), sa, sb, b_transposed=True)
    torch.cuda.synchronize()
    _assert_one_rounding_apart(c.float().cpu().numpy(), None, a8.numpy(), bt8.numpy(),
                               float(np.float32(sa) * np.float32(sb)))
    assert _capi.lib() is not None


def _epilogue_cases() -> list[tuple]:
    rng = random.Random(911)
    cases = []
    for i in range(12):
        kind = "bias" if i % 2 == 0 else "rowwise"
        Z = 1 if kind == "bias" else rng.randint(1, 3)
        M = rng.randint(1, 1300)
        N = 16 * rng.randint(1, 90) if kind == "bias" else 4 * rng.randint(1, 300)
        K = rng.choice([64 * rng.randint(1, 20), 16 * rng.randint(1, 40)])
        kn = rng.random() < 0.5 and kind == "bias"   # the row-scaled op takes B^T only
        cases.append((f"e{i}_{kind}", kind, Z, M, N, K, kn))
    return cases


EPI_CASES = _epilogue_cases()


@pytest.mark.parametrize("case", EPI_CASES, ids=[c[0] for c in EPI_CASES])
def test_random_gemm_epilogues(gpu: torch.device, case: tuple) -> None:
    """The bias epilogue (bf16(fp32(fp32(acc * s) + bias)), as a bf16
    nn.Linear rounds) and the row-scaled one (bf16((acc * s_m) * s_n), the
    unfused attention's grouped GEMM) on seeded shapes, both tile kernels
    (K % 64 picks the large tiles): every output one rounding of a value
    within the MFMA's sum error plus the epilogue's fp32 roundings of the
    exact result."""
    from oracle.quant import DECODE
    name, kind, Z, M, N, K, kn = case
    print(f"{name}: Z={Z} M={M} N={N} K={K} B {'(K, N)' if kn else '(N, K)'}", flush=True)
    g = torch.Generator().manual_seed(sum(map(ord, name)) + M)
    a8 = (torch.randn(Z, M, K, generator=g) * 30).to(torch.float8_e4m3fn)
    bt8 = (torch.randn(Z, N, K, generator=g) * 30).to(torch.float8_e4m3fn)
    if kind == "bias":
        bias = (torch.randn(N, generator=g) * 50).to(torch.bfloat16)
        sa, sb = 0.013, 0.0071
        if kn:
            got = ops.fp8_gemm(a8[0].to(gpu), bt8[0].t().contiguous().to(gpu), sa, sb,
                               bias=bias.to(gpu))
        else:
            got = ops.fp8_gemm(a8[0].to(gpu), bt8[0].to(gpu), sa, sb, b_transposed=True,
                               bias=bias.to(gpu))
        torch.cuda.synchronize()
        _assert_one_rounding_apart(got.float().cpu().numpy(), None,
                                   a8[0].view(torch.uint8).numpy(),
                                   bt8[0].view(torch.uint8).numpy(),
                                   float(np.float32(sa) * np.float32(sb)),
                                   bias.float().numpy().astype(np.float64))
        return
    rs = torch.rand(Z, M, generator=g) * 0.02 + 1e-3
    cs = torch.rand(Z, N, generator=g) * 0.02 + 1e-3
    got = ops.gemm_rowwise(a8.to(gpu), bt8.to(gpu), rs.to(gpu), cs.to(gpu)).float().cpu().numpy()
    A = DECODE[a8.view(torch.uint8).numpy()].astype(np.float64)
    B = DECODE[bt8.view(torch.uint8).numpy()].astype(np.float64)
    sc = rs.numpy().astype(np.float64)[:, :, None] * cs.numpy().astype(np.float64)[:, None, :]
    exact = np.matmul(A, B.transpose(0, 2, 1)) * sc
    eps = (2.0 ** -14 * np.matmul(np.abs(A), np.abs(B).transpose(0, 2, 1)) * sc
           + 2.0 ** -22 * np.abs(exact))
    lo = torch.from_numpy(exact - eps).float().to(torch.bfloat16).float().numpy()
    hi = torch.from_numpy(exact + eps).float().to(torch.bfloat16).float().numpy()
    bad = (got < np.minimum(lo, hi)) | (got > np.maximum(lo, hi))
    print(f"  outside the rounding interval: {int(bad.sum())}", flush=True)
    assert not bad.any(), name

