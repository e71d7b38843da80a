"""Attention that quantizes its own Q rows (rp_fp8_attn_fwd_q16).

The reference's wrapper quantizes Q, K and V, then runs the kernel on the
codes (kernels/triton_kernels/fp8_flash_attn.py:522-528, 604-644).  This
build can hand the attention launch Q as its bf16/fp16 input with Q's scale
(the quantizer then writes K's and V^T's codes only), and every workgroup
quantizes the Q rows it reads with the quantizer's own arithmetic.  The
codes are the quantizer's, so the outputs must be the two-step path's bit for
bit: one range, key splits, the balanced launch, the resident-K/V kernel,
causal masks, fp16 inputs, per-tensor scales and strided (B, S, H, D) views.
"""

from __future__ import annotations

import math

import pytest
import torch

from repercep_runtime_amd import _capi, ops

pytestmark = pytest.mark.gpu

CASES = [
    # name, B, H, Sq, Skv, D, in dtype, out dtype, kv_splits, causal, layout, granularity
    ("one_range_d128", 1, 2, 1000, 1000, 128, torch.bfloat16, torch.bfloat16, 1, False, "bhsd",
     "bh"),
    ("one_range_per_tensor", 2, 2, 777, 1300, 128, torch.bfloat16, torch.float32, 1, False,
     "bhsd", "tensor"),
    ("causal_d128", 2, 3, 1500, 1500, 128, torch.bfloat16, torch.bfloat16, 1, True, "bhsd",
     "bh"),
    ("split4_d64_fp16", 1, 3, 700, 2000, 64, torch.float16, torch.float32, 4, False, "bhsd",
     "bh"),
    ("balanced_d128", 1, 8, 8860, 8192, 128, torch.bfloat16, torch.bfloat16, 0, False, "bhsd",
     "tensor"),
    ("balanced_d256", 1, 4, 8548, 4096, 256, torch.bfloat16, torch.float32, 0, False, "bhsd",
     "bh"),
    ("resident_kv_cross_bshd", 1, 40, 9000, 512, 128, torch.bfloat16, torch.bfloat16, 1, False,
     "bshd", "tensor"),
    ("resident_kv_d64_fp16", 1, 64, 16384 + 77, 100, 64, torch.float16, torch.float16, 1, False,
     "bhsd", "bh"),
]


def _inputs(name: str, B: int, H: int, Sq: int, Skv: int, D: int, dtype: torch.dtype,
            layout: str, gpu: torch.device) -> tuple[torch.Tensor, ...]:
    g = torch.Generator().manual_seed(sum(map(ord, name)))

    def make(S: int) -> torch.Tensor:
        if layout == "bshd":   # the diffusers bridge's (B, S, H, D) memory, viewed as BHSD
            return torch.randn(B, S, H, D, generator=g).to(dtype).to(gpu).permute(0, 2, 1, 3)
        return torch.randn(B, H, S, D, generator=g).to(dtype).to(gpu)

    return make(Sq), make(Skv), make(Skv)


def _q16_call(q: torch.Tensor, k8: torch.Tensor, vt8: torch.Tensor, qs: torch.Tensor,
              ks: torch.Tensor, vs: torch.Tensor, out: torch.Tensor, sm: float, mask: int,
              kv_splits: int) -> int:
    B, H, Sq, D = q.shape
    Skv = k8.shape[2]
    st = torch.cuda.current_stream(q.device).cuda_stream
    L = _capi.lib()
    if kv_splits == 0:
        nbytes = L.rp_fp8_attn_balanced_workspace_bytes(B, H, Sq, Skv, D, mask, st)
    else:
        nbytes = L.rp_fp8_attn_workspace_bytes(B, H, Sq, D, kv_splits) if kv_splits > 1 else 0
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=q.device)
    stride = 1 if qs.numel() == B * H and B * H > 1 else 0
    odt = {torch.bfloat16: _capi.RP_OUT_BF16, torch.float16: _capi.RP_OUT_F16,
           torch.float32: _capi.RP_OUT_F32}[out.dtype]
    qdt = _capi.RP_DTYPE_F16 if q.dtype == torch.float16 else _capi.RP_DTYPE_BF16
    qsb, qsh, qss, _ = q.stride()
    rc = L.rp_fp8_attn_fwd_q16(q.data_ptr(), qdt, qsb, qsh, qss, k8.data_ptr(), vt8.data_ptr(),
                               vt8.shape[3], qs.data_ptr(), ks.data_ptr(), vs.data_ptr(), stride,
                               sm, out.data_ptr(), odt, out.stride(0), out.stride(1),
                               out.stride(2), B, H, Sq, Skv, D, mask, 0, 1, kv_splits,
                               ws.data_ptr(), ws.numel(), st)
    torch.cuda.synchronize()
    return rc


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_q16_launch_equals_the_code_launch(gpu: torch.device, case: tuple) -> None:
    name, B, H, Sq, Skv, D, dtype, odt, kv_splits, causal, layout, gran = case
    q, k, v = _inputs(name, B, H, Sq, Skv, D, dtype, layout, gpu)
    mask = _capi.RP_MASK_CAUSAL if causal else _capi.RP_MASK_NONE
    st = torch.cuda.current_stream(gpu).cuda_stream
    assert _capi.lib().rp_fp8_attn_q16_supported(B, H, Sq, Skv, D, mask, kv_splits, st) == 1
    if name.startswith("resident_kv"):
        assert _capi.lib().rp_fp8_attn_resident_kv(B, H, Sq, Skv, D, mask, 1) == 1
    sm = 1.0 / math.sqrt(D)
    qs, q8, ks, k8, vs, vt8 = ops.scale_quantize_qkv(q, k, v, gran)
    want = ops.attention_fp8(q8.view(torch.uint8), k8.view(torch.uint8), vt8.view(torch.uint8),
                             qs, ks, vs, sm, out_dtype=odt, causal=causal, kv_splits=kv_splits)
    got = torch.empty_like(want)
    print(f"{name}: q16 launch (B={B} H={H} Sq={Sq} Skv={Skv} D={D} splits={kv_splits})",
          flush=True)
    rc = _q16_call(q, k8.view(torch.uint8), vt8.view(torch.uint8), qs, ks, vs, got, sm, mask,
                   kv_splits)
    assert rc == 0, _capi.lib().rp_last_error()
    assert torch.equal(got.view(torch.uint8) if got.dtype != torch.float32 else got,
                       want.view(torch.uint8) if want.dtype != torch.float32 else want), name


def test_q16_refuses_the_multi_block_launch(gpu: torch.device) -> None:
    """A short key range past what LDS holds (8 tiles at D = 128) runs the
    multi-block kernel, which stages Q's codes through LDS: the raw-Q entry
    says so before launching anything."""
    B, H, Sq, Skv, D = 1, 16, 9000, 1024, 128
    st = torch.cuda.current_stream(gpu).cuda_stream
    L = _capi.lib()
    assert L.rp_fp8_attn_blocks_per_workgroup(B, H, Sq, Skv, D, 0, 1) > 1
    assert L.rp_fp8_attn_resident_kv(B, H, Sq, Skv, D, 0, 1) == 0
    assert L.rp_fp8_attn_q16_supported(B, H, Sq, Skv, D, 0, 1, st) == 0
    q, k, v = _inputs("multi", B, H, Sq, Skv, D, torch.bfloat16, "bhsd", gpu)
    qs, _, ks, k8, vs, vt8 = ops.scale_quantize_qkv(q, k, v)
    out = torch.empty(B, H, Sq, D, dtype=torch.bfloat16, device=gpu)
    rc = _q16_call(q, k8.view(torch.uint8), vt8.view(torch.uint8), qs, ks, vs, out,
                   D ** -0.5, 0, 1)
    assert rc == 2    # RP_ERR_UNSUPPORTED
    assert b"codes only" in _capi.lib().rp_last_error()


def test_quantizer_without_q_codes(gpu: torch.device) -> None:
    """rp_fp8_scale_quantize_qkv with q8 = NULL: every scale and the K and
    V^T codes of the full call, for small calls (whose full call folds the
    scales into the apply launch) and large ones (finalize + apply)."""
    for B, H, Sq, Skv, D in ((1, 8, 1024, 1024, 64), (1, 8, 20000, 3000, 128)):
        q, k, v = _inputs(f"nq{Sq}", B, H, Sq, Skv, D, torch.bfloat16, "bhsd", gpu)
        for gran in ("bh", "tensor"):
            qs, _, ks, k8, vs, vt8 = ops.scale_quantize_qkv(q, k, v, gran)
            arena, (o_k, o_v, o_s), G, ldv = ops._qkv_arena(q, k, v, gran, None, q_codes=False)
            torch.cuda.synchronize()
            assert o_k == 0
            nk, nv = B * H * Skv * D, B * H * D * ldv
            assert torch.equal(arena[o_s:o_s + 12 * G].view(torch.float32),
                               torch.cat([qs, ks, vs]))
            assert torch.equal(arena[:nk], k8.reshape(-1).view(torch.uint8))
            assert torch.equal(arena[o_v:o_v + nv], vt8.reshape(-1).view(torch.uint8))


def test_op_runs_the_q16_launch_with_the_code_path_bits(gpu: torch.device,
                                                        monkeypatch: pytest.MonkeyPatch) -> None:
    """fp8_flash_attention with a known launch (autotuning off: one range)
    takes the raw-Q launch where it runs the resident-K/V kernel (a
    cross-attention shape), and its output equals the two-step path's; a
    self-attention shape keeps the two-step path."""
    monkeypatch.setenv("REPERCEP_FP8_DISABLE_AUTOTUNE", "1")
    calls = []
    real = ops._qkv_q16_attention
    monkeypatch.setattr(ops, "_qkv_q16_attention",
                        lambda *a, **kw: (calls.append(1), real(*a, **kw))[1])
    for name, Sq, Skv, takes in (("op_cross", 9000, 512, True), ("op_self", 2000, 2000, False)):
        calls.clear()
        q, k, v = _inputs(name, 1, 40 if takes else 4, Sq, Skv, 128, torch.bfloat16, "bshd",
                          gpu)
        got = ops.fp8_flash_attention(q, k, v)
        assert bool(calls) == takes, name
        qs, q8, ks, k8, vs, vt8 = ops.scale_quantize_qkv(q, k, v)
        want = ops.attention_fp8(q8.view(torch.uint8), k8.view(torch.uint8),
                                 vt8.view(torch.uint8), qs, ks, vs, 128 ** -0.5,
                                 out_dtype=torch.bfloat16)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.uint8), want.view(torch.uint8)), name


@pytest.mark.parametrize("Sq,Skv", [(1000, 1000), (9000, 512)], ids=["one_range", "resident_kv"])
def test_q16_codes_at_the_extreme_scales(gpu: torch.device, Sq: int, Skv: int) -> None:
    """bf16 rows are quantized without the clamp (Q's own scale keeps every
    |x * qm| <= 426.67).  Heads whose maxima sit at that worst case
    (amax 1.043e-6), at 1e-6 and below (the scale's floor), and at large
    magnitudes: the raw-Q launch equals the code launch bit for bit."""
    B, H, D = 1, (40 if Skv == 512 else 4), 128
    if Skv == 512:
        assert _capi.lib().rp_fp8_attn_resident_kv(B, H, Sq, Skv, D, 0, 1) == 1
    q, k, v = _inputs(f"ext{Sq}", B, H, Sq, Skv, D, torch.bfloat16, "bhsd", gpu)
    worst = torch.tensor(1.043081283569336e-06).to(torch.bfloat16).float().item()
    for h, amax in enumerate((worst, 1e-6, 3e-7, 3.0e4)):
        qh = q[0, h].float()
        qh = qh / qh.abs().max() * amax
        q[0, h] = qh.to(torch.bfloat16)
        q[0, h, 7, 5] = torch.tensor(amax).to(torch.bfloat16)     # the maximum itself
    for gran in ("bh", "tensor"):
        qs, q8, ks, k8, vs, vt8 = ops.scale_quantize_qkv(q, k, v, gran)
        want = ops.attention_fp8(q8.view(torch.uint8), k8.view(torch.uint8),
                                 vt8.view(torch.uint8), qs, ks, vs, D ** -0.5,
                                 out_dtype=torch.float32, kv_splits=1)
        got = torch.empty_like(want)
        print(f"extreme scales Sq={Sq} Skv={Skv} {gran}", flush=True)
        rc = _q16_call(q, k8.view(torch.uint8), vt8.view(torch.uint8), qs, ks, vs, got,
                       D ** -0.5, 0, 1)
        assert rc == 0, _capi.lib().rp_last_error()
        assert torch.equal(got, want), gran


def test_q16_non_finite_head(gpu: torch.device) -> None:
    """A NaN in one head's Q makes that head's scale NaN: both launches give
    that head NaN everywhere and every other head the same bits."""
    B, H, Sq, Skv, D = 1, 40, 9000, 512, 128
    assert _capi.lib().rp_fp8_attn_resident_kv(B, H, Sq, Skv, D, 0, 1) == 1
    q, k, v = _inputs("nanq", B, H, Sq, Skv, D, torch.bfloat16, "bhsd", gpu)
    q[0, 2, 100, 3] = float("nan")
    qs, q8, ks, k8, vs, vt8 = ops.scale_quantize_qkv(q, k, v, "bh")
    keep = [h for h in range(H) if h != 2]
    assert torch.isnan(qs[2]) and torch.isfinite(qs[keep]).all()
    want = ops.attention_fp8(q8.view(torch.uint8), k8.view(torch.uint8), vt8.view(torch.uint8),
                             qs, ks, vs, D ** -0.5, out_dtype=torch.float32, kv_splits=1)
    got = torch.empty_like(want)
    rc = _q16_call(q, k8.view(torch.uint8), vt8.view(torch.uint8), qs, ks, vs, got, D ** -0.5,
                   0, 1)
    assert rc == 0, _capi.lib().rp_last_error()
    assert torch.isnan(got[0, 2]).all() and torch.isnan(want[0, 2]).all()
    assert torch.equal(got[0, keep], want[0, keep])
