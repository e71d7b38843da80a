"""GPU parity of the FP8 scaled GEMM.

Reference: kernels/hip/fp8_attn/fp8_gemm.hip:79-179 and its known-answer
tests tests/test_mfma_fragment_layout.py:262-315 (restated here for the
OCP e4m3fn format): all-ones -> every C == K, and small integers in [-2, 2]
compared exactly with (a @ b).bf16().
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import native
from repercep_runtime_amd import ops
from repercep_runtime_amd.workloads import C4, gemm_inputs
from oracle.quant import DECODE
from tests._helpers import bf16_bits, bf16_to_f32, bf16_ulp, codes_np, err_stats

pytestmark = pytest.mark.gpu


def _assert_one_rounding_apart(got: np.ndarray, ref: np.ndarray, a8: np.ndarray,
                               bt8: np.ndarray, scale: float) -> None:
    """The kernel and the oracle agree up to the fp32 accumulation order: within one
    bf16 ulp of the output plus a bound on the order-dependent fp32 rounding
    (2^-16 of sum |a||b|, K <= 2^14).  Also reports BASELINE's error metrics."""
    st = err_stats(got, ref)
    absab = np.abs(DECODE[a8].astype(np.float64)) @ np.abs(DECODE[bt8].astype(np.float64)).T
    tol = bf16_ulp(np.maximum(np.abs(got), np.abs(ref))) + 2.0 ** -16 * absab * abs(scale)
    bad = np.abs(got.astype(np.float64) - ref) > tol
    print(st, "elements beyond one rounding:", int(bad.sum()), flush=True)
    assert not bad.any(), f"{int(bad.sum())} elements differ by more than one rounding"
    assert st["rel_mean"] <= 1e-3


def test_all_ones_sums_to_k(gpu: torch.device) -> None:
    a = torch.ones(16, 32, device=gpu).to(torch.float8_e4m3fn)
    b = torch.ones(32, 16, device=gpu).to(torch.float8_e4m3fn)
    c = ops.fp8_gemm(a, b, 1.0, 1.0).float()
    assert torch.equal(c, torch.full((16, 16), 32.0, device=gpu))


@pytest.mark.parametrize("mnk", [(32, 32, 64), (300, 200, 256), (16, 16, 128), (5, 4, 16)])
def test_small_integers_exact(gpu: torch.device, mnk: tuple[int, int, int]) -> None:
    M, N, K = mnk
    torch.manual_seed(0)
    a_i = torch.randint(-2, 3, (M, K), dtype=torch.float32)
    b_i = torch.randint(-2, 3, (K, N), dtype=torch.float32)
    ref = (a_i @ b_i).to(torch.bfloat16).float()
    got = ops.fp8_gemm(a_i.to(gpu).to(torch.float8_e4m3fn), b_i.to(gpu).to(torch.float8_e4m3fn),
                       1.0, 1.0).float().cpu()
    assert torch.equal(got, ref), f"max abs diff {(got - ref).abs().max().item()}"


@pytest.mark.parametrize("mnk", [(257, 130 * 4, 384), (1000, 64, 512), (64, 1024, 1024)])
def test_random_vs_oracle(gpu: torch.device, mnk: tuple[int, int, int]) -> None:
    M, N, K = mnk
    g = torch.Generator().manual_seed(M + N + K)
    a8 = torch.randn(M, K, generator=g).mul(30).to(torch.float8_e4m3fn)
    bt8 = torch.randn(N, K, generator=g).mul(30).to(torch.float8_e4m3fn)
    sa, sb = 0.013, 0.0071
    got = ops.fp8_gemm(a8.to(gpu), bt8.to(gpu), sa, sb, b_transposed=True)
    ref = native.gemm_rows(codes_np(a8), codes_np(bt8), sa, sb, np.arange(M))
    _assert_one_rounding_apart(bf16_to_f32(bf16_bits(got)), bf16_to_f32(ref), codes_np(a8),
                               codes_np(bt8), sa * sb)
    # the reference's (K, N) row-major B through the transposing path, scales on device
    got2 = ops.fp8_gemm(a8.to(gpu), bt8.to(gpu).t().contiguous(),
                        torch.tensor([sa], device=gpu), torch.tensor([sb], device=gpu))
    assert torch.equal(got2, got)


def test_wan_ffn_gemm_full_shape_sampled_rows(gpu: torch.device) -> None:
    """C4: A (75600 x 5120) N(0,1), W (5120 x 13824) N(0, 0.02); per-tensor scales."""
    a, w = gemm_inputs(C4, device=gpu)
    sa, a8 = ops.scale_quantize(a, "tensor", "bhsd")
    sw, wt8 = ops.fp8_linear_weight(w)
    c = ops.fp8_gemm(a8.view(torch.uint8), wt8, sa, sw, b_transposed=True)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(1).choice(C4.M, size=48, replace=False))
    a_cpu = a[torch.from_numpy(rows).to(gpu)].cpu()
    # codes of the sampled rows under the whole-tensor scale
    sa_h = float(sa.item())
    a8_rows = native.quantize_bf16(bf16_bits(a_cpu), sa_h)
    assert np.array_equal(a8_rows, codes_np(a8)[rows])
    ws_ref, w8_ref = native.quantize_groups(bf16_bits(w.cpu()), 1)
    assert float(ws_ref[0]) == float(sw.item())
    assert np.array_equal(np.ascontiguousarray(w8_ref.T), codes_np(wt8)[:, :C4.K])
    ref = native.gemm_rows(a8_rows, codes_np(wt8)[:, :C4.K].copy(), sa_h, float(sw.item()),
                           np.arange(len(rows)))
    got = bf16_to_f32(bf16_bits(c[torch.from_numpy(rows).to(gpu)]))
    _assert_one_rounding_apart(got, bf16_to_f32(ref), a8_rows, codes_np(wt8)[:, :C4.K],
                               sa_h * float(sw.item()))
    del a, w, a8, wt8, c
    torch.cuda.empty_cache()
