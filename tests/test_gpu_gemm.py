"""GPU parity of the FP8 scaled GEMM.

Shapes with K a multiple of 64 run the large-tile kernel (one to nine 64-deep
K slices, ragged M and N); K = 48 and K = 16 run the general kernel.

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


def _bf16_rne(x: np.ndarray) -> np.ndarray:
    """float64 -> nearest bf16 value (via fp32, round to nearest even), as float64."""
    f = np.asarray(x, dtype=np.float32)
    return bf16_to_f32(np.asarray(torch.from_numpy(f).to(torch.bfloat16).view(torch.int16)
                                  .numpy().view(np.uint16))).astype(np.float64)


def _assert_one_rounding_apart(got: np.ndarray, ref: np.ndarray | None, a8: np.ndarray,
                               bt8: np.ndarray, scale: float,
                               bias: np.ndarray | None = None) -> None:
    """Every kernel output is the bf16 rounding of some value within eps of the exact
    scaled dot product, eps = 2^-14 * sum |a||b| * scale.  The f8f6f4 MFMA's dot
    product is not an exactly rounded fp32 sum (measured: up to 2^-15.5 of
    sum |a||b| away from it, identically for the 16x16x128 and 32x32x64 forms),
    so a result may round to the bf16 neighbour of the oracle's.  With a
    ``bias`` (float64 [N]) the value is exact * scale + bias, and eps widens by
    the two fp32 roundings of the epilogue (product, then sum).  Also reports
    BASELINE's error metrics against ``ref``, the oracle (exact sum rounded
    once); ``ref=None`` takes that rounding of the float64 sum here."""
    A = DECODE[a8].astype(np.float64)
    Bt = DECODE[bt8].astype(np.float64)
    exact = (A @ Bt.T) * float(np.float32(scale))
    eps = 2.0 ** -14 * (np.abs(A) @ np.abs(Bt).T) * abs(scale)
    if bias is not None:
        eps = eps + 2.0 ** -23 * (2 * np.abs(exact) + np.abs(bias))
        exact = exact + bias
    st = err_stats(got, _bf16_rne(exact) if ref is None else ref)
    lo = _bf16_rne(exact - eps)
    hi = _bf16_rne(exact + eps)
    g = got.astype(np.float64)
    bad = (g < np.minimum(lo, hi)) | (g > np.maximum(lo, hi))
    print(st, "outputs outside the rounding interval:", int(bad.sum()), flush=True)
    assert not bad.any(), f"{int(bad.sum())} outputs are not a rounding of a value near the exact sum"
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


@pytest.mark.parametrize("mnk", [(257, 130 * 4, 384), (1000, 64, 512), (64, 1024, 1024),
                                 (600, 520, 192), (300, 300, 64), (2, 8, 576), (513, 260, 48)])
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
    # the reference's (K, N) row-major B, staged and transposed in LDS by the
    # kernel (the MFMAs see the same bytes in the same order), scales on device
    got2 = ops.fp8_gemm(a8.to(gpu), bt8.to(gpu).t().contiguous(),
                        torch.tensor([sa], device=gpu), torch.tensor([sb], device=gpu))
    assert torch.equal(got2, got)


@pytest.mark.parametrize("mnk,ldb_pad", [
    ((300, 400, 320), 0),      # ragged N tile (256 + 144), K % 128 == 64: half last slice
    ((257, 512, 1024), 48),    # row-strided (K, N) view, ldb = N + 48
    ((64, 256, 64), 0),        # one 64-deep K slice
    ((513, 272, 192), 16),     # N % 256 == 16: one granule in the last tile
    ((100, 100, 4160), 0),     # N % 16 != 0: the general kernel's byte gathers
    ((33, 12, 48), 4),         # K % 64 != 0, odd ldb: the general kernel
])
def test_row_major_b_vs_oracle(gpu: torch.device, mnk: tuple[int, int, int],
                               ldb_pad: int, monkeypatch: pytest.MonkeyPatch) -> None:
    """B given as the reference passes it, (K, N) row-major (rp_fp8_gemm with
    RP_B_KN): no transpose pass runs, and the result is the (N, K) path's
    bit for bit and within one rounding of the exact sum."""
    M, N, K = mnk
    g = torch.Generator().manual_seed(7 * M + N + K)
    a8 = torch.randn(M, K, generator=g).mul(30).to(torch.float8_e4m3fn)
    b8 = torch.randn(K, N, generator=g).mul(30).to(torch.float8_e4m3fn)
    sa, sb = 0.011, 0.0093
    store = torch.zeros(K, N + ldb_pad, dtype=torch.uint8)
    store[:, :N] = b8.view(torch.uint8)
    bview = store.to(gpu)[:, :N]
    monkeypatch.setattr(ops, "transpose_fp8", lambda *_a, **_k: pytest.fail("transpose pass ran"))
    got = ops.fp8_gemm(a8.to(gpu), bview, sa, sb)
    nk = ops.fp8_gemm(a8.to(gpu), b8.t().contiguous().to(gpu), sa, sb, b_transposed=True)
    assert torch.equal(got, nk), f"max diff {(got.float() - nk.float()).abs().max().item()}"
    bt = np.ascontiguousarray(codes_np(b8).T)
    ref = native.gemm_rows(codes_np(a8), bt, sa, sb, np.arange(M))
    _assert_one_rounding_apart(bf16_to_f32(bf16_bits(got)), bf16_to_f32(ref), codes_np(a8),
                               bt, sa * sb)


def test_weight_with_unaligned_n_and_k(gpu: torch.device) -> None:
    """fp8_linear_weight on a (K, N) weight with K % 128 != 0 and N % 32 != 0
    (K = 4160, N = 100), both layouts, against the oracle: the (N, K) operand
    is a valid B^T whatever its padding, and the (K, N) codes run as they lie."""
    K, N, M = 4160, 100, 96
    g = torch.Generator().manual_seed(4160)
    w = torch.randn(K, N, generator=g).mul(0.02).to(torch.bfloat16)
    a = torch.randn(M, K, generator=g).to(torch.bfloat16)
    sa, a8 = ops.scale_quantize(a.to(gpu), "tensor", "bhsd")
    a8 = a8.view(torch.uint8).reshape(M, K)
    sw, wt8 = ops.fp8_linear_weight(w.to(gpu))
    assert wt8.shape == (N, K)
    sw2, w8 = ops.fp8_linear_weight(w.to(gpu), layout="kn")
    assert w8.shape == (K, N) and float(sw2.item()) == float(sw.item())
    ws_ref, w8_ref = native.quantize_groups(bf16_bits(w), 1)
    assert float(ws_ref[0]) == float(sw.item())
    assert np.array_equal(codes_np(w8), w8_ref) and np.array_equal(codes_np(wt8), w8_ref.T)
    c_nk = ops.fp8_gemm(a8, wt8, sa, sw, b_transposed=True)
    c_kn = ops.fp8_gemm(a8, w8, sa, sw)
    assert torch.equal(c_nk, c_kn)
    ref = native.gemm_rows(codes_np(a8), np.ascontiguousarray(w8_ref.T), float(sa.item()),
                           float(sw.item()), np.arange(M))
    _assert_one_rounding_apart(bf16_to_f32(bf16_bits(c_nk)), bf16_to_f32(ref), codes_np(a8),
                               np.ascontiguousarray(w8_ref.T), float(sa.item()) * float(sw.item()))


@pytest.mark.parametrize("mnk", [(64, 64, 256), (300, 200, 512), (5, 4, 16)])
def test_bias_epilogue_small_integers_exact(gpu: torch.device, mnk: tuple[int, int, int]) -> None:
    """rp_fp8_linear on integer operands (exact fp32 sums) with scale fp32(1/3):
    the output is bf16(fp32(fp32(acc * s) + bias)) bit for bit, which differs
    from rounding the product to bf16 before the bias is added."""
    M, N, K = mnk
    g = torch.Generator().manual_seed(M * N + K)
    a_i = torch.randint(-2, 3, (M, K), generator=g, dtype=torch.float32)
    b_i = torch.randint(-2, 3, (K, N), generator=g, dtype=torch.float32)
    bias = torch.randn(N, generator=g).mul(20).to(torch.bfloat16)
    s = np.float32(1.0 / 3.0)
    t = (a_i @ b_i) * torch.tensor(s)
    ref = (t + bias.float()).to(torch.bfloat16)
    got = ops.fp8_gemm(a_i.to(gpu).to(torch.float8_e4m3fn), b_i.to(gpu).to(torch.float8_e4m3fn),
                       float(s), 1.0, bias=bias.to(gpu)).cpu()
    assert torch.equal(got, ref), f"max abs diff {(got.float() - ref.float()).abs().max().item()}"
    if M * N >= 4096:
        twice = (t.to(torch.bfloat16).float() + bias.float()).to(torch.bfloat16)
        assert not torch.equal(twice, ref), "case does not tell one rounding from two"


@pytest.mark.parametrize("mnk", [(257, 520, 384), (1000, 64, 512), (600, 520, 192),
                                 (513, 260, 48)])
def test_bias_epilogue_vs_oracle(gpu: torch.device, mnk: tuple[int, int, int]) -> None:
    """Both GEMM kernels (256x256 tiles when K % 64 == 0, the 256x128 fallback
    otherwise) with a bias: every output within one rounding of
    exact * scale + bias, and with a zero bias bit-identical to rp_fp8_gemm."""
    M, N, K = mnk
    g = torch.Generator().manual_seed(3 * M + N + K)
    a8 = torch.randn(M, K, generator=g).mul(30).to(torch.float8_e4m3fn)
    bt8 = torch.randn(N, K, generator=g).mul(30).to(torch.float8_e4m3fn)
    bias = torch.randn(N, generator=g).mul(50).to(torch.bfloat16)
    sa, sb = 0.013, 0.0071
    got = ops.fp8_gemm(a8.to(gpu), bt8.to(gpu), sa, sb, b_transposed=True, bias=bias.to(gpu))
    bias64 = bias.float().numpy().astype(np.float64)
    _assert_one_rounding_apart(bf16_to_f32(bf16_bits(got)), None, codes_np(a8), codes_np(bt8),
                               sa * sb, bias64)
    plain = ops.fp8_gemm(a8.to(gpu), bt8.to(gpu), sa, sb, b_transposed=True)
    zero = ops.fp8_gemm(a8.to(gpu), bt8.to(gpu), sa, sb, b_transposed=True,
                        bias=torch.zeros(N, dtype=torch.bfloat16, device=gpu))
    assert torch.equal(zero, plain)


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
    # the weight as the reference passes it, (K, N) row-major: the same output
    sw2, w8 = ops.fp8_linear_weight(w, layout="kn")
    c2 = ops.fp8_gemm(a8.view(torch.uint8), w8, sa, sw2)
    assert torch.equal(c2, c)
    del a, w, a8, wt8, c, c2, w8
    torch.cuda.empty_cache()


def test_out_argument_is_checked(gpu: torch.device) -> None:
    a = torch.zeros(64, 32, device=gpu).to(torch.float8_e4m3fn)
    bt = torch.zeros(16, 32, device=gpu).to(torch.float8_e4m3fn)
    for bad in (torch.empty(64, 8, dtype=torch.bfloat16, device=gpu),      # too narrow
                torch.empty(64, 16, dtype=torch.float32, device=gpu),      # dtype
                torch.empty(16, 64, dtype=torch.bfloat16, device=gpu).t()):  # column stride
        with pytest.raises((ValueError, TypeError)):
            ops.fp8_gemm(a, bt, 1.0, 1.0, b_transposed=True, out=bad)
    wide = torch.full((64, 24), 7.0, dtype=torch.bfloat16, device=gpu)
    c = ops.fp8_gemm(a, bt, 1.0, 1.0, b_transposed=True, out=wide[:, :16])
    assert torch.equal(c, torch.zeros(64, 16, dtype=torch.bfloat16, device=gpu))
    assert torch.equal(wide[:, 16:], torch.full((64, 8), 7.0, dtype=torch.bfloat16, device=gpu))


@pytest.mark.parametrize("mnk", [(300, 260, 128), (513, 516, 192)])
def test_output_row_stride_and_offset(gpu: torch.device, mnk: tuple[int, int, int]) -> None:
    """C written into views of a wider buffer -- row strides that are and are
    not multiples of 8 elements, a base 8 but not 16 bytes aligned, N % 8 == 4
    -- equals the packed output, and the padding around it is untouched."""
    M, N, K = mnk
    g = torch.Generator().manual_seed(M + N)
    a8 = torch.randn(M, K, generator=g).mul(30).to(torch.float8_e4m3fn).to(gpu)
    bt8 = torch.randn(N, K, generator=g).mul(30).to(torch.float8_e4m3fn).to(gpu)
    plain = ops.fp8_gemm(a8, bt8, 0.01, 0.02, b_transposed=True)
    for extra, off in ((4, 0), (4, 4), (8, 4), (12, 8)):
        wide = torch.full((M, off + N + extra), 7.0, dtype=torch.bfloat16, device=gpu)
        c = ops.fp8_gemm(a8, bt8, 0.01, 0.02, b_transposed=True, out=wide[:, off:off + N])
        assert torch.equal(c, plain), (extra, off)
        pad = torch.cat([wide[:, :off], wide[:, off + N:]], dim=1)
        assert (pad == 7.0).all(), (extra, off)


def test_device_reproduces_golden_vectors(gpu: torch.device,
                                         monkeypatch: pytest.MonkeyPatch) -> None:
    """The committed known-answer vectors through the reference's (K, N)
    row-major B (staged and transposed by the kernel, no transpose pass) and
    through the K-contiguous operand, scales as host floats and as device
    tensors: every output bit for bit."""
    from tests._helpers import golden_gemm_cases

    monkeypatch.setattr(ops, "transpose_fp8", lambda *_a, **_k: pytest.fail("transpose pass ran"))
    for name, a8, b8, sa, sb, c_bits in golden_gemm_cases():
        a = torch.from_numpy(a8).to(gpu).view(torch.float8_e4m3fn)
        b = torch.from_numpy(b8).to(gpu).view(torch.float8_e4m3fn)
        c1 = ops.fp8_gemm(a, b, sa, sb)
        c2 = ops.fp8_gemm(a, b.t().contiguous(), torch.tensor([sa], device=gpu),
                          torch.tensor([sb], device=gpu), b_transposed=True)
        for c in (c1, c2):
            assert np.array_equal(bf16_bits(c), c_bits), name


def _linear_static(a8, b8, layout, bias, out, M, N, K, sa, sb):
    from repercep_runtime_amd import _capi as C
    C.check(C.lib().rp_fp8_linear(a8.data_ptr(), b8.data_ptr(), layout,
                                  bias.data_ptr() if bias is not None else None, out.data_ptr(),
                                  M, N, K, a8.stride(0), b8.stride(0), out.stride(0), sa, sb,
                                  None, None, ops._stream(a8)), "rp_fp8_linear")


@pytest.mark.parametrize("M,N,K,layout,with_bias", [
    (300, 272, 128, "kn", False),     # 4 tiles: shares of 0 and 1 tiles, nothing to pool
    (2148, 1280, 128, "kn", True),    # 45 tiles: shares of 6 and 5, every tile pooled
    (2560, 2304, 192, "nk", True),    # 90 tiles: shares of 12 and 11, every tile pooled
    (C4.M, C4.N, 512, "kn", False),   # the C4 grid (15,984 tiles): 64 pooled per share
    (C4.M, C4.N, 512, "nk", True),
])
def test_balanced_gemm_equals_static_tiles(gpu: torch.device, M: int, N: int, K: int,
                                           layout: str, with_bias: bool) -> None:
    """rp_fp8_linear_balanced (the op's launch: the last tiles of every XCD's
    share handed out through a counter) writes rp_fp8_linear's bits, on grids
    too small to pool, where every tile is pooled and the XCD shares differ by
    one tile, and on C4's grid; two calls in a row reuse the workspace (the call zeroes its
    counter itself)."""
    from repercep_runtime_amd import _capi as C
    g = torch.Generator(device=gpu).manual_seed(M + N + K)
    a8 = torch.randint(0, 126, (M, K), generator=g, device=gpu, dtype=torch.uint8)
    b8 = torch.randint(0, 126, (K, N) if layout == "kn" else (N, K), generator=g, device=gpu,
                       dtype=torch.uint8)
    lay = C.RP_B_KN if layout == "kn" else C.RP_B_NK
    bias = (torch.randn(N, generator=g, device=gpu).to(torch.bfloat16) if with_bias else None)
    ref = torch.empty((M, N), dtype=torch.bfloat16, device=gpu)
    _linear_static(a8, b8, lay, bias, ref, M, N, K, 0.01, 0.02)
    ws = torch.empty(C.RP_GEMM_BALANCED_WORKSPACE_BYTES, dtype=torch.uint8, device=gpu)
    for _ in range(2):
        out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu)
        C.check(C.lib().rp_fp8_linear_balanced(
            a8.data_ptr(), b8.data_ptr(), lay, bias.data_ptr() if bias is not None else None,
            out.data_ptr(), M, N, K, a8.stride(0), b8.stride(0), out.stride(0), 0.01, 0.02, None,
            None, ws.data_ptr(), ws.numel(), ops._stream(a8)), "rp_fp8_linear_balanced")
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
