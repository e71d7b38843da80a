"""GPU parity of the FP8 quantizer against the CPU oracle: bit-exact codes and scales.

Reference behaviour: _per_bh_scale / _quantize,
kernels/triton_kernels/fp8_flash_attn_hopper.py:374-398.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import native
from repercep_runtime_amd import ops
from repercep_runtime_amd.workloads import C1, C3_SELF, attn_inputs
from tests._helpers import bf16_bits, codes_np, vt_to_bhsd

pytestmark = pytest.mark.gpu


def _nan_code(c: np.ndarray) -> np.ndarray:
    return (c & 0x7F) == 0x7F


def _assert_codes_equal(got: np.ndarray, ref: np.ndarray) -> None:
    """Bit-exact, except that the sign of a NaN code is not specified."""
    both_nan = _nan_code(got) & _nan_code(ref)
    bad = (got != ref) & ~both_nan
    n_bad = int(bad.sum())
    if n_bad:
        idx = np.flatnonzero(bad.ravel())[:8]
        pytest.fail(f"{n_bad} code mismatches; first at {idx}: got {got.ravel()[idx]}, "
                    f"want {ref.ravel()[idx]}")


def _assert_scales_equal(got: np.ndarray, ref: np.ndarray) -> None:
    g = got.astype(np.float32)
    r = ref.astype(np.float32)
    same = (g.view(np.uint32) == r.view(np.uint32)) | (np.isnan(g) & np.isnan(r))
    assert same.all(), f"scales differ: got {g[~same][:8]}, want {r[~same][:8]}"


def _oracle(x_cpu: torch.Tensor, granularity: str) -> tuple[np.ndarray, np.ndarray]:
    bits = bf16_bits(x_cpu.contiguous())
    n = x_cpu.shape[0] * x_cpu.shape[1] if granularity == "bh" else 1
    return native.quantize_groups(bits, n)


def test_hw_e4m3_cvt_matches_torch_cast_on_every_fp32_pattern(gpu: torch.device) -> None:
    """v_cvt_pk_fp8_f32 (after the reference's +-448 clamp) vs torch's cast, all 2^32 inputs."""
    chunk = 1 << 28
    total_bad = 0
    for start in range(0, 1 << 32, chunk):
        u = torch.arange(start, start + chunk, dtype=torch.int64, device=gpu).to(torch.int32)
        x = u.view(torch.float32)
        hw = ops.selftest_e4m3(x)
        ref = x.clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8)
        nan_both = ((hw & 0x7F) == 0x7F) & ((ref & 0x7F) == 0x7F)
        bad = (hw != ref) & ~nan_both
        nb = int(bad.sum().item())
        if nb:
            i = int(torch.nonzero(bad)[0].item())
            print(f"chunk {start:#x}: {nb} mismatches, first x bits {start + i:#010x} "
                  f"hw {int(hw[i])} ref {int(ref[i])}", flush=True)
        total_bad += nb
        del u, x, hw, ref, bad, nan_both
    assert total_bad == 0


def test_scale_formula_on_every_bf16_amax(gpu: torch.device) -> None:
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    dq, qm = ops.selftest_scale(torch.from_numpy(bits.view(np.int16)).to(gpu))
    ref = np.array([native.dequant_from_amax(int(b)) for b in bits], dtype=np.float32)
    _assert_scales_equal(dq.cpu().numpy(), ref)
    with np.errstate(divide="ignore", invalid="ignore"):
        ref_qm = np.float32(1.0) / ref
    _assert_scales_equal(qm.cpu().numpy(), ref_qm)


SHAPES = [
    (1, 8, 1024, 64),
    (2, 3, 257, 128),
    (1, 1, 5, 64),
    (1, 2, 1, 128),
    (3, 1, 130, 64),
]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("granularity", ["bh", "tensor"])
def test_quantize_bhsd_bit_exact(gpu: torch.device, shape: tuple[int, ...],
                                 granularity: str) -> None:
    g = torch.Generator().manual_seed(sum(shape))
    x = torch.randn(shape, generator=g).mul(3.0).to(torch.bfloat16)
    ref_s, ref_c = _oracle(x, granularity)
    dq, codes = ops.scale_quantize(x.to(gpu), granularity, "bhsd")
    _assert_scales_equal(dq.cpu().numpy(), ref_s)
    _assert_codes_equal(codes_np(codes), ref_c)
    # separate scale / apply entry points agree with the fused one
    dq2 = ops.per_bh_scale(x.to(gpu), granularity)
    _assert_scales_equal(dq2.cpu().numpy(), ref_s)
    c2 = ops.quantize(x.to(gpu), dq2, granularity, "bhsd")
    _assert_codes_equal(codes_np(c2), ref_c)


@pytest.mark.parametrize("shape", [(1, 8, 1024, 64), (2, 3, 257, 128), (1, 2, 1, 128),
                                   (1, 1, 300, 256), (1, 3, 200, 32), (2, 2, 130, 96)])
def test_quantize_bhds_transposed_bit_exact(gpu: torch.device, shape: tuple[int, ...]) -> None:
    g = torch.Generator().manual_seed(7 + sum(shape))
    x = torch.randn(shape, generator=g).to(torch.bfloat16)
    ref_s, ref_c = _oracle(x, "bh")
    dq, vt = ops.scale_quantize(x.to(gpu), "bh", "bhds")
    B, H, S, D = shape
    vt_np = codes_np(vt)
    assert vt_np.shape == (B, H, D, (S + 127) // 128 * 128)
    _assert_scales_equal(dq.cpu().numpy(), ref_s)
    _assert_codes_equal(vt_to_bhsd(vt_np, S), ref_c)
    assert not vt_np[..., S:].any(), "padding columns must be zero"


def test_quantize_strided_bshd_view(gpu: torch.device) -> None:
    """A permuted (B, S, H, D) buffer is read in place (diffusers layout)."""
    g = torch.Generator().manual_seed(3)
    bshd = torch.randn(2, 300, 4, 128, generator=g).to(torch.bfloat16)
    x_view = bshd.to(gpu).permute(0, 2, 1, 3)          # (B, H, S, D) strided view
    ref_s, ref_c = _oracle(bshd.permute(0, 2, 1, 3).contiguous(), "bh")
    for gran in ("bh", "tensor"):
        ref_s, ref_c = _oracle(bshd.permute(0, 2, 1, 3).contiguous(), gran)
        dq, codes = ops.scale_quantize(x_view, gran, "bhsd")
        _assert_scales_equal(dq.cpu().numpy(), ref_s)
        _assert_codes_equal(codes_np(codes), ref_c)
        dqt, vt = ops.scale_quantize(x_view, gran, "bhds")
        _assert_codes_equal(vt_to_bhsd(codes_np(vt), 300), ref_c)


def _special_inputs() -> list[tuple[str, torch.Tensor]]:
    g = torch.Generator().manual_seed(11)
    base = torch.randn(2, 2, 64, 64, generator=g)
    cases = []
    z = base.clone()
    z[0, 1] = 0.0                                   # all-zero group -> amax clamps to 1e-6
    cases.append(("zero_group", z))
    n = base.clone()
    n[1, 0, 3, 5] = float("nan")                     # NaN propagates through amax
    cases.append(("nan", n))
    i = base.clone()
    i[0, 0, 7, 7] = float("inf")                     # inf amax -> q_mul 0 -> zeros and NaN
    i[1, 1, 2, 2] = float("-inf")
    cases.append(("inf", i))
    m0 = base.clone()
    m0[0, 0] = -0.0                                  # -0.0 group -> code 0x80
    m0[0, 0, 0, 0] = 0.0
    cases.append(("neg_zero", m0))
    tiny = base.clone() * 1e-7                       # amax below 1e-6
    cases.append(("tiny", tiny))
    big = base.clone() * 1e37                        # near the bf16 top
    cases.append(("huge", big))
    sub = base.clone()
    sub[1, 1] = sub[1, 1] * 1e-38                    # bf16 subnormal inputs
    cases.append(("subnormal", sub))
    return [(name, t.to(torch.bfloat16)) for name, t in cases]


@pytest.mark.parametrize("name,x", _special_inputs(), ids=[c[0] for c in _special_inputs()])
@pytest.mark.parametrize("granularity", ["bh", "tensor"])
def test_quantize_special_values(gpu: torch.device, name: str, x: torch.Tensor,
                                 granularity: str) -> None:
    ref_s, ref_c = _oracle(x, granularity)
    dq, codes = ops.scale_quantize(x.to(gpu), granularity, "bhsd")
    _assert_scales_equal(dq.cpu().numpy(), ref_s)
    _assert_codes_equal(codes_np(codes), ref_c)


def test_quantize_c1_matches_torch_restatement(gpu: torch.device) -> None:
    """C1 inputs: GPU codes equal the reference's own torch ops run on the CPU."""
    from oracle import quant

    q, k, v = attn_inputs(C1)
    for x in (q, k, v):
        dq_ref, codes_ref = quant.quantize_codes(x, "bh")
        dq, codes = ops.scale_quantize(x.to(gpu), "bh", "bhsd")
        _assert_scales_equal(dq.cpu().numpy(), dq_ref)
        _assert_codes_equal(codes_np(codes), codes_ref)


def test_quantize_wan_full_size_every_element(gpu: torch.device) -> None:
    """C3 (1, 40, 75600, 128): every code and scale of Q, K and (transposed) V."""
    q, k, v = attn_inputs(C3_SELF, device=gpu)
    for name, x, layout in (("q", q, "bhsd"), ("k", k, "bhsd"), ("v", v, "bhds")):
        dq, codes = ops.scale_quantize(x, "bh", layout)
        ref_s, ref_c = _oracle(x.cpu(), "bh")
        _assert_scales_equal(dq.cpu().numpy(), ref_s)
        got = codes_np(codes)
        if layout == "bhds":
            got = vt_to_bhsd(got, x.shape[2])
        _assert_codes_equal(got, ref_c)
        print(f"{name}: {ref_c.size} codes equal", flush=True)
        del dq, codes, got, ref_c
    del q, k, v
    torch.cuda.empty_cache()


# ------------------------------------------------------------- fp16 input
def _all_nonneg(dtype: torch.dtype) -> torch.Tensor:
    """Every non-negative value of a 16-bit float type from +0 to +inf, then a NaN."""
    top, nan = (0x7C00, 0x7E00) if dtype == torch.float16 else (0x7F80, 0x7FC0)
    bits = np.concatenate([np.arange(0, top + 1), [nan]]).astype(np.uint16)
    return torch.from_numpy(bits.view(np.int16)).view(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_scale_every_amax_matches_torch_on_the_gpu(gpu: torch.device, dtype: torch.dtype) -> None:
    """The kernel's scale function on every amax value against the reference's
    expression (``amax.clamp(min=1e-6) / (0.95 * 448)`` in the input dtype,
    fp8_flash_attn_hopper.py:381-385) evaluated by torch on this GPU, and
    against the CPU oracle."""
    from oracle import quant

    vals = _all_nonneg(dtype)
    dq, qm = ops.selftest_scale(vals.view(torch.int16).to(gpu), dtype)
    ref = (vals.to(gpu).clamp(min=1e-6) / (0.95 * 448.0)).to(torch.float32).cpu().numpy()
    _assert_scales_equal(dq.cpu().numpy(), ref)
    orc = quant.per_group_dequant(vals.reshape(1, -1, 1, 1)).numpy()
    _assert_scales_equal(dq.cpu().numpy(), orc)
    # the multiplier is the correctly rounded fp32 reciprocal, as 1.0 / scale
    qref = (1.0 / torch.from_numpy(ref)).numpy()
    _assert_scales_equal(qm.cpu().numpy(), qref)


def _f16_groups(seed: int, shape: tuple[int, ...]) -> torch.Tensor:
    """fp16 heads spanning the format: subnormal-heavy, unit, and near-max scales."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g)
    mags = torch.tensor([2e-4, 1.0, 30.0, 3e4, 0.05, 600.0])
    x = x * mags[torch.arange(shape[0] * shape[1]) % mags.numel()].reshape(shape[0], shape[1], 1, 1)
    return x.clamp(-65504, 65504).to(torch.float16)


@pytest.mark.parametrize("granularity", ["bh", "tensor"])
@pytest.mark.parametrize("layout", ["bhsd", "bhds"])
def test_fp16_quantize_bit_exact(gpu: torch.device, granularity: str, layout: str) -> None:
    from oracle import quant

    x = _f16_groups(21, (2, 3, 333, 64))
    ref_s, ref_c = quant.quantize_codes(x, granularity)
    dq, codes = ops.scale_quantize(x.to(gpu), granularity, layout)
    _assert_scales_equal(dq.cpu().numpy(), ref_s)
    c = codes_np(codes)
    if layout == "bhds":
        assert not c[..., 333:].any(), "padding columns must be zero"
        c = vt_to_bhsd(c, 333)
    _assert_codes_equal(c, ref_c)


def test_fp16_zero_scale_group_matches_torch_on_the_gpu(gpu: torch.device) -> None:
    """A head whose amax underflows the fp16 scale to zero: 1/0 = inf, so zeros
    become NaN codes and everything else +-448, exactly as the reference's
    own expression does on this GPU."""
    from oracle import quant

    x = torch.zeros(1, 2, 64, 64, dtype=torch.float16)
    x[0, 0, 3, :5] = torch.tensor([3e-6, -5e-6, 1e-7, 0.0, 9e-6]).to(torch.float16)
    x[0, 1] = _f16_groups(3, (1, 1, 64, 64))[0, 0]
    xg = x.to(gpu)
    dq, codes = ops.scale_quantize(xg, "bh", "bhsd")
    assert dq[0].item() == 0.0
    ref_dq = quant.per_group_dequant(xg)          # the reference's ops, on the GPU
    ref_c = quant.quantize(xg, ref_dq).view(torch.uint8).cpu().numpy()
    _assert_scales_equal(dq.cpu().numpy(), ref_dq.cpu().numpy())
    _assert_codes_equal(codes_np(codes), ref_c)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("granularity", ["bh", "tensor"])
@pytest.mark.parametrize("sq,skv", [(300, 700), (40000, 41000)], ids=["small", "large"])
def test_scale_quantize_qkv_equals_three_calls(gpu: torch.device, dtype: torch.dtype,
                                               granularity: str, sq: int, skv: int) -> None:
    """One library call for Q, K and V (rp_fp8_scale_quantize_qkv) gives the
    same scales and codes as three rp_fp8_scale_quantize calls; K/V longer
    than Q, and strided (permuted BSHD) inputs.  The small shapes take the
    two-launch path (each apply block folds its group's few amax partials
    itself), the large ones (per tensor: 2,400+ partials) the four-launch
    path with its own finalize launch."""
    g = torch.Generator(device=gpu).manual_seed(31)
    q = torch.randn(2, sq, 3, 128, generator=g, device=gpu).mul(2).to(dtype).permute(0, 2, 1, 3)
    k = torch.randn(2, 3, skv, 128, generator=g, device=gpu).to(dtype)
    v = torch.randn(2, skv, 3, 128, generator=g, device=gpu).mul(0.5).to(dtype).permute(0, 2, 1, 3)
    qs, q8, ks, k8, vs, vt8 = ops.scale_quantize_qkv(q, k, v, granularity)
    for (s, c), x, lay in (((qs, q8), q, "bhsd"), ((ks, k8), k, "bhsd"), ((vs, vt8), v, "bhds")):
        s2, c2 = ops.scale_quantize(x, granularity, lay)
        _assert_scales_equal(s.cpu().numpy(), s2.cpu().numpy())
        assert c.shape == c2.shape
        assert torch.equal(c.view(torch.uint8), c2.view(torch.uint8))


def test_scale_quantize_qkv_refuses_mismatched_shapes(gpu: torch.device) -> None:
    """One B, H and D go to the library for all three tensors, so any
    disagreement is refused on the host, before a launch could read past K or V."""
    q = torch.zeros(1, 2, 64, 64, dtype=torch.bfloat16, device=gpu)
    kv = torch.zeros(1, 2, 128, 64, dtype=torch.bfloat16, device=gpu)
    for k, v in ((kv[:, :1], kv[:, :1]),                                  # H differs
                 (torch.zeros(1, 2, 128, 32, dtype=torch.bfloat16, device=gpu),) * 2,  # D
                 (kv, kv[:, :, :100]),                                    # Skv differs
                 (torch.zeros(2, 2, 128, 64, dtype=torch.bfloat16, device=gpu),) * 2):  # B
        with pytest.raises(ValueError, match="share one"):
            ops.scale_quantize_qkv(q, k, v)


def test_device_reproduces_golden_vectors(gpu: torch.device) -> None:
    """The device quantizer on the committed vectors of the reference
    quantizer's torch ops: every scale and code bit for bit, both layouts."""
    from tests._helpers import golden_quant_cases, vt_to_bhsd

    for name, bits, dq_ref, codes_ref in golden_quant_cases():
        x = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).to(gpu)
        dq, codes = ops.scale_quantize(x, "bh", "bhsd")
        assert np.array_equal(dq.cpu().numpy().view(np.uint32), dq_ref.view(np.uint32)), name
        assert np.array_equal(codes_np(codes), codes_ref), name
        _, vt = ops.scale_quantize(x, "bh", "bhds")
        assert np.array_equal(vt_to_bhsd(codes_np(vt), x.shape[2]), codes_ref), name
