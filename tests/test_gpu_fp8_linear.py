"""GPU parity of the FP8 linear module: weight and activation codes bit-exact
against the quantizer oracle, the product within one bf16 rounding of the
exact sum (the GEMM's bound), and a module swap on a small DiT-like block."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import native, quant
from repercep_runtime_amd import ops
from repercep_runtime_amd.fp8_linear import FP8Linear, replace_linears_with_fp8
from tests._helpers import bf16_bits, bf16_to_f32, codes_np
from tests.test_gpu_gemm import _assert_one_rounding_apart

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape,bias", [((3, 77, 256), True), ((1000, 512), False),
                                        ((2, 1, 128), True),
                                        # row tiles wholly inside the output: the
                                        # bias epilogue's unchecked store path
                                        ((2, 300, 256), True)])
def test_fp8_linear_matches_oracle(gpu: torch.device, shape: tuple[int, ...], bias: bool) -> None:
    K, N = shape[-1], 384
    g = torch.Generator().manual_seed(sum(shape))
    lin = torch.nn.Linear(K, N, bias=bias)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(N, K, generator=g) * 0.05)
        if bias:
            lin.bias.copy_(torch.randn(N, generator=g))
    lin = lin.to(gpu).to(torch.bfloat16)
    m = FP8Linear.from_linear(lin)
    x = torch.randn(*shape, generator=g).to(torch.bfloat16)
    y = m(x.to(gpu))
    assert y.shape == (*shape[:-1], N) and y.dtype == torch.bfloat16

    w_cpu = lin.weight.detach().cpu()
    sw, w8 = quant.quantize_codes(w_cpu.reshape(1, 1, N, K), "tensor")
    assert np.array_equal(codes_np(m.qweight), w8.reshape(N, K))
    assert m.scale.item() == sw[0]
    x2 = x.reshape(-1, K)
    sa, a8 = quant.quantize_codes(x2.reshape(1, 1, -1, K), "tensor")
    a8 = a8.reshape(-1, K)
    y2 = y.reshape(-1, N)
    got = bf16_to_f32(bf16_bits(y2))
    bt8 = np.ascontiguousarray(w8.reshape(N, K))
    scale = float(np.float32(sa[0]) * np.float32(sw[0]))
    if not bias:
        ref = native.gemm_rows(a8, bt8, float(sa[0]), float(sw[0]), np.arange(a8.shape[0]))
        _assert_one_rounding_apart(got, bf16_to_f32(ref), a8, bt8, scale)
    else:
        # rp_fp8_linear: bf16(fp32(fp32(acc * s) + bias)), one bf16 rounding
        bvec = m.bias.float().cpu().numpy().astype(np.float64)
        _assert_one_rounding_apart(got, None, a8, bt8, scale, bvec)
    # against the bf16 layer: FP8 noise only
    ref = lin(x.to(gpu)).float()
    rel = (y.float() - ref).abs().mean() / ref.abs().mean()
    assert rel.item() < 0.05, rel.item()


def test_swap_on_a_dit_block(gpu: torch.device) -> None:
    g = torch.Generator().manual_seed(4)
    block = torch.nn.Sequential(torch.nn.Linear(256, 1024), torch.nn.GELU(approximate="tanh"),
                                torch.nn.Linear(1024, 256))
    with torch.no_grad():
        for p in block.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * 0.03)
    block = block.to(gpu).to(torch.bfloat16)
    x = torch.randn(2, 300, 256, generator=g).to(torch.bfloat16).to(gpu)
    ref = block(x).float()
    assert replace_linears_with_fp8(block) == 2
    out = block(x).float()
    rel = (out - ref).abs().mean() / ref.abs().mean()
    assert rel.item() < 0.06, rel.item()
    assert all(isinstance(block[i], FP8Linear) for i in (0, 2))
