"""FP8 linear layers for the DiT blocks, on the gfx950 FP8 GEMM.

The module-swap pattern is the reference's (src/repercep/runtime/quantize.py:
135-179, ``replace_linears_with_quantized`` / ``QuantizedLinearModule``): walk
a module parent-first and replace each matching ``nn.Linear`` in place, so the
swap is invisible to code that holds the parent.  The reference's swap
quantizes to INT8 and dequantizes before a bf16 matmul; this one keeps the
weight as OCP e4m3fn codes with one per-tensor scale and runs the FP8 GEMM:

    weight   W (N, K) = nn.Linear's layout, quantized once:
             dequant scale sw = bf16(max|W| clamped at 1e-6) / 425.6, codes
             e4m3fn(W / sw) -- K-contiguous rows, the GEMM's B^T operand as is
    forward  x (..., K) bf16 -> per-call per-tensor scale sa and codes (the
             attention quantizer's arithmetic), then
             y = bf16(fp32(x8 . W8^T) * sa * sw + bias)   [rp_fp8_linear: the
             product and the bias sum each rounded to fp32, as a bf16
             nn.Linear's fp32 epilogue; rp_fp8_gemm without a bias]

Same members as the reference's module: ``qweight``, ``scale`` (buffers, so
``.to()`` and state dicts work), ``bias`` (a Parameter or None),
``in_features``, ``out_features``, ``from_linear``.  Inputs must be bfloat16
on the GPU; there is no CPU path (the library raises when it cannot load).
"""

from __future__ import annotations

from typing import Any

import torch

from repercep_runtime_amd import ops


def _check_shape(in_features: int, out_features: int) -> None:
    # rp_fp8_gemm: K % 16 == 0 (16-byte rows), N % 4 == 0 (8-byte output stores)
    if in_features % 16 != 0 or out_features % 4 != 0:
        raise ValueError(f"FP8 linear needs in_features % 16 == 0 and out_features % 4 == 0 "
                         f"(got {in_features} -> {out_features})")


def quantize_weight(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(codes (N, K) uint8, dequant scale (1,) fp32) of an nn.Linear weight (N, K)."""
    if weight.dim() != 2:
        raise ValueError(f"weight must be 2-D (out_features, in_features), got {tuple(weight.shape)}")
    N, K = weight.shape
    _check_shape(K, N)
    w = weight.detach().to(torch.bfloat16).contiguous()
    scale, codes = ops.scale_quantize(w, "tensor", "bhsd")
    return codes.view(torch.uint8).reshape(N, K).contiguous(), scale


class FP8Linear(torch.nn.Module):
    """``nn.Linear`` on e4m3fn weights and activations (see the module doc)."""

    qweight: torch.Tensor
    scale: torch.Tensor
    bias: torch.nn.Parameter | None

    def __init__(self, qweight: torch.Tensor, scale: torch.Tensor,
                 bias: torch.Tensor | None = None) -> None:
        super().__init__()
        if qweight.dim() != 2 or qweight.dtype != torch.uint8:
            raise TypeError("qweight must be 2-D uint8 e4m3fn codes (out_features, in_features)")
        self.out_features, self.in_features = qweight.shape
        _check_shape(self.in_features, self.out_features)
        self.register_buffer("qweight", qweight)
        self.register_buffer("scale", scale.reshape(1).to(torch.float32))
        if bias is not None:
            self.bias = torch.nn.Parameter(bias.detach().to(torch.bfloat16).clone(),
                                           requires_grad=False)
        else:
            self.register_parameter("bias", None)

    @classmethod
    def from_linear(cls, linear: torch.nn.Linear) -> FP8Linear:
        """Quantize an existing (GPU) ``nn.Linear`` and wrap the result."""
        qweight, scale = quantize_weight(linear.weight)
        return cls(qweight, scale, linear.bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.dtype != torch.bfloat16:
            raise TypeError(f"FP8Linear takes bfloat16 input (got {x.dtype})")
        if x.shape[-1] != self.in_features:
            raise ValueError(f"last dim {x.shape[-1]} != in_features {self.in_features}")
        lead = x.shape[:-1]
        x2 = x.reshape(-1, self.in_features)
        if x2.shape[0] == 0:
            return x.new_empty(*lead, self.out_features)
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        sa, a8 = ops.scale_quantize(x2, "tensor", "bhsd")
        y = ops.fp8_gemm(a8.view(torch.uint8), self.qweight, sa, self.scale, b_transposed=True,
                         bias=self.bias)
        return y.reshape(*lead, self.out_features)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, e4m3fn per-tensor")


def replace_linears_with_fp8(module: torch.nn.Module, *, name_filter: str | None = None) -> int:
    """In-place swap every matching ``nn.Linear`` for an :class:`FP8Linear`;
    returns the number swapped.  ``name_filter`` is a substring of the dotted
    name, as in the reference (runtime/quantize.py:135-179).  Layers whose
    shape the GEMM cannot take (in_features % 16, out_features % 4) are left
    as they are."""
    count = 0

    def _recurse(parent: Any, prefix: str) -> None:
        nonlocal count
        for child_name, child in list(parent.named_children()):
            dotted = f"{prefix}.{child_name}" if prefix else child_name
            if isinstance(child, torch.nn.Linear) and (name_filter is None or name_filter in dotted):
                if child.in_features % 16 == 0 and child.out_features % 4 == 0:
                    setattr(parent, child_name, FP8Linear.from_linear(child))
                    count += 1
                continue
            _recurse(child, dotted)

    _recurse(module, "")
    return count


__all__ = ["FP8Linear", "quantize_weight", "replace_linears_with_fp8"]
