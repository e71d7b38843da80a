"""Writes tests/golden/quant_bf16.npz: small bf16 inputs with the per-(b, h)
dequant scales and e4m3fn codes of the reference's OCP quantizer.

The expected values come from torch's CPU ops in the order the reference
applies them (kernels/triton_kernels/fp8_flash_attn_hopper.py:374-398),
restated here -- the reference itself is not imported:

    amax    = |x|.reshape(B*H, -1).amax(1).clamp(min=1e-6)      (bf16)
    dequant = (amax / (0.95 * 448)).to(float32)                  (bf16 divide)
    codes   = (x.float() * (1.0 / dequant)).clamp(+-448).to(float8_e4m3fn)

For bf16 inputs CPU torch computes exactly what the reference's GPU torch
does (the device parity test of every bf16 amax shows the divide agrees), so
the vectors stand for the reference's outputs.  Run from the repository root:
python tests/golden/make_quant_vectors.py
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

FP8_MAX = 448.0


def reference_quantizer(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    B, H, S, D = x.shape
    amax = x.abs().reshape(B * H, -1).amax(dim=1).clamp(min=1e-6)
    dequant = (amax / (0.95 * FP8_MAX)).to(torch.float32)
    q_mul = (1.0 / dequant).reshape(B, H, 1, 1)
    codes = (x.to(torch.float32) * q_mul).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return dequant, codes


def inputs() -> dict[str, torch.Tensor]:
    g = torch.Generator().manual_seed(2024)
    cases = {"randn": torch.randn(1, 2, 64, 64, generator=g) * 3.0}
    mixed = torch.randn(2, 2, 37, 128, generator=g)
    mixed[0, 0] = 0.0                                  # zero head: amax clamps to 1e-6
    mixed[0, 1] *= 1e-8                                # subnormal-scale head
    mixed[1, 0, 5, 7] = 3.0e4                          # one outlier dominates its head
    mixed[1, 1] = -mixed[1, 1].abs()                   # all-negative head
    cases["mixed"] = mixed
    cases["ties"] = (torch.arange(1 * 1 * 16 * 32, dtype=torch.float32) / 7.0 - 30.0
                     ).reshape(1, 1, 16, 32)
    return {k: v.to(torch.bfloat16) for k, v in cases.items()}


def main() -> None:
    out = {}
    for name, x in inputs().items():
        dq, codes = reference_quantizer(x)
        out[f"{name}_x_bits"] = x.view(torch.int16).numpy().view(np.uint16)
        out[f"{name}_dequant"] = dq.numpy()
        out[f"{name}_codes"] = codes.view(torch.uint8).numpy()
    path = Path(__file__).with_name("quant_bf16.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({path.stat().st_size} bytes, {len(out) // 3} cases)")


if __name__ == "__main__":
    main()
