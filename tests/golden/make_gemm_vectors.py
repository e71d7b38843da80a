"""Writes tests/golden/gemm_small_int.npz: FP8 GEMM operands and outputs in
the exact regime of the reference's own known-answer test
(tests/test_mfma_fragment_layout.py:262-315 of the reference: all-ones gives
K, small integers are exact).

Expected outputs follow the reference test's emulation,
C = bf16((A8.float() @ B8.float()) * (a_scale * b_scale)), restated with CPU
torch.  Integer operands with power-of-two scales make every sum exact in
fp32, so the vectors hold for any summation order.  A is (M, K) and B is
(K, N), both row-major e4m3fn codes, as the reference's fp8_gemm takes them.
Run from the repository root: python tests/golden/make_gemm_vectors.py
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch


def cases() -> dict[str, tuple[torch.Tensor, torch.Tensor, float, float]]:
    g = torch.Generator().manual_seed(7)
    return {
        "ones": (torch.ones(16, 32), torch.ones(32, 16), 1.0, 1.0),
        "int2": (torch.randint(-2, 3, (40, 64), generator=g).float(),
                 torch.randint(-2, 3, (64, 24), generator=g).float(), 0.5, 0.25),
        "int4_ragged": (torch.randint(-4, 5, (5, 48), generator=g).float(),
                        torch.randint(-4, 5, (48, 12), generator=g).float(), 1.0, 2.0),
        "int8_deep": (torch.randint(-8, 9, (33, 256), generator=g).float(),
                      torch.randint(-1, 2, (256, 20), generator=g).float(), 0.125, 1.0),
    }


def main() -> None:
    out = {}
    for name, (a, b, sa, sb) in cases().items():
        a8, b8 = a.to(torch.float8_e4m3fn), b.to(torch.float8_e4m3fn)
        c = ((a8.float() @ b8.float()) * (sa * sb)).to(torch.bfloat16)
        out[f"{name}_a8"] = a8.view(torch.uint8).numpy()
        out[f"{name}_b8"] = b8.view(torch.uint8).numpy()
        out[f"{name}_scales"] = np.array([sa, sb], dtype=np.float32)
        out[f"{name}_c_bits"] = c.view(torch.int16).numpy().view(np.uint16)
    path = Path(__file__).with_name("gemm_small_int.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({path.stat().st_size} bytes, {len(out) // 4} cases)")


if __name__ == "__main__":
    main()
