"""Shared helpers for the tests: error metrics and oracle adapters."""

from __future__ import annotations

import numpy as np
import torch

# BASELINE.json tolerance for attention/GEMM outputs vs the torch-emulated FP8 result.
MAX_ABS_TOL = 2e-2
MEAN_ABS_TOL = 2e-3


def err_stats(got: np.ndarray, ref: np.ndarray) -> dict[str, float]:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    d = np.abs(got - ref)
    return {
        "max_abs": float(d.max()),
        "mean_abs": float(d.mean()),
        "rel_mean": float(d.mean() / (np.abs(ref).mean() + 1e-30)),
    }


def baseline_tolerance(ref: np.ndarray) -> tuple[float, float]:
    """(max_abs, mean_abs) bounds: BASELINE.json's 2e-2 / 2e-3 for outputs whose peak
    magnitude is at most 1 (every BASELINE attention config), scaled by the peak
    above that -- an e4m3 step of P is ~6% of a dominant key's weight, so an
    order-of-rounding flip moves larger outputs proportionally more."""
    scale = max(1.0, float(np.abs(ref).max()))
    return MAX_ABS_TOL * scale, MEAN_ABS_TOL * scale


def bf16_ulp(x: np.ndarray) -> np.ndarray:
    """Spacing of bf16 numbers at |x| (normal range)."""
    ax = np.maximum(np.abs(np.asarray(x, dtype=np.float64)), 2.0 ** -126)
    return 2.0 ** (np.floor(np.log2(ax)) - 7)


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def codes_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def vt_to_bhsd(vt: np.ndarray, S: int) -> np.ndarray:
    """(B, H, D, ldv) transposed V codes -> (B, H, S, D)."""
    return np.ascontiguousarray(np.swapaxes(vt[..., :S], -1, -2))


def golden_quant_cases() -> list[tuple[str, np.ndarray, np.ndarray, np.ndarray]]:
    """(name, bf16 input bits (B, H, S, D), dequant scales, codes) from
    tests/golden/quant_bf16.npz (written by tests/golden/make_quant_vectors.py:
    torch's CPU ops in the reference quantizer's order)."""
    from pathlib import Path

    data = np.load(Path(__file__).with_name("golden") / "quant_bf16.npz")
    names = sorted({k.rsplit("_x_bits", 1)[0] for k in data.files if k.endswith("_x_bits")})
    return [(n, data[f"{n}_x_bits"], data[f"{n}_dequant"], data[f"{n}_codes"]) for n in names]


def golden_gemm_cases() -> list[tuple[str, np.ndarray, np.ndarray, float, float, np.ndarray]]:
    """(name, A8 (M, K), B8 (K, N) codes, a_scale, b_scale, C bf16 bits) from
    tests/golden/gemm_small_int.npz (tests/golden/make_gemm_vectors.py)."""
    from pathlib import Path

    data = np.load(Path(__file__).with_name("golden") / "gemm_small_int.npz")
    names = sorted({k.rsplit("_a8", 1)[0] for k in data.files if k.endswith("_a8")})
    return [(n, data[f"{n}_a8"], data[f"{n}_b8"], float(data[f"{n}_scales"][0]),
             float(data[f"{n}_scales"][1]), data[f"{n}_c_bits"]) for n in names]
