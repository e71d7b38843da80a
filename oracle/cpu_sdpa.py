"""The reference's CPU attention path, restated for the CPU baseline -- TEST/BENCH ONLY.

The reference's registry ends its CPU candidate list with ``AMXSDPAAttention``
(src/repercep/attention/registry.py:126), whose ``__call__`` is one
``torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=causal,
scale=scale)`` on CPU tensors in (B, H, S, D) layout
(src/repercep/attention/amx_sdpa.py:76-94).  This module makes that one call
so bench.py can time it on the GPU box's host cores; it is a reported
baseline, not an optimisation target and not part of the product.
"""

from __future__ import annotations

import os

import torch


def cpu_threads() -> int:
    """Threads the baseline uses: every core this process may run on."""
    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    return torch.get_num_threads()


def sdpa_cpu(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, causal: bool = False,
             scale: float | None = None) -> torch.Tensor:
    """AMXSDPAAttention.__call__ (amx_sdpa.py:92-94)."""
    return torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=causal, scale=scale)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"
