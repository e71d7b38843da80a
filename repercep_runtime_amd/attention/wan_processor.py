"""Install the FP8 backend on a Wan pipeline's attention processors.

Mirrors the reference's Wan bridge (src/repercep/attention/wan_processor.py:
26-116).  Wan's diffusers transformer owns its attention processors, so
selecting an ``AttentionOp`` does not reach it.  Recent diffusers releases
route ``WanAttnProcessor`` through ``dispatch_attention_fn(...,
backend=processor._attention_backend)``; setting that attribute to the
registered ``"repercep_fp8"`` backend sends Wan's attention calls to
``diffusers_backend._repercep_fp8_attention`` and from there to the gfx950
kernel, while the processor itself (projections, QK-norm, rotary embedding)
stays diffusers' own.

The same opt-in as the reference: ``REPERCEP_FP8_ATTENTION`` set to one of
its accepted values.  Without diffusers, or with a release that lacks the
processor class, nothing is installed and the pipeline keeps its path.
"""

from __future__ import annotations

import logging
import os
from typing import Any

logger = logging.getLogger(__name__)

#: Values of REPERCEP_FP8_ATTENTION that opt in (the reference's set).
FP8_ENV_VALUES = frozenset({"1", "true", "on", "triton", "scaled_mm", "fa", "flash"})

#: Pipeline attributes that hold Wan transformers (A14B has two experts).
TRANSFORMER_ATTRS = ("transformer", "transformer_2")


def maybe_install_repercep_wan_attention(pipe: Any) -> bool:
    """Install when ``REPERCEP_FP8_ATTENTION`` opts in; True if at least one
    transformer took the processor."""
    if os.environ.get("REPERCEP_FP8_ATTENTION", "").lower() not in FP8_ENV_VALUES:
        return False
    return install_repercep_wan_attention(pipe) > 0


def install_repercep_wan_attention(pipe: Any) -> int:
    """Give every Wan transformer of ``pipe`` a ``WanAttnProcessor`` bound to
    the FP8 backend; returns how many accepted it."""
    processor_cls = _wan_attn_processor_class()
    if processor_cls is None:
        return 0
    from repercep_runtime_amd.attention import diffusers_backend

    try:
        backend = diffusers_backend.register_repercep_fp8_backend()
        processor = processor_cls()
    except Exception as exc:  # diffusers-version dependent
        logger.debug("wan attention: backend or processor unavailable (%s: %s)",
                     type(exc).__name__, exc)
        return 0
    processor._attention_backend = backend
    processor._repercep_attention_backend = diffusers_backend.REPERCEP_FP8_BACKEND_NAME

    installed = 0
    for transformer in wan_transformers(pipe):
        setter = getattr(transformer, "set_attn_processor", None)
        if not callable(setter):
            logger.debug("wan attention: %s has no set_attn_processor",
                         type(transformer).__name__)
            continue
        try:
            setter(processor)
        except Exception as exc:  # model-version dependent
            logger.warning("wan attention: %s refused the processor (%s: %s)",
                           type(transformer).__name__, type(exc).__name__, exc)
            continue
        installed += 1
    return installed


def wan_transformers(pipe: Any) -> tuple[Any, ...]:
    return tuple(t for t in (getattr(pipe, a, None) for a in TRANSFORMER_ATTRS) if t is not None)


def _wan_attn_processor_class() -> type | None:
    try:
        from diffusers.models.transformers.transformer_wan import WanAttnProcessor
    except Exception as exc:  # diffusers absent or too old
        logger.debug("wan attention: WanAttnProcessor unavailable (%s: %s)",
                     type(exc).__name__, exc)
        return None
    return WanAttnProcessor


__all__ = ["install_repercep_wan_attention", "maybe_install_repercep_wan_attention"]
