"""Install the FP8 backend on a Wan pipeline's attention processors.

Reference counterpart: src/repercep/attention/wan_processor.py:26-116.
Wan's diffusers transformer owns its attention processors, so selecting an
``AttentionOp`` does not reach it.  Recent diffusers releases route
``WanAttnProcessor`` through ``dispatch_attention_fn(...,
backend=processor._attention_backend)``; a processor whose attribute names
the registered ``"repercep_fp8"`` backend sends Wan's attention calls to
``diffusers_backend._repercep_fp8_attention`` and from there to the gfx950
kernel, while the processor itself (projections, QK-norm, rotary embedding)
stays diffusers' own.

The opt-in is the reference's: ``REPERCEP_FP8_ATTENTION`` set to one of its
accepted values.  Without diffusers, or with a release that lacks the
processor class, nothing is installed and the pipeline keeps its path.
"""

from __future__ import annotations

import logging
import os
from typing import Any, Iterator

logger = logging.getLogger(__name__)

#: Values of REPERCEP_FP8_ATTENTION that opt in (the reference's set).
FP8_ENV_VALUES = frozenset({"1", "true", "on", "triton", "scaled_mm", "fa", "flash"})

#: Pipeline attributes that may hold a Wan transformer: Wan-2.2 A14B runs a
#: high-noise and a low-noise expert.
EXPERT_ATTRS = ("transformer", "transformer_2")


def maybe_install_repercep_wan_attention(pipe: Any) -> bool:
    """Install when ``REPERCEP_FP8_ATTENTION`` opts in; True if at least one
    transformer took the processor."""
    if os.environ.get("REPERCEP_FP8_ATTENTION", "").lower() not in FP8_ENV_VALUES:
        return False
    return install_repercep_wan_attention(pipe) > 0


def install_repercep_wan_attention(pipe: Any) -> int:
    """Give every Wan transformer of ``pipe`` one shared ``WanAttnProcessor``
    bound to the FP8 backend; returns how many transformers accepted it."""
    processor = _fp8_bound_processor()
    if processor is None:
        return 0
    return sum(_hand_over(expert, processor) for expert in _experts(pipe))


def _fp8_bound_processor() -> Any | None:
    """A fresh diffusers ``WanAttnProcessor`` whose dispatch backend is the
    registered FP8 backend, or None when diffusers cannot provide one."""
    try:
        from diffusers.models.transformers.transformer_wan import WanAttnProcessor
    except Exception as exc:  # diffusers absent, or a release without the class
        logger.debug("wan attention: no WanAttnProcessor (%s: %s)", type(exc).__name__, exc)
        return None
    from repercep_runtime_amd.attention import diffusers_backend

    try:
        backend = diffusers_backend.register_repercep_fp8_backend()
        processor = WanAttnProcessor()
    except Exception as exc:  # the dispatcher's internals differ in this release
        logger.debug("wan attention: cannot bind the FP8 backend (%s: %s)",
                     type(exc).__name__, exc)
        return None
    processor._attention_backend = backend
    # the backend's registered name, read by callers that check which
    # backend a processor is bound to (reference wan_processor.py:73)
    processor._repercep_attention_backend = diffusers_backend.REPERCEP_FP8_BACKEND_NAME
    return processor


def _experts(pipe: Any) -> Iterator[Any]:
    for attr in EXPERT_ATTRS:
        expert = getattr(pipe, attr, None)
        if expert is not None:
            yield expert


def _hand_over(expert: Any, processor: Any) -> bool:
    """``expert.set_attn_processor(processor)``; False when the transformer
    has no such method or refuses."""
    set_processor = getattr(expert, "set_attn_processor", None)
    if not callable(set_processor):
        logger.debug("wan attention: %s takes no attention processor", type(expert).__name__)
        return False
    try:
        set_processor(processor)
    except Exception as exc:  # model-version dependent
        logger.warning("wan attention: %s refused the FP8 processor (%s: %s)",
                       type(expert).__name__, type(exc).__name__, exc)
        return False
    return True


__all__ = ["install_repercep_wan_attention", "maybe_install_repercep_wan_attention"]
