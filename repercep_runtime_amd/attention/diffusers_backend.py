"""The diffusers-layout entry point of the FP8 path.

Mirrors src/repercep/attention/diffusers_backend.py:52-399 of the reference:
``_repercep_fp8_attention`` has the signature diffusers' dispatcher
introspects, takes and returns (B, S, H, D) tensors, routes qualifying calls
to the FP8 kernels and everything else to a native-SDPA fallback, and guards
against non-finite output by recomputing that call with SDPA.

The FP8 branch differs from the reference in how it moves data: the
reference makes three ``permute(0, 2, 1, 3).contiguous()`` copies on the way
in and a permute on the way out (diffusers_backend.py:264-286); here the
quantizer reads the permuted (B, H, S, D) *views* directly (strided rows)
and the attention kernel writes into a (B, S, H, D) output through its
strides, so no layout copy is made.

Registration with diffusers happens on import when diffusers is installed;
without it the module still provides the backend function and the routing
logic (diffusers is not a dependency of this package).
"""

from __future__ import annotations

import logging
import os
from typing import TYPE_CHECKING, Any

if TYPE_CHECKING:
    import torch

logger = logging.getLogger(__name__)

REPERCEP_FP8_BACKEND_NAME = "repercep_fp8"

#: Sequence-length crossover below which the FP8 path is not taken
#: (the reference's measured gfx942 crossover, diffusers_backend.py:44).
_FP8_MIN_SEQ_LEN = int(os.environ.get("REPERCEP_FP8_MIN_SEQ_LEN", "4096"))
_FP8_SUPPORTED_HEAD_DIMS = frozenset({32, 64, 128, 256})   # diffusers_backend.py:49
#: Shortest key sequence the cross-attention branch takes (text encoders
#: give 512 tokens in Wan/Cosmos).
_FP8_MIN_KV_LEN = 128


def _route_should_use_fp8(query: Any, key: Any, value: Any) -> bool:
    """Whether one (B, S, H, D) call goes to the FP8 kernels.

    Same rules as the reference (diffusers_backend.py:52-79) -- BF16 or
    FP16, head dim in the compiled set, query length past the crossover --
    except that
    cross-attention (K/V sequence length != Q's) qualifies too, since the
    gfx950 kernel supports it.
    """
    import torch

    if query.dtype not in (torch.bfloat16, torch.float16):   # diffusers_backend.py:69
        return False
    if key.dtype != query.dtype or value.dtype != query.dtype:
        return False
    if query.dim() != 4 or key.shape != value.shape:
        return False
    if (key.shape[0], key.shape[2], key.shape[3]) != (query.shape[0], query.shape[2],
                                                      query.shape[3]):
        return False
    if query.shape[-1] not in _FP8_SUPPORTED_HEAD_DIMS:
        return False
    if key.shape[1] < _FP8_MIN_KV_LEN:
        return False
    return bool(query.shape[1] >= _FP8_MIN_SEQ_LEN)


def _native_fallback(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, *,
                     attn_mask: torch.Tensor | None, dropout_p: float, is_causal: bool,
                     scale: float | None, enable_gqa: bool) -> torch.Tensor:
    """diffusers' native attention: permute to (B, H, S, D), SDPA, permute back."""
    import torch

    if (attn_mask is not None and attn_mask.ndim == 2 and attn_mask.shape[0] == query.shape[0]
            and attn_mask.shape[1] == key.shape[1]):
        attn_mask = attn_mask.unsqueeze(1).unsqueeze(1)
    out = torch.nn.functional.scaled_dot_product_attention(
        query=query.permute(0, 2, 1, 3), key=key.permute(0, 2, 1, 3),
        value=value.permute(0, 2, 1, 3), attn_mask=attn_mask, dropout_p=dropout_p,
        is_causal=is_causal, scale=scale, enable_gqa=enable_gqa)
    return out.permute(0, 2, 1, 3)


def _repercep_fp8_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                            attn_mask: torch.Tensor | None = None, dropout_p: float = 0.0,
                            is_causal: bool = False, scale: float | None = None,
                            enable_gqa: bool = False, return_lse: bool = False,
                            _parallel_config: Any = None) -> torch.Tensor:
    """The ``"repercep_fp8"`` backend function: (B, S, H, D) in and out."""
    import torch

    if return_lse:
        raise ValueError("repercep_fp8 backend does not support return_lse=True.")
    fallback = dict(attn_mask=attn_mask, dropout_p=dropout_p, is_causal=is_causal, scale=scale,
                    enable_gqa=enable_gqa)
    if os.environ.get("REPERCEP_FP8_ATTENTION", "").lower() in ("fa", "flash"):
        return _native_fallback(query, key, value, **fallback)
    if _parallel_config is not None:
        return _native_fallback(query, key, value, **fallback)
    if (attn_mask is not None or dropout_p != 0.0 or enable_gqa
            or not _route_should_use_fp8(query, key, value)):
        return _native_fallback(query, key, value, **fallback)

    op = getattr(_repercep_fp8_attention, "_op", None)
    if op is None:
        from repercep_runtime_amd.attention.fp8_hip import FP8HipAttention

        op = FP8HipAttention()
        _repercep_fp8_attention._op = op  # type: ignore[attr-defined]
    if not op.available or query.device.type != "cuda":
        return _native_fallback(query, key, value, **fallback)

    from repercep_runtime_amd.ops import fp8_flash_attention

    out = torch.empty_like(query, memory_format=torch.contiguous_format)
    fp8_flash_attention(query.permute(0, 2, 1, 3), key.permute(0, 2, 1, 3),
                        value.permute(0, 2, 1, 3), causal=is_causal, scale=scale,
                        out=out.permute(0, 2, 1, 3))
    if not torch.isfinite(out).all():
        logger.warning("repercep_fp8: non-finite output at shape %s; falling back to native SDPA",
                       tuple(query.shape))
        return _native_fallback(query, key, value, **fallback)
    return out


def _ensure_backend_name_registered() -> Any:
    """Make ``AttentionBackendName("repercep_fp8")`` resolve (diffusers' sealed enum)."""
    from diffusers.models.attention_dispatch import AttentionBackendName

    if REPERCEP_FP8_BACKEND_NAME in AttentionBackendName._value2member_map_:
        return AttentionBackendName._value2member_map_[REPERCEP_FP8_BACKEND_NAME]
    member = str.__new__(AttentionBackendName, REPERCEP_FP8_BACKEND_NAME)
    member._name_ = "REPERCEP_FP8"
    member._value_ = REPERCEP_FP8_BACKEND_NAME
    AttentionBackendName._member_map_["REPERCEP_FP8"] = member
    AttentionBackendName._value2member_map_[REPERCEP_FP8_BACKEND_NAME] = member
    if "REPERCEP_FP8" not in AttentionBackendName._member_names_:
        AttentionBackendName._member_names_.append("REPERCEP_FP8")
    return member


def register_repercep_fp8_backend() -> Any:
    """Register the backend with diffusers' dispatcher (idempotent)."""
    import inspect

    from diffusers.models.attention_dispatch import _AttentionBackendRegistry

    member = _ensure_backend_name_registered()
    if member not in _AttentionBackendRegistry._backends:
        _AttentionBackendRegistry._backends[member] = _repercep_fp8_attention
        _AttentionBackendRegistry._constraints[member] = []
        _AttentionBackendRegistry._supported_arg_names[member] = set(
            inspect.signature(_repercep_fp8_attention).parameters.keys())
    return member


def activate_repercep_fp8_backend() -> bool:
    from diffusers.models.attention_dispatch import _AttentionBackendRegistry

    member = register_repercep_fp8_backend()
    if _AttentionBackendRegistry._active_backend == member:
        return False
    _AttentionBackendRegistry.set_active_backend(member)
    return True


def maybe_activate_from_env() -> bool:
    """Activate the backend iff ``REPERCEP_FP8_ATTENTION`` is set (reference :364-388)."""
    fp8_env = os.environ.get("REPERCEP_FP8_ATTENTION", "").lower()
    if fp8_env not in ("1", "true", "on", "triton", "scaled_mm", "fa", "flash"):
        return False
    return activate_repercep_fp8_backend()


try:
    register_repercep_fp8_backend()
except Exception as exc:  # diffusers absent or its internals changed
    logger.debug("repercep_fp8: registration deferred (%s: %s)", type(exc).__name__, exc)


__all__ = [
    "REPERCEP_FP8_BACKEND_NAME",
    "activate_repercep_fp8_backend",
    "maybe_activate_from_env",
    "register_repercep_fp8_backend",
]
