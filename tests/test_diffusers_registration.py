"""Registration of the ``"repercep_fp8"`` backend with diffusers' dispatcher (CPU).

diffusers is not installed here, so a stand-in
``diffusers.models.attention_dispatch`` module provides the two objects the
registration touches, shaped as diffusers defines them: ``AttentionBackendName``,
a sealed ``str`` Enum, and ``_AttentionBackendRegistry`` with its class-level
``_backends`` / ``_constraints`` / ``_supported_arg_names`` maps,
``_active_backend`` and ``set_active_backend``.  A minimal
``dispatch_attention_fn`` looks the backend up and calls it with the
arguments its ``_supported_arg_names`` allow, as diffusers' does.

Reference behaviour: src/repercep/attention/diffusers_backend.py:289-388
(enum injection, idempotent registration, activation, the env opt-in).
"""

from __future__ import annotations

import contextlib
import enum
import inspect
import sys
import types
from typing import Any, Iterator

import pytest
import torch

from repercep_runtime_amd.attention import diffusers_backend as db
from repercep_runtime_amd.attention import wan_processor


def _make_dispatch_module() -> types.ModuleType:
    class AttentionBackendName(str, enum.Enum):
        FLASH = "flash"
        NATIVE = "native"
        _NATIVE_MATH = "_native_math"

    class _AttentionBackendRegistry:
        _backends: dict = {}
        _constraints: dict = {}
        _supported_arg_names: dict = {}
        _active_backend = AttentionBackendName.NATIVE

        @classmethod
        def set_active_backend(cls, backend: Any) -> None:
            cls._active_backend = backend

        @classmethod
        def get_active_backend(cls) -> tuple[Any, Any]:
            return cls._active_backend, cls._backends[cls._active_backend]

    def _native(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False,
                scale=None, enable_gqa=False):
        o = torch.nn.functional.scaled_dot_product_attention(
            query.permute(0, 2, 1, 3), key.permute(0, 2, 1, 3), value.permute(0, 2, 1, 3),
            attn_mask=attn_mask, dropout_p=dropout_p, is_causal=is_causal, scale=scale)
        return o.permute(0, 2, 1, 3)

    R = _AttentionBackendRegistry
    R._backends[AttentionBackendName.NATIVE] = _native
    R._constraints[AttentionBackendName.NATIVE] = []
    R._supported_arg_names[AttentionBackendName.NATIVE] = set(
        inspect.signature(_native).parameters)

    def dispatch_attention_fn(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False,
                              scale=None, enable_gqa=False, *, backend=None):
        name = AttentionBackendName(backend) if backend is not None else R._active_backend
        fn = R._backends[name]
        kwargs = dict(query=query, key=key, value=value, attn_mask=attn_mask,
                      dropout_p=dropout_p, is_causal=is_causal, scale=scale,
                      enable_gqa=enable_gqa)
        kwargs = {k: v for k, v in kwargs.items() if k in R._supported_arg_names[name]}
        return fn(**kwargs)

    mod = types.ModuleType("diffusers.models.attention_dispatch")
    mod.AttentionBackendName = AttentionBackendName
    mod._AttentionBackendRegistry = _AttentionBackendRegistry
    mod.dispatch_attention_fn = dispatch_attention_fn
    return mod


@contextlib.contextmanager
def fake_diffusers(wan_processor_cls: type | None = None) -> Iterator[types.ModuleType]:
    names = ["diffusers", "diffusers.models", "diffusers.models.attention_dispatch",
             "diffusers.models.transformers", "diffusers.models.transformers.transformer_wan"]
    saved = {n: sys.modules.get(n) for n in names}
    dispatch = _make_dispatch_module()
    for n in names:
        sys.modules[n] = types.ModuleType(n)
    sys.modules["diffusers.models.attention_dispatch"] = dispatch
    if wan_processor_cls is not None:
        sys.modules[names[-1]].WanAttnProcessor = wan_processor_cls  # type: ignore[attr-defined]
    else:
        del sys.modules[names[-1]]
    try:
        yield dispatch
    finally:
        for n, m in saved.items():
            if m is None:
                sys.modules.pop(n, None)
            else:
                sys.modules[n] = m


def test_enum_member_is_injected_once_and_resolves_both_ways() -> None:
    with fake_diffusers() as d:
        E = d.AttentionBackendName
        before = list(E)
        m = db._ensure_backend_name_registered()
        assert isinstance(m, E) and isinstance(m, str)
        assert m == "repercep_fp8" and m.value == "repercep_fp8" and m.name == "REPERCEP_FP8"
        assert E("repercep_fp8") is m          # lookup by value (what dispatch does)
        assert E["REPERCEP_FP8"] is m          # lookup by name
        assert db._ensure_backend_name_registered() is m
        assert list(E) == before + [m]         # iteration lists it once, after the originals
        assert E("flash") is E.FLASH and E.NATIVE.value == "native"


def test_registration_is_idempotent_and_introspects_the_signature() -> None:
    with fake_diffusers() as d:
        R = d._AttentionBackendRegistry
        m = db.register_repercep_fp8_backend()
        assert R._backends[m] is db._repercep_fp8_attention
        assert R._constraints[m] == []
        assert R._supported_arg_names[m] == {
            "query", "key", "value", "attn_mask", "dropout_p", "is_causal", "scale",
            "enable_gqa", "return_lse", "_parallel_config"}
        snapshot = (dict(R._backends), dict(R._constraints), dict(R._supported_arg_names))
        assert db.register_repercep_fp8_backend() is m
        assert (R._backends, R._constraints, R._supported_arg_names) == snapshot
        assert R._active_backend is d.AttentionBackendName.NATIVE   # registering activates nothing


def test_activation_switches_once() -> None:
    with fake_diffusers() as d:
        R = d._AttentionBackendRegistry
        assert db.activate_repercep_fp8_backend() is True
        assert R._active_backend == "repercep_fp8"
        assert R.get_active_backend()[1] is db._repercep_fp8_attention
        assert db.activate_repercep_fp8_backend() is False
        assert R._active_backend == "repercep_fp8"


@pytest.mark.parametrize("value,active", [
    ("1", True), ("true", True), ("ON", True), ("triton", True), ("scaled_mm", True),
    ("fa", True), ("flash", True), ("", False), ("0", False), ("off", False), ("sdpa", False),
])
def test_env_opt_in(monkeypatch: pytest.MonkeyPatch, value: str, active: bool) -> None:
    monkeypatch.setenv("REPERCEP_FP8_ATTENTION", value)
    with fake_diffusers() as d:
        R = d._AttentionBackendRegistry
        assert db.maybe_activate_from_env() is active
        assert (R._active_backend == "repercep_fp8") is active
        if active:
            assert db.maybe_activate_from_env() is False   # already active


def test_dispatch_reaches_the_backend_and_falls_back_on_cpu(
        monkeypatch: pytest.MonkeyPatch) -> None:
    """diffusers' dispatcher, given the registered name, calls the bridge with
    the arguments it declares; CPU tensors take the bridge's native fallback,
    whose result is SDPA's."""
    monkeypatch.delenv("REPERCEP_FP8_ATTENTION", raising=False)
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(2, 40, 3, 32, generator=g) for _ in range(3))
    calls = []
    real = db._repercep_fp8_attention

    def spy(*a, **kw):
        calls.append(kw)
        return real(*a, **kw)

    with fake_diffusers() as d:
        db.register_repercep_fp8_backend()
        m = d.AttentionBackendName("repercep_fp8")
        d._AttentionBackendRegistry._backends[m] = spy
        out = d.dispatch_attention_fn(q, k, v, is_causal=True, backend="repercep_fp8")
        ref = d.dispatch_attention_fn(q, k, v, is_causal=True, backend="native")
    assert calls and calls[0]["is_causal"] is True
    torch.testing.assert_close(out, ref, rtol=0, atol=0)


def test_wan_installer_with_the_real_registration(monkeypatch: pytest.MonkeyPatch) -> None:
    """End to end on the stand-ins: the Wan processor's dispatch backend is the
    injected enum member itself."""
    class FakeWanAttnProcessor:
        _attention_backend = None

    class T:
        def set_attn_processor(self, p: Any) -> None:
            self.p = p

    pipe = types.SimpleNamespace(transformer=T(), transformer_2=T())
    monkeypatch.setenv("REPERCEP_FP8_ATTENTION", "1")
    with fake_diffusers(FakeWanAttnProcessor) as d:
        assert wan_processor.maybe_install_repercep_wan_attention(pipe) is True
        member = d.AttentionBackendName("repercep_fp8")
        assert pipe.transformer.p._attention_backend is member
        assert pipe.transformer_2.p is pipe.transformer.p
        assert d._AttentionBackendRegistry._backends[member] is db._repercep_fp8_attention
