"""The Wan processor installer (CPU only).

Re-expresses the reference's installer tests (tests/test_wan.py:242-294)
against ``repercep_runtime_amd.attention.wan_processor``, with a stand-in
``diffusers.models.transformers.transformer_wan`` module (diffusers is not
installed here).
"""

from __future__ import annotations

import contextlib
import sys
import types
from typing import Any, Iterator

import pytest

from repercep_runtime_amd.attention import diffusers_backend, wan_processor


class FakeTransformer:
    def __init__(self) -> None:
        self.processor: Any | None = None

    def set_attn_processor(self, processor: Any) -> None:
        self.processor = processor


@contextlib.contextmanager
def fake_wan_module(processor_cls: type) -> Iterator[None]:
    names = ["diffusers", "diffusers.models", "diffusers.models.transformers",
             "diffusers.models.transformers.transformer_wan"]
    saved = {n: sys.modules.get(n) for n in names}
    for n in names:
        sys.modules[n] = types.ModuleType(n)
    sys.modules[names[-1]].WanAttnProcessor = processor_cls  # type: ignore[attr-defined]
    try:
        yield
    finally:
        for n, m in saved.items():
            if m is None:
                sys.modules.pop(n, None)
            else:
                sys.modules[n] = m


def test_installer_noops_without_env(monkeypatch: pytest.MonkeyPatch) -> None:
    pipe = types.SimpleNamespace(transformer=FakeTransformer(), transformer_2=None)
    monkeypatch.delenv("REPERCEP_FP8_ATTENTION", raising=False)
    assert wan_processor.maybe_install_repercep_wan_attention(pipe) is False
    assert pipe.transformer.processor is None
    monkeypatch.setenv("REPERCEP_FP8_ATTENTION", "off")
    assert wan_processor.maybe_install_repercep_wan_attention(pipe) is False


@pytest.mark.parametrize("value", ["fa", "1", "TRUE", "triton"])
def test_installer_sets_the_fp8_backend_on_both_experts(monkeypatch: pytest.MonkeyPatch,
                                                        value: str) -> None:
    class FakeWanAttnProcessor:
        pass

    pipe = types.SimpleNamespace(transformer=FakeTransformer(), transformer_2=FakeTransformer())
    monkeypatch.setenv("REPERCEP_FP8_ATTENTION", value)
    monkeypatch.setattr(diffusers_backend, "register_repercep_fp8_backend",
                        lambda: "repercep-backend")
    with fake_wan_module(FakeWanAttnProcessor):
        assert wan_processor.maybe_install_repercep_wan_attention(pipe) is True
    for t in (pipe.transformer, pipe.transformer_2):
        assert isinstance(t.processor, FakeWanAttnProcessor)
        assert t.processor._attention_backend == "repercep-backend"
        assert t.processor._repercep_attention_backend == "repercep_fp8"
    # one processor object shared by both experts, as diffusers' setter allows
    assert pipe.transformer.processor is pipe.transformer_2.processor


def test_installer_without_diffusers_keeps_the_native_path(
        monkeypatch: pytest.MonkeyPatch) -> None:
    pipe = types.SimpleNamespace(transformer=FakeTransformer())
    monkeypatch.setenv("REPERCEP_FP8_ATTENTION", "1")
    monkeypatch.setitem(sys.modules, "diffusers", None)   # import fails
    assert wan_processor.install_repercep_wan_attention(pipe) == 0
    assert pipe.transformer.processor is None


def test_installer_skips_transformers_that_refuse(monkeypatch: pytest.MonkeyPatch) -> None:
    class FakeWanAttnProcessor:
        pass

    class Refusing(FakeTransformer):
        def set_attn_processor(self, processor: Any) -> None:
            raise RuntimeError("no")

    pipe = types.SimpleNamespace(transformer=Refusing(), transformer_2=object())
    monkeypatch.setattr(diffusers_backend, "register_repercep_fp8_backend", lambda: "b")
    with fake_wan_module(FakeWanAttnProcessor):
        assert wan_processor.install_repercep_wan_attention(pipe) == 0
    pipe.transformer_2 = FakeTransformer()
    with fake_wan_module(FakeWanAttnProcessor):
        assert wan_processor.install_repercep_wan_attention(pipe) == 1
