"""FP8 linear module (host side, CPU only): construction, shape rules, state
dicts, and the reference's parent-first module swap
(src/repercep/runtime/quantize.py:135-179) with its name filter."""

from __future__ import annotations

import pytest
import torch

from repercep_runtime_amd import fp8_linear
from repercep_runtime_amd.fp8_linear import FP8Linear, replace_linears_with_fp8


def _fake(n: int, k: int, bias: bool = True) -> FP8Linear:
    return FP8Linear(torch.zeros(n, k, dtype=torch.uint8), torch.tensor([0.5]),
                     torch.ones(n) if bias else None)


def test_members_and_state_dict() -> None:
    m = _fake(64, 32)
    assert (m.out_features, m.in_features) == (64, 32)
    assert m.qweight.dtype == torch.uint8 and m.scale.dtype == torch.float32
    assert m.bias is not None and m.bias.dtype == torch.bfloat16 and not m.bias.requires_grad
    sd = m.state_dict()
    assert set(sd) == {"qweight", "scale", "bias"}
    m2 = _fake(64, 32)
    m2.load_state_dict(sd)
    assert "in_features=32, out_features=64" in repr(m2)
    assert _fake(8, 16, bias=False).bias is None


@pytest.mark.parametrize("n,k", [(64, 24), (30, 32)])
def test_shapes_the_gemm_cannot_take_are_refused(n: int, k: int) -> None:
    with pytest.raises(ValueError, match="in_features % 16"):
        _fake(n, k)


def test_forward_needs_bf16() -> None:
    with pytest.raises(TypeError, match="bfloat16"):
        _fake(8, 16)(torch.zeros(2, 16))


class _Block(torch.nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.ff = torch.nn.Sequential(torch.nn.Linear(32, 64), torch.nn.GELU(),
                                      torch.nn.Linear(64, 32))
        self.proj = torch.nn.Linear(32, 48)
        self.odd = torch.nn.Linear(20, 32)       # in_features % 16 != 0: kept


def test_swap_is_parent_first_and_filtered(monkeypatch: pytest.MonkeyPatch) -> None:
    monkeypatch.setattr(fp8_linear, "quantize_weight",
                        lambda w: (torch.zeros(w.shape, dtype=torch.uint8), torch.tensor([1.0])))
    net = torch.nn.ModuleDict({"dit": _Block(), "vae": _Block()})
    assert replace_linears_with_fp8(net, name_filter="dit.ff") == 2
    assert isinstance(net["dit"].ff[0], FP8Linear) and isinstance(net["dit"].ff[2], FP8Linear)
    assert isinstance(net["dit"].proj, torch.nn.Linear)
    assert replace_linears_with_fp8(net) == 4     # dit.proj, vae.ff x2, vae.proj
    assert isinstance(net["vae"].odd, torch.nn.Linear) and isinstance(net["dit"].odd, torch.nn.Linear)
    assert net["vae"].proj.out_features == 48
