"""Host-side logic of the drop-in (CPU only): the AttentionOp surface, op
selection, the ROCm backend seam, the (B, S, H, D) dispatcher bridge, the
workload definitions and the bench's one-GPU contract.

The structural tests re-express the reference's own
(tests/test_attention_fp8.py:37-73, tests/test_attention_diffusers_backend.py)
against this package's classes.
"""

from __future__ import annotations

import inspect
import json
import os
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from repercep_runtime_amd import _capi, ops
from repercep_runtime_amd.attention import (
    AttentionKind,
    AttentionOp,
    AttentionShape,
    FP8HipAttention,
    NaiveAttention,
)
from repercep_runtime_amd.attention import diffusers_backend as db
from repercep_runtime_amd.backend.protocol import Backend
from repercep_runtime_amd.backend.rocm import _GFX_TO_ARCH, ROCmBackend
from repercep_runtime_amd.hardware import MI300X, MI355X, DeviceArch, DType, Vendor
from repercep_runtime_amd.workloads import (
    ATTN_CONFIGS,
    C1,
    C2,
    C3_CROSS,
    C3_SELF,
    C4,
    C5,
    AttnConfig,
    attn_inputs,
)

ROOT = Path(__file__).resolve().parent.parent


# ------------------------------------------------------------ AttentionOp
def test_fp8_op_satisfies_protocol() -> None:
    op = FP8HipAttention()
    assert isinstance(op, AttentionOp)
    assert op.name == "fp8-hip-flash"
    assert isinstance(NaiveAttention(), AttentionOp)


def test_fp8_op_supports() -> None:
    op = FP8HipAttention()
    assert op.available  # the library loads on any host; compute needs the GPU
    ok = AttentionShape(batch=1, heads=2, seq_len_q=256, seq_len_kv=256, head_dim=64)
    assert op.supports(ok, DType.BF16)
    assert op.supports(AttentionShape(1, 40, 75600, 512, 128), DType.BF16)        # cross
    assert op.supports(AttentionShape(1, 2, 256, 256, 128, AttentionKind.CAUSAL), DType.BF16)
    assert not op.supports(AttentionShape(1, 2, 64, 64, 64), DType.BF16)          # min length
    assert not op.supports(AttentionShape(1, 2, 256, 256, 96), DType.BF16)        # head dim
    assert not op.supports(AttentionShape(1, 2, 256, 256, 64, AttentionKind.NEIGHBORHOOD),
                           DType.BF16)
    assert op.supports(ok, DType.FP16)                                            # as fp8_triton.py:85
    assert not op.supports(ok, DType.FP32)
    for d in (32, 256):                                                            # the full set
        assert op.supports(AttentionShape(1, 2, 256, 256, d), DType.BF16)


def test_fp8_op_raises_runtime_error_when_unavailable() -> None:
    op = FP8HipAttention()
    op._fn = None
    op._import_error = "HipLibraryError: missing"
    assert not op.available
    assert not op.supports(AttentionShape(1, 2, 256, 256, 64), DType.BF16)
    x = torch.zeros(1, 1, 4, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="not available"):
        op(x, x, x)


def test_product_path_has_no_cpu_fallback() -> None:
    x = torch.zeros(1, 2, 256, 64, dtype=torch.bfloat16)
    for fn in (lambda: ops.fp8_flash_attention(x, x, x), lambda: ops.scale_quantize(x),
               lambda: ops.per_bh_scale(x)):
        with pytest.raises(ValueError, match="GPU tensor"):
            fn()
    a8 = torch.zeros(16, 16, dtype=torch.uint8)
    with pytest.raises(ValueError, match="GPU tensor"):
        ops.fp8_gemm(a8, a8, 1.0, 1.0)


def _run(code: str, **env: str) -> str:
    e = dict(os.environ)
    e.pop("REPERCEP_FP8_ATTENTION", None)
    e.update(env)
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=e, capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    return r.stdout.strip()


def test_missing_library_fails_loudly() -> None:
    out = _run(
        "from repercep_runtime_amd import _capi\n"
        "from repercep_runtime_amd.attention import FP8HipAttention\n"
        "op = FP8HipAttention()\n"
        "try:\n"
        "    _capi.lib(); print('loaded')\n"
        "except _capi.HipLibraryError as e:\n"
        "    print('raised', op.available)\n",
        REPERCEP_FP8_LIB="/nonexistent/librepercep_fp8.so")
    assert out == "raised False"


_SELECT = (
    "from repercep_runtime_amd.attention import select_attention_op, AttentionShape\n"
    "from repercep_runtime_amd.hardware import MI355X, DType, DeviceArch, Vendor\n"
    "s = AttentionShape(1, 40, 75600, 75600, 128)\n"
    "print(select_attention_op(MI355X, s, DType.BF16).name,"
    " select_attention_op(MI355X, AttentionShape(1, 2, 64, 64, 64), DType.BF16).name,"
    " select_attention_op(DeviceArch(Vendor.NVIDIA, 'sm_90', 'hopper'), s, DType.BF16).name)\n"
)


@pytest.mark.parametrize("env,want", [
    ({}, "naive-sdpa naive-sdpa naive-sdpa"),
    # the fused kernel where it qualifies (Skv >= 128), the unfused scaled-mm
    # op below that, the floor on other vendors (reference registry.py:84-92)
    ({"REPERCEP_FP8_ATTENTION": "1"}, "fp8-hip-flash fp8-hip-scaled-mm naive-sdpa"),
    ({"REPERCEP_FP8_ATTENTION": "triton"}, "fp8-hip-flash naive-sdpa naive-sdpa"),
    # scaled_mm: the unfused op only -- its 4 GiB scores cap rules out the Wan shape
    ({"REPERCEP_FP8_ATTENTION": "scaled_mm"}, "naive-sdpa fp8-hip-scaled-mm naive-sdpa"),
    ({"REPERCEP_FP8_ATTENTION": "te"}, "naive-sdpa naive-sdpa naive-sdpa"),
    ({"REPERCEP_FP8_ATTENTION": "off"}, "naive-sdpa naive-sdpa naive-sdpa"),
])
def test_registry_env_selection(env: dict, want: str) -> None:
    assert _run(_SELECT, **env) == want


# ------------------------------------------------------------- backend
def test_rocm_backend_maps_gfx950() -> None:
    assert _GFX_TO_ARCH["gfx950"] is MI355X
    assert MI355X == DeviceArch(Vendor.AMD, "gfx950", "CDNA4")
    assert _GFX_TO_ARCH["gfx942"] is MI300X
    assert str(MI355X) == "amd:gfx950"
    b = ROCmBackend()
    assert isinstance(b, Backend)
    assert b.default_dtype() is DType.BF16
    assert "fp8-hip-flash" in b.capabilities().attention_ops


# ------------------------------------------------------- diffusers bridge
def test_bridge_signature_matches_reference() -> None:
    """diffusers introspects these names (diffusers_backend.py:160-171 of the reference)."""
    names = list(inspect.signature(db._repercep_fp8_attention).parameters)
    assert names == ["query", "key", "value", "attn_mask", "dropout_p", "is_causal", "scale",
                     "enable_gqa", "return_lse", "_parallel_config"]
    assert db.REPERCEP_FP8_BACKEND_NAME == "repercep_fp8"


def _bshd(S: int, H: int = 2, D: int = 64, dtype=torch.bfloat16, Skv: int | None = None):
    g = torch.Generator().manual_seed(S)
    q = torch.randn(1, S, H, D, generator=g).to(dtype)
    kv = torch.randn(1, Skv or S, H, D, generator=g).to(dtype)
    return q, kv, kv.clone()


def test_bridge_routing_rules() -> None:
    q, k, v = _bshd(4096)
    assert db._route_should_use_fp8(q, k, v)
    assert not db._route_should_use_fp8(*_bshd(1024))                       # crossover
    assert db._route_should_use_fp8(*_bshd(4096, dtype=torch.float16))      # fp16 (:69)
    assert not db._route_should_use_fp8(*_bshd(4096, dtype=torch.float32))  # dtype
    assert db._route_should_use_fp8(*_bshd(4096, D=256))                    # head dims (:49)
    assert db._route_should_use_fp8(*_bshd(4096, D=32))
    assert not db._route_should_use_fp8(*_bshd(4096, D=96))                 # head dim
    assert db._route_should_use_fp8(*_bshd(4096, D=128, Skv=512))           # cross-attention
    assert not db._route_should_use_fp8(*_bshd(4096, Skv=64))               # short K/V
    qh, kh, vh = _bshd(4096)
    assert not db._route_should_use_fp8(qh, kh[:, :, :1], vh[:, :, :1])     # head mismatch


def test_bridge_falls_back_to_sdpa_off_gpu() -> None:
    q, k, v = _bshd(4096, H=1)
    ref = torch.nn.functional.scaled_dot_product_attention(
        q.permute(0, 2, 1, 3), k.permute(0, 2, 1, 3), v.permute(0, 2, 1, 3)).permute(0, 2, 1, 3)
    out = db._repercep_fp8_attention(q, k, v)
    assert out.shape == q.shape and torch.equal(out, ref)
    with pytest.raises(ValueError, match="return_lse"):
        db._repercep_fp8_attention(q, k, v, return_lse=True)


# ------------------------------------------------------------- workloads
def test_workload_flops_match_published_counts() -> None:
    """Algorithmic FLOPs per call of the BASELINE configurations."""
    assert C1.flops == pytest.approx(2.147e9, rel=1e-3)
    assert C2.flops == pytest.approx(5.197e13, rel=1e-3)
    assert C3_SELF.flops == pytest.approx(1.1705e14, rel=1e-3)
    assert C3_CROSS.flops == pytest.approx(7.93e11, rel=1e-3)
    assert C5.flops == pytest.approx(1.083e9, rel=1e-3)
    assert C4.flops == pytest.approx(1.0702e13, rel=1e-3)
    assert C3_SELF.quant_elems * 5 == 5_806_080_000


@pytest.mark.parametrize("cfg", [AttnConfig("t", 1, 1, 37, 37, 64, causal=True),
                                 AttnConfig("p", 1, 1, 24, 40, 64, prefix=16, suffix=8)])
def test_visible_pairs_brute_force(cfg: AttnConfig) -> None:
    import numpy as np

    from oracle.attention import visible

    mask = 1 if cfg.causal else 2
    vis = visible(np.arange(cfg.Sq), np.arange(cfg.Skv), mask, cfg.prefix or 0, cfg.suffix or 1)
    assert int(vis.sum()) == cfg.visible_pairs_per_head()


def test_inputs_are_seeded_and_match_recipe() -> None:
    q, k, _ = attn_inputs(C1)
    g = torch.Generator().manual_seed(0)
    assert torch.equal(q, torch.randn(1, 8, 1024, 64, generator=g).to(torch.bfloat16))
    assert torch.equal(k, torch.randn(1, 8, 1024, 64, generator=g).to(torch.bfloat16))
    assert set(ATTN_CONFIGS) >= {"c1_cpu_runnable", "c3_wan_self", "c5_shared_prefix"}


# ------------------------------------------------------------ bench / entry
def test_bench_refuses_more_than_one_gpu() -> None:
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_graft_entry_points_exist() -> None:
    import __graft_entry__ as g

    assert callable(g.build) and callable(g.smoke)


def test_traffic_profile_is_well_formed() -> None:
    data = json.loads((ROOT / "profiles" / "traffic.json").read_text())
    k = data["c3_wan_self"]["attn_fwd_kernel"]
    assert k["hbm_bytes_per_launch"] == k["hbm_read_bytes_per_launch"] + \
        k["hbm_write_bytes_per_launch"]
    # the balanced launch (288 of 296 query blocks per head unsplit, the
    # rest split 4 ways): the kernel writes the bf16 output of the unsplit
    # rows once and the fp32 partials (O, m, l) of the split rows; the merge
    # reads those partials and writes the bf16 output of the split rows
    main_rows, tail_rows = 288 * 256, 75600 - 288 * 256
    out_main = 40 * main_rows * 128 * 2
    partials = 4 * 40 * tail_rows * (128 + 2) * 4
    assert abs(k["hbm_write_bytes_per_launch"] - (out_main + partials)) < 1e6
    c = data["c3_wan_self"]["attn_combine_kernel"]
    assert abs(c["hbm_write_bytes_per_launch"] - 40 * tail_rows * 128 * 2) < 1e6
    assert abs(c["hbm_read_bytes_per_launch"] - partials) < 0.05 * partials


def test_scaled_mm_op_contract() -> None:
    """FP8HipScaledMMAttention keeps the reference's supports() rules
    (src/repercep/attention/fp8_scaled_mm.py:87-105): head dims {64, 96, 128,
    192, 256}, FULL/CAUSAL, lengths >= 16 and multiples of 16, bf16 scores at
    most 4 GiB."""
    from repercep_runtime_amd.attention import AttentionOp, FP8HipScaledMMAttention
    from repercep_runtime_amd.attention.types import AttentionKind

    op = FP8HipScaledMMAttention()
    assert isinstance(op, AttentionOp) and op.name == "fp8-hip-scaled-mm"
    assert op.available        # the library loads on a CPU host too
    ok = AttentionShape(1, 4, 512, 512, 128)
    assert op.supports(ok, DType.BF16) and op.supports(ok, DType.FP16)
    assert not op.supports(ok, DType.FP32)
    assert not op.supports(AttentionShape(1, 4, 512, 512, 32), DType.BF16)
    assert op.supports(AttentionShape(1, 4, 512, 512, 96), DType.BF16)
    assert not op.supports(AttentionShape(1, 4, 520, 512, 128), DType.BF16)
    assert not op.supports(AttentionShape(1, 4, 8, 8, 128), DType.BF16)
    assert not op.supports(AttentionShape(1, 4, 512, 512, 128, kind=AttentionKind.NEIGHBORHOOD),
                           DType.BF16)
    assert op.supports(AttentionShape(1, 1, 46336, 46336, 128), DType.BF16)   # 4.0 GiB
    assert not op.supports(AttentionShape(1, 1, 46352, 46352, 128), DType.BF16)
