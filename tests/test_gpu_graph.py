"""The FP8 attention path (and the GEMM) under HIP graph capture (torch.cuda.graph): small
calls are bound by host launch work, which a captured graph removes.  Every
replay, with new inputs copied into the captured buffers and eager work and
synchronisations between replays, equals an eager call bit for bit."""

from __future__ import annotations

import pytest
import torch

from repercep_runtime_amd import ops
from repercep_runtime_amd.workloads import C1, C5, attn_inputs

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("cfg", [C1, C5], ids=["c1", "c5_shared_prefix"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_captured_attention_replays_match_eager(gpu: torch.device, cfg, dtype) -> None:
    kw = dict(prefix_len=cfg.prefix, suffix_len=cfg.suffix) if cfg.prefix else {}
    q, k, v = (t.to(dtype) for t in attn_inputs(cfg, device=gpu))
    sq, sk, sv = q.clone(), k.clone(), v.clone()          # the captured inputs
    ops.fp8_flash_attention(sq, sk, sv, kv_splits=1, **kw)   # warm up outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        sout = ops.fp8_flash_attention(sq, sk, sv, kv_splits=1, **kw)
    g = torch.Generator(device=gpu).manual_seed(7)
    for rep in range(4):
        if rep:   # new inputs for every later replay
            for src in (sq, sk, sv):
                src.copy_(torch.randn(src.shape, generator=g, device=gpu).to(dtype))
        graph.replay()
        torch.cuda.synchronize()
        want = ops.fp8_flash_attention(sq.clone(), sk.clone(), sv.clone(), kv_splits=1, **kw)
        _ = torch.randn(1024, device=gpu).sum().item()      # unrelated eager work + sync
        assert torch.equal(sout, want), f"replay {rep} differs from eager"


def test_captured_balanced_launch_replays_match_eager(gpu: torch.device) -> None:
    """The balanced launch (kv_splits=0) of a shape whose plan splits the last
    round's blocks on 256 CUs: one mixed attention launch and the merge,
    with its workspace from the capture's pool; every replay equals an eager
    call bit for bit."""
    q, k, v = (torch.randn(1, 8, n, 128, device=gpu).to(torch.bfloat16)
               for n in (8860, 8192, 8192))
    sq, sk, sv = q.clone(), k.clone(), v.clone()
    ops.fp8_flash_attention(sq, sk, sv, kv_splits=0)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        sout = ops.fp8_flash_attention(sq, sk, sv, kv_splits=0)
    g = torch.Generator(device=gpu).manual_seed(11)
    for rep in range(3):
        if rep:
            for src in (sq, sk, sv):
                src.copy_(torch.randn(src.shape, generator=g, device=gpu).to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        want = ops.fp8_flash_attention(sq.clone(), sk.clone(), sv.clone(), kv_splits=0)
        _ = torch.randn(1024, device=gpu).sum().item()
        assert torch.equal(sout, want), f"replay {rep} differs from eager"


def test_captured_balanced_gemm_replays_match_eager(gpu: torch.device) -> None:
    """ops.fp8_gemm's balanced launch (its counter cleared by a kernel of the
    call, tiles handed out through it) captured with its workspace from the
    capture's pool: every replay, with new operands, equals an eager call bit
    for bit."""
    M, N, K = 2148, 1280, 256    # 45 tiles: every tile goes through the counter
    g = torch.Generator(device=gpu).manual_seed(13)
    a8 = torch.randint(0, 126, (M, K), generator=g, device=gpu, dtype=torch.uint8)
    b8 = torch.randint(0, 126, (K, N), generator=g, device=gpu, dtype=torch.uint8)
    ops.fp8_gemm(a8, b8, 0.01, 0.02)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        sout = ops.fp8_gemm(a8, b8, 0.01, 0.02)
    for rep in range(3):
        if rep:
            a8.copy_(torch.randint(0, 126, (M, K), generator=g, device=gpu, dtype=torch.uint8))
            b8.copy_(torch.randint(0, 126, (K, N), generator=g, device=gpu, dtype=torch.uint8))
        graph.replay()
        torch.cuda.synchronize()
        want = ops.fp8_gemm(a8.clone(), b8.clone(), 0.01, 0.02)
        _ = torch.randn(1024, device=gpu).sum().item()
        assert torch.equal(sout.view(torch.int16), want.view(torch.int16)), f"replay {rep}"
