"""The allocation-free Q/K/V quantizer entry point (rp_fp8_scale_quantize_qkv_noalloc).

It has no counterpart in the reference: it serves callers that cannot
allocate device memory.  Through the C ABI it must give exactly the scales
and codes of rp_fp8_scale_quantize_qkv (the workspace entry point) on
consecutive calls that share its static device scratch, the second smaller
than the first, and refuse shapes whose scratch would not fit before touching
the device.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from repercep_runtime_amd import _capi

FAKE = 1 << 20           # 16-byte aligned non-null address; never dereferenced


def _bhsd(x: torch.Tensor) -> tuple[int, int, int]:
    return x.stride(0), x.stride(1), x.stride(2)


def _run(entry: str, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, gran: int,
         workspace: bool) -> tuple[torch.Tensor, ...]:
    L = _capi.lib()
    B, H, Sq, D = q.shape
    Skv = k.shape[2]
    G = B * H if gran == _capi.RP_SCALE_PER_BH else 1
    ldv = -(-Skv // 128) * 128
    dev = q.device
    dq = torch.full((3 * G,), float("nan"), dtype=torch.float32, device=dev)
    q8 = torch.full((B, H, Sq, D), 0x55, dtype=torch.uint8, device=dev)
    k8 = torch.full((B, H, Skv, D), 0x55, dtype=torch.uint8, device=dev)
    vt8 = torch.full((B, H, D, ldv), 0x55, dtype=torch.uint8, device=dev)
    dt = _capi.RP_DTYPE_BF16 if q.dtype == torch.bfloat16 else _capi.RP_DTYPE_F16
    args = [q.data_ptr(), k.data_ptr(), v.data_ptr(), dt, B, H, Sq, Skv, D, *_bhsd(q),
            *_bhsd(k), *_bhsd(v), gran, dq.data_ptr(), q8.data_ptr(), k8.data_ptr(),
            vt8.data_ptr(), ldv]
    stream = torch.cuda.current_stream(dev).cuda_stream
    if workspace:
        nbytes = L.rp_fp8_quant_qkv_workspace_bytes(B, H, Sq, Skv, D, gran)
        ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=dev)
        rc = getattr(L, entry)(*args, ws.data_ptr(), ws.numel(), stream)
    else:
        rc = getattr(L, entry)(*args, stream)
    _capi.check(rc, entry)
    torch.cuda.synchronize()
    return dq, q8, k8, vt8


def _case(seed: int, B: int, H: int, Sq: int, Skv: int, D: int, dtype: torch.dtype,
          bshd: bool, dev: torch.device) -> tuple[torch.Tensor, ...]:
    g = torch.Generator().manual_seed(seed)

    def t(S: int, scale: float) -> torch.Tensor:
        x = (torch.randn(B, S, H, D, generator=g) * scale).to(dtype).to(dev)
        return x.permute(0, 2, 1, 3) if bshd else x.permute(0, 2, 1, 3).contiguous()

    return t(Sq, 1.0), t(Skv, 3.0), t(Skv, 0.5)


@pytest.mark.gpu
def test_noalloc_equals_workspace_entry_on_consecutive_calls() -> None:
    """Two calls in a row, the second on smaller tensors (fewer partial maxima
    than the first left in the scratch), each bit-identical to the workspace
    entry point: scales, Q/K codes and V^T codes with its zero tail."""
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a host without a GPU")
    dev = torch.device("cuda", 0)
    cases = [
        # seed, B, H, Sq, Skv, D, dtype, strided (B, S, H, D) views, granularity
        (1, 2, 5, 3000, 2100, 128, torch.bfloat16, True, _capi.RP_SCALE_PER_BH),
        (2, 1, 2, 300, 129, 64, torch.float16, False, _capi.RP_SCALE_PER_TENSOR),
        (3, 1, 3, 777, 640, 128, torch.bfloat16, False, _capi.RP_SCALE_PER_BH),
    ]
    for seed, B, H, Sq, Skv, D, dtype, bshd, gran in cases:
        q, k, v = _case(seed, B, H, Sq, Skv, D, dtype, bshd, dev)
        ref = _run("rp_fp8_scale_quantize_qkv", q, k, v, gran, workspace=True)
        got = _run("rp_fp8_scale_quantize_qkv_noalloc", q, k, v, gran, workspace=False)
        names = ("scales", "q8", "k8", "vt8")
        for name, a, b in zip(names, got, ref):
            if name == "scales":
                assert torch.equal(a.view(torch.int32), b.view(torch.int32)), (seed, name)
            else:
                assert torch.equal(a, b), (seed, name, int((a != b).sum()))
        assert torch.isfinite(got[0]).all()


def test_noalloc_refuses_shapes_beyond_its_scratch() -> None:
    """Shapes whose partial maxima exceed RP_QKV_NOALLOC_SCRATCH_BYTES are
    refused with RP_ERR_WORKSPACE before any device call (fake pointers; no
    GPU needed), and the message names the size."""
    L = _capi.lib()
    D = 128
    S = 1 << 22                        # 4 Mi rows of 128: 512 Mi elements per head
    H = 4
    need = L.rp_fp8_quant_qkv_workspace_bytes(1, H, S, S, D, _capi.RP_SCALE_PER_BH)
    assert need > _capi.RP_QKV_NOALLOC_SCRATCH_BYTES
    st = (H * S * D, S * D, D)
    rc = L.rp_fp8_scale_quantize_qkv_noalloc(
        FAKE, FAKE, FAKE, _capi.RP_DTYPE_BF16, 1, H, S, S, D, *st, *st, *st,
        _capi.RP_SCALE_PER_BH, FAKE, FAKE, FAKE, FAKE, S, None)
    assert rc == 3  # RP_ERR_WORKSPACE
    msg = L.rp_last_error().decode()
    assert str(need) in msg and "scratch" in msg
    # argument errors come first, as in the workspace entry point
    rc = L.rp_fp8_scale_quantize_qkv_noalloc(
        None, FAKE, FAKE, _capi.RP_DTYPE_BF16, 1, 1, 128, 128, D, *st, *st, *st,
        _capi.RP_SCALE_PER_BH, FAKE, FAKE, FAKE, FAKE, 128, None)
    assert rc == 1  # RP_ERR_INVALID_ARGUMENT
    assert isinstance(L.rp_fp8_scale_quantize_qkv_noalloc, ctypes._CFuncPtr)


@pytest.mark.gpu
def test_noalloc_replays_from_a_captured_graph() -> None:
    """After one eager call on the device, the entry point can be captured:
    replays with new inputs copied in between (and the program's own eager
    work and synchronisations between replays) give the eager results bit
    for bit every time."""
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a host without a GPU")
    dev = torch.device("cuda", 0)
    L = _capi.lib()
    B, H, Sq, Skv, D = 1, 3, 777, 640, 128
    gran = _capi.RP_SCALE_PER_BH
    q, k, v = _case(7, B, H, Sq, Skv, D, torch.bfloat16, False, dev)
    ldv = -(-Skv // 128) * 128
    xq, xk, xv = q.clone(), k.clone(), v.clone()    # the graph's input buffers
    dq = torch.empty(3 * B * H, dtype=torch.float32, device=dev)
    q8 = torch.empty(B, H, Sq, D, dtype=torch.uint8, device=dev)
    k8 = torch.empty(B, H, Skv, D, dtype=torch.uint8, device=dev)
    vt8 = torch.zeros(B, H, D, ldv, dtype=torch.uint8, device=dev)

    def call() -> None:
        stream = torch.cuda.current_stream(dev).cuda_stream
        rc = L.rp_fp8_scale_quantize_qkv_noalloc(
            xq.data_ptr(), xk.data_ptr(), xv.data_ptr(), _capi.RP_DTYPE_BF16, B, H, Sq, Skv, D,
            *_bhsd(xq), *_bhsd(xk), *_bhsd(xv), gran, dq.data_ptr(), q8.data_ptr(),
            k8.data_ptr(), vt8.data_ptr(), ldv, stream)
        _capi.check(rc, "rp_fp8_scale_quantize_qkv_noalloc")

    call()                       # the eager first call resolves the scratch address
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    for seed in (11, 12, 13):
        nq, nk, nv = _case(seed, B, H, Sq, Skv, D, torch.bfloat16, False, dev)
        want = _run("rp_fp8_scale_quantize_qkv", nq, nk, nv, gran, workspace=True)
        xq.copy_(nq)
        xk.copy_(nk)
        xv.copy_(nv)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(dq.view(torch.int32), want[0].view(torch.int32)), seed
        assert torch.equal(q8, want[1]), seed
        assert torch.equal(k8, want[2]), seed
        assert torch.equal(vt8[..., :Skv], want[3][..., :Skv]), seed
