"""Kernel-layer entry points of the FP8 hot path (torch tensors in, torch tensors out).

This module plays the role of the reference's kernel module
(kernels/triton_kernels/fp8_flash_attn.py and its OCP siblings, plus
kernels/hip/fp8_attn/binding.cpp): it validates shapes, allocates outputs and
scratch with torch's caching allocator, and calls librepercep_fp8.so through
its C ABI on torch's current stream.  All arithmetic happens in the gfx950
kernels; nothing here computes on the CPU.

Numerics (OCP e4m3fn, FP8_MAX = 448):
  per_bh_scale   dequant = bf16(max(amax|x|, bf16(1e-6)) / (0.95 * 448))
                 -- kernels/triton_kernels/fp8_flash_attn_hopper.py:374-385
  quantize       e4m3fn(clamp(x * (1 / dequant), -448, 448)), RNE
                 -- fp8_flash_attn_hopper.py:388-398
  fp8_flash_attention
                 FA-2 FP8 forward -- kernels/triton_kernels/fp8_flash_attn.py:480-645
  fp8_gemm       bf16(fp32(A8 . B8) * a_scale * b_scale), B (K, N) as the
                 reference takes it or (N, K)
                 -- kernels/hip/fp8_attn/binding.cpp:25-57, fp8_gemm.hip:79-179
"""

from __future__ import annotations

import functools
import math
from typing import Callable, Literal

import torch

from repercep_runtime_amd import _capi as C
from repercep_runtime_amd import tuning

FP8_E4M3_MAX = 448.0
#: head dims compiled into the attention kernel
SUPPORTED_HEAD_DIMS = frozenset({32, 64, 128, 256})
#: keys per tile of the attention kernel.  Numerically significant: the
#: running max after each tile sets the grid P is quantized on.
BLOCK_N = 128
#: query rows per block of the attention kernel (one workgroup's rows)
BLOCK_M = 256
#: query rows per workgroup of the short-query (wave-split) launch, and the
#: head dims it is compiled for
WSPLIT_BLOCK_MS = (32, 64, 128)
WSPLIT_HEAD_DIMS = frozenset({64, 128})
#: row padding of the transposed V operand
V_PAD = 128

Granularity = Literal["bh", "tensor"]
_GRAN = {"bh": C.RP_SCALE_PER_BH, "tensor": C.RP_SCALE_PER_TENSOR}
_IN_DTYPES = {torch.bfloat16: C.RP_DTYPE_BF16, torch.float16: C.RP_DTYPE_F16}
_OUT_DTYPES = {torch.bfloat16: C.RP_OUT_BF16, torch.float16: C.RP_OUT_F16,
               torch.float32: C.RP_OUT_F32}


# torch's accessor of the current stream's raw handle (what its own kernels
# launch on), without building a Stream object on every call
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t: torch.Tensor) -> int:
    if _raw_stream is not None:
        return _raw_stream(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def _check_cuda(name: str, t: torch.Tensor) -> None:
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor (got device {t.device})")


def _on_device_of(ref: torch.Tensor, **tensors: torch.Tensor | None) -> None:
    """Every given tensor (None skipped) lives on ``ref``'s GPU: the kernels
    launch on that device and dereference each pointer there."""
    for name, t in tensors.items():
        if t is None:
            continue
        _check_cuda(name, t)
        if t.device != ref.device:
            raise ValueError(f"{name} is on {t.device}, the other operands on {ref.device}")


def _bhsd_view(x: torch.Tensor) -> tuple[int, int, int, int, int, int, int]:
    """(B, H, S, D, sb, sh, ss) for a 4-D (B, H, S, D) tensor with unit stride on D."""
    if x.dim() != 4:
        raise ValueError(f"expected a 4-D (B, H, S, D) tensor, got shape {tuple(x.shape)}")
    if x.stride(3) != 1:
        raise ValueError("the last (head) dimension must be contiguous")
    B, H, S, D = x.shape
    sb, sh, ss, _ = x.stride()
    return B, H, S, D, sb, sh, ss


def _as4d(x: torch.Tensor) -> torch.Tensor:
    if x.dim() == 4:
        return x
    if x.dim() == 2:
        return x.reshape(1, 1, *x.shape) if x.is_contiguous() else x.unsqueeze(0).unsqueeze(0)
    raise ValueError(f"expected a 2-D or 4-D tensor, got {x.dim()}-D")


def _check_bf16(name: str, x: torch.Tensor) -> None:
    _check_cuda(name, x)
    if x.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16 (got {x.dtype})")


def _in_dtype(name: str, x: torch.Tensor) -> int:
    """RP_DTYPE_* of a quantizer input: bfloat16 or float16, on the GPU."""
    _check_cuda(name, x)
    dt = _IN_DTYPES.get(x.dtype)
    if dt is None:
        raise TypeError(f"{name} must be bfloat16 or float16 (got {x.dtype})")
    return dt


def per_bh_scale(x: torch.Tensor, granularity: Granularity = "bh") -> torch.Tensor:
    """Dequant scale per (batch, head) -- shape (B*H,) -- or per tensor -- shape (1,).

    Same result as the reference's ``_per_bh_scale`` on the GPU (bit for
    bit), for bfloat16 or float16 ``x``.  A 2-D input is treated as one
    (1, 1, S, D) head.
    """
    dt = _in_dtype("x", x)
    x4 = _as4d(x)
    B, H, S, D, sb, sh, ss = _bhsd_view(x4)
    n = B * H if granularity == "bh" else 1
    out = torch.empty(n, dtype=torch.float32, device=x.device)
    ws_bytes = C.lib().rp_fp8_quant_workspace_bytes(B, H, S, D, _GRAN[granularity])
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=x.device)
    C.check(C.lib().rp_fp8_scale(x4.data_ptr(), dt, B, H, S, D, sb, sh, ss, _GRAN[granularity],
                                 out.data_ptr(), ws.data_ptr(), ws.numel(), _stream(x)),
            "rp_fp8_scale")
    return out


def quantize(x: torch.Tensor, dequant: torch.Tensor, granularity: Granularity = "bh",
             layout: Literal["bhsd", "bhds"] = "bhsd") -> torch.Tensor:
    """e4m3fn codes of ``x`` (torch.float8_e4m3fn) under the given dequant scales.

    layout "bhsd": (B, H, S, D) contiguous, like the reference's
    ``_quantize(x, s).contiguous()``.  layout "bhds": (B, H, D, ldv) with
    ldv = S rounded up to 128 and zero padding -- V transposed per head, the
    operand layout of the attention kernel.
    """
    dt = _in_dtype("x", x)
    _on_device_of(x, dequant=dequant)
    x4 = _as4d(x)
    B, H, S, D, sb, sh, ss = _bhsd_view(x4)
    dq = dequant.to(torch.float32).contiguous()
    if dq.numel() != (B * H if granularity == "bh" else 1):
        raise ValueError(f"dequant has {dq.numel()} scales for granularity {granularity!r}")
    if layout == "bhsd":
        codes = torch.empty((B, H, S, D), dtype=torch.uint8, device=x.device)
        lay, ld = C.RP_LAYOUT_BHSD, 0
    else:
        ld = _round_up(S, V_PAD)
        codes = torch.empty((B, H, D, ld), dtype=torch.uint8, device=x.device)
        lay = C.RP_LAYOUT_BHDS
    C.check(C.lib().rp_fp8_quantize(x4.data_ptr(), dt, B, H, S, D, sb, sh, ss, _GRAN[granularity],
                                    dq.data_ptr(), codes.data_ptr(), lay, ld, _stream(x)),
            "rp_fp8_quantize")
    codes = codes.view(torch.float8_e4m3fn)
    return codes if x.dim() == 4 or layout == "bhds" else codes.reshape(x.shape)


def scale_quantize(x: torch.Tensor, granularity: Granularity = "bh",
                   layout: Literal["bhsd", "bhds"] = "bhsd") -> tuple[torch.Tensor, torch.Tensor]:
    """(dequant scales, codes) in one stream-ordered call (amax, scale, apply)."""
    dt = _in_dtype("x", x)
    x4 = _as4d(x)
    B, H, S, D, sb, sh, ss = _bhsd_view(x4)
    g = _GRAN[granularity]
    dq = torch.empty(B * H if granularity == "bh" else 1, dtype=torch.float32, device=x.device)
    if layout == "bhsd":
        codes = torch.empty((B, H, S, D), dtype=torch.uint8, device=x.device)
        lay, ld = C.RP_LAYOUT_BHSD, 0
    else:
        ld = _round_up(S, V_PAD)
        codes = torch.empty((B, H, D, ld), dtype=torch.uint8, device=x.device)
        lay = C.RP_LAYOUT_BHDS
    ws_bytes = C.lib().rp_fp8_quant_workspace_bytes(B, H, S, D, g)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=x.device)
    C.check(C.lib().rp_fp8_scale_quantize(x4.data_ptr(), dt, B, H, S, D, sb, sh, ss, g,
                                          dq.data_ptr(), codes.data_ptr(), lay, ld,
                                          ws.data_ptr(), ws.numel(), _stream(x)),
            "rp_fp8_scale_quantize")
    codes = codes.view(torch.float8_e4m3fn)
    if x.dim() != 4 and layout == "bhsd":
        codes = codes.reshape(x.shape)
    return dq, codes


@functools.lru_cache(maxsize=256)
def _qkv_ws_bytes(B: int, H: int, Sq: int, Skv: int, D: int, g: int) -> int:
    return int(C.lib().rp_fp8_quant_qkv_workspace_bytes(B, H, Sq, Skv, D, g))


def _align(n: int, a: int = 256) -> int:
    return (n + a - 1) // a * a


def scale_quantize_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                       granularity: Granularity = "bh", *, stream: int | None = None
                       ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                                  torch.Tensor, torch.Tensor]:
    """(q_scale, q8, k_scale, k8, v_scale, vt8) of one attention call from one
    library call (rp_fp8_scale_quantize_qkv: four kernel launches instead of
    nine) into one device allocation: the same scales and codes as three
    ``scale_quantize`` calls (V transposed, "bhds"), with a fraction of the
    host work, which is what bounds small calls.  (B, H, S, D) inputs, bf16 or
    fp16, any strides with a contiguous head dim; K and V share their shape."""
    arena, (o_k, o_v, o_s), G, ldv = _qkv_arena(q, k, v, granularity, stream)
    B, H, Sq, D = q.shape
    Skv = k.shape[2]
    nq, nk, nv = B * H * Sq * D, B * H * Skv * D, B * H * D * ldv
    dq = arena[o_s:o_s + 3 * G * 4].view(torch.float32)
    q8 = arena[:nq].view(B, H, Sq, D).view(torch.float8_e4m3fn)
    k8 = arena[o_k:o_k + nk].view(B, H, Skv, D).view(torch.float8_e4m3fn)
    vt8 = arena[o_v:o_v + nv].view(B, H, D, ldv).view(torch.float8_e4m3fn)
    return dq[:G], q8, dq[G:2 * G], k8, dq[2 * G:], vt8


def _qkv_arena(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, granularity: Granularity,
               stream: int | None, q_codes: bool = True, dtype_code: int | None = None
               ) -> tuple[torch.Tensor, tuple[int, int, int], int, int]:
    """The quantizer call of ``scale_quantize_qkv`` into one uint8 arena:
    (arena, (byte offsets of k8, vt8 and the 3G fp32 scales; q8 at 0), G =
    scales per tensor, ldv).  ``fp8_flash_attention`` launches from the
    arena's pointers without building tensor views.  ``q_codes=False``
    computes Q's scale without its codes (the arena then starts with k8),
    for the attention launch that quantizes Q itself.
    (``dtype_code``: the caller has checked q, k and v for one supported
    dtype, this RP_DTYPE_* code.)"""
    if dtype_code is None:
        dt = _in_dtype("q", q)
        for name, t in (("k", k), ("v", v)):
            if _in_dtype(name, t) != dt:
                raise TypeError(f"q, k, v dtypes differ ({q.dtype}, {k.dtype}, {v.dtype})")
    else:
        dt = dtype_code
    B, H, Sq, D, qsb, qsh, qss = _bhsd_view(q)
    _, _, Skv, _, ksb, ksh, kss = _bhsd_view(k)
    _, _, _, _, vsb, vsh, vss = _bhsd_view(v)
    if k.shape[:2] != q.shape[:2] or k.shape[3] != D or v.shape != k.shape:
        raise ValueError(f"k and v must share one (B, H, Skv, D) shape with q's B, H and D "
                         f"(q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)})")
    _on_device_of(q, k=k, v=v)
    g = _GRAN[granularity]
    G = B * H if granularity == "bh" else 1
    ldv = _round_up(Skv, V_PAD)
    nq, nk, nv = B * H * Sq * D, B * H * Skv * D, B * H * D * ldv
    ws = _qkv_ws_bytes(B, H, Sq, Skv, D, g)
    o_k = _align(nq) if q_codes else 0
    o_v = o_k + _align(nk)
    o_s = o_v + _align(nv)
    o_w = o_s + _align(3 * G * 4)
    arena = torch.empty(o_w + max(ws, 16), dtype=torch.uint8, device=q.device)
    base = arena.data_ptr()
    C.check(C.lib().rp_fp8_scale_quantize_qkv(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), dt, B, H, Sq, Skv, D, qsb, qsh, qss,
        ksb, ksh, kss, vsb, vsh, vss, g, base + o_s, base if q_codes else None, base + o_k,
        base + o_v, ldv, base + o_w, ws, _stream(q) if stream is None else stream),
        "rp_fp8_scale_quantize_qkv")
    return arena, (o_k, o_v, o_s), G, ldv


_ROPE = {None: C.RP_ROPE_NONE, "half": C.RP_ROPE_HALF, "interleaved": C.RP_ROPE_INTERLEAVED}


def _norm_operands(x: torch.Tensor, weight: torch.Tensor | None,
                   rope: tuple[torch.Tensor, torch.Tensor] | None
                   ) -> tuple[int | None, int | None, int | None]:
    """Device pointers of a prologue's weight and cos/sin tables (None when
    absent), checked against x's (B, H, S, D) shape."""
    _, _, S, D = x.shape
    w_ptr = cos_ptr = sin_ptr = None
    if weight is not None:
        _check_bf16("weight", weight)
        _on_device_of(x, weight=weight)
        if weight.shape != (D,) or not weight.is_contiguous():
            raise ValueError(f"weight must be a contiguous ({D},) bf16 vector")
        w_ptr = weight.data_ptr()
    if rope is not None:
        cos, sin = rope
        _on_device_of(x, cos=cos, sin=sin)
        for name, t in (("cos", cos), ("sin", sin)):
            if t.dtype != torch.float32 or t.shape != (S, D) or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous float32 ({S}, {D}) table")
        cos_ptr, sin_ptr = cos.data_ptr(), sin.data_ptr()
    return w_ptr, cos_ptr, sin_ptr


def rmsnorm_scale_quantize(x: torch.Tensor, weight: torch.Tensor | None = None,
                           eps: float = 1e-6,
                           rope: tuple[torch.Tensor, torch.Tensor] | None = None,
                           rope_layout: Literal["half", "interleaved"] = "half",
                           granularity: Granularity = "bh") -> tuple[torch.Tensor, torch.Tensor]:
    """(dequant scales, BHSD codes) of RMSNorm(x) [* weight] [rotated], fused.

    The attention processors' ``norm_q``/``norm_k`` (RMSNorm over the head
    dim, fp32 math; reference docs/walkthroughs/02-architecture.md:114-123)
    and, with ``rope = (cos, sin)`` fp32 (S, D) tables, diffusers'
    ``apply_rotary_emb(use_real=True)`` ("half" pairs d with d +- D/2, as
    ``use_real_unbind_dim=-2``; "interleaved" pairs 2k with 2k+1), computed
    inside the quantizer's two passes: the normalised tensor never reaches
    HBM.  ``x`` is (B, H, S, D) bf16 with a unit stride on D.
    """
    _check_bf16("x", x)
    if x.dim() != 4:
        raise ValueError("x must be (B, H, S, D)")
    B, H, S, D, sb, sh, ss = _bhsd_view(x)
    w_ptr, cos_ptr, sin_ptr = _norm_operands(x, weight, rope)
    mode = _ROPE[rope_layout if rope is not None else None]
    g = _GRAN[granularity]
    dq = torch.empty(B * H if granularity == "bh" else 1, dtype=torch.float32, device=x.device)
    codes = torch.empty((B, H, S, D), dtype=torch.uint8, device=x.device)
    ws_bytes = C.lib().rp_fp8_rmsnorm_quant_workspace_bytes(B, H, S, D, g)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=x.device)
    C.check(C.lib().rp_fp8_rmsnorm_scale_quantize(
        x.data_ptr(), B, H, S, D, sb, sh, ss, w_ptr, float(eps), cos_ptr, sin_ptr, mode, g,
        dq.data_ptr(), codes.data_ptr(), ws.data_ptr(), ws.numel(), _stream(x)),
        "rp_fp8_rmsnorm_scale_quantize")
    return dq, codes.view(torch.float8_e4m3fn)


def rmsnorm_scale_quantize_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
                               norm_q_weight: torch.Tensor | None = None,
                               norm_k_weight: torch.Tensor | None = None, eps: float = 1e-6,
                               rope_q: tuple[torch.Tensor, torch.Tensor] | None = None,
                               rope_k: tuple[torch.Tensor, torch.Tensor] | None = None,
                               rope_layout: Literal["half", "interleaved"] = "half",
                               granularity: Granularity = "bh"
                               ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                                          torch.Tensor, torch.Tensor]:
    """(q_scale, q8, k_scale, k8, v_scale, vt8) of one attention call with the
    QK-norm prologue, from one library call (rp_fp8_rmsnorm_scale_quantize_qkv:
    three kernel launches instead of nine) into one device allocation: the
    same scales and codes as ``rmsnorm_scale_quantize`` of Q and of K and
    ``scale_quantize(v, granularity, "bhds")``.  (B, H, S, D) bf16 inputs
    with a unit stride on D; K and V share their shape; rotary tables for
    both Q and K or for neither."""
    for name, t in (("q", q), ("k", k), ("v", v)):
        _check_bf16(name, t)
    B, H, Sq, D, qsb, qsh, qss = _bhsd_view(q)
    _, _, Skv, _, ksb, ksh, kss = _bhsd_view(k)
    _, _, _, _, vsb, vsh, vss = _bhsd_view(v)
    if k.shape[:2] != q.shape[:2] or k.shape[3] != D or v.shape != k.shape:
        raise ValueError(f"k and v must share one (B, H, Skv, D) shape with q's B, H and D "
                         f"(q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)})")
    if (rope_q is None) != (rope_k is None):
        raise ValueError("rotary tables must be given for both q and k or for neither")
    _on_device_of(q, k=k, v=v)
    qw, qc, qsn = _norm_operands(q, norm_q_weight, rope_q)
    kw, kc, ksn = _norm_operands(k, norm_k_weight, rope_k)
    mode = _ROPE[rope_layout if rope_q is not None else None]
    g = _GRAN[granularity]
    G = B * H if granularity == "bh" else 1
    ldv = _round_up(Skv, V_PAD)
    nq, nk, nv = B * H * Sq * D, B * H * Skv * D, B * H * D * ldv
    ws = int(C.lib().rp_fp8_rmsnorm_quant_qkv_workspace_bytes(B, H, Sq, Skv, D, g))
    o_k = _align(nq)
    o_v = o_k + _align(nk)
    o_s = o_v + _align(nv)
    o_w = o_s + _align(3 * G * 4)
    arena = torch.empty(o_w + max(ws, 16), dtype=torch.uint8, device=q.device)
    base = arena.data_ptr()
    C.check(C.lib().rp_fp8_rmsnorm_scale_quantize_qkv(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), B, H, Sq, Skv, D, qsb, qsh, qss, ksb, ksh, kss,
        vsb, vsh, vss, qw, kw, float(eps), qc, qsn, kc, ksn, mode, g, base + o_s, base,
        base + o_k, base + o_v, ldv, base + o_w, ws, _stream(q)),
        "rp_fp8_rmsnorm_scale_quantize_qkv")
    dq = arena[o_s:o_s + 3 * G * 4].view(torch.float32)
    q8 = arena[:nq].view(B, H, Sq, D).view(torch.float8_e4m3fn)
    k8 = arena[o_k:o_k + nk].view(B, H, Skv, D).view(torch.float8_e4m3fn)
    vt8 = arena[o_v:o_v + nv].view(B, H, D, ldv).view(torch.float8_e4m3fn)
    return dq[:G], q8, dq[G:2 * G], k8, dq[2 * G:], vt8


def fp8_flash_attention_qknorm(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
                               norm_q_weight: torch.Tensor | None = None,
                               norm_k_weight: torch.Tensor | None = None, eps: float = 1e-6,
                               rope_q: tuple[torch.Tensor, torch.Tensor] | None = None,
                               rope_k: tuple[torch.Tensor, torch.Tensor] | None = None,
                               rope_layout: Literal["half", "interleaved"] = "half",
                               causal: bool = False, scale: float | None = None,
                               granularity: Granularity = "bh", out: torch.Tensor | None = None,
                               out_dtype: torch.dtype | None = None,
                               kv_splits: int | None = None) -> torch.Tensor:
    """``fp8_flash_attention`` on pre-norm Q and K: the attention processor's
    QK-RMSNorm (and rotary embedding) runs fused into Q's and K's quantizers,
    and V's quantizer shares their launches (``rmsnorm_scale_quantize_qkv``).  Same result as
    normalising (and rotating) Q and K in torch first, up to the summation
    order of the RMSNorm's mean (see rp_prologue.hip)."""
    for name, t in (("q", q), ("k", k), ("v", v)):
        _check_bf16(name, t)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be 4-D (B, H, S, D)")
    B, H, Sq, D = q.shape
    if k.shape != v.shape or k.shape[0] != B or k.shape[1] != H or k.shape[3] != D:
        raise ValueError(f"shape mismatch: q {tuple(q.shape)}, k {tuple(k.shape)}, "
                         f"v {tuple(v.shape)}")
    if D not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"head_dim {D} not in compiled tile shapes {sorted(SUPPORTED_HEAD_DIMS)}")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if (rope_q is None) == (rope_k is None):
        qs, q8, ks, k8, vs, vt8 = rmsnorm_scale_quantize_qkv(
            q, k, v, norm_q_weight=norm_q_weight, norm_k_weight=norm_k_weight, eps=eps,
            rope_q=rope_q, rope_k=rope_k, rope_layout=rope_layout, granularity=granularity)
    else:   # rotary tables for one of Q and K only
        qs, q8 = rmsnorm_scale_quantize(q, norm_q_weight, eps, rope_q, rope_layout, granularity)
        ks, k8 = rmsnorm_scale_quantize(k, norm_k_weight, eps, rope_k, rope_layout, granularity)
        vs, vt8 = scale_quantize(v, granularity, "bhds")
    Skv = k.shape[2]
    block_m = BLOCK_M
    if kv_splits is None:
        block_m, kv_splits = tuned_launch(B, H, Sq, Skv, D, causal)
    return attention_fp8(q8.view(torch.uint8), k8.view(torch.uint8), vt8.view(torch.uint8),
                         qs, ks, vs, scale, out=out, out_dtype=out_dtype or q.dtype,
                         causal=causal, kv_splits=kv_splits, block_m=block_m)


def _round_up(v: int, m: int) -> int:
    return (v + m - 1) // m * m


def attention_fp8(q8: torch.Tensor, k8: torch.Tensor, vt8: torch.Tensor, q_scale: torch.Tensor,
                  k_scale: torch.Tensor, v_scale: torch.Tensor, sm_scale: float, *,
                  out: torch.Tensor | None = None, out_dtype: torch.dtype = torch.bfloat16,
                  causal: bool = False, prefix_len: int | None = None,
                  suffix_len: int | None = None, kv_splits: int = 1,
                  block_m: int = BLOCK_M) -> torch.Tensor:
    """FP8 attention on already-quantized operands.

    q8 (B, H, Sq, D), k8 (B, H, Skv, D) contiguous codes; vt8 (B, H, D, ldv)
    transposed V codes; scales of length B*H (per head) or 1 (per tensor).
    ``out`` may be any (B, H, Sq, D)-shaped view with a contiguous last dim
    (e.g. a permuted (B, S, H, D) buffer).  ``prefix_len``/``suffix_len``
    select the shared-prefix candidate mask.  ``kv_splits`` > 1 runs the key
    range in that many parts and merges them (``rp_fp8_attn_fwd_split``);
    0 runs the balanced launch (``rp_fp8_attn_fwd_balanced``): the query
    blocks that fill whole rounds of workgroups over one key range, the rest
    key-split.  ``block_m`` 32, 64 or 128 (head dims 64 and 128) runs the
    short-query launch (``rp_fp8_attn_fwd_wsplit``): that many query rows per
    workgroup, the keys split over its waves and merged in the same launch;
    ``kv_splits`` must then be left at 1.
    """
    _check_cuda("q8", q8)
    _on_device_of(q8, k8=k8, vt8=vt8, q_scale=q_scale, k_scale=k_scale, v_scale=v_scale,
                  out=out)
    for name, t in (("q8", q8), ("k8", k8), ("vt8", vt8)):
        if t.dtype not in (torch.float8_e4m3fn, torch.uint8):
            raise TypeError(f"{name} must hold e4m3fn codes (float8_e4m3fn or uint8), got {t.dtype}")
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    B, H, Sq, D = q8.shape
    Skv = k8.shape[2]
    if k8.shape != (B, H, Skv, D) or vt8.shape[:3] != (B, H, D):
        raise ValueError(f"operand shapes disagree: q8 {tuple(q8.shape)}, k8 {tuple(k8.shape)}, "
                         f"vt8 {tuple(vt8.shape)}")
    ldv = vt8.shape[3]
    n = q_scale.numel()
    if not (n == k_scale.numel() == v_scale.numel()) or n not in (1, B * H):
        raise ValueError("scales must all have B*H or 1 elements")
    stride = 1 if n == B * H and B * H > 1 else 0
    if out is None:
        out = torch.empty((B, H, Sq, D), dtype=out_dtype, device=q8.device)
    if out.shape != (B, H, Sq, D) or out.stride(3) != 1:
        raise ValueError("out must be (B, H, Sq, D) with a contiguous last dimension")
    odt = _OUT_DTYPES.get(out.dtype)
    if odt is None:
        raise TypeError(f"out dtype {out.dtype} not supported (bfloat16, float16 or float32)")
    if prefix_len is not None:
        mask, pre, suf = C.RP_MASK_SHARED_PREFIX, int(prefix_len), int(suffix_len or 0)
    else:
        mask, pre, suf = (C.RP_MASK_CAUSAL if causal else C.RP_MASK_NONE), 0, 1
    qs = q_scale.to(torch.float32).contiguous()
    ks = k_scale.to(torch.float32).contiguous()
    vs = v_scale.to(torch.float32).contiguous()
    args = (q8.data_ptr(), k8.data_ptr(), vt8.data_ptr(), ldv, qs.data_ptr(), ks.data_ptr(),
            vs.data_ptr(), stride, float(sm_scale), out.data_ptr(), odt, out.stride(0),
            out.stride(1), out.stride(2), B, H, Sq, Skv, D, mask, pre, suf)
    _launch_attention(args, kv_splits, block_m, q8.device, _stream(q8))
    return out


def _launch_attention(args: tuple, kv_splits: int, block_m: int, device: torch.device,
                      stream: int) -> None:
    """The attention launch of ``attention_fp8`` on checked arguments (the
    common leading arguments of the rp_fp8_attn_fwd* entry points)."""
    if kv_splits < 0:
        raise ValueError(f"kv_splits={kv_splits} must be >= 0")
    L = C.lib()
    if block_m != BLOCK_M:
        if block_m not in WSPLIT_BLOCK_MS or kv_splits != 1:
            raise ValueError(f"block_m={block_m} (kv_splits={kv_splits}): the short-query launch "
                             f"takes block_m in {WSPLIT_BLOCK_MS} and kv_splits=1")
        C.check(L.rp_fp8_attn_fwd_wsplit(*args, int(block_m), stream), "rp_fp8_attn_fwd_wsplit")
    elif kv_splits == 1:
        C.check(L.rp_fp8_attn_fwd(*args, stream), "rp_fp8_attn_fwd")
    elif kv_splits == 0:
        # whole rounds of workgroups over one key range, the query blocks of
        # the last partial round key-split so that they fill the GPU
        B, H, Sq, Skv, D, mask = args[14], args[15], args[16], args[17], args[18], args[19]
        nbytes = L.rp_fp8_attn_balanced_workspace_bytes(B, H, Sq, Skv, D, mask, stream)
        ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
        C.check(L.rp_fp8_attn_fwd_balanced(*args, ws.data_ptr(), ws.numel(), stream),
                "rp_fp8_attn_fwd_balanced")
    else:
        B, H, Sq, D = args[14], args[15], args[16], args[18]
        nbytes = L.rp_fp8_attn_workspace_bytes(B, H, Sq, D, int(kv_splits))
        ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
        C.check(L.rp_fp8_attn_fwd_split(*args, int(kv_splits), ws.data_ptr(), ws.numel(),
                                         stream), "rp_fp8_attn_fwd_split")


def fp8_flash_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
                        causal: bool = False, scale: float | None = None,
                        granularity: Granularity = "bh", out: torch.Tensor | None = None,
                        out_dtype: torch.dtype | None = None, prefix_len: int | None = None,
                        suffix_len: int | None = None, kv_splits: int | None = None
                        ) -> torch.Tensor:
    """Fused FP8 flash attention, (B, H, S, D) bf16 or fp16 in, (B, H, Sq, D) out.

    Mirrors the reference's ``fp8_flash_attention``
    (kernels/triton_kernels/fp8_flash_attn.py:480-645): quantize Q/K/V with
    per-(B, H) amax scales, run the FA-2 FP8 kernel with softmax temperature
    ``scale`` (default 1/sqrt(D)), return the result in q's dtype.  Unlike
    the reference, K/V may have a different sequence length than Q
    (cross-attention), inputs may be strided (e.g. permuted (B, S, H, D)
    views -- no copies are made), and the output is written directly in
    q's dtype (or into ``out``) rather than cast from fp32.

    The launch configuration resolves as in the reference (:482-499):
    ``kv_splits`` if given; else the fallback when
    ``REPERCEP_FP8_DISABLE_AUTOTUNE`` is set; else the on-disk cache entry for
    the shape; else a timed search over ``tuning.candidate_configs`` whose
    winner is recorded (see ``repercep_runtime_amd.tuning``).
    """
    dt = _in_dtype("q", q)
    _in_dtype("k", k)
    _in_dtype("v", v)
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError(f"q, k, v dtypes differ ({q.dtype}, {k.dtype}, {v.dtype})")
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be 4-D (B, H, S, D)")
    B, H, Sq, D = q.shape
    if k.shape != v.shape or k.shape[0] != B or k.shape[1] != H or k.shape[3] != D:
        raise ValueError(f"shape mismatch: q {tuple(q.shape)}, k {tuple(k.shape)}, "
                         f"v {tuple(v.shape)}")
    if D not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"head_dim {D} not in compiled tile shapes {sorted(SUPPORTED_HEAD_DIMS)}")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    st = _stream(q)
    Skv = k.shape[2]
    if out is None:
        out = torch.empty((B, H, Sq, D), dtype=out_dtype or q.dtype, device=q.device)
    else:
        _on_device_of(q, out=out)
    if out.shape != (B, H, Sq, D) or out.stride(3) != 1:
        raise ValueError("out must be (B, H, Sq, D) with a contiguous last dimension")
    odt = _OUT_DTYPES.get(out.dtype)
    if odt is None:
        raise TypeError(f"out dtype {out.dtype} not supported (bfloat16, float16 or float32)")
    if prefix_len is not None:
        mask, pre, suf = C.RP_MASK_SHARED_PREFIX, int(prefix_len), int(suffix_len or 0)
    else:
        mask, pre, suf = (C.RP_MASK_CAUSAL if causal else C.RP_MASK_NONE), 0, 1
    # a resident-K/V launch known without a timed search quantizes Q itself:
    # Q is read as it lies instead of written as codes and read back
    if kv_splits is not None:
        known = {"KV_SPLITS": int(kv_splits)}
    else:
        known = _known_launch(B, H, Sq, Skv, D, causal, prefix_len, suffix_len)
    if known is not None:
        block_m, splits = launch_of(known)
        if (block_m == BLOCK_M and q.data_ptr() % 16 == 0
                and all(x % 8 == 0 for x in q.stride()[:3]) and q.stride(3) == 1
                and q16_pays(B, H, Sq, Skv, D, mask, splits, st)):
            _qkv_q16_attention(q, k, v, granularity, st, out, odt, float(scale), mask, pre, suf,
                               splits)
            return out
    arena, (o_k, o_v, o_s), G, ldv = _qkv_arena(q, k, v, granularity, st, dtype_code=dt)
    base = arena.data_ptr()
    # the quantizer's own outputs in the arena: contiguous codes, fp32
    # scales, one per head or one per tensor
    stride = 1 if G == B * H and B * H > 1 else 0
    args = (base, base + o_k, base + o_v, ldv, base + o_s, base + o_s + 4 * G,
            base + o_s + 8 * G, stride, float(scale), out.data_ptr(), odt,
            out.stride(0), out.stride(1), out.stride(2), B, H, Sq, Skv, D, mask, pre, suf)

    def run(cfg: dict) -> torch.Tensor:
        block_m, splits = launch_of(cfg)
        # the arena stays referenced while the launches are queued
        _launch_attention(args, splits, block_m, arena.device, st)
        return out

    if known is not None:
        return run(known)
    return run(_resolve_launch(B, H, Sq, Skv, D, causal, prefix_len, suffix_len, run))


def _known_launch(B: int, H: int, Sq: int, Skv: int, D: int, causal: bool,
                  prefix_len: int | None, suffix_len: int | None) -> dict | None:
    """The launch configuration ``_resolve_launch`` returns for a shape when
    it needs no timed search (autotuning off, or a cached entry), else None."""
    if tuning.autotune_disabled():
        return dict(tuning.FALLBACK_CONFIG)
    cfg = tuning.resolve_config(B, H, Sq, Skv, D, causal, prefix_len, suffix_len)
    return cfg or None


def scale_quantize_kv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                      granularity: Granularity = "bh"
                      ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                                 torch.Tensor]:
    """(q_scale, k_scale, k8, v_scale, vt8): ``scale_quantize_qkv`` without
    Q's codes (rp_fp8_scale_quantize_qkv with q8 = NULL), for
    ``attention_fp8_q16``, which quantizes Q's rows itself."""
    arena, (o_k, o_v, o_s), G, ldv = _qkv_arena(q, k, v, granularity, None, q_codes=False)
    B, H, _, D = q.shape
    Skv = k.shape[2]
    nk, nv = B * H * Skv * D, B * H * D * ldv
    dq = arena[o_s:o_s + 3 * G * 4].view(torch.float32)
    k8 = arena[o_k:o_k + nk].view(B, H, Skv, D).view(torch.float8_e4m3fn)
    vt8 = arena[o_v:o_v + nv].view(B, H, D, ldv).view(torch.float8_e4m3fn)
    return dq[:G], dq[G:2 * G], k8, dq[2 * G:], vt8


def q16_pays(B: int, H: int, Sq: int, Skv: int, D: int, mask: int, kv_splits: int,
             stream: int) -> bool:
    """Whether ``fp8_flash_attention`` hands this launch Q as it lies: the
    resident-K/V launch (one key range).  Its step (Q's amax, K/V codes,
    attention) measured 0.94-0.95 -> 0.86 ms at C3 cross, the attention kernel
    0.54 -> 0.63 ms with Q's quantization inside it; the self-attention
    launches are VALU-bound through many more key tiles per Q row and gained
    nothing (C3 self: quantize 0.92 -> 0.73 ms, attention +0.15-0.25 ms)."""
    if kv_splits not in (0, 1):
        return False
    L = C.lib()
    return bool(L.rp_fp8_attn_resident_kv(B, H, Sq, Skv, D, mask, 1)
                and L.rp_fp8_attn_q16_supported(B, H, Sq, Skv, D, mask, kv_splits, stream))


def attention_q16_supported(B: int, H: int, Sq: int, Skv: int, D: int, causal: bool = False,
                            prefix_len: int | None = None, kv_splits: int = 1) -> bool:
    """Whether ``attention_fp8_q16`` runs this shape with ``kv_splits``
    (rp_fp8_attn_q16_supported: every launch but the multi-block one)."""
    mask = (C.RP_MASK_SHARED_PREFIX if prefix_len is not None
            else C.RP_MASK_CAUSAL if causal else C.RP_MASK_NONE)
    return bool(C.lib().rp_fp8_attn_q16_supported(B, H, Sq, Skv, D, mask, int(kv_splits),
                                                    torch.cuda.current_stream().cuda_stream))


def attention_fp8_q16(q: torch.Tensor, k8: torch.Tensor, vt8: torch.Tensor,
                      q_scale: torch.Tensor, k_scale: torch.Tensor, v_scale: torch.Tensor,
                      sm_scale: float, *, out: torch.Tensor | None = None,
                      out_dtype: torch.dtype | None = None, causal: bool = False,
                      prefix_len: int | None = None, suffix_len: int | None = None,
                      kv_splits: int = 1) -> torch.Tensor:
    """``attention_fp8`` with Q as its bf16/fp16 (B, H, Sq, D) input
    (any 16-byte aligned strides, contiguous head dim) and its scale(s):
    each workgroup quantizes the Q rows it reads with the quantizer's
    arithmetic (rp_fp8_attn_fwd_q16), so the output equals
    ``attention_fp8`` on ``scale_quantize_qkv``'s codes bit for bit.
    ``kv_splits`` 0 (balanced), 1 or more; no short-query launch."""
    qdt = _in_dtype("q", q)
    _on_device_of(q, k8=k8, vt8=vt8, q_scale=q_scale, k_scale=k_scale, v_scale=v_scale,
                  out=out)
    B, H, Sq, D, qsb, qsh, qss = _bhsd_view(q)
    for name, t in (("k8", k8), ("vt8", vt8)):
        if t.dtype not in (torch.float8_e4m3fn, torch.uint8) or not t.is_contiguous():
            raise ValueError(f"{name} must hold contiguous e4m3fn codes")
    Skv = k8.shape[2]
    if k8.shape != (B, H, Skv, D) or vt8.shape[:3] != (B, H, D):
        raise ValueError(f"operand shapes disagree: q {tuple(q.shape)}, k8 {tuple(k8.shape)}, "
                         f"vt8 {tuple(vt8.shape)}")
    n = q_scale.numel()
    if not (n == k_scale.numel() == v_scale.numel()) or n not in (1, B * H):
        raise ValueError("scales must all have B*H or 1 elements")
    if kv_splits < 0:
        raise ValueError(f"kv_splits={kv_splits} must be >= 0")
    stride = 1 if n == B * H and B * H > 1 else 0
    if out is None:
        out = torch.empty((B, H, Sq, D), dtype=out_dtype or q.dtype, device=q.device)
    if out.shape != (B, H, Sq, D) or out.stride(3) != 1:
        raise ValueError("out must be (B, H, Sq, D) with a contiguous last dimension")
    odt = _OUT_DTYPES.get(out.dtype)
    if odt is None:
        raise TypeError(f"out dtype {out.dtype} not supported (bfloat16, float16 or float32)")
    if prefix_len is not None:
        mask, pre, suf = C.RP_MASK_SHARED_PREFIX, int(prefix_len), int(suffix_len or 0)
    else:
        mask, pre, suf = (C.RP_MASK_CAUSAL if causal else C.RP_MASK_NONE), 0, 1
    qs = q_scale.to(torch.float32).contiguous()
    ks = k_scale.to(torch.float32).contiguous()
    vs = v_scale.to(torch.float32).contiguous()
    st = _stream(q)
    L = C.lib()
    if kv_splits == 0:
        nbytes = L.rp_fp8_attn_balanced_workspace_bytes(B, H, Sq, Skv, D, mask, st)
    else:
        nbytes = L.rp_fp8_attn_workspace_bytes(B, H, Sq, D, kv_splits) if kv_splits > 1 else 0
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=q.device)
    C.check(L.rp_fp8_attn_fwd_q16(
        q.data_ptr(), qdt, qsb, qsh, qss, k8.data_ptr(), vt8.data_ptr(), vt8.shape[3],
        qs.data_ptr(), ks.data_ptr(), vs.data_ptr(), stride, float(sm_scale), out.data_ptr(),
        odt, out.stride(0), out.stride(1), out.stride(2), B, H, Sq, Skv, D, mask, pre, suf,
        int(kv_splits), ws.data_ptr(), ws.numel(), st), "rp_fp8_attn_fwd_q16")
    return out


def _qkv_q16_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                       granularity: Granularity, st: int, out: torch.Tensor, odt: int,
                       scale: float, mask: int, pre: int, suf: int, kv_splits: int) -> None:
    """Scales of Q, K and V with K's and V^T's codes (rp_fp8_scale_quantize_qkv
    with no Q codes), then the attention that quantizes Q's rows itself
    (rp_fp8_attn_fwd_q16): the same codes and output as the two-step path."""
    B, H, Sq, D = q.shape
    Skv = k.shape[2]
    arena, (o_k, o_v, o_s), G, ldv = _qkv_arena(q, k, v, granularity, st, q_codes=False)
    base = arena.data_ptr()
    stride = 1 if G == B * H and B * H > 1 else 0
    L = C.lib()
    if kv_splits == 0:
        nbytes = L.rp_fp8_attn_balanced_workspace_bytes(B, H, Sq, Skv, D, mask, st)
    else:
        nbytes = L.rp_fp8_attn_workspace_bytes(B, H, Sq, D, kv_splits) if kv_splits > 1 else 0
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=q.device)
    qsb, qsh, qss, _ = q.stride()
    C.check(L.rp_fp8_attn_fwd_q16(
        q.data_ptr(), _IN_DTYPES[q.dtype], qsb, qsh, qss, base + o_k, base + o_v, ldv,
        base + o_s, base + o_s + 4 * G, base + o_s + 8 * G, stride, scale, out.data_ptr(), odt,
        out.stride(0), out.stride(1), out.stride(2), B, H, Sq, Skv, D, mask, pre, suf,
        kv_splits, ws.data_ptr(), ws.numel(), st), "rp_fp8_attn_fwd_q16")


def _time_call(fn: Callable[[], object], reps: int = 10, rounds: int = 3) -> float:
    """Seconds per call on the current stream: the best of ``rounds`` runs of
    ``reps`` back-to-back calls (after one warmup), so that launch overhead
    overlaps the GPU work it precedes."""
    fn()
    best = math.inf
    for _ in range(rounds):
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(reps):
            fn()
        t1.record()
        t1.synchronize()
        best = min(best, t0.elapsed_time(t1) * 1e-3 / reps)
    return best


def launch_of(cfg: dict) -> tuple[int, int]:
    """(block_m, kv_splits) ``attention_fp8`` runs for a launch configuration:
    a ``BLOCK_M`` below 256 selects the short-query launch, whose split
    count follows from its shape (``KV_SPLITS`` in such an entry only
    records it)."""
    block_m = int(cfg.get("BLOCK_M", BLOCK_M))
    if block_m != BLOCK_M:
        return block_m, 1
    return block_m, int(cfg.get("KV_SPLITS", 1))


def tuned_launch(B: int, H: int, Sq: int, Skv: int, D: int, causal: bool = False,
                 prefix_len: int | None = None, suffix_len: int | None = None
                 ) -> tuple[int, int]:
    """The (block_m, kv_splits) ``fp8_flash_attention`` uses for a shape
    without searching: the fallback when autotuning is disabled, else the
    cached entry; on a miss the one candidate of a shape that needs no search
    (the balanced launch of a large grid), else the fallback."""
    if tuning.autotune_disabled():
        return launch_of(tuning.FALLBACK_CONFIG)
    cfg = tuning.resolve_config(B, H, Sq, Skv, D, causal, prefix_len, suffix_len)
    if cfg:
        return launch_of(cfg)
    cands = tuning.candidate_configs(B, H, Sq, Skv, D=D)
    return launch_of(cands[0] if len(cands) == 1 else tuning.FALLBACK_CONFIG)


def tuned_kv_splits(B: int, H: int, Sq: int, Skv: int, D: int, causal: bool = False,
                    prefix_len: int | None = None, suffix_len: int | None = None) -> int:
    """The key split count of ``tuned_launch`` (1 for a short-query launch,
    whose splits run inside its workgroups)."""
    return tuned_launch(B, H, Sq, Skv, D, causal, prefix_len, suffix_len)[1]


def _resolve_launch(B: int, H: int, Sq: int, Skv: int, D: int, causal: bool,
                    prefix_len: int | None, suffix_len: int | None,
                    run: Callable[[dict], torch.Tensor]) -> dict:
    """Launch configuration for a shape: fallback, cache, or timed search."""
    if tuning.autotune_disabled():
        return dict(tuning.FALLBACK_CONFIG)
    cfg = tuning.resolve_config(B, H, Sq, Skv, D, causal, prefix_len, suffix_len)
    if not cfg:
        cands = tuning.candidate_configs(B, H, Sq, Skv, D=D)
        cfg = tuning.autotune(cands, lambda c: _time_call(lambda: run(c)))
        tuning.record_config(B, H, Sq, Skv, D, causal, cfg, prefix_len, suffix_len)
    return cfg


def transpose_fp8(x8: torch.Tensor) -> torch.Tensor:
    """(R, C) -> (C, R) byte transpose of an FP8 matrix on the GPU."""
    _check_cuda("x8", x8)
    if x8.dim() != 2 or x8.stride(1) != 1:
        raise ValueError("expected a 2-D row-major matrix")
    R, Cc = x8.shape
    out = torch.empty((Cc, R), dtype=torch.uint8, device=x8.device)
    C.check(C.lib().rp_fp8_transpose(x8.data_ptr(), out.data_ptr(), R, Cc, x8.stride(0), R,
                                     _stream(x8)), "rp_fp8_transpose")
    return out.view(x8.dtype) if x8.dtype != torch.uint8 else out


def fp8_gemm(a8: torch.Tensor, b8: torch.Tensor, a_scale: float | torch.Tensor,
             b_scale: float | torch.Tensor, *, b_transposed: bool = False,
             out: torch.Tensor | None = None, bias: torch.Tensor | None = None) -> torch.Tensor:
    """C (M, N) bf16 = bf16(fp32(A8 . B8) * a_scale * b_scale).

    Same contract as the reference's ``fp8_gemm(A, B, a_scale, b_scale)``
    (kernels/hip/fp8_attn/binding.cpp:25-57) with OCP e4m3fn operands: A8 is
    (M, K) row-major and B8 (K, N) row-major, which the kernel stages and
    transposes in LDS itself (``RP_B_KN``: no transpose pass, no copy) -- or,
    with ``b_transposed``, B^T (N, K), the nn.Linear weight layout
    (``RP_B_NK``).  Either operand may be a row-strided view (unit stride
    along its rows, row stride >= the row length; A's and B^T's row strides
    multiples of 16).  Scales may be Python floats or one-element device
    tensors (read on the device, no host sync).  ``bias`` (bf16 [N]) is added
    to the fp32 product before the bf16 rounding (``rp_fp8_linear``, an
    nn.Linear epilogue; the reference GEMM has none).
    """
    _check_cuda("a8", a8)
    _on_device_of(a8, b8=b8, out=out, bias=bias,
                  a_scale=a_scale if isinstance(a_scale, torch.Tensor) else None,
                  b_scale=b_scale if isinstance(b_scale, torch.Tensor) else None)
    if a8.dim() != 2 or b8.dim() != 2:
        raise ValueError("A and B must be 2-D")
    for name, t in (("A", a8), ("B", b8)):
        if t.dtype not in (torch.float8_e4m3fn, torch.uint8):
            raise TypeError(f"{name} must be float8_e4m3fn (got {t.dtype})")
        if t.stride(1) != 1 or t.stride(0) < t.shape[1]:
            raise ValueError(f"{name} must have unit column stride and a row stride of at "
                             f"least its row length (got strides {t.stride()})")
    M, K = a8.shape
    if b_transposed:
        N, Kb = b8.shape
        layout = C.RP_B_NK
    else:
        Kb, N = b8.shape
        layout = C.RP_B_KN
    if Kb != K:
        raise ValueError(f"K mismatch: A {tuple(a8.shape)}, B {tuple(b8.shape)}"
                         f"{' (transposed)' if b_transposed else ''}")
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=a8.device)
    else:
        _check_bf16("out", out)
        if out.shape != (M, N) or out.stride(1) != 1:
            raise ValueError(f"out must be a ({M}, {N}) bf16 tensor with unit column stride, "
                             f"got {tuple(out.shape)} strides {out.stride()}")
    a_dev = a_scale.to(torch.float32).contiguous() if isinstance(a_scale, torch.Tensor) else None
    b_dev = b_scale.to(torch.float32).contiguous() if isinstance(b_scale, torch.Tensor) else None
    args = (M, N, K, a8.stride(0), b8.stride(0), out.stride(0),
            0.0 if a_dev is not None else float(a_scale),
            0.0 if b_dev is not None else float(b_scale),
            a_dev.data_ptr() if a_dev is not None else None,
            b_dev.data_ptr() if b_dev is not None else None, _stream(a8))
    if bias is not None:
        _check_bf16("bias", bias)
        if bias.shape != (N,) or not bias.is_contiguous():
            raise ValueError(f"bias must be a contiguous ({N},) tensor, got {tuple(bias.shape)}")
        if bias.data_ptr() % 8 != 0:          # the epilogue reads 4 bias values at a time
            bias = bias.clone()
    # the balanced launch (tiles pooled across XCDs) needs a small workspace
    # for its counter; the outputs are rp_fp8_gemm's / rp_fp8_linear's bits
    ws = torch.empty(C.RP_GEMM_BALANCED_WORKSPACE_BYTES, dtype=torch.uint8, device=a8.device)
    *sizes, stream = args
    C.check(C.lib().rp_fp8_linear_balanced(
        a8.data_ptr(), b8.data_ptr(), layout, bias.data_ptr() if bias is not None else None,
        out.data_ptr(), *sizes, ws.data_ptr(), ws.numel(), stream), "rp_fp8_linear_balanced")
    return out


def fp8_linear_weight(w: torch.Tensor, layout: Literal["nk", "kn"] = "nk"
                      ) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantize a bf16 weight W (K, N) once, per tensor: (dequant scale (1,),
    codes).  ``layout="nk"`` gives the (N, K) operand for
    ``fp8_gemm(..., b_transposed=True)`` -- written transposed by the
    quantizer itself when N % 32 == 0 (a row-strided (N, K) view of its
    128-padded rows), else quantized as it lies and transposed once;
    ``layout="kn"`` gives the (K, N) codes as they lie, for
    ``fp8_gemm(..., b_transposed=False)``."""
    _check_bf16("w", w)
    if w.dim() != 2:
        raise ValueError(f"w must be 2-D (K, N), got {tuple(w.shape)}")
    K, N = w.shape
    if layout == "kn" or N % 32 != 0:
        # one group: the contiguous weight viewed as rows of 8 elements
        if (K * N) % 8 != 0:
            raise ValueError(f"K * N must be a multiple of 8 (got {K} x {N})")
        dq, codes = scale_quantize(w.contiguous().reshape(1, 1, K * N // 8, 8), "tensor", "bhsd")
        codes = codes.view(torch.uint8).reshape(K, N)
        return (dq, codes) if layout == "kn" else (dq, transpose_fp8(codes))
    dq, codes = scale_quantize(w.reshape(1, 1, K, N), "tensor", "bhds")
    # codes: (1, 1, N, ldk) with ldk = K rounded up to 128; the (N, K) view
    return dq, codes.view(torch.uint8)[0, 0, :, :K]


# --------------------------------------------------------------- row-wise FP8
# The reference's unfused FP8 attention (src/repercep/attention/
# fp8_scaled_mm.py:58-221): per-row scales, two scaled grouped GEMMs around a
# bf16 softmax.  Each step is one library call here.

def rowwise_quantize(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(dequant scales x.shape[:-1] fp32, codes x.shape e4m3fn): one scale per
    row of the last axis, as the reference's ``_rowwise_quantize``
    (fp8_scaled_mm.py:107-133) computes it with the OCP constants
    (``rp_fp8_rowwise_quantize``).  ``x`` is bf16 or fp16 with a unit stride
    on its last axis and rows that flatten to one row stride."""
    dt = _in_dtype("x", x)
    if x.dim() < 1 or x.stride(-1) != 1:
        raise ValueError("x needs a unit stride along its last axis")
    cols = x.shape[-1]
    x2 = x.reshape(-1, cols)      # a view whenever the rows share one stride
    rows = x2.shape[0]
    ldx = x2.stride(0) if rows > 1 else cols
    dq = torch.empty(rows, dtype=torch.float32, device=x.device)
    codes = torch.empty((rows, cols), dtype=torch.uint8, device=x.device)
    C.check(C.lib().rp_fp8_rowwise_quantize(x2.data_ptr(), dt, rows, cols, ldx, dq.data_ptr(),
                                            codes.data_ptr(), cols, _stream(x)),
            "rp_fp8_rowwise_quantize")
    return dq.reshape(x.shape[:-1]), codes.view(torch.float8_e4m3fn).reshape(x.shape)


def transpose16(x: torch.Tensor) -> torch.Tensor:
    """(..., R, C) -> contiguous (..., C, R) for a 16-bit tensor (``rp_transpose16``)."""
    _check_cuda("x", x)
    if x.element_size() != 2 or x.dim() < 2:
        raise TypeError("transpose16 takes a 16-bit tensor of at least 2 dims")
    x3 = x.contiguous().reshape(-1, x.shape[-2], x.shape[-1])
    nb, R, Cc = x3.shape
    out = torch.empty((nb, Cc, R), dtype=x.dtype, device=x.device)
    C.check(C.lib().rp_transpose16(x3.data_ptr(), out.data_ptr(), nb, R, Cc, Cc, R, R * Cc,
                                   R * Cc, _stream(x)), "rp_transpose16")
    return out.reshape(*x.shape[:-2], Cc, R)


def gemm_rowwise(a8: torch.Tensor, bt8: torch.Tensor, row_scale: torch.Tensor,
                 col_scale: torch.Tensor) -> torch.Tensor:
    """Batched C (Z, M, N) bf16 = bf16((fp32(A8 . B8) * row_scale[m]) * col_scale[n])
    for A8 (Z, M, K) and B^T (Z, N, K) e4m3fn codes, row_scale (Z, M),
    col_scale (Z, N): the reference's ``torch._scaled_grouped_mm(A, B^T.t(),
    scale_a, scale_b, out_dtype=bf16)`` (fp8_scaled_mm.py:149-157, 172-178),
    on ``rp_fp8_gemm_rowwise``."""
    _check_cuda("a8", a8)
    _on_device_of(a8, bt8=bt8, row_scale=row_scale, col_scale=col_scale)
    if a8.dim() != 3 or bt8.dim() != 3:
        raise ValueError("a8 and bt8 must be (Z, M, K) and (Z, N, K)")
    for name, t in (("a8", a8), ("bt8", bt8)):
        if t.dtype not in (torch.float8_e4m3fn, torch.uint8) or not t.is_contiguous():
            raise TypeError(f"{name} must be contiguous e4m3fn codes")
    Z, M, K = a8.shape
    Zb, N, Kb = bt8.shape
    if Zb != Z or Kb != K:
        raise ValueError(f"shapes disagree: a8 {tuple(a8.shape)}, bt8 {tuple(bt8.shape)}")
    rs = row_scale.to(torch.float32).contiguous()
    cs = col_scale.to(torch.float32).contiguous()
    if rs.shape != (Z, M) or cs.shape != (Z, N):
        raise ValueError(f"row_scale must be ({Z}, {M}) and col_scale ({Z}, {N})")
    if N % 4 != 0:
        raise ValueError(f"N = {N} must be a multiple of 4")
    out = torch.empty((Z, M, N), dtype=torch.bfloat16, device=a8.device)
    C.check(C.lib().rp_fp8_gemm_rowwise(a8.data_ptr(), bt8.data_ptr(), C.RP_B_NK, out.data_ptr(),
                                        M, N, K, K, K, N, rs.data_ptr(), cs.data_ptr(), Z, M * K,
                                        N * K, M * N, M, N, _stream(a8)), "rp_fp8_gemm_rowwise")
    return out


def softmax_rowwise_quantize(scores: torch.Tensor, scale: float, causal: bool = False
                             ) -> tuple[torch.Tensor, torch.Tensor]:
    """(dequant (Z, Sq) fp32, P codes (Z, Sq, Skv) e4m3fn) of
    P = softmax(bf16(scores * scale)) in bf16 (causal: key j visible to query
    q iff j <= q), row-wise quantized -- the reference's ``scores * scale``,
    masked_fill, torch.softmax and ``_rowwise_quantize(p)``
    (fp8_scaled_mm.py:159-171) in one pass per row."""
    _check_bf16("scores", scores)
    if scores.dim() != 3 or not scores.is_contiguous():
        raise ValueError("scores must be a contiguous (Z, Sq, Skv) tensor")
    Z, Sq, Skv = scores.shape
    dq = torch.empty((Z, Sq), dtype=torch.float32, device=scores.device)
    codes = torch.empty((Z, Sq, Skv), dtype=torch.uint8, device=scores.device)
    C.check(C.lib().rp_fp8_softmax_rowwise_quantize(scores.data_ptr(), Z * Sq, Skv, Skv, Sq,
                                                    int(causal), float(scale), dq.data_ptr(),
                                                    codes.data_ptr(), Skv, _stream(scores)),
            "rp_fp8_softmax_rowwise_quantize")
    return dq, codes.view(torch.float8_e4m3fn)


def fp8_scaled_mm_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
                            causal: bool = False, scale: float | None = None) -> torch.Tensor:
    """The unfused FP8 attention of the reference's ``FP8ScaledMMAttention``
    (fp8_scaled_mm.py:135-221) on the gfx950 kernels, (B, H, S, D) bf16 or
    fp16 in, q's dtype out: row-wise Q and K codes, scores = the row-scaled
    FP8 GEMM in bf16, P = softmax(scores * scale) in bf16 with its row-wise
    codes, V^T's row-wise codes (one scale per head-dim index), and the
    row-scaled P.V GEMM.  The (B*H, Sq, Skv) bf16 scores are materialised,
    as in the reference."""
    for name, t in (("q", q), ("k", k), ("v", v)):
        _in_dtype(name, t)
    if q.dim() != 4 or k.shape != v.shape or k.shape[0] != q.shape[0] or \
            k.shape[1] != q.shape[1] or k.shape[3] != q.shape[3]:
        raise ValueError(f"shape mismatch: q {tuple(q.shape)}, k {tuple(k.shape)}, "
                         f"v {tuple(v.shape)}")
    b, h, sq, d = q.shape
    skv = k.shape[2]
    bh = b * h
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    cdt = torch.bfloat16     # the reference computes in bf16 (fp8_scaled_mm.py:146-149)
    qs, q8 = rowwise_quantize(q.to(cdt).reshape(bh, sq, d))
    ks, k8 = rowwise_quantize(k.to(cdt).reshape(bh, skv, d))
    scores = gemm_rowwise(q8.view(torch.uint8), k8.view(torch.uint8), qs, ks)
    ps, p8 = softmax_rowwise_quantize(scores, scale, causal)
    del scores
    vt = transpose16(v.to(cdt).reshape(bh, skv, d))          # (bh, d, skv)
    vs, vt8 = rowwise_quantize(vt)
    out = gemm_rowwise(p8.view(torch.uint8), vt8.view(torch.uint8), ps, vs)
    return out.reshape(b, h, sq, d).to(q.dtype)


def selftest_e4m3(x: torch.Tensor) -> torch.Tensor:
    """Device e4m3fn code of clamp(x, -448, 448) for fp32 x (pins the hardware cvt)."""
    _check_cuda("x", x)
    x = x.to(torch.float32).contiguous()
    out = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    C.check(C.lib().rp_selftest_e4m3(x.data_ptr(), out.data_ptr(), x.numel(), _stream(x)),
            "rp_selftest_e4m3")
    return out


def selftest_scale(amax_bits: torch.Tensor, dtype: torch.dtype = torch.bfloat16
                   ) -> tuple[torch.Tensor, torch.Tensor]:
    """Device dequant scale and multiplier for bf16 or fp16 (``dtype``) amax bit
    patterns (int16/uint16)."""
    _check_cuda("amax_bits", amax_bits)
    dt = _IN_DTYPES[dtype]
    a = amax_bits.contiguous()
    dq = torch.empty(a.shape, dtype=torch.float32, device=a.device)
    qm = torch.empty(a.shape, dtype=torch.float32, device=a.device)
    C.check(C.lib().rp_selftest_scale(a.data_ptr(), dt, dq.data_ptr(), qm.data_ptr(), a.numel(),
                                      _stream(a)), "rp_selftest_scale")
    return dq, qm
