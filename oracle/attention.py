"""Attention oracle -- TEST INFRASTRUCTURE ONLY.

``emulate`` is a numpy, tile-exact restatement of the FP8 FA-2 kernel body
of kernels/triton_kernels/fp8_flash_attn.py:294-391 for the OCP format
(P cast as in fp8_flash_attn_hopper.py:322):

    qk_scale = (sm_scale * q_scale) * k_scale            :329
    per key tile of ``block_n`` columns                  :334
      s      = fp32(Q8 . K8^T) * qk_scale                :346-347
      masked -> -inf                                     :350-356
      m_new  = max(m, rowmax s)                          :359
      alpha  = exp(m - m_new); p = exp(s - m_new)        :360-361
      l      = l*alpha + sum(p)   (fp32 p, unquantized)  :362
      acc   *= alpha                                     :365
      p8     = e4m3fn(p * 448)                           :375 (hopper :322)
      acc   += fp32(p8 . V8) * (v_scale / 448)           :376-380
    out = acc / l                                        :385

The result is fp32; the reference casts it to the input dtype on the host
(:645).  ``block_n`` is numerically significant (the running max at each tile
sets P's quantization grid); callers match the kernel's tile width.

``mutation`` lets the tests plant a plausible mistake in the oracle and show
that a pin catches it; it is never set outside tests.

Parity: pinned.  tests/test_oracle_attention.py checks (a) the P-quant-free
path against an exact fp64 softmax for multi-tile, ragged, causal and
shared-prefix cases, (b) hand-derived answers for the P quantization and the
unquantized denominator, (c) Skv = 1 and key/value permutation invariants,
(d) the C restatement against this module, and (e) the error against torch
SDPA at the reference's published Ada shape (docs/FP8_ON_ADA.md:56-67).
The bit pattern of the reference Triton kernel's own output is not
observable here (Triton's exp and MFMA accumulation order on gfx942), so
outputs are compared within tolerance, not bit for bit.
"""

from __future__ import annotations

import numpy as np

from oracle.quant import DECODE, encode_e4m3fn

P_SCALE = np.float32(448.0)


def visible(q: np.ndarray, kv: np.ndarray, mask: int, prefix: int = 0, suffix: int = 1) -> np.ndarray:
    """Boolean (len(q), len(kv)) visibility matrix for the supported masks:
    0 none, 1 causal (kv <= q), 2 shared-prefix candidates."""
    q = q[:, None]
    kv = kv[None, :]
    if mask == 0:
        return np.ones((q.shape[0], kv.shape[1]), dtype=bool)
    if mask == 1:
        return kv <= q
    j = kv - prefix
    return (kv < prefix) | ((j >= 0) & (j // suffix == q // suffix) & (j <= q))


def emulate(q8: np.ndarray, k8: np.ndarray, v8: np.ndarray, q_scale: float, k_scale: float,
            v_scale: float, sm_scale: float, rows: np.ndarray | None = None, *,
            block_n: int = 128, mask: int = 0, prefix: int = 0, suffix: int = 1,
            pquant: bool = True, mutation: str | None = None) -> np.ndarray:
    """fp32 output rows (len(rows), D) for one (b, h) slice of e4m3fn codes."""
    Sq, D = q8.shape
    Skv = k8.shape[0]
    rows = np.arange(Sq) if rows is None else np.asarray(rows)
    Q = DECODE[q8[rows]].astype(np.float64)
    K = DECODE[k8].astype(np.float64)
    V = DECODE[v8].astype(np.float64)
    f32 = np.float32
    qk_scale = (f32(sm_scale) * f32(q_scale)) * f32(k_scale)
    if mutation == "drop_q_scale":
        qk_scale = f32(sm_scale) * f32(k_scale)
    pv_scale = f32(v_scale) / P_SCALE
    R = rows.size
    m = np.full(R, -np.inf, dtype=f32)
    l = np.zeros(R, dtype=f32)
    acc = np.zeros((R, D), dtype=f32)
    for n0 in range(0, Skv, block_n):
        kv = np.arange(n0, n0 + block_n)
        valid = kv < Skv
        kvc = np.minimum(kv, Skv - 1)
        s = (Q @ K[kvc].T).astype(f32) * qk_scale
        vis = visible(rows, kv, mask, prefix, suffix) & valid[None, :]
        if mutation == "causal_off_by_one" and mask == 1:
            vis = (kv[None, :] < rows[:, None]) & valid[None, :]
        s = np.where(vis, s, f32(-np.inf))
        with np.errstate(invalid="ignore"):
            m_new = np.maximum(m, s.max(axis=1))
            alpha = np.exp(m - m_new).astype(f32)
            p = np.exp(s - m_new[:, None]).astype(f32)
        if mutation == "no_rescale":
            alpha = np.ones_like(alpha)
        if pquant:
            p8 = DECODE[encode_e4m3fn(p * P_SCALE)]
            if mutation == "p_scale_240":
                p8 = DECODE[encode_e4m3fn(p * f32(240.0))] * f32(448.0 / 240.0)
        else:
            p8 = p * P_SCALE
        if mutation == "l_from_quantized_p":
            l = l * alpha + (p8.astype(np.float64).sum(axis=1) / 448.0).astype(f32)
        else:
            l = l * alpha + p.astype(np.float64).sum(axis=1).astype(f32)
        acc = acc * alpha[:, None]
        Vt = np.where(valid[:, None], V[kvc], 0.0)
        pv = (p8.astype(np.float64) @ Vt).astype(f32)
        acc = acc + pv * pv_scale
        m = m_new
    return acc / l[:, None]


def exact_softmax_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, sm_scale: float,
                            rows: np.ndarray | None = None, *, mask: int = 0, prefix: int = 0,
                            suffix: int = 1) -> np.ndarray:
    """Textbook softmax(sm * q k^T) v in float64 on already-dequantized inputs."""
    rows = np.arange(q.shape[0]) if rows is None else np.asarray(rows)
    s = (q[rows].astype(np.float64) @ k.astype(np.float64).T) * float(sm_scale)
    vis = visible(rows, np.arange(k.shape[0]), mask, prefix, suffix)
    s = np.where(vis, s, -np.inf)
    s = s - s.max(axis=1, keepdims=True)
    w = np.exp(s)
    w /= w.sum(axis=1, keepdims=True)
    return w @ v.astype(np.float64)
