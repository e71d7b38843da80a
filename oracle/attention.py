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

``emulate_key_splits`` restates this build's key-split launch (no reference
counterpart) from ``emulate`` over sub-ranges; it is pinned by (f) equality
with ``emulate`` for one range and (g) the P-quant-free merge against the exact
softmax, with and without a causal mask.

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
            pquant: bool = True, mutation: str | None = None, kv_offset: int = 0,
            state: bool = False):
    """fp32 output rows (len(rows), D) for one (b, h) slice of e4m3fn codes.

    ``kv_offset`` places k8/v8 at that absolute key position (for the masks);
    ``state`` returns the unnormalised (acc, l, m) instead of acc / l, with a
    row that sees no key in the range left at acc = l = 0, m = -inf (the
    reference never meets such a row: its first tile always holds key 0)."""
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
        vis = visible(rows, kv + kv_offset, mask, prefix, suffix) & valid[None, :]
        if mutation == "causal_off_by_one" and mask == 1:
            vis = (kv[None, :] < rows[:, None]) & valid[None, :]
        s = np.where(vis, s, f32(-np.inf))
        with np.errstate(invalid="ignore"):
            m_new = np.maximum(m, s.max(axis=1))
            if state:  # rows with nothing visible yet keep alpha = 1, p = 0
                m_ref = np.where(m_new == -np.inf, f32(0), m_new)
                alpha = np.where(m == -np.inf, f32(1), np.exp(m - m_ref)).astype(f32)
                p = np.exp(s - m_ref[:, None]).astype(f32)
            else:
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
    if state:
        return acc, l, m
    return acc / l[:, None]


def emulate_key_splits(q8: np.ndarray, k8: np.ndarray, v8: np.ndarray, q_scale: float,
                       k_scale: float, v_scale: float, sm_scale: float,
                       rows: np.ndarray | None = None, *, split_keys: int, block_n: int = 128,
                       mask: int = 0, prefix: int = 0, suffix: int = 1,
                       pquant: bool = True) -> np.ndarray:
    """The key-split launch: ``emulate`` over each range of ``split_keys``
    keys from its own running max, merged as out = sum_j w_j acc_j /
    sum_j w_j l_j with w_j = exp(m_j - max_j m_j) over the ranges where the
    row saw a key.  Not a reference function: the reference runs one range."""
    Skv = k8.shape[0]
    parts = [emulate(q8, k8[a:a + split_keys], v8[a:a + split_keys], q_scale, k_scale, v_scale,
                     sm_scale, rows, block_n=block_n, mask=mask, prefix=prefix, suffix=suffix,
                     pquant=pquant, kv_offset=a, state=True) for a in range(0, Skv, split_keys)]
    ms = np.stack([p[2] for p in parts]).astype(np.float64)
    seen = np.stack([p[1] for p in parts]) != 0
    mmax = np.where(seen, ms, -np.inf).max(axis=0)
    w = np.where(seen, np.exp(np.where(seen, ms, 0.0) - mmax), 0.0)
    num = sum(w[j][:, None] * parts[j][0].astype(np.float64) for j in range(len(parts)))
    den = sum(w[j] * parts[j][1].astype(np.float64) for j in range(len(parts)))
    return (num / den[:, None]).astype(np.float32)


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
