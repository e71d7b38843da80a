"""GPU parity of the FP8 flash-attention forward against the tile-exact CPU oracle.

Reference behaviour: kernels/triton_kernels/fp8_flash_attn.py:294-391 (kernel
body) and :480-645 (wrapper), OCP P cast per fp8_flash_attn_hopper.py:322.
The oracle runs with the kernel's key-tile width (BLOCK_N = 128) because the
running max after each tile sets P's quantization grid.

Tolerances: BASELINE.json's max-abs 2e-2 / mean-abs 2e-3 against the
torch-emulated FP8 result -- scaled by the output's peak magnitude only in
the tests that declare ``scaled=True`` because their outputs exceed 1 by
construction (see tests/_helpers.baseline_tolerance) -- plus a relative mean
error bound of 1e-2: the kernel and the oracle run the same algorithm, so they differ
only by fp32 rounding (exp2 vs exp, summation order) and the rare P code
that rounding flips.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention, native
from repercep_runtime_amd import ops
from repercep_runtime_amd.workloads import C1, C3_CROSS, C3_SELF, C5, AttnConfig, attn_inputs
from tests._helpers import baseline_tolerance, bf16_bits, codes_np, err_stats, vt_to_bhsd

pytestmark = pytest.mark.gpu

REL_TOL = 1e-2


def _oracle_rows(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, heads: list[int],
                 rows: np.ndarray, *, sm_scale: float, mask: int = 0, prefix: int = 0,
                 suffix: int = 1, granularity: str = "bh") -> tuple[np.ndarray, dict]:
    """Oracle output (len(heads), len(rows), D) for (B=1) CPU tensors."""
    B, H, Sq, D = q.shape
    n = B * H if granularity == "bh" else 1
    qs, q8 = native.quantize_groups(bf16_bits(q), n)
    ks, k8 = native.quantize_groups(bf16_bits(k), n)
    vs, v8 = native.quantize_groups(bf16_bits(v), n)
    outs = []
    for h in heads:
        si = h if granularity == "bh" else 0
        outs.append(native.attn_rows(q8[0, h], k8[0, h], v8[0, h], qs[si], ks[si], vs[si],
                                     sm_scale, rows, block_n=ops.BLOCK_N, mask=mask,
                                     prefix=prefix, suffix=suffix))
    return np.stack(outs), {"q8": q8, "k8": k8, "v8": v8, "qs": qs, "ks": ks, "vs": vs}


def _check(got: np.ndarray, ref: np.ndarray, what: str, rel_tol: float = REL_TOL,
           scaled: bool = False) -> dict:
    """BASELINE's absolute bounds (max-abs 2e-2, mean-abs 2e-3) and the
    relative mean bound.  ``scaled=True`` -- declared only by tests whose
    outputs exceed 1 by construction (a handful of keys, peaked rows) --
    scales the absolute bounds by the output's peak (see
    tests/_helpers.baseline_tolerance); the relative bound never scales."""
    st = err_stats(got, ref)
    max_tol, mean_tol = baseline_tolerance(ref) if scaled else (2e-2, 2e-3)
    print(f"{what}: {st} (tol max {max_tol:.3g}, mean {mean_tol:.3g}"
          f"{', scaled by the output peak' if scaled else ''})", flush=True)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    assert st["max_abs"] <= max_tol, f"{what}: {st}"
    assert st["mean_abs"] <= mean_tol, f"{what}: {st}"
    assert st["rel_mean"] <= rel_tol, f"{what}: {st}"
    return st


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_c1_all_rows(gpu: torch.device, out_dtype: torch.dtype) -> None:
    """BASELINE config 1, (1, 8, 1024, 64): every output element vs the oracle."""
    q, k, v = attn_inputs(C1)
    sm = 1.0 / math.sqrt(C1.D)
    out = ops.fp8_flash_attention(q.to(gpu), k.to(gpu), v.to(gpu), out_dtype=out_dtype)
    ref, _ = _oracle_rows(q, k, v, list(range(C1.H)), np.arange(C1.Sq), sm_scale=sm)
    got = out.float().cpu().numpy()[0]
    if out_dtype == torch.bfloat16:
        ref = torch.from_numpy(ref).to(torch.bfloat16).float().numpy()
    _check(got, ref, f"c1 {out_dtype}")


CASES = [
    # name, B, H, Sq, Skv, D, causal
    ("self_ragged_d128", 1, 2, 1000, 1000, 128, False),
    ("self_ragged_d64", 2, 1, 777, 777, 64, False),
    ("cross_d128", 1, 2, 300, 512, 128, False),
    ("cross_short_kv", 1, 1, 1000, 131, 128, False),
    ("single_key", 1, 1, 64, 1, 128, False),
    ("single_query", 1, 3, 1, 300, 64, False),
    ("causal_d128", 1, 2, 700, 700, 128, True),
    ("causal_d64", 1, 2, 513, 513, 64, True),
    ("tiny", 1, 1, 5, 7, 64, False),
    # head dim 32: one 64-deep QK step whose upper k-slots are zero padding
    ("self_ragged_d32", 1, 2, 600, 600, 32, False),
    ("causal_d32", 2, 1, 300, 300, 32, True),
    ("tiny_d32", 1, 1, 5, 7, 32, False),
    # head dim 256: two workgroups per query block, one per half of V^T / O
    ("self_ragged_d256", 1, 2, 700, 700, 256, False),
    ("cross_d256", 1, 1, 300, 450, 256, False),
    ("causal_d256", 1, 2, 513, 513, 256, True),
    ("tiny_d256", 1, 1, 5, 7, 256, False),
    # causal with unequal lengths: the reference's top-left mask kv <= q
    # (fp8_flash_attn.py:350-352); rows past Skv see every key
    ("causal_q_longer", 1, 2, 700, 300, 128, True),
    ("causal_kv_longer", 1, 2, 300, 700, 64, True),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_shapes_vs_oracle(gpu: torch.device, case: tuple) -> None:
    name, B, H, Sq, Skv, D, causal = case
    g = torch.Generator().manual_seed(sum(map(ord, name)))
    q = torch.randn(B, H, Sq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, H, Skv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, H, Skv, D, generator=g).to(torch.bfloat16)
    sm = 1.0 / math.sqrt(D)
    out = ops.fp8_flash_attention(q.to(gpu), k.to(gpu), v.to(gpu), causal=causal,
                                  out_dtype=torch.float32).cpu().numpy()
    rows = np.arange(Sq)
    for b in range(B):
        ref, _ = _oracle_rows(q[b:b + 1], k[b:b + 1], v[b:b + 1], list(range(H)), rows,
                              sm_scale=sm, mask=1 if causal else 0)
        _check(out[b], ref, f"{name} b={b}")


@pytest.mark.parametrize("out_dtype", [None, torch.float32, torch.bfloat16])
def test_fp16_inputs_vs_oracle(gpu: torch.device, out_dtype: torch.dtype | None) -> None:
    """fp16 Q/K/V (the reference accepts them: fp8_triton.py:85): fp16 scales
    and codes, and the output in q's dtype by default."""
    from oracle import quant

    g = torch.Generator().manual_seed(16)
    B, H, S, D = 1, 2, 700, 128
    q, k, v = (torch.randn(B, H, S, D, generator=g).mul(m).to(torch.float16)
               for m in (1.0, 2.0, 0.5))
    out = ops.fp8_flash_attention(q.to(gpu), k.to(gpu), v.to(gpu), out_dtype=out_dtype)
    assert out.dtype == (out_dtype or torch.float16)
    qs, q8 = quant.quantize_codes(q)
    ks, k8 = quant.quantize_codes(k)
    vs, v8 = quant.quantize_codes(v)
    for h in range(H):
        ref = native.attn_rows(q8[0, h], k8[0, h], v8[0, h], qs[h], ks[h], vs[h], D ** -0.5,
                               np.arange(S), block_n=ops.BLOCK_N)
        if out.dtype != torch.float32:
            ref = torch.from_numpy(ref).to(out.dtype).float().numpy()
        _check(out[0, h].float().cpu().numpy(), ref, f"fp16 in, {out.dtype} out, h={h}")


def test_fp16_and_bf16_outputs_are_one_rounding_of_fp32(gpu: torch.device) -> None:
    """The 16-bit outputs, direct and through the split-merge kernel, are the
    fp32 result rounded once to nearest even, like the reference's
    ``out.to(q.dtype)`` (fp8_flash_attn.py:645)."""
    g = torch.Generator().manual_seed(18)
    q, k, v = (torch.randn(1, 2, 200, 64, generator=g).to(torch.float16) for _ in range(3))
    qg, kg, vg = q.to(gpu), k.to(gpu), v.to(gpu)
    o1 = ops.fp8_flash_attention(qg, kg, vg, out_dtype=torch.float32, kv_splits=1)
    o4 = ops.fp8_flash_attention(qg, kg, vg, kv_splits=1)
    assert o4.dtype == torch.float16
    assert torch.equal(o4, o1.to(torch.float16))   # one RNE of the same fp32 value
    s32 = ops.fp8_flash_attention(qg, kg, vg, out_dtype=torch.float32, kv_splits=4)
    s16 = ops.fp8_flash_attention(qg, kg, vg, kv_splits=4)
    assert torch.equal(s16, s32.to(torch.float16))
    # likewise bf16 output: the reference's fp32 result cast once (:645)
    for n, o32 in ((1, o1), (4, s32)):
        ob = ops.fp8_flash_attention(qg, kg, vg, out_dtype=torch.bfloat16, kv_splits=n)
        assert torch.equal(ob, o32.to(torch.bfloat16))


MULTI_CASES = [
    # name, B, H, Sq, Skv, D, dtype, out_dtype: shapes on which a workgroup
    # streams several query blocks (rp_fp8_attn_blocks_per_workgroup > 1);
    # ragged Sq, a key range shorter than one tile, a shifted last tile
    ("d64_one_partial_tile", 1, 64, 16384 + 77, 100, 64, torch.bfloat16, torch.float32),
    ("d128_shifted_tail", 2, 20, 12000, 300, 128, torch.bfloat16, torch.bfloat16),
    ("d32_fp16", 1, 48, 8192 + 5, 512, 32, torch.float16, torch.float16),
    ("d128_wan_cross_like", 1, 40, 9000, 512, 128, torch.bfloat16, torch.float32),
    # 16-bit outputs at D = 128 with two or more key tiles per block leave
    # through the staged (whole-line) stores; two tiles is the shortest
    # window the Q buffer they borrow stays idle
    ("d128_wan_cross_like_bf16", 1, 40, 9000, 512, 128, torch.bfloat16, torch.bfloat16),
    ("d128_two_tiles_fp16", 1, 24, 7003, 256, 128, torch.float16, torch.float16),
    # key ranges past what LDS holds (more than 4 tiles at D = 128, 8 at
    # D = 64): the multi-block kernel, with its staged stores at D = 128
    ("d128_six_tiles_bf16", 1, 24, 9000, 700, 128, torch.bfloat16, torch.bfloat16),
    ("d128_eight_tiles_f32", 1, 16, 9000, 1024, 128, torch.bfloat16, torch.float32),
    ("d64_nine_tiles", 1, 32, 12000, 1100, 64, torch.bfloat16, torch.bfloat16),
]


@pytest.mark.parametrize("case", MULTI_CASES, ids=[c[0] for c in MULTI_CASES])
def test_multi_block_launches_vs_oracle(gpu: torch.device, case: tuple) -> None:
    """Rows at the start, at block boundaries and at the end of workgroups'
    block streams, against the oracle.  The shapes have a multi-block plan;
    those whose keys fit LDS (head dim 64/128, up to 4 or 8 tiles) run the
    resident-K/V kernel, the rest the multi-block kernel."""
    from oracle import quant
    from repercep_runtime_amd import _capi

    name, B, H, Sq, Skv, D, dtype, out_dtype = case
    per = _capi.lib().rp_fp8_attn_blocks_per_workgroup(B, H, Sq, Skv, D, 0, 1)
    assert per > 1, f"{name}: not a multi-block plan"
    kvres = _capi.lib().rp_fp8_attn_resident_kv(B, H, Sq, Skv, D, 0, 1)
    fits = D in (64, 128) and -(-Skv // 128) <= (4 if D == 128 else 8)
    assert kvres == int(fits), name
    g = torch.Generator().manual_seed(sum(map(ord, name)))
    q = torch.randn(B, H, Sq, D, generator=g).to(dtype)
    k = torch.randn(B, H, Skv, D, generator=g).to(dtype)
    v = torch.randn(B, H, Skv, D, generator=g).to(dtype)
    out = ops.fp8_flash_attention(q.to(gpu), k.to(gpu), v.to(gpu), out_dtype=out_dtype)
    out = out.float().cpu().numpy()
    blk = 256 * per   # query rows of one workgroup
    rows = set()
    for w0 in range(0, Sq, blk):
        for r in (w0, w0 + 1, w0 + 255, w0 + 256, w0 + 257, w0 + blk - 1, w0 + blk // 2):
            rows.add(min(r, Sq - 1))
    rows |= {Sq - 1, Sq - 2}
    rows = np.array(sorted(rows))
    for b in range(B):
        sl = slice(b, b + 1)
        qs, q8 = quant.quantize_codes(q[sl])
        ks, k8 = quant.quantize_codes(k[sl])
        vs, v8 = quant.quantize_codes(v[sl])
        for h in (0, H // 2, H - 1):
            ref = native.attn_rows(q8[0, h], k8[0, h], v8[0, h], qs[h], ks[h], vs[h],
                                   D ** -0.5, rows, block_n=ops.BLOCK_N)
            if out_dtype != torch.float32:
                ref = torch.from_numpy(ref).to(out_dtype).float().numpy()
            _check(out[b, h, rows], ref, f"{name} per={per} b={b} h={h}")


def test_per_tensor_granularity(gpu: torch.device) -> None:
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(1, 4, 600, 128, generator=g).mul(1 + i).to(torch.bfloat16)
               for i in range(3))
    out = ops.fp8_flash_attention(q.to(gpu), k.to(gpu), v.to(gpu), granularity="tensor",
                                  out_dtype=torch.float32).cpu().numpy()[0]
    ref, _ = _oracle_rows(q, k, v, [0, 1, 2, 3], np.arange(600), sm_scale=128 ** -0.5,
                          granularity="tensor")
    # V = 3 N(0, 1): outputs reach ~3, so one flipped P code moves them ~3x more
    _check(out, ref, "per-tensor", scaled=True)


def test_custom_softmax_scale(gpu: torch.device) -> None:
    g = torch.Generator().manual_seed(9)
    q, k, v = (torch.randn(1, 2, 256, 64, generator=g).to(torch.bfloat16) for _ in range(3))
    out = ops.fp8_flash_attention(q.to(gpu), k.to(gpu), v.to(gpu), scale=0.3,
                                  out_dtype=torch.float32).cpu().numpy()[0]
    ref, _ = _oracle_rows(q, k, v, [0, 1], np.arange(256), sm_scale=0.3)
    # 2.4x the default temperature: peaked rows whose outputs exceed 1
    _check(out, ref, "scale=0.3", scaled=True)


def test_shared_prefix_candidates_c5(gpu: torch.device) -> None:
    """512-token shared prefix + 16 candidates x 8 suffix tokens."""
    q, k, v = attn_inputs(C5)
    out = ops.fp8_flash_attention(q.to(gpu), k.to(gpu), v.to(gpu), prefix_len=C5.prefix,
                                  suffix_len=C5.suffix, out_dtype=torch.float32)
    ref, _ = _oracle_rows(q, k, v, list(range(C5.H)), np.arange(C5.Sq),
                          sm_scale=C5.D ** -0.5, mask=2, prefix=C5.prefix, suffix=C5.suffix)
    _check(out.cpu().numpy()[0], ref, "c5 shared prefix")


def test_shared_prefix_candidates_are_isolated_on_gpu(gpu: torch.device) -> None:
    """C5 layout: exchanging two candidates' suffix keys and values (a
    permutation: scales and codes of everything else unchanged) leaves every
    other candidate's kernel output bit-identical and changes the two
    exchanged ones -- a candidate attends to the shared prefix and its own
    suffix only."""
    q, k, v = attn_inputs(C5)
    P, L = C5.prefix, C5.suffix
    n_cand = C5.Sq // L
    a, b = 2, 11
    idx = torch.arange(C5.Skv)
    ia = torch.arange(P + a * L, P + (a + 1) * L)
    ib = torch.arange(P + b * L, P + (b + 1) * L)
    idx[ia], idx[ib] = ib, ia
    run = lambda kk, vv: ops.fp8_flash_attention(  # noqa: E731
        q.to(gpu), kk.to(gpu), vv.to(gpu), prefix_len=P, suffix_len=L,
        out_dtype=torch.float32, kv_splits=1).cpu()
    base = run(k, v)
    swapped = run(k[:, :, idx], v[:, :, idx])
    for c in range(n_cand):
        rows = slice(c * L, (c + 1) * L)
        same = torch.equal(swapped[:, :, rows], base[:, :, rows])
        assert same == (c not in (a, b)), c


SPLIT_CASES = [
    # name, B, H, Sq, Skv, D, causal, prefix, suffix, split counts
    ("c1", 1, 8, 1024, 1024, 64, False, None, None, (2, 3, 8)),
    # 8 tiles, the last shifted back; with 8 splits it opens its own range
    ("ragged_cross", 1, 2, 700, 1000, 128, False, None, None, (2, 8)),
    ("causal", 1, 2, 1000, 1000, 128, True, None, None, (2, 4, 8)),
    ("c5_prefix", 1, 32, 128, 640, 128, False, 512, 8, (2, 3, 5)),
    ("short_kv", 1, 2, 300, 100, 64, False, None, None, (4,)),   # one tile: no split
    ("two_tiles_ragged", 2, 1, 257, 131, 128, False, None, None, (2,)),
    ("d256", 1, 2, 300, 1000, 256, False, None, None, (2, 8)),
    ("d256_causal", 1, 1, 600, 600, 256, True, None, None, (3,)),
    ("d32", 1, 2, 300, 1000, 32, False, None, None, (3,)),
    # causal, 256 queries against 1000 keys: splits past every query hold
    # nothing (their running max stays -inf) and the merge ignores them
    ("causal_kv_longer", 1, 2, 256, 1000, 128, True, None, None, (2, 4)),
]


@pytest.mark.parametrize("case", SPLIT_CASES, ids=[c[0] for c in SPLIT_CASES])
def test_key_splits_vs_oracle(gpu: torch.device, case: tuple) -> None:
    """Key-split launches (rp_fp8_attn_fwd_split) against the unsplit oracle:
    each range keeps its own running max, which moves P's quantization grid
    as the reference's BLOCK_N choice does, so the bound is the FP8
    tolerance, not the unsplit kernel's bit pattern."""
    name, B, H, Sq, Skv, D, causal, prefix, suffix, counts = case
    g = torch.Generator().manual_seed(sum(map(ord, name)))
    q = torch.randn(B, H, Sq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, H, Skv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, H, Skv, D, generator=g).to(torch.bfloat16)
    mask = 2 if prefix is not None else (1 if causal else 0)
    qg, kg, vg = q.to(gpu), k.to(gpu), v.to(gpu)
    base = ops.fp8_flash_attention(qg, kg, vg, causal=causal, prefix_len=prefix,
                                   suffix_len=suffix, out_dtype=torch.float32, kv_splits=1)
    n_kb = -(-Skv // 128)
    for n in counts:
        out = ops.fp8_flash_attention(qg, kg, vg, causal=causal, prefix_len=prefix,
                                      suffix_len=suffix, out_dtype=torch.float32,
                                      kv_splits=n).cpu().numpy()
        if Skv <= 128:   # a single key tile cannot split: the unsplit kernel's bits
            assert np.array_equal(out, base.cpu().numpy()), name
        # the kernel's plan: equal ranges of whole tiles (rp_attn.hip split_plan)
        split_keys = -(-n_kb // min(n, n_kb)) * 128
        for b in range(B):
            sl = slice(b, b + 1)
            qs8, ks8, vs8 = (native.quantize_groups(bf16_bits(t[sl]), H) for t in (q, k, v))
            for h in range(H):
                ref = attention.emulate_key_splits(
                    qs8[1][0, h], ks8[1][0, h], vs8[1][0, h], qs8[0][h], ks8[0][h], vs8[0][h],
                    D ** -0.5, split_keys=split_keys, mask=mask, prefix=prefix or 0,
                    suffix=suffix or 1)
                _check(out[b, h], ref, f"{name} kv_splits={n} b={b} h={h}")
            # against the one-range oracle only the FP8 tolerance holds: each
            # range quantizes P against its own running max
            ref1, _ = _oracle_rows(q[sl], k[sl], v[sl], list(range(H)), np.arange(Sq),
                                   sm_scale=D ** -0.5, mask=mask, prefix=prefix or 0,
                                   suffix=suffix or 1)
            _check(out[b], ref1, f"{name} kv_splits={n} b={b} vs one range", rel_tol=5e-2)


BALANCED_CASES = [
    # name, B, H, Sq, Skv, D, out dtype; on 256 CUs the plans are (32, 8):
    # 24 (D=128) / 16 (D=256, two halves) tail workgroups split 8 ways
    ("d128", 1, 8, 8860, 8192, 128, torch.float32),
    ("d128_bf16", 1, 8, 8860, 8192, 128, torch.bfloat16),
    ("d256", 1, 4, 8548, 4096, 256, torch.float32),
]


@pytest.mark.parametrize("case", BALANCED_CASES, ids=[c[0] for c in BALANCED_CASES])
def test_balanced_launch_vs_oracle(gpu: torch.device, case: tuple) -> None:
    """rp_fp8_attn_fwd_balanced (kv_splits=0): the query blocks of the
    unsplit launch are the plain launch's bits; the rows of the key-split
    tail match the split emulation with the plan's split count (bit-exact
    codes in, the usual tolerance out) and the one-range oracle to the FP8
    tolerance."""
    import ctypes

    from repercep_runtime_amd import _capi

    name, B, H, Sq, Skv, D, odt = case
    cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    m, s = ctypes.c_int(), ctypes.c_int()
    assert _capi.lib().rp_fp8_attn_balanced_plan(B, H, Sq, Skv, D, 0, cus, ctypes.byref(m),
                                                 ctypes.byref(s)) == 0
    main, splits = m.value, s.value
    if cus == 256:
        assert (main, splits) == (32, 8)
    if splits == 1:
        pytest.skip(f"no tail split on {cus} CUs")
    g = torch.Generator().manual_seed(sum(map(ord, name)))
    q = torch.randn(B, H, Sq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, H, Skv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, H, Skv, D, generator=g).to(torch.bfloat16)
    qg, kg, vg = q.to(gpu), k.to(gpu), v.to(gpu)
    one = ops.fp8_flash_attention(qg, kg, vg, out_dtype=odt, kv_splits=1)
    bal = ops.fp8_flash_attention(qg, kg, vg, out_dtype=odt, kv_splits=0)
    torch.cuda.synchronize()
    r0 = main * ops.BLOCK_M
    assert torch.equal(bal[:, :, :r0].view(torch.int16 if odt != torch.float32 else torch.int32),
                       one[:, :, :r0].view(torch.int16 if odt != torch.float32 else torch.int32))
    tail = np.arange(r0, Sq)
    n_kb = -(-Skv // 128)
    split_keys = -(-n_kb // min(splits, n_kb)) * 128
    qs8, ks8, vs8 = (native.quantize_groups(bf16_bits(t), B * H) for t in (q, k, v))
    got = bal[0, :, r0:].float().cpu().numpy()
    for h in range(H):
        ref = attention.emulate_key_splits(qs8[1][0, h], ks8[1][0, h], vs8[1][0, h], qs8[0][h],
                                           ks8[0][h], vs8[0][h], D ** -0.5, tail,
                                           split_keys=split_keys)
        if odt != torch.float32:
            ref = torch.from_numpy(ref).to(odt).float().numpy()
        _check(got[h], ref, f"{name} tail h={h}")
    ref1, _ = _oracle_rows(q, k, v, list(range(H)), tail, sm_scale=D ** -0.5)
    _check(got, ref1, f"{name} tail vs one range", rel_tol=5e-2)


@pytest.mark.parametrize("shape", [(1, 4, 1000, 1000, 128, True), (1, 2, 3000, 512, 128, False),
                                   (1, 32, 2048, 4224, 128, False), (1, 8, 2048, 2048, 64, False),
                                   (2, 3, 700, 900, 256, True)],
                         ids=["causal", "multi_block", "whole_rounds", "under_a_round",
                              "d256_causal"])
def test_balanced_launch_without_a_split_is_the_plain_launch(gpu: torch.device,
                                                              shape: tuple) -> None:
    """Where the balanced plan splits nothing (a mask, a multi-block launch,
    rounds already full), kv_splits=0 runs exactly the one-range launch."""
    import ctypes

    from repercep_runtime_amd import _capi

    B, H, Sq, Skv, D, causal = shape
    cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    m, s = ctypes.c_int(), ctypes.c_int()
    assert _capi.lib().rp_fp8_attn_balanced_plan(B, H, Sq, Skv, D, int(causal), cus,
                                                 ctypes.byref(m), ctypes.byref(s)) == 0
    assert s.value == 1
    g = torch.Generator(device=gpu).manual_seed(Sq + Skv)
    q = torch.randn(B, H, Sq, D, generator=g, device=gpu).to(torch.bfloat16)
    k = torch.randn(B, H, Skv, D, generator=g, device=gpu).to(torch.bfloat16)
    v = torch.randn(B, H, Skv, D, generator=g, device=gpu).to(torch.bfloat16)
    one = ops.fp8_flash_attention(q, k, v, causal=causal, kv_splits=1)
    bal = ops.fp8_flash_attention(q, k, v, causal=causal, kv_splits=0)
    assert torch.equal(one, bal)


def test_autotune_records_and_reuses_a_split_count(gpu: torch.device, tmp_path,
                                                   monkeypatch: pytest.MonkeyPatch) -> None:
    """Cache miss -> timed search over the candidates, winner recorded under
    the reference's key; the next call reads it without timing anything."""
    from repercep_runtime_amd import tuning

    path = tmp_path / "cache.json"
    monkeypatch.setenv("REPERCEP_FP8_AUTOTUNE_CACHE", str(path))
    monkeypatch.delenv("REPERCEP_FP8_DISABLE_AUTOTUNE")
    q, k, v = attn_inputs(C1)
    qg, kg, vg = q.to(gpu), k.to(gpu), v.to(gpu)
    out = ops.fp8_flash_attention(qg, kg, vg, out_dtype=torch.float32).cpu().numpy()[0]
    cfg = tuning.resolve_config(1, C1.H, C1.Sq, C1.Skv, C1.D, False)
    assert cfg["KV_SPLITS"] in (1, 2, 4, 8), cfg
    print("autotuned C1 launch:", cfg, flush=True)
    assert "B1_H8_Sq1024_Skv1024_D64_C0" in tuning.cache_load()
    # the winner depends on the box's timings: check it against the oracle of
    # its own key ranges (rp_attn.hip split_plan: equal ranges of whole tiles)
    block_m, n = ops.launch_of(cfg)   # a short-query winner computes the one-range result
    n_kb = -(-C1.Skv // 128)
    qs8, ks8, vs8 = (native.quantize_groups(bf16_bits(t), C1.H) for t in (q, k, v))
    for h in range(C1.H):
        if n == 1:
            ref = native.attn_rows(qs8[1][0, h], ks8[1][0, h], vs8[1][0, h], qs8[0][h],
                                   ks8[0][h], vs8[0][h], C1.D ** -0.5, np.arange(C1.Sq),
                                   block_n=ops.BLOCK_N)
        else:
            ref = attention.emulate_key_splits(
                qs8[1][0, h], ks8[1][0, h], vs8[1][0, h], qs8[0][h], ks8[0][h], vs8[0][h],
                C1.D ** -0.5, split_keys=-(-n_kb // min(n, n_kb)) * 128)
        _check(out[h], ref, f"c1 autotuned block_m={block_m} kv_splits={n} h={h}")

    def no_timing(*_a, **_k):
        raise AssertionError("cache hit must not time candidates")

    monkeypatch.setattr(ops, "_time_call", no_timing)
    again = ops.fp8_flash_attention(qg, kg, vg, out_dtype=torch.float32).cpu().numpy()[0]
    # the recorded launch run directly: (block_m, kv_splits) of the entry
    qs, q8, ks, k8, vs, vt8 = ops.scale_quantize_qkv(qg, kg, vg)
    direct = ops.attention_fp8(q8.view(torch.uint8), k8.view(torch.uint8),
                               vt8.view(torch.uint8), qs, ks, vs, C1.D ** -0.5,
                               out_dtype=torch.float32, kv_splits=n,
                               block_m=block_m).cpu().numpy()[0]
    assert np.array_equal(again, direct)


def test_output_into_strided_bshd_buffer(gpu: torch.device) -> None:
    """Kernel writes through output strides: a permuted (B, S, H, D) buffer."""
    g = torch.Generator().manual_seed(21)
    q, k, v = (torch.randn(2, 300, 3, 128, generator=g).to(torch.bfloat16) for _ in range(3))
    qg, kg, vg = q.to(gpu), k.to(gpu), v.to(gpu)
    out = torch.full((2, 300, 3, 128), float("nan"), dtype=torch.bfloat16, device=gpu)
    ops.fp8_flash_attention(qg.permute(0, 2, 1, 3), kg.permute(0, 2, 1, 3),
                            vg.permute(0, 2, 1, 3), out=out.permute(0, 2, 1, 3))
    ref_bhsd = ops.fp8_flash_attention(qg.permute(0, 2, 1, 3).contiguous(),
                                       kg.permute(0, 2, 1, 3).contiguous(),
                                       vg.permute(0, 2, 1, 3).contiguous())
    assert torch.equal(out.permute(0, 2, 1, 3), ref_bhsd)


def test_codes_seen_by_kernel_match_oracle_codes(gpu: torch.device) -> None:
    """The attention wrapper's quantized operands are the oracle's codes, bit for bit."""
    q, k, v = attn_inputs(C1)
    _, q8_ref = native.quantize_groups(bf16_bits(q), C1.B * C1.H)
    _, v8_ref = native.quantize_groups(bf16_bits(v), C1.B * C1.H)
    qs, q8 = ops.scale_quantize(q.to(gpu), "bh", "bhsd")
    vs, vt8 = ops.scale_quantize(v.to(gpu), "bh", "bhds")
    assert np.array_equal(codes_np(q8), q8_ref)
    assert np.array_equal(vt_to_bhsd(codes_np(vt8), C1.Skv), v8_ref)


def _group_scales_codes(x: torch.Tensor, heads: list[int], granularity: str
                        ) -> tuple[dict, dict, float | None]:
    """Oracle dequant scale and codes of the listed heads of a (1, H, S, D) bf16
    CPU tensor: per (b, h) from the head alone, per tensor from the amax of
    the whole tensor (third value; None per head)."""
    bits = bf16_bits(x)
    whole = None
    if granularity == "tensor":
        whole = float(native.dequant_from_amax(native.amax_bf16(bits)))
    scales, codes = {}, {}
    for h in heads:
        s = whole if whole is not None else float(native.dequant_from_amax(
            native.amax_bf16(bits[0, h])))
        scales[h] = s
        codes[h] = native.quantize_bf16(bits[0, h], s)
    return scales, codes, whole


def _wan_sample(gpu: torch.device, cfg: AttnConfig, heads: list[int], nrows: int,
                granularity: str, out_dtype: torch.dtype = torch.float32) -> None:
    q, k, v = attn_inputs(cfg, device=gpu)
    out = ops.fp8_flash_attention(q, k, v, out_dtype=out_dtype, granularity=granularity)
    gq = ops.scale_quantize_qkv(q, k, v, granularity)
    torch.cuda.synchronize()
    rng = np.random.default_rng(0)
    rows = np.sort(rng.choice(cfg.Sq, size=nrows, replace=False))
    # per-tensor scales need every head; per-(b,h) scales only the sampled ones
    src = (q, k, v) if granularity == "tensor" else (q[:, heads], k[:, heads], v[:, heads])
    idx = heads if granularity == "tensor" else list(range(len(heads)))
    ora = [_group_scales_codes(t.cpu(), idx, granularity) for t in src]
    # the device scales are the oracle's, bit for bit
    for (dev_s, (sc, _, whole)) in zip((gq[0], gq[2], gq[4]), ora):
        dev_s = dev_s.cpu().numpy()
        if granularity == "tensor":
            assert dev_s.shape == (1,) and dev_s[0] == np.float32(whole)
        else:
            assert all(dev_s[h] == np.float32(sc[i]) for h, i in zip(heads, idx))
    got = out[0, heads][:, torch.from_numpy(rows).to(gpu)].float().cpu().numpy()
    ref = np.stack([native.attn_rows(ora[0][1][i], ora[1][1][i], ora[2][1][i], ora[0][0][i],
                                     ora[1][0][i], ora[2][0][i], cfg.D ** -0.5, rows,
                                     block_n=ops.BLOCK_N) for i in idx])
    if out_dtype != torch.float32:   # one rounding of the fp32 result, as the reference casts
        ref = torch.from_numpy(ref).to(out_dtype).float().numpy()
    _check(got, ref, f"{cfg.name} {granularity} {out_dtype} heads {heads} rows {nrows}")
    assert torch.isfinite(out).all()
    del q, k, v, out, gq
    torch.cuda.empty_cache()


@pytest.mark.parametrize("granularity", ["bh", "tensor"])
def test_wan_self_attention_full_shape_sampled_rows(gpu: torch.device, granularity: str) -> None:
    """C3 self (1, 40, 75600, 128): full kernel run, 128 rows x 3 heads vs oracle,
    per-(b,h) scales (the reference's) and per-tensor scales (BASELINE's wording)."""
    _wan_sample(gpu, C3_SELF, [0, 17, 39], 128, granularity)


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("granularity", ["bh", "tensor"])
def test_wan_cross_attention_full_shape_sampled_rows(gpu: torch.device, granularity: str,
                                                     out_dtype: torch.dtype) -> None:
    """C3 cross (Skv = 512, the resident-K/V launch): 512 rows x 4 heads vs
    oracle, both granularities, fp32 and the bench's bf16 output."""
    from repercep_runtime_amd import _capi

    c = C3_CROSS
    assert _capi.lib().rp_fp8_attn_resident_kv(c.B, c.H, c.Sq, c.Skv, c.D, 0, 1) == 1
    _wan_sample(gpu, C3_CROSS, [0, 5, 20, 39], 512, granularity, out_dtype)


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_wan_self_balanced_launch_full_shape(gpu: torch.device, out_dtype: torch.dtype) -> None:
    """C3 self through the launch the op resolves for it when autotuning is on
    (kv_splits=0, the balanced launch) with per-tensor scales, as the bench
    runs it (bf16 output included): 64 sampled rows of the unsplit query
    blocks against the one-range oracle, 64 of the key-split tail against
    the split emulation with the plan's count."""
    import ctypes

    from repercep_runtime_amd import _capi

    cfg = C3_SELF
    cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    m, s = ctypes.c_int(), ctypes.c_int()
    assert _capi.lib().rp_fp8_attn_balanced_plan(cfg.B, cfg.H, cfg.Sq, cfg.Skv, cfg.D, 0, cus,
                                                 ctypes.byref(m), ctypes.byref(s)) == 0
    main, splits = m.value, s.value
    if cus == 256:
        assert (main, splits) == (288, 4)
    if splits == 1:
        pytest.skip(f"no tail split on {cus} CUs")
    q, k, v = attn_inputs(cfg, device=gpu)
    out = ops.fp8_flash_attention(q, k, v, out_dtype=out_dtype, granularity="tensor",
                                  kv_splits=0)
    torch.cuda.synchronize()
    heads = [0, 21, 39]
    r0 = main * ops.BLOCK_M
    rng = np.random.default_rng(3)
    rows_main = np.sort(rng.choice(r0, size=64, replace=False))
    rows_tail = np.sort(rng.choice(np.arange(r0, cfg.Sq), size=64, replace=False))
    ora = [_group_scales_codes(t.cpu(), heads, "tensor") for t in (q, k, v)]
    n_kb = -(-cfg.Skv // 128)
    split_keys = -(-n_kb // min(splits, n_kb)) * 128
    sm = cfg.D ** -0.5
    for rows, tail in ((rows_main, False), (rows_tail, True)):
        got = out[0, heads][:, torch.from_numpy(rows).to(gpu)].float().cpu().numpy()
        refs = []
        for h in heads:
            args = (ora[0][1][h], ora[1][1][h], ora[2][1][h], ora[0][0][h], ora[1][0][h],
                    ora[2][0][h], sm, rows)
            refs.append(attention.emulate_key_splits(*args, split_keys=split_keys) if tail
                        else native.attn_rows(*args, block_n=ops.BLOCK_N))
        ref = np.stack(refs)
        if out_dtype != torch.float32:
            ref = torch.from_numpy(ref).to(out_dtype).float().numpy()
        _check(got, ref, f"c3 balanced {out_dtype} {'tail' if tail else 'unsplit'} rows")
    assert torch.isfinite(out).all()
    del q, k, v, out
    torch.cuda.empty_cache()


def test_cosmos_full_shape_per_tensor_through_fused_qknorm(gpu: torch.device) -> None:
    """BASELINE config 2, Cosmos (1, 32, 56320, 128): pre-norm Q/K through the
    fused RMSNorm prologue, per-tensor scales, the full attention kernel run
    (56320 is a whole number of 128-key tiles: no shifted last tile).  The
    oracle normalises every row of Q and K on the CPU (oracle/c
    or_rmsnorm_bf16_rows, the prologue's summation order) for the
    whole-tensor amax; scales and the sampled heads' codes are bit-exact, and
    128 rows x 3 heads of the output are within tolerance."""
    from repercep_runtime_amd.workloads import C2

    assert C2.Skv % 128 == 0
    q, k, v = attn_inputs(C2, device=gpu, normalize=False)
    out = ops.fp8_flash_attention_qknorm(q, k, v, granularity="tensor", out_dtype=torch.float32)
    # the op's own quantizer call: Q/K prologue and V in shared launches
    dqq, q8, dqk, k8, dqv, vt8 = ops.rmsnorm_scale_quantize_qkv(q, k, v, granularity="tensor")
    torch.cuda.synchronize()
    heads = [0, 13, 31]
    rows = np.sort(np.random.default_rng(2).choice(C2.Sq, size=128, replace=False))
    ora = []
    for x, dq_dev, c_dev, norm in ((q, dqq, q8, True), (k, dqk, k8, True), (v, dqv, vt8, False)):
        bits = bf16_bits(x.cpu())
        if norm:
            bits = native.rmsnorm_bf16(bits, 1e-6)
        s = float(native.dequant_from_amax(native.amax_bf16(bits)))
        codes = {h: native.quantize_bf16(bits[0, h], s) for h in heads}
        assert dq_dev.cpu().numpy()[0] == np.float32(s)
        for h in heads:
            got_c = codes_np(c_dev[0, h])
            if not norm:   # V^T (D, ldv) -> (Skv, D)
                got_c = np.ascontiguousarray(got_c[:, :C2.Skv].T)
            assert np.array_equal(got_c, codes[h]), h
        ora.append((s, codes))
        del bits
    got = out[0, heads][:, torch.from_numpy(rows).to(gpu)].cpu().numpy()
    ref = np.stack([native.attn_rows(ora[0][1][h], ora[1][1][h], ora[2][1][h], ora[0][0],
                                     ora[1][0], ora[2][0], C2.D ** -0.5, rows,
                                     block_n=ops.BLOCK_N) for h in heads])
    _check(got, ref, f"c2 per-tensor heads {heads} rows 128")
    assert torch.isfinite(out).all()
    del q, k, v, out, q8, k8, vt8
    torch.cuda.empty_cache()


def test_zero_softmax_scale_gives_mean_of_visible_values(gpu: torch.device) -> None:
    """scale = 0: the reference scales the scores before masking them, so each
    row averages the values it may see (SDPA does the same).  Causal and a
    ragged key range exercise the masked paths."""
    g = torch.Generator().manual_seed(41)
    S, D = 300, 64
    q, k, v = (torch.randn(1, 2, S, D, generator=g).to(torch.bfloat16) for _ in range(3))
    from oracle import quant

    for causal in (False, True):
        out = ops.fp8_flash_attention(q.to(gpu), k.to(gpu), v.to(gpu), causal=causal, scale=0.0,
                                      out_dtype=torch.float32).cpu().numpy()[0]
        assert np.isfinite(out).all(), causal
        ref, _ = _oracle_rows(q, k, v, [0, 1], np.arange(S), sm_scale=0.0,
                              mask=1 if causal else 0)
        _check(out, ref, f"scale=0 causal={causal}")
        # closed form: the running mean of the dequantized values
        vs, v8 = native.quantize_groups(bf16_bits(v), 2)
        vd = np.stack([quant.decode_e4m3fn(v8[0, h]) * vs[h] for h in range(2)])
        mean = (np.cumsum(vd, axis=1) / np.arange(1, S + 1)[None, :, None] if causal
                else np.broadcast_to(vd.mean(axis=1, keepdims=True), vd.shape))
        assert np.abs(out - mean).max() < 2e-2, causal


# ----------------------------------------------------------------------------
# The reference's own acceptance tests, re-expressed against this package's op
# (tests/test_attention_fp8.py:102-154, tests/test_fp8_attention_ada.py:115-201).

def _sdpa_case(gpu: torch.device, shape: tuple[int, int, int, int]):
    torch.manual_seed(0)
    q = torch.randn(*shape, device=gpu, dtype=torch.bfloat16) / 8.0
    k = torch.randn(*shape, device=gpu, dtype=torch.bfloat16) / 8.0
    v = torch.randn(*shape, device=gpu, dtype=torch.bfloat16)
    return q, k, v


def _rel_vs_sdpa(out: torch.Tensor, ref: torch.Tensor) -> float:
    return ((out.float() - ref.float()).abs().mean() / ref.float().abs().mean()).item()


@pytest.mark.parametrize("shape,causal,bound", [
    ((1, 4, 256, 64), False, 0.15),      # test_attention_fp8.py:102-126
    ((1, 4, 256, 64), True, 0.15),       # test_attention_fp8.py:129-154
    ((1, 8, 4096, 128), False, 0.10),    # test_fp8_attention_ada.py:115-146
    ((1, 8, 4096, 64), False, 0.10),     # test_fp8_attention_ada.py:149-172
    ((1, 8, 4096, 128), True, 0.10),     # test_fp8_attention_ada.py:175-201
])
def test_op_matches_sdpa_like_the_reference(gpu: torch.device, shape: tuple, causal: bool,
                                            bound: float) -> None:
    from repercep_runtime_amd.attention import FP8HipAttention, NaiveAttention

    op = FP8HipAttention()
    assert op.available
    q, k, v = _sdpa_case(gpu, shape)
    ref = NaiveAttention()(q.float(), k.float(), v.float(), causal=causal)
    out = op(q, k, v, causal=causal)
    assert out.shape == ref.shape and out.dtype == torch.bfloat16
    assert torch.isfinite(out).all()
    rel = _rel_vs_sdpa(out, ref)
    print(f"{shape} causal={causal}: mean rel vs SDPA {rel:.4f}", flush=True)
    assert rel < bound


def test_diffusers_bridge_runs_fp8_kernel_on_bshd(gpu: torch.device) -> None:
    """(B, S, H, D) through the dispatcher bridge: FP8 branch taken, equal to
    the op on permuted copies, within tolerance of the oracle, close to SDPA."""
    from repercep_runtime_amd.attention import diffusers_backend as db

    g = torch.Generator(device=gpu).manual_seed(4)
    q = torch.randn(1, 4096, 4, 128, device=gpu, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 4096, 4, 128, device=gpu, generator=g).to(torch.bfloat16)
    v = torch.randn(1, 4096, 4, 128, device=gpu, generator=g).to(torch.bfloat16)
    assert db._route_should_use_fp8(q, k, v)
    out = db._repercep_fp8_attention(q, k, v)
    via_op = ops.fp8_flash_attention(q.permute(0, 2, 1, 3).contiguous(),
                                     k.permute(0, 2, 1, 3).contiguous(),
                                     v.permute(0, 2, 1, 3).contiguous())
    assert torch.equal(out, via_op.permute(0, 2, 1, 3))
    # the (B, S, H, D) result itself against the oracle on the same inputs
    rows = np.sort(np.random.default_rng(4).choice(4096, size=384, replace=False))
    bhsd = [t.permute(0, 2, 1, 3).contiguous().cpu() for t in (q, k, v)]
    oref, _ = _oracle_rows(*bhsd, list(range(4)), rows, sm_scale=128 ** -0.5)
    got = out[0, torch.from_numpy(rows).to(gpu)].permute(1, 0, 2).float().cpu().numpy()
    _check(got, torch.from_numpy(oref).to(torch.bfloat16).float().numpy(), "bridge (B,S,H,D)")
    ref = torch.nn.functional.scaled_dot_product_attention(
        q.permute(0, 2, 1, 3).float(), k.permute(0, 2, 1, 3).float(),
        v.permute(0, 2, 1, 3).float()).permute(0, 2, 1, 3)
    assert _rel_vs_sdpa(out, ref) < 0.10


def test_operands_off_the_gpu_are_refused(gpu: torch.device) -> None:
    """Scales or an output buffer in host memory would be dereferenced by the
    kernel: refused on the host before any launch, like codes of a wrong dtype."""
    q8 = torch.zeros(1, 1, 128, 64, dtype=torch.uint8, device=gpu)
    vt8 = torch.zeros(1, 1, 64, 128, dtype=torch.uint8, device=gpu)
    one = torch.ones(1, device=gpu)
    with pytest.raises(ValueError, match="GPU tensor"):
        ops.attention_fp8(q8, q8, vt8, one.cpu(), one, one, 0.125)
    with pytest.raises(ValueError, match="GPU tensor"):
        ops.attention_fp8(q8, q8, vt8, one, one, one, 0.125,
                          out=torch.empty(1, 1, 128, 64, dtype=torch.bfloat16))
    with pytest.raises(TypeError, match="codes"):
        ops.attention_fp8(q8.to(torch.bfloat16), q8, vt8, one, one, one, 0.125)
    a = torch.zeros(32, 32, dtype=torch.uint8, device=gpu)
    with pytest.raises(ValueError, match="GPU tensor"):
        ops.fp8_gemm(a, a, torch.ones(1), 1.0, b_transposed=True)
    out = ops.attention_fp8(q8, q8, vt8, one, one, one, 0.125)
    assert torch.equal(out, torch.zeros_like(out))      # all-zero codes: mean of zero V


def test_diffusers_bridge_recomputes_non_finite_output_with_sdpa(gpu: torch.device,
                                                                 monkeypatch: pytest.MonkeyPatch,
                                                                 caplog) -> None:
    """The bridge's guard (reference diffusers_backend.py, non-finite check
    after the FP8 call): a non-finite FP8 result is replaced by native SDPA's
    output for the same call, with a warning.  First forced (the FP8 call
    writes NaN), then real: an infinite V entry makes its head's FP8 output
    NaN, and the call returns exactly what SDPA returns for it."""
    import logging

    from repercep_runtime_amd.attention import diffusers_backend as db

    g = torch.Generator(device=gpu).manual_seed(6)
    q, k, v = (torch.randn(1, 4096, 2, 64, device=gpu, generator=g).to(torch.bfloat16)
               for _ in range(3))
    assert db._route_should_use_fp8(q, k, v)       # past the bridge's length crossover
    sdpa = torch.nn.functional.scaled_dot_product_attention(
        q.permute(0, 2, 1, 3), k.permute(0, 2, 1, 3), v.permute(0, 2, 1, 3)).permute(0, 2, 1, 3)

    def nan_fp8(*_a, out, **_k):
        out.fill_(float("nan"))
        return out

    with monkeypatch.context() as m:
        m.setattr(ops, "fp8_flash_attention", nan_fp8)
        with caplog.at_level(logging.WARNING):
            out = db._repercep_fp8_attention(q, k, v)
    assert torch.equal(out, sdpa)
    assert "non-finite" in caplog.text

    v_inf = v.clone()
    v_inf[0, 7, 1, 3] = float("inf")
    fp8 = ops.fp8_flash_attention(q.permute(0, 2, 1, 3), k.permute(0, 2, 1, 3),
                                  v_inf.permute(0, 2, 1, 3))
    assert not torch.isfinite(fp8[0, 1]).all() and torch.isfinite(fp8[0, 0]).all()
    out = db._repercep_fp8_attention(q, k, v_inf)
    ref = torch.nn.functional.scaled_dot_product_attention(
        q.permute(0, 2, 1, 3), k.permute(0, 2, 1, 3),
        v_inf.permute(0, 2, 1, 3)).permute(0, 2, 1, 3)
    torch.testing.assert_close(out, ref, rtol=0, atol=0, equal_nan=True)


@pytest.mark.parametrize("kind", ["sharp", "rising_max"])
def test_softmax_extremes_vs_oracle(gpu: torch.device, kind: str) -> None:
    """Rows whose scores are dominated by one key (Q and K scaled by 6), and
    keys whose scale rises along the sequence so that the running max moves at
    almost every tile (the O^T rescale and alpha path run constantly)."""
    g = torch.Generator().manual_seed(31 if kind == "sharp" else 32)
    B, H, S, D = (1, 2, 700, 128) if kind == "sharp" else (1, 2, 900, 64)
    q = torch.randn(B, H, S, D, generator=g)
    k = torch.randn(B, H, S, D, generator=g)
    v = torch.randn(B, H, S, D, generator=g)
    if kind == "sharp":
        q, k = q * 6.0, k * 6.0
    else:
        k = k * torch.linspace(0.2, 4.0, S).reshape(1, 1, S, 1)
    q, k, v = (t.to(torch.bfloat16) for t in (q, k, v))
    out = ops.fp8_flash_attention(q.to(gpu), k.to(gpu), v.to(gpu),
                                  out_dtype=torch.float32).cpu().numpy()[0]
    ref, _ = _oracle_rows(q, k, v, list(range(H)), np.arange(S), sm_scale=D ** -0.5)
    # both kinds make peaked rows (one or a few dominant keys): outputs exceed 1
    _check(out, ref, f"{kind} (1, {H}, {S}, {D})", scaled=True)


WSPLIT_CASES = [
    # name, B, H, Sq, Skv, D, mask, prefix, suffix, block_m, in dtype, out dtype, granularity
    ("c1_bm32", 1, 8, 1024, 1024, 64, 0, 0, 1, 32, torch.bfloat16, torch.bfloat16, "tensor"),
    ("c1_bm64_f32", 1, 8, 1024, 1024, 64, 0, 0, 1, 64, torch.bfloat16, torch.float32, "bh"),
    ("c1_bm128", 1, 8, 1024, 1024, 64, 0, 0, 1, 128, torch.bfloat16, torch.float32, "bh"),
    ("c5_bm32", 1, 32, 128, 640, 128, 2, 512, 8, 32, torch.bfloat16, torch.float32, "tensor"),
    ("c5_bm64_bf16", 1, 32, 128, 640, 128, 2, 512, 8, 64, torch.bfloat16, torch.bfloat16,
     "tensor"),
    # a ragged last tile, shifted back, opening the last split
    ("causal_ragged", 1, 2, 700, 700, 128, 1, 0, 1, 32, torch.bfloat16, torch.float32, "bh"),
    # splits wholly past a block's queries: skipped, left out of the merge
    ("causal_kv_longer", 1, 2, 300, 1000, 64, 1, 0, 1, 64, torch.float16, torch.float16, "bh"),
    ("cross_ragged", 2, 2, 300, 1000, 128, 0, 0, 1, 64, torch.bfloat16, torch.float32, "bh"),
    ("short_kv", 1, 1, 100, 100, 64, 0, 0, 1, 32, torch.bfloat16, torch.float32, "bh"),
    # 18 tiles: six splits of three tiles per wave
    ("three_tiles_per_wave", 1, 2, 256, 2200, 128, 0, 0, 1, 32, torch.bfloat16, torch.float32,
     "bh"),
    ("ragged_sq", 1, 3, 77, 513, 64, 0, 0, 1, 128, torch.bfloat16, torch.float32, "bh"),
]


@pytest.mark.parametrize("case", WSPLIT_CASES, ids=[c[0] for c in WSPLIT_CASES])
def test_wave_split_launch_vs_oracle(gpu: torch.device, case: tuple) -> None:
    """rp_fp8_attn_fwd_wsplit against the one-range oracle (the reference's
    loop over 128-key tiles): each wave starts from the running max of the
    tiles before its run, so P is quantized on the reference's grid and the
    usual tolerance holds, not only the key-split one; the run plan is the
    host's (tuning.wsplit_plan); rows past Sq of a strided output are left
    untouched."""
    import ctypes

    from oracle import quant
    from repercep_runtime_amd import _capi, tuning

    name, B, H, Sq, Skv, D, mask, prefix, suffix, bm, dt, odt, gran = case
    st, ns = ctypes.c_int(), ctypes.c_int()
    assert _capi.lib().rp_fp8_attn_wsplit_plan(Skv, bm, ctypes.byref(st), ctypes.byref(ns)) == 0
    assert (st.value, ns.value) == tuning.wsplit_plan(Skv, bm)
    g = torch.Generator().manual_seed(sum(map(ord, name)))
    q = torch.randn(B, H, Sq, D, generator=g).to(dt)
    k = torch.randn(B, H, Skv, D, generator=g).to(dt)
    v = torch.randn(B, H, Skv, D, generator=g).to(dt)
    qs, q8, ks, k8, vs, vt8 = ops.scale_quantize_qkv(q.to(gpu), k.to(gpu), v.to(gpu), gran)
    big = torch.full((B, H, Sq + 3, D), float("nan"), dtype=odt, device=gpu)
    out = big[:, :, :Sq]
    ops.attention_fp8(q8.view(torch.uint8), k8.view(torch.uint8), vt8.view(torch.uint8), qs, ks,
                      vs, D ** -0.5, out=out, causal=mask == 1,
                      prefix_len=prefix if mask == 2 else None,
                      suffix_len=suffix if mask == 2 else None, block_m=bm)
    torch.cuda.synchronize()
    assert torch.isnan(big[:, :, Sq:].float()).all(), "rows past Sq were written"
    got = out.float().cpu().numpy()
    for b in range(B):
        sl = slice(b, b + 1)
        cq, c8q = quant.quantize_codes(q[sl], gran)
        ck, c8k = quant.quantize_codes(k[sl], gran)
        cv, c8v = quant.quantize_codes(v[sl], gran)
        for h in range(H):
            si = h if gran == "bh" else 0
            ref = native.attn_rows(c8q[0, h], c8k[0, h], c8v[0, h], cq[si], ck[si], cv[si],
                                   D ** -0.5, np.arange(Sq), block_n=ops.BLOCK_N, mask=mask,
                                   prefix=prefix, suffix=suffix)
            if odt != torch.float32:
                ref = torch.from_numpy(ref).to(odt).float().numpy()
            _check(got[b, h], ref, f"{name} b={b} h={h} runs={ns.value}x{st.value}")


def test_wave_split_launch_equals_one_range_launch(gpu: torch.device) -> None:
    """Same tiles, same running maxima: the short-query launch and the
    256-row one-range launch agree to fp32 rounding of the merge (which
    multiplies out the rescale factors of later tiles), far inside the FP8
    tolerance, at every block height."""
    q, k, v = attn_inputs(C1)
    qs, q8, ks, k8, vs, vt8 = ops.scale_quantize_qkv(q.to(gpu), k.to(gpu), v.to(gpu), "tensor")
    args = (q8.view(torch.uint8), k8.view(torch.uint8), vt8.view(torch.uint8), qs, ks, vs,
            C1.D ** -0.5)
    one = ops.attention_fp8(*args, out_dtype=torch.float32).cpu().numpy()
    for bm in ops.WSPLIT_BLOCK_MS:
        ws = ops.attention_fp8(*args, out_dtype=torch.float32, block_m=bm).cpu().numpy()
        st = err_stats(ws, one)
        print(f"block_m={bm} vs the one-range launch: {st}", flush=True)
        assert st["max_abs"] <= 1e-3 and st["rel_mean"] <= 1e-4, (bm, st)


def test_wave_split_launch_refuses_other_shapes(gpu: torch.device) -> None:
    """Head dims outside {64, 128} and other block heights are refused with
    the library's message, before any launch."""
    q8 = torch.zeros(1, 1, 128, 32, dtype=torch.uint8, device=gpu)
    vt8 = torch.zeros(1, 1, 32, 128, dtype=torch.uint8, device=gpu)
    one = torch.ones(1, device=gpu)
    with pytest.raises(RuntimeError, match="head dim 32"):
        ops.attention_fp8(q8, q8, vt8, one, one, one, 0.125, block_m=32)
    q8 = torch.zeros(1, 1, 128, 64, dtype=torch.uint8, device=gpu)
    vt8 = torch.zeros(1, 1, 64, 128, dtype=torch.uint8, device=gpu)
    with pytest.raises(ValueError, match="block_m"):
        ops.attention_fp8(q8, q8, vt8, one, one, one, 0.125, block_m=48)
    with pytest.raises(ValueError, match="block_m"):
        ops.attention_fp8(q8, q8, vt8, one, one, one, 0.125, block_m=64, kv_splits=2)
