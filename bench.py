"""Benchmark of the MI355X FP8 attention hot path (one JSON line on stdout).

Default workload: BASELINE config 3, Wan-2.2 self-attention
(B=1, H=40, S=75600, D=128, non-causal), bf16 inputs resident in HBM.
One step = the whole hot path on one batch: amax scale + e4m3fn quantization
of Q, K and V (V written transposed) followed by the FP8 flash-attention
forward writing bf16 output -- the work of the reference's
``fp8_flash_attention`` call.  As ``fp8_flash_attention`` does for a
256-row launch, the step hands the attention Q as it lies with its scale and
the kernel quantizes Q's rows itself (the same codes) on resident-K/V
launches (``--codes-q`` runs the two-step form there too).  Scales are per tensor by default, as BASELINE
configs 2-5 state them (``--granularity bh`` runs the reference's per-(B,H)
scales; the attention kernel's work is the same either way).

``value`` is whole-step throughput in TFLOP/s (algorithmic FLOPs
4*B*H*S^2*D per step / step time).  ``roofline`` is the attention kernel's
own MFMA roofline, its average launch time measured with HIP events on the
stream the kernel runs on; its ``traffic`` (HBM bytes per launch) is read from
profiles/traffic.json, which the rocprofv3 counter runs wrote, and says so in
``traffic_source``.  ``quantize`` reports the quantizer's HBM rate (5 bytes
per element).  ``cpu_baseline`` times the reference's own CPU attention path
(AMXSDPAAttention: one torch SDPA call in bf16 on all host cores) on a
bounded sample, and ``cpu_oracle`` the C restatement of the reference's FP8
attention (the test oracle) on another.  Beside them, as the reference's
scripts/bench_fp8.py reports its FP8 op: ``whole_op`` times the op as a caller
runs it (``FP8HipAttention.__call__``, host work included) and ``sdpa_gpu``
times torch SDPA in bf16 on the same GPU and inputs.  Step and kernel times
are medians over the timed calls (HIP events on the launch stream).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config NAME]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import tempfile
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

FP8_PEAK_TFLOPS = 5000.0  # MI355X dense FP8 MFMA, published
HBM_PEAK_GBPS = 8000.0    # MI355X HBM3E, published
GRAPH_CALLS = 20          # attention launches per captured graph (--graph)
TRAFFIC_SOURCE = ("profiles/traffic.json: FETCH_SIZE + WRITE_SIZE per launch from two "
                  "rocprofv3 --pmc runs of this bench, scaled by a plain copy's readings; "
                  "not measured in this run")


def log(*a: object) -> None:
    print(*a, file=sys.stderr, flush=True)


def _traffic_from_profiles(kernel: str, workload: str) -> float | None:
    """HBM bytes per launch recorded by the rocprofv3 counter runs under profiles/."""
    f = ROOT / "profiles" / "traffic.json"
    if not f.exists():
        return None
    try:
        data = json.loads(f.read_text())
        return float(data[workload][kernel]["hbm_bytes_per_launch"])
    except (KeyError, ValueError, TypeError, json.JSONDecodeError):
        return None


def _grow(run, start: int, limit: int, budget_s: float) -> tuple[int, float, int]:
    """Grow a row count by 4x until one timed run takes about budget_s / 4 or
    more.  A workload whose whole row count runs faster than that is timed
    over repeated calls instead (one millisecond-scale call is mostly noise).
    Returns (rows, mean seconds per call, calls timed)."""
    rows = min(start, limit)
    run(rows)  # warm-up (thread pool, allocator, page faults)
    t = run(rows)
    while rows < limit and t < budget_s / 4:
        rows = min(limit, rows * 4)
        t = run(rows)
    calls = 1
    if t < budget_s / 4:
        calls = max(1, min(10000, int(budget_s / 4 / max(t, 1e-6))))
        t = sum(run(rows) for _ in range(calls)) / calls
    return rows, t, calls


def _calls_note(t: float, calls: int) -> str:
    return f"in {t:.2f} s" if calls == 1 else f"in {t * 1e3:.3f} ms (mean of {calls} calls)"


def _secs(t: float) -> str:
    return f"{t:.0f} s" if t >= 10 else (f"{t:.2f} s" if t >= 0.1 else f"{t * 1e3:.3f} ms")


def cpu_oracle_timing(cfg, budget_s: float) -> dict:
    """The CPU oracle (C restatement of the reference's FP8 attention, OpenMP
    over query rows) on one head of the workload: a row slice of the queries
    against all keys, scaled to the workload's FLOPs.  Reported beside the
    baseline, not as it."""
    import numpy as np
    import torch

    from oracle import native
    from oracle.cpu_sdpa import cpu_model

    gen = torch.Generator().manual_seed(cfg.seed)
    k = torch.randn(cfg.Skv, cfg.D, generator=gen).to(torch.bfloat16)
    v = torch.randn(cfg.Skv, cfg.D, generator=gen).to(torch.bfloat16)
    q = torch.randn(min(cfg.Sq, 65536), cfg.D, generator=gen).to(torch.bfloat16)
    bits = [t.view(torch.int16).numpy().view(np.uint16) for t in (q, k, v)]
    (qs,), q8 = native.quantize_groups(bits[0], 1)
    (ks,), k8 = native.quantize_groups(bits[1], 1)
    (vs,), v8 = native.quantize_groups(bits[2], 1)
    threads = native.num_threads()

    def run(rows: int) -> float:
        idx = np.arange(rows, dtype=np.int32)
        t0 = time.perf_counter()
        native.attn_rows(q8, k8, v8, qs, ks, vs, cfg.D ** -0.5, idx)
        return time.perf_counter() - t0

    rows, t, calls = _grow(run, 16, q8.shape[0], budget_s)
    tflops = 4.0 * rows * cfg.Skv * cfg.D / t / 1e12
    return {
        "value": round(tflops, 5),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"C oracle (tile-exact FP8 emulation, {threads} OpenMP threads, "
                   f"{cpu_model()}): 1 head, {rows} query rows x {cfg.Skv} keys x D={cfg.D} "
                   f"{_calls_note(t, calls)}; full {cfg.name} extrapolates to "
                   f"{_secs(cfg.flops / (tflops * 1e12))}"),
    }


def cpu_sdpa_baseline(cfg, budget_s: float) -> dict:
    """The reference's CPU attention path -- the registry's CPU floor
    AMXSDPAAttention, whose call is one torch SDPA in bf16
    (src/repercep/attention/amx_sdpa.py:76-94, registry.py:126) -- on all host
    cores, on one head: a row slice of the queries against all keys, scaled
    to the workload's FLOPs."""
    import torch

    from oracle.cpu_sdpa import cpu_model, cpu_threads, sdpa_cpu

    threads = cpu_threads()
    gen = torch.Generator().manual_seed(cfg.seed)
    k = torch.randn(1, 1, cfg.Skv, cfg.D, generator=gen).to(torch.bfloat16)
    v = torch.randn(1, 1, cfg.Skv, cfg.D, generator=gen).to(torch.bfloat16)

    def run(rows: int) -> float:
        q = torch.randn(1, 1, rows, cfg.D, generator=gen).to(torch.bfloat16)
        t0 = time.perf_counter()
        sdpa_cpu(q, k, v)
        return time.perf_counter() - t0

    rows, t, calls = _grow(run, 256, cfg.Sq, budget_s)
    tflops = 4.0 * rows * cfg.Skv * cfg.D / t / 1e12
    return {"value": round(tflops, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": (f"the reference's CPU attention path (AMXSDPAAttention = torch SDPA "
                       f"bf16, {threads} threads, {cpu_model()}): 1 head, {rows} query rows x "
                       f"{cfg.Skv} keys x D={cfg.D} {_calls_note(t, calls)}; full {cfg.name} "
                       f"extrapolates to {_secs(cfg.flops / (tflops * 1e12))}")}


def bench_attention(args, cfg) -> dict:
    import torch

    from repercep_runtime_amd import _capi, ops
    from repercep_runtime_amd.workloads import QUANT_BYTES_PER_ELEM, attn_inputs

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    log(f"[bench] generating {cfg.name} inputs on {dev}")
    # configs with QK RMSNorm take pre-norm Q/K: the norm runs fused into
    # their quantizers inside the step (rmsnorm_scale_quantize_qkv)
    fused_norm = cfg.rmsnorm_qk
    gran = args.granularity
    q, k, v = attn_inputs(cfg, device=dev, normalize=not fused_norm)
    sm = cfg.D ** -0.5
    prefix = cfg.prefix
    out = torch.empty_like(q)
    st = torch.cuda.current_stream(dev)
    # launch configuration as the op resolves it (a timed search on a cache
    # miss for shapes too small to fill the GPU unsplit; see tuning.py)
    if fused_norm:
        ops.fp8_flash_attention_qknorm(q, k, v, causal=cfg.causal, out=out, granularity=gran)
    else:
        ops.fp8_flash_attention(q, k, v, causal=cfg.causal, prefix_len=prefix,
                                suffix_len=cfg.suffix, out=out, granularity=gran)
    if args.kv_splits is not None or args.block_m is not None:
        block_m = args.block_m or ops.BLOCK_M
        splits = 1 if args.kv_splits is None else args.kv_splits
    else:
        block_m, splits = ops.tuned_launch(cfg.B, cfg.H, cfg.Sq, cfg.Skv, cfg.D, cfg.causal,
                                           prefix, cfg.suffix)
    # what fp8_flash_attention runs for a resident-K/V launch: the quantizer
    # writes K's and V^T's codes and every scale, the attention quantizes its
    # own Q rows (the same codes, the same output)
    mask = 1 if cfg.causal else (2 if prefix is not None else 0)
    q16 = (not fused_norm and block_m == ops.BLOCK_M and not args.codes_q
           and ops.q16_pays(cfg.B, cfg.H, cfg.Sq, cfg.Skv, cfg.D, mask, splits,
                            ops._stream(q)))
    log(f"[bench] block_m {block_m} kv_splits {splits} q_in_attention {q16}")

    def step(ev=None):
        if ev is not None:
            ev[0].record(st)
        if fused_norm:
            qs, q8, ks, k8, vs, vt8 = ops.rmsnorm_scale_quantize_qkv(q, k, v, granularity=gran)
        elif q16:
            qs, ks, k8, vs, vt8 = ops.scale_quantize_kv(q, k, v, gran)
        else:   # one library call for Q, K, V
            qs, q8, ks, k8, vs, vt8 = ops.scale_quantize_qkv(q, k, v, gran)
        if ev is not None:
            ev[1].record(st)
        if q16:
            ops.attention_fp8_q16(q, k8.view(torch.uint8), vt8.view(torch.uint8), qs, ks, vs, sm,
                                  out=out, causal=cfg.causal, prefix_len=prefix,
                                  suffix_len=cfg.suffix, kv_splits=splits)
        else:
            ops.attention_fp8(q8.view(torch.uint8), k8.view(torch.uint8), vt8.view(torch.uint8),
                              qs, ks, vs, sm, out=out, causal=cfg.causal, prefix_len=prefix,
                              suffix_len=cfg.suffix, kv_splits=splits, block_m=block_m)
        if ev is not None:
            ev[2].record(st)

    log(f"[bench] warmup {args.warmup}")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # whole-step timing: one event between consecutive steps, so the K steps
    # run back to back and each step's time is one interval; ms_per_step is
    # their median, the bracketed mean is reported beside it
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    torch.cuda.synchronize()
    marks[0].record(st)
    for i in range(args.steps):
        step()
        marks[i + 1].record(st)
    torch.cuda.synchronize()
    per_step = [marks[i].elapsed_time(marks[i + 1]) for i in range(args.steps)]
    ms_per_step = statistics.median(per_step)
    mean_ms = marks[0].elapsed_time(marks[-1]) / args.steps
    log(f"[bench] {args.steps} steps: median {ms_per_step:.3f} ms/step (mean {mean_ms:.3f})")

    # per-kernel split (same stream, separate pass so the events do not perturb the above)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    for e in evs:
        step(e)
    torch.cuda.synchronize()
    quant_ms = statistics.median(e[0].elapsed_time(e[1]) for e in evs)
    attn_ms = statistics.median(e[1].elapsed_time(e[2]) for e in evs)
    log(f"[bench] split (medians): quantize {quant_ms:.3f} ms, attention kernel {attn_ms:.3f} ms")

    whole = _whole_op_timing(args, cfg, q, k, v, st)
    sdpa = _sdpa_gpu_timing(args, cfg, q, k, v, st)
    if whole.get("ms") and sdpa.get("ms"):
        sdpa["speedup_of_fp8_whole_op"] = round(sdpa["ms"] / whole["ms"], 3)

    graph = None
    if args.graph:
        # the same step captured in a HIP graph and replayed: what a serving
        # loop runs when host launch work bounds small calls
        g = torch.cuda.CUDAGraph()
        s2 = torch.cuda.Stream(dev)
        s2.wait_stream(st)
        with torch.cuda.stream(s2):
            step()   # warm the capture stream's allocator pool
        st.wait_stream(s2)
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            step()
        g_ms, _ = _time_calls(g.replay, args.steps, args.warmup, st)
        # the attention launch alone: GRAPH_CALLS calls on the same codes in
        # one graph, so one replay interval holds GRAPH_CALLS kernel times
        qs, q8, ks, k8, vs, vt8 = ops.scale_quantize_qkv(q, k, v, gran)
        attn = lambda: ops.attention_fp8(  # noqa: E731
            q8.view(torch.uint8), k8.view(torch.uint8), vt8.view(torch.uint8), qs, ks, vs, sm,
            out=out, causal=cfg.causal, prefix_len=prefix, suffix_len=cfg.suffix,
            kv_splits=splits, block_m=block_m)
        with torch.cuda.stream(s2):
            attn()
        st.wait_stream(s2)
        torch.cuda.synchronize()
        ga = torch.cuda.CUDAGraph()
        with torch.cuda.graph(ga):
            for _ in range(GRAPH_CALLS):
                attn()
        ga_ms, _ = _time_calls(ga.replay, max(3, args.steps // 4), 2, st)
        graph = {"ms_per_step": round(g_ms, 4),
                 "value": round(cfg.flops / (g_ms * 1e-3) / 1e12, 2),
                 "attention_ms_per_call": round(ga_ms / GRAPH_CALLS, 5),
                 "note": "the step captured once with torch.cuda.graph, then replayed back "
                         f"to back (median replay interval); attention_ms_per_call: a graph "
                         f"of {GRAPH_CALLS} attention launches on the same codes, replayed, "
                         f"per launch"}
        log(f"[bench] graph attention: {ga_ms / GRAPH_CALLS * 1e3:.2f} us per call")
        log(f"[bench] graph replay: {g_ms:.4f} ms/step")

    tflops_step = cfg.flops / (ms_per_step * 1e-3) / 1e12
    tflops_attn = cfg.flops / (attn_ms * 1e-3) / 1e12
    # the launches between the attention events: a balanced launch whose plan
    # splits the last round's blocks is followed by the merge of their rows
    mask = 1 if cfg.causal else (2 if prefix is not None else 0)
    merged = splits != 1 and (splits > 1 or _capi.lib().rp_fp8_attn_balanced_workspace_bytes(
        cfg.B, cfg.H, cfg.Sq, cfg.Skv, cfg.D, mask, ops._stream(q)) > 0)
    attn_launches = ("attn_fwd_kernel + attn_combine_kernel (the merge of the key-split rows)"
                     if merged else "attn_fwd_kernel")
    if merged and splits == 0:   # the balanced launch clears its item counter first
        attn_launches = "attn_zero_counter_kernel + " + attn_launches
    kernel = "attn_fwd_kernel"
    if not merged and splits in (0, 1) and _capi.lib().rp_fp8_attn_resident_kv(
            cfg.B, cfg.H, cfg.Sq, cfg.Skv, cfg.D, mask, 1):
        # a plain launch whose key range fits LDS runs the resident-K/V kernel
        kernel = attn_launches = "attn_kvres_kernel"
        if q16:
            attn_launches += " (quantizing Q's rows from the bf16 input as it reads them)"
    if block_m != ops.BLOCK_M:   # the short-query launch merges its splits itself
        kernel = attn_launches = "attn_wsplit_kernel"
    qbytes = QUANT_BYTES_PER_ELEM * cfg.quant_elems
    if q16:   # Q is read once by the quantizer (its amax), its codes never stored
        qbytes -= (QUANT_BYTES_PER_ELEM - 2) * cfg.B * cfg.H * cfg.Sq * cfg.D
    q_gbps = qbytes / (quant_ms * 1e-3) / 1e9
    res = {
        "metric": "FP8 attn TFLOP/s + % FP8-MFMA peak (Wan-2.2 S=75600); quantize GB/s",
        "value": round(tflops_step, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "ms_per_step_mean": round(mean_ms, 4),
        "timing": ("ms_per_step and every *_ms figure: the median over the timed calls of "
                   "HIP-event intervals on the launch stream; ms_per_step_mean: the "
                   "bracketed region / steps"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3fn (fp32 accumulate, bf16 out)",
        "data": "synthetic: seeded N(0,1) bf16 Q/K/V generated on the GPU",
        "config": {"workload": cfg.name, "B": cfg.B, "H": cfg.H, "Sq": cfg.Sq, "Skv": cfg.Skv,
                   "D": cfg.D, "causal": cfg.causal,
                   "scale_granularity": "per tensor" if gran == "tensor" else "per (b,h)",
                   "block_m": block_m, "kv_splits": splits, "flops_per_step": cfg.flops},
        "roofline": {
            "bound": "mfma",
            "achieved": round(tflops_attn, 2),
            "peak": FP8_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(tflops_attn / FP8_PEAK_TFLOPS, 4),
            "traffic": _traffic_from_profiles(kernel, cfg.name),
            "traffic_source": TRAFFIC_SOURCE,
            "kernel": kernel,
            "kernel_ms": round(attn_ms, 4),
            "kernel_ms_covers": attn_launches,
        },
        "quantize": {
            "achieved_GBps": round(q_gbps, 1),
            "peak_GBps": HBM_PEAK_GBPS,
            "frac": round(q_gbps / HBM_PEAK_GBPS, 4),
            "ms": round(quant_ms, 4),
            "bytes": qbytes,
            "note": ("Q, K with RMSNorm fused, V plain: one multi-tensor amax pass + "
                     "finalize + apply (V transposed); 5 B/element" if fused_norm else
                     "Q's scale and K, V codes: one multi-tensor amax pass + finalize + "
                     "apply of K and V (V transposed); Q read once (2 B/element), K and V "
                     "5 B/element; the attention kernel quantizes Q's rows as it reads "
                     "them" if q16 else
                     "Q, K, V: one multi-tensor amax pass + finalize + apply (V "
                     "transposed), 5 B/element"),
        },
        "whole_op_ms": whole.get("ms"),
        "whole_op": whole,
        "sdpa_gpu": sdpa,
        **({"graph": graph} if graph else {}),
    }
    del q, k, v, out
    return res


def _time_calls(fn, steps: int, warmup: int, st) -> tuple[float, float]:
    """(median ms per call from HIP events around each call, mean wall ms per
    call over the same calls, host time included, synchronised at the end --
    the reference's scripts/bench_fp8.py:47-76 measurement)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    t0 = time.perf_counter()
    marks[0].record(st)
    for i in range(steps):
        fn()
        marks[i + 1].record(st)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps * 1e3
    return statistics.median(marks[i].elapsed_time(marks[i + 1]) for i in range(steps)), wall


def _whole_op_timing(args, cfg, q, k, v, st) -> dict:
    """The op as a caller runs it: ``FP8HipAttention.__call__`` -- quantize,
    launch-configuration lookup, attention and the output allocation, host
    work included -- on the config's inputs (QK-normalised ones for a config
    whose processor normalises Q and K before dispatch).  The shared-prefix
    config has no AttentionOp form (the Protocol takes no mask): it times
    ``ops.fp8_flash_attention`` with its prefix arguments."""
    import torch

    from repercep_runtime_amd import ops
    from repercep_runtime_amd.attention import FP8HipAttention
    from repercep_runtime_amd.workloads import rmsnorm_heads

    if cfg.rmsnorm_qk:
        q, k = rmsnorm_heads(q), rmsnorm_heads(k)
    if cfg.prefix is not None:
        what = "ops.fp8_flash_attention(q, k, v, prefix_len, suffix_len)"
        fn = lambda: ops.fp8_flash_attention(q, k, v, prefix_len=cfg.prefix,  # noqa: E731
                                             suffix_len=cfg.suffix)
    else:
        op = FP8HipAttention()
        what = "FP8HipAttention()(q, k, v" + (", causal=True)" if cfg.causal else ")")
        fn = lambda: op(q, k, v, causal=cfg.causal)  # noqa: E731
    ms, wall = _time_calls(fn, args.steps, args.warmup, st)
    log(f"[bench] whole op: {ms:.4f} ms (wall {wall:.4f} ms)")
    return {"call": what, "ms": round(ms, 4), "wall_ms": round(wall, 4),
            "TFLOPs": round(cfg.flops / (ms * 1e-3) / 1e12, 2),
            "note": "bf16 in, bf16 out; ms: median of event intervals, wall_ms: mean wall "
                    "time per call, host work included"}


def _sdpa_gpu_timing(args, cfg, q, k, v, st) -> dict:
    """torch SDPA in bf16 on the same GPU and inputs (the reference's
    NaiveAttention, which its bench_fp8.py sets beside the FP8 op), restricted
    to the fused flash and memory-efficient backends: the math backend would
    materialise the (Sq, Skv) scores of every head."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from repercep_runtime_amd.workloads import rmsnorm_heads

    if cfg.rmsnorm_qk:
        q, k = rmsnorm_heads(q), rmsnorm_heads(k)
    mask = None
    if cfg.prefix is not None:
        # the shared-prefix candidates: query i sees the prefix, and suffix key
        # j (kv - prefix) of its own candidate when j <= i
        i = torch.arange(cfg.Sq, device=q.device)[:, None]
        kv = torch.arange(cfg.Skv, device=q.device)[None, :]
        j = kv - cfg.prefix
        mask = (kv < cfg.prefix) | ((j >= 0) & (j // cfg.suffix == i // cfg.suffix) & (j <= i))
    try:
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            fn = lambda: F.scaled_dot_product_attention(  # noqa: E731
                q, k, v, attn_mask=mask, is_causal=cfg.causal)
            ms, wall = _time_calls(fn, args.steps, args.warmup, st)
    except Exception as exc:  # no fused backend for this shape or mask
        log(f"[bench] sdpa: {type(exc).__name__}: {exc}")
        return {"ms": None, "error": f"{type(exc).__name__}: {str(exc)[:200]}"}
    log(f"[bench] sdpa bf16: {ms:.4f} ms (wall {wall:.4f} ms)")
    return {"call": "torch.nn.functional.scaled_dot_product_attention (bf16, flash or "
                    "memory-efficient backend)",
            "ms": round(ms, 4), "wall_ms": round(wall, 4),
            "TFLOPs": round(cfg.flops / (ms * 1e-3) / 1e12, 2),
            "torch": torch.__version__}


def cpu_gemm_baseline(cfg, budget_s: float) -> dict:
    """The GEMM row's CPU path: the layer the FP8 GEMM replaces, a bf16
    nn.Linear, is one torch matmul on the host -- timed on all host cores over
    a slice of the activation rows against the whole weight, scaled to the
    workload's FLOPs."""
    import torch

    from oracle.cpu_sdpa import cpu_model, cpu_threads

    threads = cpu_threads()
    gen = torch.Generator().manual_seed(cfg.seed)
    w = (torch.randn(cfg.K, cfg.N, generator=gen) * 0.02).to(torch.bfloat16)

    def run(rows: int) -> float:
        a = torch.randn(rows, cfg.K, generator=gen).to(torch.bfloat16)
        t0 = time.perf_counter()
        torch.matmul(a, w)
        return time.perf_counter() - t0

    rows, t, calls = _grow(run, 64, cfg.M, budget_s)
    tflops = 2.0 * rows * cfg.N * cfg.K / t / 1e12
    return {"value": round(tflops, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": (f"the layer's CPU path (bf16 nn.Linear = one torch matmul, {threads} "
                       f"threads, {cpu_model()}): {rows} rows x K={cfg.K} x N={cfg.N} "
                       f"{_calls_note(t, calls)}; full {cfg.name} extrapolates to "
                       f"{_secs(cfg.flops / (tflops * 1e12))}")}


def bench_gemm(args, cfg) -> dict:
    import torch

    from repercep_runtime_amd import ops
    from repercep_runtime_amd.workloads import gemm_inputs

    dev = torch.device("cuda", 0)
    a, w = gemm_inputs(cfg, device=dev)
    # weights quantized once, like a loaded layer, in both B layouts: (K, N) as
    # the reference's fp8_gemm takes B, and (N, K) as nn.Linear stores it
    sw, wt8 = ops.fp8_linear_weight(w, layout="nk")
    _, w8 = ops.fp8_linear_weight(w, layout="kn")
    kn = args.b_layout == "kn"
    b_main, b_other = (w8, wt8) if kn else (wt8, w8)
    out = torch.empty((cfg.M, cfg.N), dtype=torch.bfloat16, device=dev)
    st = torch.cuda.current_stream(dev)

    def step(ev=None):
        if ev is not None:
            ev[0].record(st)
        sa, a8 = ops.scale_quantize(a, "tensor", "bhsd")
        if ev is not None:
            ev[1].record(st)
        ops.fp8_gemm(a8.view(torch.uint8), b_main, sa, sw, b_transposed=not kn, out=out)
        if ev is not None:
            ev[2].record(st)

    for _ in range(args.warmup):
        step()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    for e in evs:
        step(e)
    torch.cuda.synchronize()
    step_ms = statistics.median(e[0].elapsed_time(e[2]) for e in evs)
    gemm_ms = statistics.median(e[1].elapsed_time(e[2]) for e in evs)
    quant_ms = statistics.median(e[0].elapsed_time(e[1]) for e in evs)
    tf = cfg.flops / (gemm_ms * 1e-3) / 1e12
    # the other B layout on the same codes: same kernel family, same output bits
    sa, a8 = ops.scale_quantize(a, "tensor", "bhsd")
    a8 = a8.view(torch.uint8)
    other = torch.empty_like(out)
    run_other = lambda: ops.fp8_gemm(a8, b_other, sa, sw, b_transposed=kn, out=other)
    other_ms, _ = _time_calls(run_other, args.steps, args.warmup, st)
    ops.fp8_gemm(a8, b_main, sa, sw, b_transposed=not kn, out=out)
    same = bool(torch.equal(out, other))
    library = _library_gemm(args, cfg, a, wt8, sw, out, st) if args.library_gemm else None
    return {
        "metric": "FP8 scaled GEMM TFLOP/s (Wan FFN up-projection)",
        "value": round(cfg.flops / (step_ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp8_e4m3fn (fp32 accumulate, bf16 out)",
        "data": "synthetic: seeded A ~ N(0,1), W ~ N(0,0.02) bf16",
        "config": {"workload": cfg.name, "M": cfg.M, "K": cfg.K, "N": cfg.N,
                   "b_layout": "(K, N) row-major" if kn else "(N, K)"},
        "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": FP8_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tf / FP8_PEAK_TFLOPS, 4),
                     "traffic": _traffic_from_profiles("gemm256_kernel", cfg.name),
                     "traffic_source": TRAFFIC_SOURCE,
                     "kernel": "gemm256_kernel", "kernel_ms": round(gemm_ms, 4),
                     "kernel_ms_covers": "gemm_zero_counter_kernel + gemm256_kernel (the "
                                         "balanced launch: rp_fp8_linear_balanced)"},
        "quantize": {"ms": round(quant_ms, 4),
                     "achieved_GBps": round(5 * cfg.M * cfg.K / (quant_ms * 1e-3) / 1e9, 1)},
        "other_b_layout": {"b_layout": "(N, K)" if kn else "(K, N) row-major",
                           "kernel_ms": round(other_ms, 4),
                           "TFLOPs": round(cfg.flops / (other_ms * 1e-3) / 1e12, 2),
                           "bit_identical_output": same},
        **({"library_gemm": library} if library else {}),
    }


def _library_gemm(args, cfg, a, wt8, sw, out, st) -> dict:
    """Time the vendor library's FP8 GEMM (torch._scaled_mm, hipBLASLt on
    ROCm) on the same operands and scales, for comparison only; also report
    how far its bf16 output is from this build's."""
    import torch

    from repercep_runtime_amd import ops

    sa, a8 = ops.scale_quantize(a, "tensor", "bhsd")
    ops.fp8_gemm(a8.view(torch.uint8), wt8, sa, sw, b_transposed=True, out=out)
    A = a8.view(torch.float8_e4m3fn).reshape(cfg.M, cfg.K)
    B = wt8.view(torch.float8_e4m3fn).t()
    run = lambda: torch._scaled_mm(A, B, scale_a=sa.reshape(()), scale_b=sw.reshape(()),
                                   out_dtype=torch.bfloat16)
    # the same timing as this build's kernels: median of the intervals
    # between events recorded after each back-to-back call
    ms, _ = _time_calls(run, args.steps, args.warmup, st)
    ref = run()
    torch.cuda.synchronize()
    diff = (ref.float() - out.float()).abs()
    return {"op": "torch._scaled_mm", "ms": round(ms, 4),
            "TFLOPs": round(cfg.flops / (ms * 1e-3) / 1e12, 2),
            "max_abs_diff_vs_ours": float(diff.max()),
            "max_abs_out": float(out.float().abs().max())}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c3_wan_self",
                    help="c1_cpu_runnable | c2_cosmos_self | c3_wan_self | c3_wan_cross | "
                         "c5_shared_prefix | c4_wan_ffn_up")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="run one device-to-device copy of this many MiB first, so a "
                         "rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE run can scale the counters "
                         "against a plain copy of known size")
    ap.add_argument("--graph", action="store_true",
                    help="attention configs: also time the step captured in a HIP graph and "
                         "replayed (small calls are bound by host launch work)")
    ap.add_argument("--library-gemm", action="store_true",
                    help="c4_wan_ffn_up only: also time the vendor library's FP8 GEMM "
                         "(torch._scaled_mm) on the same operands, for comparison")
    ap.add_argument("--granularity", choices=("tensor", "bh"), default="tensor",
                    help="attention configs: scale groups -- per tensor (BASELINE's configs) "
                         "or per (b, h) (the reference wrapper's)")
    ap.add_argument("--b-layout", choices=("kn", "nk"), default="kn",
                    help="c4_wan_ffn_up: the weight operand as the reference's fp8_gemm takes B, "
                         "(K, N) row-major (kn), or transposed (nk); the other is timed beside it")
    ap.add_argument("--block-m", type=int, default=None, choices=(32, 64, 128, 256),
                    help="attention configs: force the query rows per workgroup (32, 64, 128: "
                         "the short-query launch with its keys split over the waves)")
    ap.add_argument("--codes-q", action="store_true",
                    help="write Q's codes in the quantizer and read them in the attention "
                         "launch, instead of the attention quantizing Q's rows itself")
    ap.add_argument("--kv-splits", type=int, default=None,
                    help="attention configs: force a launch configuration (1: one key range, "
                         "0: the balanced launch, n > 1: n key splits) instead of the one the "
                         "op resolves")
    ap.add_argument("--cpu-budget", type=float, default=12.0,
                    help="seconds of CPU work for the cpu_baseline sample (0 disables)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE={world}); the FP8 attention path shards over heads with no "
              f"collective, so one GPU's throughput is the per-GPU figure", file=sys.stderr)
        return 2

    # a run's own launch-configuration cache, unless the caller names one
    os.environ.setdefault("REPERCEP_FP8_AUTOTUNE_CACHE", os.path.join(
        tempfile.gettempdir(), f"repercep_bench_autotune_{os.getpid()}.json"))

    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1

    from repercep_runtime_amd.workloads import ATTN_CONFIGS, C4

    if args.copy_calibration_mib > 0:
        n = args.copy_calibration_mib << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] calibration copy of {args.copy_calibration_mib} MiB done")
        del src, dst
    if args.config == C4.name:
        res = bench_gemm(args, C4)
        if args.cpu_budget > 0:
            log("[bench] timing the CPU baseline")
            res["cpu_baseline"] = cpu_gemm_baseline(C4, args.cpu_budget)
    else:
        cfg = ATTN_CONFIGS[args.config]
        res = bench_attention(args, cfg)
        if args.cpu_budget > 0:
            log("[bench] timing the CPU baseline")
            res["cpu_baseline"] = cpu_sdpa_baseline(cfg, args.cpu_budget)
            res["cpu_oracle"] = cpu_oracle_timing(cfg, args.cpu_budget / 3)
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
