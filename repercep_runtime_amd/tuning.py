"""Per-shape launch configuration of the FP8 attention kernel, cached on disk.

Keeps the reference's persistent autotune cache
(kernels/triton_kernels/fp8_flash_attn.py:52-94, 453-477): a JSON object that
maps ``B{B}_H{H}_Sq{Sq}_Skv{Skv}_D{D}_C{causal}`` to a launch configuration,
written atomically (temporary file, then rename), with a missing, unreadable
or corrupt file read as empty.  ``REPERCEP_FP8_AUTOTUNE_CACHE`` overrides the
path and ``REPERCEP_FP8_DISABLE_AUTOTUNE`` selects the fixed fallback
configuration, as in the reference (:482-499, :551-559).

The gfx950 kernel has one tile shape: 256 query rows in eight waves
(``BLOCK_M``) against 128-key tiles (``BLOCK_N``).  What varies per shape is
``KV_SPLITS``: the number of contiguous key ranges run by separate
workgroups and merged afterwards (``rp_fp8_attn_fwd_split``).  Splitting pays
when the (query block, head) grid alone would leave most of the 256 compute
units idle -- short sequences, few heads -- and costs a merge pass otherwise.
``KV_SPLITS`` 0 is the balanced launch (``rp_fp8_attn_fwd_balanced``): the
query blocks that fill whole rounds of workgroups run over one key range and
the rest key-split, in one launch, so that the last round is not left
mostly idle; grids of two or more rounds get it without a search (2.6%
faster at the Wan shape).  Like the reference's BLOCK_N, a split moves P's
quantization grid (each range keeps its own running max) within the FP8
tolerance.

Entries with ``BLOCK_M`` 32, 64 or 128 (and ``SPLIT_IN_WORKGROUP``) select
the short-query launch (``rp_fp8_attn_fwd_wsplit``) for head dims 64 and
128: that many query rows per workgroup of eight waves, each wave a run of
the key tiles, merged in the workgroup.  Its waves exchange their tiles'
maxima first, so it computes the one-range result (the reference's running
max at every tile); the timed search offers it for grids of a few rounds.

Entries carry the reference's four keys with the values this kernel runs,
so they also validate under the reference's resolver (:463-471); an absent
``KV_SPLITS`` means 1, the way absent backend knobs mean "default" there.
Shared-prefix calls, which the reference does not have, append
``_P{prefix}S{suffix}`` to the key.
"""

from __future__ import annotations

import json
import os
from pathlib import Path
from typing import Callable

_DEFAULT_CACHE_PATH = Path.home() / ".cache" / "repercep" / "fp8_hip_autotune.json"
_DEFAULT_CACHE_STR = str(_DEFAULT_CACHE_PATH)

BLOCK_M = 256
BLOCK_N = 128
#: Compute units of an MI355X; the count used when no GPU is visible (CPU
#: tests, planning ahead of a launch).  On a GPU the current device's count
#: is used, the same number the C launch plans read from the stream's device.
NUM_CUS = 256

_cus_by_device: dict[int, int] = {}


def num_cus() -> int:
    """Compute units of torch's current CUDA device, or ``NUM_CUS`` without one."""
    try:
        import torch
    except ImportError:  # pragma: no cover - torch is a dependency
        return NUM_CUS
    if not torch.cuda.is_available():
        return NUM_CUS
    dev = torch.cuda.current_device()
    if dev not in _cus_by_device:
        _cus_by_device[dev] = int(torch.cuda.get_device_properties(dev).multi_processor_count)
    return _cus_by_device[dev]

#: Used when autotuning is disabled, and the first candidate of every timed
#: search.
FALLBACK_CONFIG = {"BLOCK_M": BLOCK_M, "BLOCK_N": BLOCK_N, "num_warps": 8, "num_stages": 2,
                   "KV_SPLITS": 1}

_REQUIRED = ("BLOCK_M", "BLOCK_N", "num_warps", "num_stages")
SPLIT_CHOICES = (1, 2, 4, 8, 16, 32)

#: Query rows per workgroup of the short-query launch (rp_fp8_attn_fwd_wsplit:
#: eight waves, the key tiles of each 32-row group run by 256 / BLOCK_M of
#: them and merged in the workgroup, numerically the one-range launch) and
#: the head dims it is built for.
WSPLIT_BLOCK_MS = (32, 64, 128)
WSPLIT_HEAD_DIMS = (64, 128)
#: Its workgroups may cover the GPU this many times over.
WSPLIT_MAX_ROUNDS = 4


def wsplit_plan(Skv: int, block_m: int) -> tuple[int, int]:
    """(key tiles per wave, waves with tiles) of the short-query launch: at
    most 256 / block_m equal runs of whole 128-key tiles (rp_attn.hip
    split_plan)."""
    n_kb = -(-Skv // BLOCK_N)
    want = max(1, min(8 * 32 // block_m, n_kb))
    tiles = -(-n_kb // want)
    return tiles, -(-n_kb // tiles)


def wsplit_config(Skv: int, block_m: int) -> dict:
    """The cache entry of a short-query launch.  ``num_warps`` is its eight
    waves; ``num_stages`` keeps the reference grid's value although the
    kernel stages nothing in LDS; ``KV_SPLITS`` records how many waves of a
    query group run key tiles (their runs merge inside the workgroup into
    the one-range result, so unlike a key-split launch this moves no P
    grid)."""
    return {"BLOCK_M": block_m, "BLOCK_N": BLOCK_N, "num_warps": 8, "num_stages": 2,
            "KV_SPLITS": wsplit_plan(Skv, block_m)[1], "SPLIT_IN_WORKGROUP": True}


def cache_path() -> Path:
    override = os.environ.get("REPERCEP_FP8_AUTOTUNE_CACHE")
    return Path(override) if override else _DEFAULT_CACHE_PATH


#: (path, mtime_ns, size) -> parsed cache; the file is re-read only when it
#: changes, so a winner another process records is still picked up on the
#: next call (the reference re-reads the file every call,
#: fp8_flash_attn.py:459-468) without a JSON parse per attention call.
_memo: tuple[tuple[str, int, int], dict] | None = None


def _cache_view() -> dict:
    """The parsed cache file, shared with the memo (callers must not modify
    it): one os.stat per call, a JSON parse only when the file changed."""
    global _memo
    override = os.environ.get("REPERCEP_FP8_AUTOTUNE_CACHE")
    path = override if override else _DEFAULT_CACHE_STR
    try:
        st = os.stat(path)
    except OSError:
        return {}
    stamp = (path, st.st_mtime_ns, st.st_size)
    if _memo is not None and _memo[0] == stamp:
        return _memo[1]
    try:
        with open(path, "r") as fh:
            data = json.load(fh)
    except (OSError, ValueError):
        return {}
    data = data if isinstance(data, dict) else {}
    _memo = (stamp, data)
    return data


def cache_load() -> dict:
    return dict(_cache_view())


def cache_save(cache: dict) -> None:
    path = cache_path()
    path.parent.mkdir(parents=True, exist_ok=True)
    tmp = path.with_name(f"{path.name}.{os.getpid()}.tmp")
    with tmp.open("w") as fh:
        json.dump(cache, fh, indent=2, sort_keys=True)
    tmp.replace(path)


def cache_key(B: int, H: int, Sq: int, Skv: int, D: int, causal: bool,
              prefix_len: int | None = None, suffix_len: int | None = None) -> str:
    key = f"B{B}_H{H}_Sq{Sq}_Skv{Skv}_D{D}_C{int(bool(causal))}"
    if prefix_len is not None:
        key += f"_P{int(prefix_len)}S{int(suffix_len or 0)}"
    return key


def runnable(cfg: object) -> bool:
    """Whether this kernel can launch ``cfg`` (entries written by the
    reference's Triton autotuner may name other tile shapes).  A short-query
    entry (``BLOCK_M`` 32, 64 or 128) must carry ``SPLIT_IN_WORKGROUP``: a
    Triton winner with the same tile numbers describes another kernel."""
    if not isinstance(cfg, dict) or not all(k in cfg for k in _REQUIRED):
        return False
    splits = cfg.get("KV_SPLITS", 1)
    if not (isinstance(splits, int) and not isinstance(splits, bool) and splits >= 0):
        return False
    if cfg["BLOCK_N"] != BLOCK_N:
        return False
    if cfg["BLOCK_M"] == BLOCK_M:
        return True
    return cfg["BLOCK_M"] in WSPLIT_BLOCK_MS and cfg.get("SPLIT_IN_WORKGROUP") is True


def resolve_config(B: int, H: int, Sq: int, Skv: int, D: int, causal: bool,
                   prefix_len: int | None = None, suffix_len: int | None = None) -> dict:
    """The cached configuration for this shape, or {} on a miss."""
    cfg = _cache_view().get(cache_key(B, H, Sq, Skv, D, causal, prefix_len, suffix_len))
    return dict(cfg) if runnable(cfg) else {}


def record_config(B: int, H: int, Sq: int, Skv: int, D: int, causal: bool, cfg: dict,
                  prefix_len: int | None = None, suffix_len: int | None = None) -> None:
    cache = cache_load()
    cache[cache_key(B, H, Sq, Skv, D, causal, prefix_len, suffix_len)] = dict(cfg)
    cache_save(cache)


def autotune_disabled() -> bool:
    return os.environ.get("REPERCEP_FP8_DISABLE_AUTOTUNE", "") in ("1", "true", "on")


def candidate_configs(B: int, H: int, Sq: int, Skv: int, cus: int | None = None,
                      D: int | None = None) -> list[dict]:
    """Configurations worth timing for a shape: split counts that leave every
    range at least one key tile (as the kernel plans them: equal whole-tile
    ranges, so a request is rounded to the count it yields) and keep the grid
    within a few workgroups per compute unit.  A shape whose unsplit grid
    already covers the GPU twice gets the balanced launch alone (the plain
    launch where its plan splits nothing: a full last round, a mask).
    ``cus`` defaults to the current device's compute units (``num_cus``).
    For head dims the short-query launch is built for (``D`` given), its
    block heights follow, those whose grid covers the GPU at most
    ``WSPLIT_MAX_ROUNDS`` times."""
    cus = num_cus() if cus is None else int(cus)
    n_kb = -(-Skv // BLOCK_N)
    work = -(-Sq // BLOCK_M) * B * H
    if work >= 2 * cus:
        return [{**FALLBACK_CONFIG, "KV_SPLITS": 0}]
    counts: list[int] = []
    for want in sorted(set(SPLIT_CHOICES) | {n_kb}):
        if want > n_kb:
            continue
        tiles = -(-n_kb // want)
        s = -(-n_kb // tiles)
        if s not in counts and (s == 1 or work * s <= 8 * cus):
            counts.append(s)
    cands = [{**FALLBACK_CONFIG, "KV_SPLITS": s} for s in counts]
    if D in WSPLIT_HEAD_DIMS:
        for bm in WSPLIT_BLOCK_MS:
            if -(-Sq // bm) * B * H <= WSPLIT_MAX_ROUNDS * cus:
                cands.append(wsplit_config(Skv, bm))
    return cands


#: A later (more split) candidate must beat the best earlier one by this
#: factor: below it the difference is timing noise, and fewer splits keep the
#: unsplit kernel's P grid and skip the merge pass.
MIN_GAIN = 0.95


def autotune(candidates: list[dict], timer: Callable[[dict], float]) -> dict:
    """The fastest candidate by ``timer(cfg)`` (seconds per call), taking
    candidates in order and moving on only for a gain beyond ``MIN_GAIN``."""
    if not candidates:
        raise ValueError("no candidate configurations")
    if len(candidates) == 1:
        return dict(candidates[0])
    best, best_t = candidates[0], timer(candidates[0])
    for c in candidates[1:]:
        t = timer(c)
        if t < best_t * MIN_GAIN:
            best, best_t = c, t
    return dict(best)
