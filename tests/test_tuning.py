"""The launch-configuration cache (CPU only).

Re-expresses the reference's cache tests (tests/test_attention_fp8.py:161-371:
round trip, corruption, search-grid constraints, legacy entries) against
``repercep_runtime_amd.tuning``, plus this build's own rules: entries naming
tile shapes this kernel does not run are misses, and the split search is
confined to shapes that leave the GPU idle.
"""

from __future__ import annotations

import json
from pathlib import Path

import pytest

from repercep_runtime_amd import _capi, ops, tuning
from repercep_runtime_amd.workloads import C1, C3_CROSS, C3_SELF, C5


@pytest.fixture()
def cache_file(tmp_path: Path, monkeypatch: pytest.MonkeyPatch) -> Path:
    path = tmp_path / "fp8_autotune.json"
    monkeypatch.setenv("REPERCEP_FP8_AUTOTUNE_CACHE", str(path))
    monkeypatch.delenv("REPERCEP_FP8_DISABLE_AUTOTUNE", raising=False)
    return path


def test_cache_roundtrip(cache_file: Path) -> None:
    assert tuning.cache_load() == {}
    assert tuning.resolve_config(2, 32, 109120, 109120, 128, False) == {}

    cfg = {**tuning.FALLBACK_CONFIG, "KV_SPLITS": 4}
    tuning.record_config(2, 32, 109120, 109120, 128, False, cfg)
    assert cache_file.exists()
    data = json.loads(cache_file.read_text())
    assert "B2_H32_Sq109120_Skv109120_D128_C0" in data        # the reference's key encoding
    assert tuning.resolve_config(2, 32, 109120, 109120, 128, False) == cfg

    assert tuning.resolve_config(1, 8, 8192, 8192, 128, False) == {}   # other shape: miss
    assert tuning.resolve_config(2, 32, 109120, 109120, 128, True) == {}  # causal differs

    other = dict(tuning.FALLBACK_CONFIG)
    tuning.record_config(1, 8, 8192, 8192, 128, False, other)
    assert len(tuning.cache_load()) == 2                         # earlier entry kept
    assert tuning.resolve_config(2, 32, 109120, 109120, 128, False) == cfg
    assert tuning.resolve_config(1, 8, 8192, 8192, 128, False) == other
    assert not list(cache_file.parent.glob("*.tmp"))             # atomic write left nothing


def test_corrupt_cache_is_a_miss(cache_file: Path) -> None:
    cache_file.write_text("{ this is not valid json")
    assert tuning.cache_load() == {}
    assert tuning.resolve_config(2, 32, 109120, 109120, 128, False) == {}
    cache_file.write_text("[1, 2, 3]")                           # valid JSON, wrong type
    assert tuning.cache_load() == {}
    tuning.record_config(1, 1, 1, 1, 64, False, dict(tuning.FALLBACK_CONFIG))
    assert tuning.resolve_config(1, 1, 1, 1, 64, False) == tuning.FALLBACK_CONFIG


def test_foreign_and_legacy_entries(cache_file: Path) -> None:
    key = tuning.cache_key(1, 8, 8192, 8192, 128, False)
    # a Triton winner the reference recorded: a tile shape this kernel does not run
    triton_cfg = {"BLOCK_M": 128, "BLOCK_N": 64, "num_warps": 4, "num_stages": 2}
    cache_file.write_text(json.dumps({key: triton_cfg}))
    assert tuning.resolve_config(1, 8, 8192, 8192, 128, False) == {}
    # the reference's four keys with this kernel's tile shape and no split knob
    legacy = {"BLOCK_M": 256, "BLOCK_N": 128, "num_warps": 8, "num_stages": 2}
    cache_file.write_text(json.dumps({key: legacy}))
    assert tuning.resolve_config(1, 8, 8192, 8192, 128, False) == legacy
    assert ops.tuned_kv_splits(1, 8, 8192, 8192, 128) == 1
    balanced = {**legacy, "KV_SPLITS": 0}       # the balanced launch
    cache_file.write_text(json.dumps({key: balanced}))
    assert tuning.resolve_config(1, 8, 8192, 8192, 128, False) == balanced
    assert ops.tuned_kv_splits(1, 8, 8192, 8192, 128) == 0
    for bad in ({**legacy, "KV_SPLITS": -1}, {**legacy, "KV_SPLITS": "4"},
                {**legacy, "KV_SPLITS": True}, {"BLOCK_M": 256}):
        cache_file.write_text(json.dumps({key: bad}))
        assert tuning.resolve_config(1, 8, 8192, 8192, 128, False) == {}


def test_our_entries_satisfy_the_reference_grid_constraints() -> None:
    """What the reference's resolver and grid test demand of an entry
    (fp8_flash_attn.py:463-471, tests/test_attention_fp8.py:232-255)."""
    for cfg in [tuning.FALLBACK_CONFIG] + tuning.candidate_configs(1, 8, 1024, 1024):
        bm, bn = cfg["BLOCK_M"], cfg["BLOCK_N"]
        assert bm >= 32 and bn >= 32 and bn <= 2 * bm and bm * bn <= 256 * 256
        assert cfg["num_warps"] in (4, 8, 16) and cfg["num_stages"] in (2, 3)


def test_prefix_key_and_disable_switch(cache_file: Path, monkeypatch: pytest.MonkeyPatch) -> None:
    assert tuning.cache_key(1, 32, 128, 640, 128, False, 512, 8) == \
        "B1_H32_Sq128_Skv640_D128_C0_P512S8"
    tuning.record_config(1, 32, 128, 640, 128, False, {**tuning.FALLBACK_CONFIG, "KV_SPLITS": 5},
                         512, 8)
    assert ops.tuned_kv_splits(1, 32, 128, 640, 128, False, 512, 8) == 5
    assert ops.tuned_kv_splits(1, 32, 128, 640, 128, False) == 1   # no prefix: other key
    monkeypatch.setenv("REPERCEP_FP8_DISABLE_AUTOTUNE", "1")
    assert tuning.autotune_disabled()
    assert ops.tuned_kv_splits(1, 32, 128, 640, 128, False, 512, 8) == 1


def test_candidates_only_split_small_grids() -> None:
    # 11,840 workgroups: no search, the balanced launch
    balanced = [{**tuning.FALLBACK_CONFIG, "KV_SPLITS": 0}]
    assert tuning.candidate_configs(C3_SELF.B, C3_SELF.H, C3_SELF.Sq, C3_SELF.Skv) == balanced
    assert tuning.candidate_configs(C3_CROSS.B, C3_CROSS.H, C3_CROSS.Sq,
                                    C3_CROSS.Skv) == balanced
    small = tuning.candidate_configs(C1.B, C1.H, C1.Sq, C1.Skv)   # 32 workgroups, 8 key tiles
    assert [c["KV_SPLITS"] for c in small] == [1, 2, 4, 8]
    # 5 key tiles: requests 1, 2, 4, 5 give ranges of 5, 3, 2, 1 tiles
    c5 = tuning.candidate_configs(1, C5.H, C5.Sq, C5.Skv)
    assert [c["KV_SPLITS"] for c in c5] == [1, 2, 3, 5]
    # 17 tiles: requests 8 and 16 give ranges of 3 and 2 tiles, i.e. 6 and 9 splits
    assert [c["KV_SPLITS"] for c in tuning.candidate_configs(1, 1, 256, 17 * 128)] == \
        [1, 2, 4, 6, 9, 17]
    assert [c["KV_SPLITS"] for c in tuning.candidate_configs(1, 1, 256, 100)] == [1]


def test_candidates_follow_the_compute_unit_count(monkeypatch: pytest.MonkeyPatch) -> None:
    # C1's 32 workgroups on 24 CUs: 8 splits would exceed the cap of eight
    # workgroups per CU; on 16 CUs they are two rounds (the balanced launch)
    assert [c["KV_SPLITS"] for c in tuning.candidate_configs(1, 8, 1024, 1024, cus=24)] == [1, 2, 4]
    assert [c["KV_SPLITS"] for c in tuning.candidate_configs(1, 8, 1024, 1024, cus=16)] == [0]
    # 64 workgroups: two rounds on 32 CUs (the balanced launch), not on 256
    assert tuning.candidate_configs(1, 16, 1024, 1024, cus=32) == [
        {**tuning.FALLBACK_CONFIG, "KV_SPLITS": 0}]
    assert len(tuning.candidate_configs(1, 16, 1024, 1024, cus=256)) > 1
    # the default is the current device's count
    monkeypatch.setattr(tuning, "num_cus", lambda: 32)
    assert tuning.candidate_configs(1, 16, 1024, 1024) == [
        {**tuning.FALLBACK_CONFIG, "KV_SPLITS": 0}]


def test_a_large_grid_resolves_to_the_balanced_launch_without_a_search(cache_file: Path) -> None:
    assert ops.tuned_kv_splits(C3_SELF.B, C3_SELF.H, C3_SELF.Sq, C3_SELF.Skv, C3_SELF.D) == 0
    assert ops.tuned_kv_splits(C1.B, C1.H, C1.Sq, C1.Skv, C1.D) == 1   # searched: 1 on a miss
    assert not cache_file.exists()


def test_autotune_picks_the_fastest() -> None:
    cands = [{**tuning.FALLBACK_CONFIG, "KV_SPLITS": s} for s in (1, 2, 4)]
    times = {1: 3.0, 2: 1.0, 4: 2.0}
    assert tuning.autotune(cands, lambda c: times[c["KV_SPLITS"]])["KV_SPLITS"] == 2
    # within the noise margin the fewer-split candidate stays
    times = {1: 1.0, 2: 0.97, 4: 0.96}
    assert tuning.autotune(cands, lambda c: times[c["KV_SPLITS"]])["KV_SPLITS"] == 1
    times = {1: 1.0, 2: 0.97, 4: 0.5}
    assert tuning.autotune(cands, lambda c: times[c["KV_SPLITS"]])["KV_SPLITS"] == 4
    calls = []
    assert tuning.autotune(cands[:1], lambda c: calls.append(c) or 0.0) == cands[0]
    assert calls == []                                            # nothing to time
    with pytest.raises(ValueError):
        tuning.autotune([], lambda c: 0.0)


def _split_call(L, kv_splits: int, ws, nbytes: int) -> int:
    fake = 1 << 20
    return L.rp_fp8_attn_fwd_split(fake, fake, fake, 1024, fake, fake, fake, 1, 0.125, fake, 0,
                                   8 * 1024 * 64, 1024 * 64, 64, 1, 8, 1024, 1024, 64, 0, 0, 1,
                                   kv_splits, ws, nbytes, None)


def test_split_entry_point_checks_and_sizing() -> None:
    L = _capi.lib()
    assert L.rp_fp8_attn_workspace_bytes(1, 8, 1024, 64, 1) == 0
    n8 = L.rp_fp8_attn_workspace_bytes(1, 8, 1024, 64, 8)
    rows = 8 * 8 * 1024
    assert n8 == rows * 2 * 4 + rows * 64 * 4                    # (m, l) + fp32 O per row
    assert L.rp_fp8_attn_workspace_bytes(0, 8, 1024, 64, 8) == 0
    assert _split_call(L, 0, None, 0) == 1
    assert "kv_splits" in L.rp_last_error().decode()
    assert _split_call(L, 8, None, 0) == 1
    assert "workspace" in L.rp_last_error().decode()
    assert _split_call(L, 8, 1 << 20, n8 - 1) == 1                # one byte short
    assert _split_call(L, 8, (1 << 20) + 64, n8) == 1             # misaligned
    assert "256-byte" in L.rp_last_error().decode()


def test_cache_is_reread_when_the_file_changes(cache_file: Path) -> None:
    """The parsed cache is kept between calls, but a file another process
    rewrites is picked up on the next lookup (as the reference's per-call
    read would)."""
    import os

    legacy = dict(tuning.FALLBACK_CONFIG)
    tuning.record_config(1, 8, 8192, 8192, 128, False, legacy)
    assert ops.tuned_kv_splits(1, 8, 8192, 8192, 128) == 1
    key = tuning.cache_key(1, 8, 8192, 8192, 128, False)
    cache_file.write_text(json.dumps({key: {**legacy, "KV_SPLITS": 4}}))
    st = cache_file.stat()
    os.utime(cache_file, ns=(st.st_atime_ns, st.st_mtime_ns + 1_000_000))
    assert ops.tuned_kv_splits(1, 8, 8192, 8192, 128) == 4
    cache_file.unlink()
    assert ops.tuned_kv_splits(1, 8, 8192, 8192, 128) == 1        # gone: a miss


def test_short_query_entries(cache_file: Path) -> None:
    """Short-query launches (BLOCK_M 32/64/128, keys split over the waves):
    candidates only for head dims 64 and 128 and grids of a few rounds, each
    carrying the split count of its plan and the SPLIT_IN_WORKGROUP marker;
    a reference Triton winner with the same tile numbers but no marker is
    another kernel's entry and reads as a miss."""
    c1 = tuning.candidate_configs(C1.B, C1.H, C1.Sq, C1.Skv, cus=256, D=C1.D)
    ws = [c for c in c1 if c["BLOCK_M"] != 256]
    assert [(c["BLOCK_M"], c["KV_SPLITS"]) for c in ws] == [(32, 8), (64, 4), (128, 2)]
    assert all(c["SPLIT_IN_WORKGROUP"] is True and c["BLOCK_N"] == 128 for c in ws)
    assert [c for c in c1 if c["BLOCK_M"] == 256][0] == tuning.FALLBACK_CONFIG
    assert all(c["BLOCK_M"] == 256 for c in
               tuning.candidate_configs(C1.B, C1.H, C1.Sq, C1.Skv, cus=256, D=32))
    c5 = tuning.candidate_configs(1, C5.H, C5.Sq, C5.Skv, cus=256, D=C5.D)
    assert [(c["BLOCK_M"], c["KV_SPLITS"]) for c in c5 if c["BLOCK_M"] != 256] == \
        [(32, 5), (64, 3), (128, 2)]
    # 18 key tiles over eight waves: six splits of three tiles
    assert tuning.wsplit_plan(18 * 128, 32) == (3, 6)
    assert tuning.wsplit_plan(100, 32) == (1, 1)
    key = tuning.cache_key(1, 8, 1024, 1024, 64, False)
    entry = tuning.wsplit_config(1024, 32)
    cache_file.write_text(json.dumps({key: entry}))
    assert tuning.resolve_config(1, 8, 1024, 1024, 64, False) == entry
    assert ops.tuned_launch(1, 8, 1024, 1024, 64) == (32, 1)
    assert ops.tuned_kv_splits(1, 8, 1024, 1024, 64) == 1
    triton_128 = {"BLOCK_M": 128, "BLOCK_N": 128, "num_warps": 8, "num_stages": 2}
    cache_file.write_text(json.dumps({key: triton_128}))
    assert tuning.resolve_config(1, 8, 1024, 1024, 64, False) == {}
    assert ops.launch_of({**tuning.FALLBACK_CONFIG, "KV_SPLITS": 4}) == (256, 4)


def test_short_query_plan_matches_the_library() -> None:
    import ctypes

    L = _capi.lib()
    for skv in (1, 100, 128, 129, 640, 1024, 1000, 2200, 8192):
        for bm in (32, 64, 128):
            st, ns = ctypes.c_int(), ctypes.c_int()
            assert L.rp_fp8_attn_wsplit_plan(skv, bm, ctypes.byref(st), ctypes.byref(ns)) == 0
            assert (st.value, ns.value) == tuning.wsplit_plan(skv, bm), (skv, bm)
    st, ns = ctypes.c_int(), ctypes.c_int()
    assert L.rp_fp8_attn_wsplit_plan(128, 48, ctypes.byref(st), ctypes.byref(ns)) == 1
    assert L.rp_fp8_attn_wsplit_plan(0, 32, ctypes.byref(st), ctypes.byref(ns)) == 1
