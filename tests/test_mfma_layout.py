"""Structural spec of the gfx950 matrix-core layouts the kernels rely on (CPU only).

The counterpart of the reference's MFMA fragment-layout spec
(tests/test_mfma_fragment_layout.py:84-235: bijection, per-lane coverage,
negative controls, coupling to the source constants), for the layouts this
build's kernels use:

* v_mfma_f32_32x32x64_f8f6f4 and v_mfma_f32_16x16x128_f8f6f4: operand and
  accumulator lane maps (the maps the kernels' epilogues and operand reads
  assume, which the GPU parity tests confirm end to end);
* the attention kernel's K-row permutation ``key_of`` (rp_attn.hip), which
  lets the S^T accumulator feed the P.V product without leaving registers;
* the GEMM's LDS swizzles (rp_gemm.hip) and, for a (K, N) B operand, the
  ds_read_b64_tr_b8 transpose reads that assemble each lane's 32 K bytes.

The index expressions are read out of the kernel sources and evaluated here
(C and Python agree on the precedence of * + << >> & ^), so a change in a
kernel's indexing is checked on the CPU before it costs a GPU run.
"""

from __future__ import annotations

import re
from pathlib import Path

import numpy as np
import pytest

CSRC = Path(__file__).resolve().parent.parent / "repercep_runtime_amd" / "csrc"
ATTN = (CSRC / "rp_attn.hip").read_text()
GEMM = (CSRC / "rp_gemm.hip").read_text()


def _expr(src: str, pattern: str) -> str:
    m = re.search(pattern, src)
    assert m, f"pattern not found in the kernel source: {pattern}"
    return m.group(1)


def _fn(expr: str, *names: str):
    """A Python function of ``names`` evaluating a C integer expression."""
    code = compile(expr, "<kernel expr>", "eval")
    return lambda *args: eval(code, {"min": min}, dict(zip(names, args)))


# ---------------------------------------------------------- lane maps
def op_32x32x64(lane: int, byte: int) -> tuple[int, int]:
    """Operand (A or B) element held by byte ``byte`` of lane ``lane``: row
    (or column) lane % 32, k-slot 32 * (lane / 32) + byte."""
    return lane % 32, 32 * (lane // 32) + byte


def acc_32x32(lane: int, reg: int) -> tuple[int, int]:
    """Accumulator element of register ``reg``: row 8(reg/4) + 4(lane/32) + reg%4,
    column lane % 32."""
    return 8 * (reg // 4) + 4 * (lane // 32) + reg % 4, lane % 32


def op_16x16x128(lane: int, byte: int) -> tuple[int, int]:
    return lane % 16, 32 * (lane // 16) + byte


def acc_16x16(lane: int, reg: int) -> tuple[int, int]:
    return 4 * (lane // 16) + reg, lane % 16


@pytest.mark.parametrize("fn,lanes,per_lane,shape", [
    (op_32x32x64, 64, 32, (32, 64)), (acc_32x32, 64, 16, (32, 32)),
    (op_16x16x128, 64, 32, (16, 128)), (acc_16x16, 64, 4, (16, 16)),
])
def test_lane_maps_are_bijections(fn, lanes: int, per_lane: int, shape: tuple) -> None:
    seen = np.zeros(shape, dtype=int)
    for lane in range(lanes):
        for e in range(per_lane):
            r, c = fn(lane, e)
            seen[r, c] += 1
    assert (seen == 1).all()


def test_lane_map_negative_control() -> None:
    """A map that forgets the lane-half term covers half the tile twice."""
    seen = np.zeros((32, 32), dtype=int)
    for lane in range(64):
        for reg in range(16):
            seen[8 * (reg // 4) + reg % 4, lane % 32] += 1
    assert not (seen == 1).all()


def test_epilogues_use_the_accumulator_maps() -> None:
    """The GEMM epilogues index outputs by these maps: 32x32 -- column lq (m),
    rows 8q + 4lg + r (n, four consecutive per store); 16x16 -- column li,
    rows 4lg + r."""
    assert "const int64_t m = m0 + wm * 128 + 32 * i + lq;" in GEMM
    assert "const int64_t n = n0 + wn * 128 + 32 * j + 8 * q + 4 * lg;" in GEMM
    assert "const int64_t m = m0 + wm * G::WM + 16 * i + li;" in GEMM
    assert "const int64_t n = n0 + wn * G::WN + 16 * j + 4 * lg;" in GEMM
    for lane in range(64):
        lq, lg = lane & 31, lane >> 5
        for q in range(4):
            for r in range(4):
                assert acc_32x32(lane, 4 * q + r) == (8 * q + 4 * lg + r, lq)


# --------------------------------------------- attention: key_of and P
KEY_OF = _fn(_expr(ATTN, r"int key_of\(int h, int rho\) \{\s*return ([^;]+);"), "h", "rho")
HH = _fn(_expr(ATTN, r"const int hh = (2 \* m \+ \(wd >> 2\));"), "m", "wd")
R0 = _fn(_expr(ATTN, r"const int r = (4 \* \(wd & 3\));"), "wd")


def test_key_of_is_a_permutation_of_the_tile() -> None:
    keys = sorted(KEY_OF(h, rho) for h in range(4) for rho in range(32))
    assert keys == list(range(128))


def _p_operand_key(key_of, m: int, lane: int, byte: int) -> int:
    """Key whose P value byte ``byte`` of lane ``lane`` carries in the P.V
    B operand of 64-key chunk m: the softmax packs s[hh][r + i] (i < 4) into
    byte 4 wd + i, and s[hh][reg] is the S^T accumulator of key tile hh,
    register reg, whose row is key_of(hh, row of the accumulator map)."""
    wd, i = byte // 4, byte % 4
    hh, reg = HH(m, wd), R0(wd) + i
    rho, col = acc_32x32(lane, reg)
    assert col == lane % 32                 # the lane's own query
    return key_of(hh, rho)


def test_p_operand_matches_the_pv_mfma_k_slots() -> None:
    """P never leaves registers: byte b of lane l in chunk m holds the score
    of key 64m + (k-slot of the 32x32x64 operand map), the key whose V^T
    column the A operand (V^T, keys in natural order) pairs with it."""
    for m in range(2):
        for lane in range(64):
            for byte in range(32):
                _, kslot = op_32x32x64(lane, byte)
                assert _p_operand_key(KEY_OF, m, lane, byte) == 64 * m + kslot


def test_identity_key_order_fails_the_p_operand_check() -> None:
    """Negative control: K rows in natural order put the wrong keys in P."""
    identity = lambda h, rho: 32 * h + rho    # noqa: E731
    bad = sum(_p_operand_key(identity, m, lane, b) != 64 * m + op_32x32x64(lane, b)[1]
              for m in range(2) for lane in range(64) for b in range(32))
    assert bad > 0


# -------------------------------------------------- GEMM LDS layouts
SW_NK = _fn(_expr(GEMM, r"const int s16 = \((slot \^ \(\(row >> 1\) & 7\))\) \* 16;"),
            "slot", "row")
SWZ = _fn(_expr(GEMM, r"const int swz = ([^;]+);"), "lq")
SW_KN = _fn(_expr(GEMM, r"const int gran = min\((slot \^ \(2 \* \(row & 7\)\)), last\);"),
            "slot", "row")
KN_ROW = _fn(_expr(GEMM, r"const int row = (32 \* lg \+ \(i >> 1\));"), "lg", "i")
KN_GR = _fn(_expr(GEMM, r"const int gr = (8 \* wn \+ 2 \* j \+ \(\(lane >> 4\) & 1\));"),
            "wn", "j", "lane")
KN_OFF = _fn(_expr(GEMM, r"kn_off\[j\] = \(uint32_t\)\(kG2Half \+ ([^;]+)\);"), "row", "kG2Tile",
             "gr", "i")
TILE = 256   # kG2Tile


def _bank_groups_distinct(addrs: list[int], width: int) -> bool:
    """No two accesses of one LDS cycle share a 16-byte bank group (64 banks
    of 4 bytes = 16 groups), accesses of ``width`` bytes."""
    groups = []
    for a in addrs:
        groups += [((a + o) // 16) % 16 for o in range(0, width, 16)] if width >= 16 \
            else [(a // 16) % 16]
    return len(groups) == len(set(groups))


def test_nk_swizzle_round_trip_and_conflict_free_reads() -> None:
    """(N, K) operands: the load puts K granule slot ^ ((row >> 1) & 7) at LDS
    slot `slot` of 128-byte row `row`; the operand read of granule 2lg (+1) of
    row lq finds it at (2lg ^ swz) with swz = (lq >> 1) & 7, and the 16 lanes
    of one ds_read_b128 group (rows lq .. lq+15 of a 32-row block, one
    granule each) hit 16 distinct bank groups."""
    for row in range(32):
        slot_of = {SW_NK(slot, row): slot for slot in range(8)}   # K granule -> LDS slot
        for lg in range(2):
            for g in (2 * lg, 2 * lg + 1):
                assert slot_of[g] == (g ^ SWZ(row))   # where the read looks
    for base in (0, 16):
        for g in range(8):
            addrs = [(base + r) * 128 + 16 * (g ^ SWZ(base + r)) for r in range(16)]
            assert _bank_groups_distinct(addrs, 16)
    # negative control: without the swizzle a group's 16 rows share 2 bank groups
    assert not _bank_groups_distinct([r * 128 for r in range(16)], 16)


def _tr8(addrs: list[int], lds: np.ndarray) -> list[list[int]]:
    """ds_read_b64_tr_b8 as measured on gfx950: lane l, byte j comes from the
    8 bytes lane 16(l/16) + 2j + (l%16)/8 points at, byte l % 8."""
    out = []
    for lane in range(64):
        src = [16 * (lane // 16) + 2 * j + (lane % 16) // 8 for j in range(8)]
        out.append([int(lds[addrs[s] + lane % 8]) for s in src])
    return out


@pytest.mark.parametrize("wn", [0, 1])
def test_kn_transpose_reads_assemble_the_b_operand(wn: int) -> None:
    """(K, N) B: a 128 x 256 byte slice stored with N granule g of K row r at
    slot g ^ 2(r & 7); the four transpose reads at kn_off[j] + 8t rows give
    lane l the bytes B[k][n] with n = 32j + l % 32 (+ 128 wn) and
    k = 32(l/32) + 8t + byte: the 32x32x64 operand map of B^T row n."""
    rng = np.random.default_rng(wn)
    B = rng.integers(0, 256, size=(128, TILE), dtype=np.uint8)
    lds = np.zeros(128 * TILE, dtype=np.uint8)
    for r in range(128):
        for slot in range(16):
            g = SW_KN(slot, r)
            lds[r * TILE + 16 * slot: r * TILE + 16 * slot + 16] = B[r, 16 * g: 16 * g + 16]
    for j in range(4):
        base = []
        for lane in range(64):
            i, lg = lane & 15, lane >> 5
            base.append(KN_OFF(KN_ROW(lg, i), TILE, KN_GR(wn, j, lane), i))
        for t in range(4):
            got = _tr8([a + 8 * t * TILE for a in base], lds)
            for lane in range(64):
                n = 128 * wn + 32 * j + lane % 32
                for byte in range(8):
                    k = 32 * (lane // 32) + 8 * t + byte
                    assert got[lane][byte] == B[k, n], (j, t, lane, byte)


def test_kn_swizzle_is_a_permutation_and_reads_conflict_free() -> None:
    for r in range(128):
        assert sorted(SW_KN(s, r) for s in range(16)) == list(range(16))
    # 32 lanes of one transpose read (two 16-lane groups: adjacent N granules,
    # eight K rows) touch each 16-byte bank group exactly once
    for wn in range(2):
        for j in range(4):
            addrs = []
            for lane in range(32):
                i, lg = lane & 15, lane >> 5
                addrs.append(KN_OFF(KN_ROW(lg, i), TILE, KN_GR(wn, j, lane), i))
            groups = sorted(((a // 16) % 16) for a in addrs[::2])
            assert groups == list(range(16)), (wn, j)
    # negative control: an unswizzled slice puts a group's eight rows in one bank group
    assert len({((r * TILE + 16 * 3) // 16) % 16 for r in range(8)}) == 1
