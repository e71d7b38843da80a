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
KN_OFF = _fn(_expr(GEMM, r"kn_off\[j\] = \(uint32_t\)\(([^;]+)\);"), "row", "kG2Tile", "gr", "i")
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


# ------------------------------------------- GEMM epilogue: C through LDS
EPI_W = _fn(_expr(GEMM, r"const int cs = (\(\(8 \* j \+ 2 \* q \+ lg\) \^ lq\));"),
            "j", "q", "lg", "lq")
EPI_R = _fn(_expr(GEMM, r"const int cg = (\(c \^ \(\(r & 31\) >> 1\)\));"), "c", "r")
C_PITCH = 256   # kCPitch: 128 bf16 columns of a wave's part


def test_epilogue_staging_round_trip_and_conflict_free() -> None:
    """The 128 x 128 bf16 part of a wave: lane (lq, lg) writes the 4 columns
    32j + 8q + 4lg .. +3 of row 32i + lq (the 32x32 accumulator map) as 8-byte
    slot cs of the row; reading 16 bytes at granule cg of row r (halves
    swapped for odd r) returns columns 8c .. 8c+7 in order.  One write
    instruction's 32 lanes of a half-wave fill 32 distinct 8-byte slots (all
    64 banks), one read's 16 lanes of a row 16 distinct granules."""
    lds = {}
    for i in range(4):
        for j in range(4):
            for q in range(4):
                slots = {0: [], 1: []}
                for lane in range(64):
                    lq, lg = lane & 31, lane >> 5
                    row = 32 * i + lq
                    off = row * C_PITCH + 8 * EPI_W(j, q, lg, lq)
                    assert 0 <= off - row * C_PITCH < C_PITCH
                    cols = [32 * j + 8 * q + 4 * lg + e for e in range(4)]
                    for e in range(4):
                        assert off + 2 * e not in lds
                        lds[off + 2 * e] = (row, cols[e])
                    slots[lg].append((off % 256) // 8)
                assert all(sorted(v) == list(range(32)) for v in slots.values())
    assert len(lds) == 128 * 128
    for k in range(32):
        for lane in range(64):
            r, c = 4 * k + (lane >> 4), lane & 15
            base = r * C_PITCH + 16 * EPI_R(c, r)
            got = [lds[base + 2 * e] for e in range(8)]
            if r & 1:
                got = got[4:] + got[:4]
            assert got == [(r, 8 * c + e) for e in range(8)], (k, lane)
        for grp in range(4):
            r = 4 * k + grp
            assert sorted(EPI_R(c, r) for c in range(16)) == list(range(16))
    # negative control: without the XOR the 32 rows of one write instruction
    # (pitch 256 bytes = one sweep of the banks) all land on the same slot
    plain = {((32 + lq) * C_PITCH + 8 * (8 * 1 + 2 * 2 + 0)) % 256 for lq in range(32)}
    assert len(plain) == 1


# --------------------------------------- GEMM: the slot ring of the loads
RING_LINES = (
    "const uint8_t* sta = smem + (H == 0 ? sa : wrap(sa + 2)) * kG2Half;",
    "const uint8_t* stb = smem + (H == 0 ? wrap(sa + 1) : wrap(sa + 3)) * kG2Half;",
    "const int lslot = H == 0 ? wrap(sa + 4) : sa;",
    "if ((t & 1) == 1 && load)",
    "issue(H * kG2ALoads + (t >> 1), kk + 2, lslot, std::integral_constant<bool, STEADY>{});",
    "const bool more = STEADY || u + 1 < nsub;",
    "const bool load = STEADY || kk + 2 < nslice;",
    "const int nsteady = max(0, nslice - 3);",
    "if (load) g2_wait_vmem<kG2ALoads>();",
    "for (int n = 0; n < kG2Loads; ++n) issue(n, 0, n < kG2ALoads ? 0 : 1, std::false_type{});",
    "for (int n = 0; n < kG2Loads; ++n) issue(n, 1, n < kG2ALoads ? 2 : 3, std::false_type{});",
    "if (H == 1) sa = wrap(sa + 2);",
    "constexpr int kG2Slots = 5;",
)


def _ring_schedule(nsub: int, slots: int = 5) -> None:
    """Replays the large-tile kernel's load/read schedule (the lines above)
    for one tile: every operand read finds its slice part landed (the vmcnt
    waits) and in its slot, and no load overwrites a part that some wave may
    still read (the last read of a part precedes a barrier that precedes the
    load).  Units are the A (0) or B^T (1) part of a slice, 8 loads each."""
    nslice, half, nfull = (nsub + 1) // 2, nsub & 1, nsub // 2
    wrap = lambda x: x - slots if x >= slots else x   # noqa: E731
    issued, landed, slot, reads, pending = [], set(), {}, {}, set()
    need = lambda s: 1 if (half and s == nslice - 1) else 2   # noqa: E731

    def issue(unit, sl):
        old = slot.get(sl)
        assert old is None or (reads.get(old, 0) == need(old[0]) and old not in pending), \
            (nsub, unit, sl, old)
        slot[sl] = unit
        issued.append(unit)

    def wait(k):                       # all but the k most recent units landed
        landed.update(issued[:len(issued) - k])

    def read(s, sla, slb):
        for part, sl in ((0, sla), (1, slb)):
            assert slot[sl] == (s, part) and (s, part) in landed, (nsub, s, part)
            reads[(s, part)] = reads.get((s, part), 0) + 1
            pending.add((s, part))

    issue((0, 0), 0)
    issue((0, 1), 1)
    if nslice > 1:
        issue((1, 0), 2)
        issue((1, 1), 3)
        wait(2)
    else:
        wait(0)
    pending.clear()                    # barrier
    read(0, 0, 1)
    sa = 0
    steps = [(kk, h) for kk in range(nfull) for h in (0, 1)] + ([(nfull, 0)] if half else [])
    for kk, h in steps:
        more, load = 2 * kk + h + 1 < nsub, kk + 2 < nslice
        if kk < max(0, nslice - 3):    # a steady sub-step: both taken as true,
            assert more and load and kk + 2 < nslice - 1   # the slice loaded full
        if h == 1:
            if more:
                wait(1 if load else 0)
            pending.clear()            # barrier
        if more:
            if h == 0:
                read(kk, sa, wrap(sa + 1))
            else:
                read(kk + 1, wrap(sa + 2), wrap(sa + 3))
        if load:
            issue((kk + 2, h), wrap(sa + 4) if h == 0 else sa)
        if h == 1:
            sa = wrap(sa + 2)
    assert len(issued) == 2 * nslice
    assert all(reads[(s, p)] == need(s) for s in range(nslice) for p in (0, 1))


def test_gemm_slot_ring_schedule() -> None:
    for line in RING_LINES:
        assert line in GEMM, line
    for nsub in range(1, 41):
        _ring_schedule(nsub)


def test_gemm_slot_ring_negative_controls() -> None:
    """With four slots the same schedule puts slice k+2's A part over a part
    that is still read (or has not been read yet): the replay fails."""
    with pytest.raises(AssertionError):
        _ring_schedule(12, slots=4)


# ----------------------------- quantizer: the V^T tile's LDS swizzle
QUANT = (CSRC / "rp_quant_dev.h").read_text()   # the transposed apply body
VT_W = _fn(_expr(QUANT, r"const int qs = (4 \* \(q \^ \(8 \* \(c & 3\)\)\));"), "q", "c")
VT_R = _fn(_expr(QUANT, r"const int sch = (ch \^ \(2 \* \(\(dr >> 3\) & 3\)\));"), "ch", "dr")


def test_vt_tile_round_trip_and_banks() -> None:
    """quant_apply_t_kernel: thread (q = t >> 3, c = t & 7) writes the dword of
    codes s = 4q .. 4q+3 of each column d in [8c, 8c+8) at byte qs of row d;
    reading 16 bytes at chunk ch of row dr gives the codes of s chunk sch.
    Write instructions hit each bank at most twice, reads never twice."""
    lds = {}
    for t in range(256):
        q, c = t >> 3, t & 7
        for d in range(8 * c, 8 * c + 8):
            off = d * 128 + VT_W(q, c)
            assert off not in lds
            lds[off] = (d, q)
    for t in range(256):
        for k in range(2):
            dr, ch = (t >> 3) + 32 * k, t & 7
            got = [lds[dr * 128 + 16 * ch + 4 * i] for i in range(4)]
            assert got == [(dr, 4 * VT_R(ch, dr) + i) for i in range(4)]
    for w in range(4):                         # one wave's write of column offset e
        for e in range(8):
            banks = [((8 * (l & 7) + e) * 128 + VT_W(8 * w + (l >> 3), l & 7)) // 4 % 64
                     for l in range(64)]
            assert max(banks.count(b) for b in set(banks)) <= 2
    # negative control: the unswizzled dword (4q) piles eight lanes on a bank
    banks = [((8 * (l & 7)) * 128 + 4 * (l >> 3)) // 4 % 64 for l in range(64)]
    assert max(banks.count(b) for b in set(banks)) == 8
