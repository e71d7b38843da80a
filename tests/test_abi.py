"""The C-ABI library loads on a CPU-only host and exports what its header declares.

No compute call is made here (there is no GPU): only host-side entry points
(version, status strings, workspace sizing) and argument checks that every
entry point performs before it touches the device.
"""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from repercep_runtime_amd import _capi

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "repercep_fp8.h"
FAKE = 1 << 20           # 16-byte aligned non-null address; never dereferenced


def _declared() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"^[A-Za-z_][\w\s\*]*?\b(rp_\w+)\s*\(", text, flags=re.M))


def test_header_declarations_match_binding() -> None:
    declared = _declared()
    assert declared, "no declarations parsed"
    assert declared == set(_capi.EXPORTS)


def test_library_exports_every_declared_symbol() -> None:
    assert _capi.LIB_PATH.exists(), "build first: python -c 'import __graft_entry__ as g; g.build()'"
    nm = subprocess.run(["nm", "-D", "--defined-only", str(_capi.LIB_PATH)], check=True,
                        capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in nm.splitlines() if " T " in line}
    missing = _declared() - exported
    assert not missing, f"not exported: {sorted(missing)}"
    L = _capi.lib()
    for name in _declared():
        assert isinstance(getattr(L, name), ctypes._CFuncPtr)


def test_no_oracle_or_torch_symbols_in_library() -> None:
    """The product library is self-contained: it links neither the oracle nor torch."""
    deps = subprocess.run(["readelf", "-d", str(_capi.LIB_PATH)], check=True,
                          capture_output=True, text=True).stdout
    assert "fp8_oracle" not in deps and "libtorch" not in deps and "libc10" not in deps
    nm = subprocess.run(["nm", "-D", str(_capi.LIB_PATH)], check=True, capture_output=True,
                        text=True).stdout
    assert " or_" not in nm


def test_version_and_status_strings() -> None:
    L = _capi.lib()
    assert L.rp_abi_version() == 3
    assert L.rp_status_string(0) == b"ok"
    assert L.rp_status_string(1) == b"invalid argument"
    assert L.rp_status_string(2) == b"unsupported shape or layout"
    assert L.rp_status_string(3) == b"workspace missing or too small"
    assert L.rp_status_string(4) == b"kernel launch failed"
    assert L.rp_status_string(99) == b"unknown status"


def test_workspace_sizing_is_host_only() -> None:
    L = _capi.lib()
    small = L.rp_fp8_quant_workspace_bytes(1, 8, 1024, 64, _capi.RP_SCALE_PER_BH)
    big = L.rp_fp8_quant_workspace_bytes(1, 40, 75600, 128, _capi.RP_SCALE_PER_BH)
    assert 0 < small <= big < (64 << 20)
    assert L.rp_fp8_quant_workspace_bytes(0, 8, 1024, 64, 0) == 0        # invalid -> 0


def _attn(L, **kw) -> int:
    a = dict(q8=FAKE, k8=FAKE, vt8=FAKE, ldv=128, qs=FAKE, ks=FAKE, vs=FAKE, stride=1,
             sm=0.125, out=FAKE, odt=0, osb=8 * 128 * 128, osh=128 * 128, oss=128, B=1, H=8,
             Sq=128, Skv=128, D=128, mask=0, prefix=0, suffix=1, stream=None)
    a.update(kw)
    return L.rp_fp8_attn_fwd(*a.values())


@pytest.mark.parametrize("kw,status,msg", [
    (dict(q8=None), 1, "null pointer"),
    (dict(D=96), 2, "head dim"),
    (dict(D=512), 2, "head dim"),
    (dict(D=16), 2, "head dim"),
    (dict(Sq=0), 1, "non-positive"),
    (dict(ldv=100), 1, "ldv"),
    (dict(mask=7), 1, "unknown mask"),
    (dict(mask=2, suffix=0), 1, "shared-prefix"),
    (dict(odt=5), 1, "out_dtype"),
    (dict(stride=3), 1, "scale_stride"),
    (dict(k8=FAKE + 8), 2, "aligned"),
    (dict(sm=-0.125), 1, "sm_scale"),
    (dict(sm=float("nan")), 1, "sm_scale"),
])
def test_attention_argument_checks(kw: dict, status: int, msg: str) -> None:
    L = _capi.lib()
    assert _attn(L, **kw) == status
    assert msg in L.rp_last_error().decode()


NK, KN = _capi.RP_B_NK, _capi.RP_B_KN


@pytest.mark.parametrize("args,status,msg", [
    # a8, b8, layout, c, M, N, K, lda, ldb, ldc
    ((None, FAKE, NK, FAKE, 64, 64, 64, 64, 64, 64), 1, "null pointer"),
    ((FAKE, FAKE, NK, FAKE, 64, 64, 0, 64, 64, 64), 1, "bad sizes"),
    ((FAKE, FAKE, NK, FAKE, 64, 64, 40, 40, 40, 64), 2, "multiples of 16"),
    ((FAKE, FAKE, NK, FAKE + 4, 64, 64, 64, 64, 64, 64), 2, "aligned"),
    ((FAKE, FAKE, 7, FAKE, 64, 64, 64, 64, 64, 64), 1, "B layout"),
    # (N, K) B: ldb >= K, a multiple of 16, B 16-byte aligned
    ((FAKE, FAKE, NK, FAKE, 64, 128, 64, 64, 48, 128), 1, "bad sizes"),
    ((FAKE, FAKE, NK, FAKE, 64, 64, 64, 64, 72, 64), 2, "multiples of 16"),
    ((FAKE, FAKE + 8, NK, FAKE, 64, 64, 64, 64, 64, 64), 2, "aligned"),
    # (K, N) B: ldb >= N (no alignment needed: the general kernel gathers bytes)
    ((FAKE, FAKE, KN, FAKE, 64, 128, 64, 64, 100, 128), 1, "bad sizes"),
])
def test_gemm_argument_checks(args: tuple, status: int, msg: str) -> None:
    L = _capi.lib()
    assert L.rp_fp8_gemm(*args, 1.0, 1.0, None, None, None) == status
    assert msg in L.rp_last_error().decode()


def test_linear_argument_checks() -> None:
    """rp_fp8_linear runs the GEMM's checks, then needs an 8-byte aligned bias
    (the epilogue reads four bf16 values at once); a null bias is rp_fp8_gemm."""
    L = _capi.lib()
    ok = (FAKE, FAKE, NK, FAKE, FAKE, 64, 64, 64, 64, 64, 64, 1.0, 1.0, None, None, None)
    bad = list(ok); bad[3] = FAKE + 2
    assert L.rp_fp8_linear(*bad) == 2 and "bias" in L.rp_last_error().decode()
    bad = list(ok); bad[0] = None
    assert L.rp_fp8_linear(*bad) == 1 and "null" in L.rp_last_error().decode()
    bad = list(ok); bad[6] = 6
    assert L.rp_fp8_linear(*bad) == 2 and "multiples" in L.rp_last_error().decode()


def test_balanced_linear_argument_checks() -> None:
    """rp_fp8_linear_balanced refuses a missing, short or unaligned workspace
    before any launch, then runs rp_fp8_linear's checks."""
    L = _capi.lib()
    n = _capi.RP_GEMM_BALANCED_WORKSPACE_BYTES
    ok = (FAKE, FAKE, NK, None, FAKE, 64, 64, 64, 64, 64, 64, 1.0, 1.0, None, None)
    for ws, nbytes in ((None, n), (FAKE, n - 1), (FAKE + 16, n)):
        assert L.rp_fp8_linear_balanced(*ok, ws, nbytes, None) == 3
        assert "workspace" in L.rp_last_error().decode()
    bad = list(ok); bad[3] = FAKE + 2
    assert L.rp_fp8_linear_balanced(*bad, FAKE, n, None) == 2
    assert "bias" in L.rp_last_error().decode()
    bad = list(ok); bad[6] = 6
    assert L.rp_fp8_linear_balanced(*bad, FAKE, n, None) == 2


def test_quantizer_argument_checks() -> None:
    L = _capi.lib()
    bf16, f16 = _capi.RP_DTYPE_BF16, _capi.RP_DTYPE_F16
    assert L.rp_fp8_scale(None, bf16, 1, 1, 16, 64, 1024, 1024, 64, 0, FAKE, FAKE, 4096,
                          None) == 1
    assert L.rp_fp8_scale_quantize(FAKE, f16, 1, 1, 16, 64, 1024, 1024, 64, 5, FAKE, FAKE, 0, 0,
                                   FAKE, 4096, None) != 0
    assert "granularity" in L.rp_last_error().decode()
    for dt in (2, -1):   # fp32 and unknown inputs are refused before any launch
        assert L.rp_fp8_scale(FAKE, dt, 1, 1, 16, 64, 1024, 1024, 64, 0, FAKE, FAKE, 4096,
                              None) == 1
        assert "input dtype" in L.rp_last_error().decode()
        assert L.rp_fp8_quantize(FAKE, dt, 1, 1, 16, 64, 1024, 1024, 64, 0, FAKE, FAKE, 0, 0,
                                 None) == 1
        assert L.rp_selftest_scale(FAKE, dt, FAKE, FAKE, 4, None) == 1


def _norm(L, **kw) -> int:
    a = dict(x=FAKE, B=1, H=2, S=64, D=128, sb=2 * 64 * 128, sh=64 * 128, ss=128, w=None,
             eps=1e-6, cos=None, sin=None, rope=0, gran=0, dq=FAKE, codes=FAKE, ws=FAKE,
             nbytes=1 << 20, stream=None)
    a.update(kw)
    return L.rp_fp8_rmsnorm_scale_quantize(*a.values())


@pytest.mark.parametrize("kw,status,msg", [
    (dict(x=None), 1, "null pointer"),
    (dict(D=96), 2, "head dim"),
    (dict(S=0), 1, "non-positive"),
    (dict(gran=5), 1, "granularity"),
    (dict(rope=3), 1, "rope_mode"),
    (dict(rope=1), 1, "cos and sin"),
    (dict(eps=-1.0), 1, "eps"),
    (dict(eps=float("inf")), 1, "eps"),
    (dict(ss=127), 2, "aligned"),
    (dict(nbytes=0), 3, "workspace"),
])
def test_rmsnorm_quantize_argument_checks(kw: dict, status: int, msg: str) -> None:
    L = _capi.lib()
    assert _norm(L, **kw) == status
    assert msg in L.rp_last_error().decode()


def test_rmsnorm_workspace_sizing() -> None:
    L = _capi.lib()
    # one partial per 16384 elements of a group (64 rows x 128 per (b, h) -> 1 block
    # each), padded to 256 bytes, then one fp32 inverse norm per row
    assert L.rp_fp8_rmsnorm_quant_workspace_bytes(1, 2, 64, 128, 0) == 256 + 2 * 64 * 4
    assert L.rp_fp8_rmsnorm_quant_workspace_bytes(1, 2, 64, 128, 1) == 256 + 2 * 64 * 4
    assert L.rp_fp8_rmsnorm_quant_workspace_bytes(1, 40, 75600, 128, 0) == \
        (40 * 591 * 4 + 255) // 256 * 256 + 40 * 75600 * 4
    assert L.rp_fp8_rmsnorm_quant_workspace_bytes(1, 2, 64, 96, 0) == 0


def _norm_qkv(L, **kw) -> int:
    B, H, Sq, Skv, D = 1, 2, 64, 96, 128
    a = dict(q=FAKE, k=FAKE, v=FAKE, B=B, H=H, Sq=Sq, Skv=Skv, D=D,
             qsb=H * Sq * D, qsh=Sq * D, qss=D, ksb=H * Skv * D, ksh=Skv * D, kss=D,
             vsb=H * Skv * D, vsh=Skv * D, vss=D, qw=None, kw=None, eps=1e-6,
             qc=None, qs=None, kc=None, ks=None, rope=0, gran=0, dq=FAKE, q8=FAKE, k8=FAKE,
             vt8=FAKE, ldv=128, ws=FAKE, nbytes=1 << 20, stream=None)
    a.update(kw)
    return L.rp_fp8_rmsnorm_scale_quantize_qkv(*a.values())


@pytest.mark.parametrize("kw,status,msg", [
    (dict(v=None), 1, "null pointer"),
    (dict(vt8=None), 1, "null pointer"),
    (dict(k8=None), 1, "null pointer"),
    (dict(D=96), 2, "head dim"),
    (dict(Skv=0), 1, "non-positive"),
    (dict(gran=5), 1, "granularity"),
    (dict(rope=3), 1, "rope_mode"),
    (dict(rope=1, qc=FAKE, qs=FAKE), 1, "cos and sin"),     # K's tables missing
    (dict(eps=-1.0), 1, "eps"),
    (dict(kss=127), 2, "aligned"),
    (dict(vss=127), 2, "aligned"),
    (dict(ldv=64), 2, "ldv"),                                # below Skv
    (dict(ldv=200), 2, "ldv"),                               # not a multiple of 128
    (dict(nbytes=0), 3, "workspace"),
    (dict(ws=FAKE + 16), 3, "workspace"),                    # not 256-byte aligned
])
def test_rmsnorm_quantize_qkv_argument_checks(kw: dict, status: int, msg: str) -> None:
    """The fused Q/K-norm + V entry refuses bad arguments on the host, before
    any launch, with the single-tensor call's messages."""
    L = _capi.lib()
    assert _norm_qkv(L, **kw) == status
    assert msg in L.rp_last_error().decode()


def test_rmsnorm_qkv_workspace_sizing() -> None:
    """Q's, K's and V's partial maxima (one per 16384 elements of a group),
    each run padded to 256 bytes, then Q's and K's fp32 inverse norms."""
    L = _capi.lib()
    pad = lambda n: (n + 255) // 256 * 256  # noqa: E731
    B, H, Sq, Skv, D = 1, 40, 75600, 512, 128
    nq = H * -(-Sq * D // 16384)
    nk = H * -(-Skv * D // 16384)
    assert L.rp_fp8_rmsnorm_quant_qkv_workspace_bytes(B, H, Sq, Skv, D, 0) == \
        pad(4 * nq) + 2 * pad(4 * nk) + pad(4 * H * Sq) + 4 * H * Skv
    # per tensor: one group, the same block count
    assert L.rp_fp8_rmsnorm_quant_qkv_workspace_bytes(B, H, Sq, Skv, D, 1) == \
        pad(4 * nq) + 2 * pad(4 * nk) + pad(4 * H * Sq) + 4 * H * Skv
    assert L.rp_fp8_rmsnorm_quant_qkv_workspace_bytes(1, 2, 64, 64, 96, 0) == 0
    assert L.rp_fp8_rmsnorm_quant_qkv_workspace_bytes(1, 2, 64, 0, 128, 0) == 0


def test_multi_block_launch_plan() -> None:
    """Which shapes stream several query blocks per workgroup (short,
    unmasked key ranges with many query blocks), and that the others keep
    one block per workgroup."""
    L = _capi.lib()
    plan = L.rp_fp8_attn_blocks_per_workgroup
    assert plan(1, 40, 75600, 512, 128, 0, 1) == 50          # Wan cross: 240 workgroups
    assert plan(1, 40, 75600, 75600, 128, 0, 1) == 1         # Wan self: long key range
    assert plan(1, 40, 75600, 512, 128, 1, 1) == 1           # causal mask
    assert plan(1, 40, 75600, 512, 128, 2, 1) == 1           # shared-prefix mask
    assert plan(1, 40, 75600, 512, 256, 0, 1) == 1           # head dim 256 (two halves)
    assert plan(1, 40, 75600, 512, 128, 0, 4) == 1           # key splits
    assert plan(1, 40, 75600, 100, 128, 0, 8) > 1            # one tile: no split happens
    assert plan(1, 8, 1024, 1024, 64, 0, 1) == 1             # C1: 32 blocks in all
    assert plan(1, 40, 75600, 4096, 128, 0, 1) > 1           # 32 tiles: still pays
    assert plan(1, 40, 75600, 4097, 128, 0, 1) == 1          # 33 tiles: off
    assert plan(0, 40, 75600, 512, 128, 0, 1) == 0           # invalid


def test_balanced_launch_plan() -> None:
    """rp_fp8_attn_balanced_plan: the query blocks per head that fill whole
    rounds of workgroups on `cus` compute units run unsplit, the rest key-split
    2, 4 or 8 ways when that shortens the last round; masks, multi-block
    shapes, whole rounds and unknown CU counts keep one plain launch."""
    L = _capi.lib()

    def plan(B, H, Sq, Skv, D, mask=0, cus=256):
        m, s = ctypes.c_int(), ctypes.c_int()
        assert L.rp_fp8_attn_balanced_plan(B, H, Sq, Skv, D, mask, cus, ctypes.byref(m),
                                           ctypes.byref(s)) == 0
        return m.value, s.value

    # C3 self: 40 heads x 296 blocks; 288 per head fill 45 rounds, the last
    # 8 x 40 = 320 workgroups split 4 ways take 1.25 round-equivalents
    assert plan(1, 40, 75600, 75600, 128) == (288, 4)
    # C2: 32 heads x 220 blocks; 216 fill 27 rounds, 128 tail workgroups x 2
    assert plan(1, 32, 56320, 56320, 128) == (216, 2)
    assert plan(1, 20, 75600, 75600, 256) == (288, 4)        # D=256: two halves per block
    assert plan(1, 8, 8860, 8192, 128) == (32, 8)            # 24 tail workgroups
    assert plan(1, 40, 75600, 75600, 128, mask=1) == (296, 1)     # causal
    assert plan(1, 40, 75600, 75600, 128, mask=2) == (296, 1)     # shared prefix
    assert plan(1, 40, 75600, 512, 128) == (296, 1)          # multi-block launch instead
    assert plan(1, 32, 65536, 65536, 128) == (256, 1)        # whole rounds already
    assert plan(1, 8, 8860, 512, 128) == (35, 1)             # 4 key tiles: 8 ways too few
    assert plan(1, 40, 75600, 75600, 128, cus=0) == (296, 1)      # CU count unknown
    # 304 CUs: 266 blocks per head fill whole rounds, the other 1200
    # workgroups take 3.95 rounds unsplit, which splitting cannot shorten
    assert plan(1, 40, 75600, 75600, 128, cus=304) == (296, 1)
    assert L.rp_fp8_attn_balanced_plan(1, 1, 1, 1, 128, 0, 256, None, None) != 0
    # workspace for the split tail only: 4 splits x 40 heads x 1872 rows
    rows = 4 * 40 * (75600 - 288 * 256)
    ml = (rows * 8 + 255) // 256 * 256
    assert L.rp_fp8_attn_workspace_bytes(1, 40, 75600 - 288 * 256, 128, 4) == ml + rows * 512


def test_qkv_quantizer_argument_checks() -> None:
    L = _capi.lib()
    args = [FAKE, FAKE, FAKE, _capi.RP_DTYPE_BF16, 1, 2, 64, 128, 64,
            2 * 64 * 64, 64 * 64, 64, 2 * 128 * 64, 128 * 64, 64, 2 * 128 * 64, 128 * 64, 64,
            0, FAKE, FAKE, FAKE, FAKE, 128, FAKE, 1 << 20, None]
    bad = list(args); bad[1] = None
    assert L.rp_fp8_scale_quantize_qkv(*bad) == 1 and "null" in L.rp_last_error().decode()
    bad = list(args); bad[3] = 7
    assert L.rp_fp8_scale_quantize_qkv(*bad) == 1 and "dtype" in L.rp_last_error().decode()
    bad = list(args); bad[23] = 100                      # ldv < Skv
    assert L.rp_fp8_scale_quantize_qkv(*bad) == 2 and "ldv" in L.rp_last_error().decode()


def test_rowwise_argument_checks() -> None:
    """The row-wise entry points check their arguments before any launch."""
    L = _capi.lib()
    bf16 = _capi.RP_DTYPE_BF16
    assert L.rp_fp8_rowwise_quantize(None, bf16, 4, 64, 64, FAKE, FAKE, 64, None) == 1
    assert L.rp_fp8_rowwise_quantize(FAKE, 7, 4, 64, 64, FAKE, FAKE, 64, None) == 1
    assert L.rp_fp8_rowwise_quantize(FAKE, bf16, 4, 60, 64, FAKE, FAKE, 64, None) == 2
    assert "multiples of 8" in L.rp_last_error().decode()
    assert L.rp_fp8_rowwise_quantize(FAKE, bf16, 4, 64, 32, FAKE, FAKE, 64, None) == 1
    assert L.rp_transpose16(FAKE, FAKE, 1, 8, 8, 4, 8, 64, 64, None) == 1
    assert L.rp_fp8_softmax_rowwise_quantize(FAKE, 4, 63, 64, 4, 0, 0.1, FAKE, FAKE, 64,
                                             None) == 2
    assert L.rp_fp8_softmax_rowwise_quantize(FAKE, 4, 64, 64, 4, 0, float("nan"), FAKE, FAKE,
                                             64, None) == 1
    # row-wise GEMM: both scale vectors, aligned column scales, a sane batch
    args = (FAKE, FAKE, _capi.RP_B_NK, FAKE, 64, 64, 64, 64, 64, 64)
    assert L.rp_fp8_gemm_rowwise(*args, None, FAKE, 1, 0, 0, 0, 0, 0, None) == 1
    assert L.rp_fp8_gemm_rowwise(*args, FAKE, FAKE + 4, 1, 0, 0, 0, 0, 0, None) == 1
    assert L.rp_fp8_gemm_rowwise(*args, FAKE, FAKE, 0, 0, 0, 0, 0, 0, None) == 2
    assert L.rp_fp8_gemm_rowwise(*args, FAKE, FAKE, 2, 8, 0, 0, 0, 0, None) == 2
