"""The documented ctypes binding a maintainer would add to the reference
(kernels/hip/fp8_attn/ beside binding.cpp) declares the entry points exactly
as the product binding does.

The example is taken from the repository's integration guide, pointed at the
built library and executed (declarations and function definitions only, no
GPU call).  Every ``_L.<symbol>.argtypes`` / ``.restype`` it sets must equal
``repercep_runtime_amd._capi``'s, so the example cannot drift from the ABI.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

from repercep_runtime_amd import _capi

ROOT = Path(__file__).resolve().parent.parent
GUIDE = ROOT / "INTEGRATION.md"


def _binding_block() -> str:
    text = GUIDE.read_text()
    start = text.index("### ctypes binding")
    m = re.search(r"```python\n(.*?)```", text[start:], flags=re.S)
    assert m, "no python block after the ctypes binding heading"
    return m.group(1)


def test_binding_example_matches_product_declarations() -> None:
    src = _binding_block()
    assert 'ctypes.CDLL("/path/to/librepercep_fp8.so")' in src
    src = src.replace('"/path/to/librepercep_fp8.so"', repr(str(_capi.LIB_PATH)))
    ns: dict = {}
    exec(compile(src, "binding_example", "exec"), ns)     # defines, calls nothing on a GPU
    stub = ns["_L"]
    real = _capi.lib()
    declared = sorted(set(re.findall(r"_L\.(rp_\w+)\.(?:argtypes|restype)", src)))
    assert len(declared) >= 6, declared
    for name in declared:
        assert name in _capi.EXPORTS, name
        s_fn, r_fn = getattr(stub, name), getattr(real, name)
        if f"_L.{name}.argtypes" in src:
            assert list(s_fn.argtypes) == list(r_fn.argtypes), name
        if f"_L.{name}.restype" in src:
            assert s_fn.restype == r_fn.restype, name
        else:   # the example relies on ctypes' default int return
            assert r_fn.restype in (ctypes.c_int, None), name
    assert callable(ns["fp8_flash_attention"])
