"""MI355X-native (gfx950) FP8 attention hot path of miteshs/repercep-runtime.

Importable spelling of the ``repercep-runtime_amd`` package.  Layers:

* ``csrc/``      hand-written HIP kernels for gfx950 and their C ABI
                 (declared in include/repercep_fp8.h), built into
                 ``lib/librepercep_fp8.so`` by ``build.py``;
* ``_capi``      ctypes binding of that library (no fallback: a missing
                 library raises);
* ``ops``        kernel-layer torch entry points (quantize, attention, GEMM);
* ``attention``  the reference's AttentionOp surface (protocol, registry,
                 FP8 op, diffusers-layout bridge);
* ``backend``    the reference's Backend seam with MI355X added;
* ``workloads``  the BASELINE configurations and their seeded inputs.
"""

__version__ = "0.1.0"
