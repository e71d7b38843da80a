"""CPU oracle for the FP8 attention hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the numerics of miteshs/repercep-runtime's
FP8 path (OCP e4m3fn, the gfx950 format).  It is the checker, never the thing
measured or shipped: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it.  The product package
``repercep_runtime_amd`` never imports it and fails loudly when its HIP
library is missing.

Modules
-------
quant       torch-CPU restatement of the reference quantizer
            (kernels/triton_kernels/fp8_flash_attn_hopper.py:374-398) and a
            numpy e4m3fn encoder/decoder written from the format definition.
attention   numpy tile-exact emulation of the FA-2 FP8 kernel body
            (kernels/triton_kernels/fp8_flash_attn.py:294-391) plus exact
            fp64 softmax references used to pin it.
gemm        emulation of kernels/hip/fp8_attn/fp8_gemm.hip:79-156.
native      ctypes binding of the C restatement in oracle/c/fp8_oracle.c
            (same numerics, OpenMP, used for full-size parity checks).
cpu_sdpa    the reference's CPU attention floor (AMXSDPAAttention,
            src/repercep/attention/amx_sdpa.py:76-94), timed as the CPU baseline.

Parity status of each function is recorded in its module docstring.
"""
