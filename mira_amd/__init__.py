"""mira_amd: MIRA's W8A8 quantized-inference path as an MI355X (gfx950) target.

The package is the `rocm` execution target of the MIRA tensor compiler
(myramay/MIRA) for one hot path -- W8A8 inference -- plus the host-side
mirror of the reference interfaces it plugs into:

    target.RocmTarget / RocmExecutable   the Target/Executable plugin (mira/backends/base.py)
    _lib                                 ctypes binding of libmira_rocm.so (include/mira_rocm.h)
    csrc/                                the HIP kernels (int8 MFMA GEMM / implicit-GEMM conv,
                                         fused dequant/epilogue/requant, quantizer, depthwise,
                                         pooling) and their C ABI
    ir, types, ops, passes, quantize,    mirrors of the reference's IR, type rules, passes,
    partition, compiler                  W8A8 rewrite, partitioner and driver
    hosteval                             compile-time constant folding and calibration
    models                               graph builders for the benchmark configurations
"""
from .compiler import CompiledProgram, compile_graph, compile_ir, get_target  # noqa: F401

__all__ = ["compile_ir", "compile_graph", "get_target", "CompiledProgram"]
