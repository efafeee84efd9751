"""mira_amd: MIRA's W8A8 quantized-inference path as an MI355X (gfx950) target.

The package is the `rocm` execution target of the MIRA tensor compiler
(myramay/MIRA) for one hot path, W8A8 inference.  MIRA's own compiler,
quantizer and partitioner produce the graphs; this package runs them:

    target.RocmTarget / RocmExecutable   the Target/Executable plugin (mira/backends/base.py:13-26)
    _lib                                 ctypes binding of libmira_rocm.so (include/mira_rocm.h)
    pack                                 host-side byte order of int8 weights and activations
    build                                hipcc build of libmira_rocm.so for gfx950
    csrc/                                the HIP kernels (int8 MFMA GEMM / implicit-GEMM conv,
                                         fused dequant/epilogue/requant, quantizer, depthwise,
                                         pooling, the float ops of a transformer decode step)
                                         and their C ABI

`get_target` / `TARGETS` are the branch a MIRA checkout adds to its backend
registry (mira/backends/__init__.py:5-25).
"""
from __future__ import annotations

TARGETS = ["rocm"]


def get_target(name: str, **options):
    """The rocm branch of MIRA's get_target: options device (int), debug_acc (bool),
    approx_f32 (bool: also run softmax, f32 matmuls of two tensors and libm epilogue steps,
    to f32 rounding instead of bit for bit) and graph_loops (bool, default True: a while loop
    run on the device replays its condition and body steps as HIP graphs)."""
    if name != "rocm":
        raise ValueError(f"unknown target '{name}' (this package provides: rocm)")
    from .target import RocmTarget
    unknown = set(options) - {"device", "debug_acc", "approx_f32", "graph_loops"}
    if unknown:
        raise ValueError(f"unknown rocm target options: {sorted(unknown)}")
    return RocmTarget(device=options.get("device", 0), debug_acc=options.get("debug_acc", False),
                      approx_f32=options.get("approx_f32", False), graph_loops=options.get("graph_loops", True))


__all__ = ["get_target", "TARGETS"]
