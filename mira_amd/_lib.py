"""ctypes binding of libmira_rocm.so (declarations in include/mira_rocm.h).

The library is the only compute path of the rocm target: if it is missing or
was built for another ABI, loading raises instead of falling back to anything.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path
from typing import Optional

LIB_PATH = Path(__file__).resolve().parent / "libmira_rocm.so"
ABI_VERSION = 12
MAX_EPI = 8

# enum mr_epi_fn
EPI_FN = {"add": 1, "sub": 2, "mul": 3, "div": 4, "maximum": 5, "minimum": 6, "relu": 7,
          "gelu": 8, "sigmoid": 9, "tanh": 10}
EPI_UNARY = ("relu", "gelu", "sigmoid", "tanh")
EPI_APPROX = ("gelu", "sigmoid", "tanh")     # libm steps: not bit-identical to NumPy
EPI_OUT_F16 = 1     # mr_epilogue.flags: round results to f16 (the op's dtype is f16)
EPI_OUT_H16 = 2     # ... and store them as IEEE halves (out_f32 points to halves)
EPI_FULL_H16 = 4    # full-shape operands hold IEEE halves
# enum mr_ew_fn (mr_elementwise_f32 beyond the epilogue codes)
EW_FN = {"add": 1, "sub": 2, "mul": 3, "div": 4, "maximum": 5, "minimum": 6, "relu": 7,
         "greater": 11, "greater_equal": 12, "equal": 13, "neg": 14, "abs": 15}
EW_UNARY = ("relu", "neg", "abs")
# enum mr_bcast
BC_SCALAR, BC_COL, BC_ROW, BC_FULL = 0, 1, 2, 3

EXPORTS = [
    "mr_abi_version", "mr_last_error", "mr_sizeof", "mr_init",
    "mr_quantize_rows", "mr_quantize_nchw_nhwc", "mr_quantize_f16_nchw_nhwc",
    "mr_qmatmul", "mr_qmatmul_f32in", "mr_qmatmul_lnin", "mr_w8_matmul_f32", "mr_w8_conv2d_f32", "mr_qconv2d", "mr_qconv2d_maxpool",
    "mr_qconv2d_maxpool_f32in", "mr_dwconv2d_f32", "mr_qconv1x1_dw3x3", "mr_qstem3x3_dw3x3",
    "mr_maxpool2d_f32", "mr_mean_hw_f32", "mr_pad_hw_f32", "mr_round_f16_f32",
    "mr_nchw_to_nhwc_f32", "mr_nchw_to_nhwc_pad_f32", "mr_nhwc_to_nchw_f32",
    "mr_layernorm_f32", "mr_softmax_f32", "mr_bmm_f32", "mr_transpose_f32", "mr_copy_rows_f32",
    "mr_attention_decode_f32", "mr_decode_embed", "mr_decode_commit", "mr_elementwise_f32",
    "mr_elementwise_i32", "mr_cast_32", "mr_gather_rows_32", "mr_dynamic_slice_32", "mr_dynamic_update_slice_32",
    "mr_argmax_f32", "mr_where_32",
]
DT = {"f32": 0, "f16": 1, "i32": 2}       # enum mr_dtype
DECODE_MAX_CACHES = 16      # MR_DECODE_MAX_CACHES


class EpiStep(C.Structure):
    _fields_ = [("fn", C.c_int32), ("swapped", C.c_int32), ("mode", C.c_int32), ("reserved", C.c_int32),
                ("ptr", C.c_void_p), ("ld", C.c_int64)]


class Epilogue(C.Structure):
    _fields_ = [("n_steps", C.c_int32), ("flags", C.c_int32), ("steps", EpiStep * MAX_EPI),
                ("scale", C.c_void_p), ("out_f32", C.c_void_p), ("ldo", C.c_int64),
                ("out_i8", C.c_void_p), ("ldq", C.c_int64), ("out_xs", C.c_float), ("reserved1", C.c_int32),
                ("out_acc", C.c_void_p), ("ldacc", C.c_int64)]


class ConvGeom(C.Structure):
    _fields_ = [(n, C.c_int32) for n in
                ("n", "h", "w", "c", "c_pad", "o", "oh", "ow", "kh", "kw", "sh", "sw", "ph", "pw", "dh", "dw")]


class RocmError(RuntimeError):
    """A libmira_rocm.so entry point returned an error status."""


_lib: Optional[C.CDLL] = None

_i32, _i64, _f32, _p = C.c_int32, C.c_int64, C.c_float, C.c_void_p
_SIGS = {
    "mr_abi_version": ([], C.c_int),
    "mr_last_error": ([], C.c_char_p),
    "mr_sizeof": ([C.c_char_p], _i64),
    "mr_init": ([C.c_int], C.c_int),
    "mr_quantize_rows": ([_p, _i64, _i64, _i64, _p, _i64, _f32, _p], C.c_int),
    "mr_quantize_nchw_nhwc": ([_p, _i32, _i32, _i32, _i32, _p, _i32, _f32, _p], C.c_int),
    "mr_quantize_f16_nchw_nhwc": ([_p, _i32, _i32, _i32, _i32, _p, _i32, _f32, _p], C.c_int),
    "mr_qmatmul": ([_p, _i64, _p, _i64, _i64, _i64, _i64, _i64, C.POINTER(Epilogue), _p], C.c_int),
    "mr_qmatmul_f32in": ([_p, _i64, _f32, _p, _i64, _i64, _i64, _i64, _i64, C.POINTER(Epilogue), _p], C.c_int),
    "mr_qmatmul_lnin": ([_p, _i64, _p, _p, _f32, _i32, _f32, _p, _i64, _i64, _i64, _i64, _i64, C.POINTER(Epilogue),
                         _p], C.c_int),
    "mr_w8_matmul_f32": ([_p, _i64, _p, _p, _i32, _i64, _i64, _i64, _i64, _i64, C.POINTER(Epilogue), _p], C.c_int),
    "mr_qconv2d": ([_p, C.POINTER(ConvGeom), _p, _i64, _i64, C.POINTER(Epilogue), _p], C.c_int),
    "mr_w8_conv2d_f32": ([_p, C.POINTER(ConvGeom), _p, _p, _i32, _i64, _i64, C.POINTER(Epilogue), _p], C.c_int),
    "mr_qconv2d_maxpool": ([_p, C.POINTER(ConvGeom), _p, _i64, _i64, C.POINTER(Epilogue), _i32, _i32, _i32, _i32,
                            _f32, _i32, _i32, _p], C.c_int),
    "mr_qconv2d_maxpool_f32in": ([_p, _f32, _i32, C.POINTER(ConvGeom), _p, _i64, _i64, C.POINTER(Epilogue), _i32,
                                  _i32, _i32, _i32, _f32, _i32, _i32, _p], C.c_int),
    "mr_dwconv2d_f32": ([_p, C.POINTER(ConvGeom), _p, C.POINTER(Epilogue), _p], C.c_int),
    "mr_qconv1x1_dw3x3": ([_p, _i64, _p, _i64, _i64, _i64, C.POINTER(Epilogue), C.POINTER(ConvGeom), _p,
                           C.POINTER(Epilogue), _p], C.c_int),
    "mr_qstem3x3_dw3x3": ([_p, C.POINTER(ConvGeom), _p, _i64, _i64, C.POINTER(Epilogue), C.POINTER(ConvGeom), _p,
                           C.POINTER(Epilogue), _p], C.c_int),
    "mr_maxpool2d_f32": ([_p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _i32, _p, _p, _i32, _f32,
                          _p], C.c_int),
    "mr_mean_hw_f32": ([_p, _i32, _i32, _i32, _p, _p, _i32, _f32, _i32, _p], C.c_int),
    "mr_pad_hw_f32": ([_p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _p, _p], C.c_int),
    "mr_round_f16_f32": ([_p, _i64, _p, _p], C.c_int),
    "mr_nchw_to_nhwc_f32": ([_p, _i32, _i32, _i32, _i32, _p, _p], C.c_int),
    "mr_nchw_to_nhwc_pad_f32": ([_p, _i32, _i32, _i32, _i32, _p, _i32, _p], C.c_int),
    "mr_nhwc_to_nchw_f32": ([_p, _i32, _i32, _i32, _i32, _p, _p], C.c_int),
    "mr_layernorm_f32": ([_p, _i64, _i32, _p, _p, _f32, _i32, _p, _p, _i64, _f32, _p], C.c_int),
    "mr_softmax_f32": ([_p, _i64, _i32, _i32, _p, _p], C.c_int),
    "mr_bmm_f32": ([_p, _p, _i32, _p, _p, _p, _p, _i64, _i64, _i64, C.POINTER(Epilogue), _p], C.c_int),
    "mr_transpose_f32": ([_p, _i32, _p, _p, _p, _p], C.c_int),
    "mr_copy_rows_f32": ([_p, _i64, _i64, _p, _i64, _i64, _p], C.c_int),
    "mr_attention_decode_f32": ([_p, _i64, _p, _p, _i64, _i64, _p, _i64, _p, _i64, _p, _f32, _i64, _i32, _i32, _i32, _p,
                                 _i64, _p, _i64, _f32, _p], C.c_int),
    "mr_decode_embed": ([_p, _i64, _p, _p, _p, _i32, _p, _i32, _i32, _p, _i64, _p, _f32, _p], C.c_int),
    "mr_elementwise_i32": ([_i32, _p, C.POINTER(_i64), _p, C.POINTER(_i64), _p, C.POINTER(_i64), _p], C.c_int),
    "mr_cast_32": ([_p, _i64, _i32, _i32, _p, _p], C.c_int),
    "mr_gather_rows_32": ([_p, _i64, _i64, _p, _i64, _p, _p], C.c_int),
    "mr_dynamic_slice_32": ([_p, C.POINTER(_i64), _p, _i32, C.POINTER(_i64), _p, _p], C.c_int),
    "mr_dynamic_update_slice_32": ([_p, C.POINTER(_i64), _p, C.POINTER(_i64), _p, _i32, _p, _p], C.c_int),
    "mr_argmax_f32": ([_p, _i64, _i64, _p, _p], C.c_int),
    "mr_where_32": ([_p, _i32, C.POINTER(_i64), _p, C.POINTER(_i64), _p, C.POINTER(_i64), _p, C.POINTER(_i64), _p],
                    C.c_int),
    "mr_elementwise_f32": ([_i32, _p, C.POINTER(_i64), _p, C.POINTER(_i64), _p, C.POINTER(_i64), _i32, _p], C.c_int),
    "mr_decode_commit": ([_p, _i64, _i32, _i32, _p, _p, _p, _i64, _i64, _i32, _p, _i64, _p, _p, _i32, _i32, _i64, _p],
                         C.c_int),
}


def load(path: Optional[Path] = None) -> C.CDLL:
    """Load (once) and type the library; raises if it is absent or mismatched."""
    global _lib
    if _lib is not None:
        return _lib
    p = Path(path or LIB_PATH)
    if not p.exists():
        raise RocmError(f"{p} is not built: run `python -m mira_amd.build` (the rocm target has no other "
                        f"compute path)")
    # PyTorch-ROCm ships its own libamdhip64.so (soname libamdhip64.so.7).  Loading torch
    # first makes this library bind to that same HIP runtime, so torch's device pointers
    # and streams are valid here; loading it first would put two runtimes in the process.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = C.CDLL(str(p))
    for name, (args, res) in _SIGS.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    if lib.mr_abi_version() != ABI_VERSION:
        raise RocmError(f"{p}: ABI version {lib.mr_abi_version()} != {ABI_VERSION}")
    for name, cls in (("mr_epi_step", EpiStep), ("mr_epilogue", Epilogue), ("mr_conv_geom", ConvGeom)):
        if lib.mr_sizeof(name.encode()) != C.sizeof(cls):
            raise RocmError(f"{p}: sizeof({name}) {lib.mr_sizeof(name.encode())} != binding {C.sizeof(cls)}")
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = _lib.mr_last_error().decode(errors="replace") if _lib is not None else "?"
        raise RocmError(f"{what} failed (status {rc}): {msg}")


def call(name: str, *args) -> None:
    """Call an entry point and raise RocmError on a non-zero status."""
    lib = load()
    check(getattr(lib, name)(*args), name)
