"""Type rules of the ops the W8A8 path meets (the `infer` half of mira/ops.py).

Only shapes and dtypes live here: the rocm target computes on the GPU and the
compile-time calibration evaluator lives in calibrate.py.  Each rule follows
the reference op's `infer` (file:line given per rule) so graphs built or
rewritten here verify exactly where the reference's would.
"""
from __future__ import annotations

from typing import Callable

from .types import TensorType, type_of_array


class OpTypeError(Exception):
    """An op was applied to operands with incompatible shapes or dtypes."""


UNARY = {"relu", "gelu", "sigmoid", "tanh", "exp", "log", "sqrt", "abs", "neg", "sign", "erf"}
INT_UNARY = {"relu", "neg", "abs", "sign"}
BINARY = {"add", "sub", "mul", "div", "pow", "maximum", "minimum", "greater", "greater_equal", "equal"}
FLOAT_ONLY_BINARY = {"div", "pow"}
REDUCE = {"reduce_sum", "reduce_mean", "reduce_max"}


def same_dtype(types: list[TensorType], op: str) -> str:
    dts = {t.dtype for t in types}
    if len(dts) != 1:
        raise OpTypeError(f"{op}: operands have different dtypes ({', '.join(map(str, types))})")
    return dts.pop()


def broadcast_shapes(a: tuple[int, ...], b: tuple[int, ...], op: str) -> tuple[int, ...]:
    """NumPy broadcasting (mira/ops.py:53-66)."""
    out = []
    for i in range(max(len(a), len(b))):
        da = a[-1 - i] if i < len(a) else 1
        db = b[-1 - i] if i < len(b) else 1
        if da == db or db == 1:
            out.append(da)
        elif da == 1:
            out.append(db)
        else:
            raise OpTypeError(f"{op}: shapes {list(a)} and {list(b)} can't be broadcast")
    return tuple(reversed(out))


def need_float(types: list[TensorType], op: str) -> None:
    for t in types:
        if not t.is_float:
            raise OpTypeError(f"{op}: needs floating-point operands, got {t}")


def norm_axis(axis: int, rank: int, op: str) -> int:
    if not -rank <= axis < rank:
        raise OpTypeError(f"{op}: axis {axis} is out of range for rank {rank}")
    return axis % rank


def epilogue_infer(core: TensorType, ts: list[TensorType], epilogue, op: str) -> TensorType:
    """mira/ops.py:183-189: every epilogue operand must broadcast onto the core result."""
    for _fn, idx, _sw in epilogue:
        if idx is not None:
            other = ts[idx]
            if other.dtype != core.dtype or broadcast_shapes(core.shape, other.shape, op) != core.shape:
                raise OpTypeError(f"{op}: epilogue operand {other} doesn't fit result {core}")
    return core


def conv_params(a: dict):
    """(stride, padding, dilation, groups) with the reference's defaults (mira/ops.py:229-231)."""
    return tuple(a["stride"]), tuple(a["padding"]), tuple(a.get("dilation", (1, 1))), a.get("groups", 1)


def conv_out(size: int, k: int, stride: int, pad: int, dilation: int = 1) -> int:
    return (size + 2 * pad - dilation * (k - 1) - 1) // stride + 1


def _matmul(ts, a):
    """mira/ops.py:204-214."""
    x, w = ts[0], ts[1]
    dt = same_dtype([x, w], "matmul")
    need_float([x], "matmul")
    if x.rank < 2 or w.rank < 2 or x.shape[-1] != w.shape[-2]:
        raise OpTypeError(f"matmul: can't multiply {x} @ {w}")
    batch = broadcast_shapes(x.shape[:-2], w.shape[:-2], "matmul")
    return epilogue_infer(TensorType(dt, batch + (x.shape[-2], w.shape[-1])), ts, a.get("epilogue", ()), "matmul")


def _conv_core(x: TensorType, w_shape: tuple, a: dict, dt: str) -> TensorType:
    """mira/ops.py:234-253."""
    if x.rank != 4 or len(w_shape) != 4:
        raise OpTypeError(f"conv2d: expects [N, C, H, W] input and [O, C/g, KH, KW] weight, got {x}, {list(w_shape)}")
    n, c, h, wd = x.shape
    o, ci, kh, kw = w_shape
    (sh, sw), (ph, pw), (dh, dw), g = conv_params(a)
    if g < 1 or c % g or o % g or c != ci * g:
        raise OpTypeError(f"conv2d: groups={g} doesn't fit {c} input / {o} output channels")
    oh, ow = conv_out(h, kh, sh, ph, dh), conv_out(wd, kw, sw, pw, dw)
    if oh <= 0 or ow <= 0:
        raise OpTypeError("conv2d: kernel larger than padded input")
    return TensorType(dt, (n, o, oh, ow))


def _conv2d(ts, a):
    x, w = ts[0], ts[1]
    dt = same_dtype([x, w], "conv2d")
    need_float([x], "conv2d")
    return epilogue_infer(_conv_core(x, w.shape, a, dt), ts, a.get("epilogue", ()), "conv2d")


def _qmatmul(ts, a):
    """mira/ops.py:606-613."""
    x = ts[0]
    need_float([x], "qmatmul")
    k, n = a["q"].shape
    if x.rank < 2 or x.shape[-1] != k:
        raise OpTypeError(f"qmatmul: {x} doesn't match int8 weights [{k}, {n}]")
    return epilogue_infer(TensorType(a["dtype"], x.shape[:-1] + (n,)), ts, a.get("epilogue", ()), "qmatmul")


def _qconv2d(ts, a):
    """mira/ops.py:623-627."""
    x = ts[0]
    need_float([x], "qconv2d")
    core = _conv_core(x, tuple(a["q"].shape), a, x.dtype).with_dtype(a["dtype"])
    return epilogue_infer(core, ts, a.get("epilogue", ()), "qconv2d")


def _maxpool(ts, a):
    """mira/ops.py:282-290."""
    x = ts[0]
    k, s = a["size"], a["stride"]
    if x.rank != 4 or x.shape[2] < k or x.shape[3] < k:
        raise OpTypeError(f"maxpool2d: window {k} doesn't fit {x}")
    n, c, h, w = x.shape
    return TensorType(x.dtype, (n, c, (h - k) // s + 1, (w - k) // s + 1))


def _pad(ts, a):
    """mira/ops.py:461-466."""
    x = ts[0]
    pads = tuple(a["pads"])
    if len(pads) != x.rank or any(lo < 0 or hi < 0 for lo, hi in pads):
        raise OpTypeError(f"pad: need {x.rank} non-negative (before, after) pairs")
    return TensorType(x.dtype, tuple(d + lo + hi for d, (lo, hi) in zip(x.shape, pads)))


def _reduce(name):
    def infer(ts, a):
        """mira/ops.py:323-333."""
        x = ts[0]
        if name == "reduce_mean":
            need_float(ts, name)
        axes = sorted(norm_axis(ax, x.rank, name) for ax in a["axes"])
        if a["keepdims"]:
            shape = tuple(1 if i in axes else d for i, d in enumerate(x.shape))
        else:
            shape = tuple(d for i, d in enumerate(x.shape) if i not in axes)
        return TensorType(x.dtype, shape)
    return infer


def _reshape(ts, a):
    x, shape = ts[0], tuple(a["shape"])
    total = 1
    for d in shape:
        total *= d
    if total != x.numel:
        raise OpTypeError(f"reshape: can't reshape {x} to {list(shape)}")
    return TensorType(x.dtype, shape)


def _transpose(ts, a):
    x, perm = ts[0], tuple(a["perm"])
    if sorted(perm) != list(range(x.rank)):
        raise OpTypeError(f"transpose: bad perm {list(perm)}")
    return TensorType(x.dtype, tuple(x.shape[p] for p in perm))


def _unary(name):
    def infer(ts, a):
        if name not in INT_UNARY:
            need_float(ts, name)
        return ts[0]
    return infer


def _binary(name):
    def infer(ts, a):
        dt = same_dtype(ts, name)
        if name in FLOAT_ONLY_BINARY:
            need_float(ts, name)
        return TensorType(dt, broadcast_shapes(ts[0].shape, ts[1].shape, name))
    return infer


def _layernorm(ts, a):
    x, g, b = ts
    same_dtype(ts, "layernorm")
    d = x.shape[-1]
    if g.shape != (d,) or b.shape != (d,):
        raise OpTypeError("layernorm: gamma/beta must match the last axis")
    return x


def _softmax(ts, a):
    need_float(ts, "softmax")
    norm_axis(a["axis"], ts[0].rank, "softmax")
    return ts[0]


def _gather(ts, a):
    table, idx = ts
    if idx.dtype != "i32":
        raise OpTypeError("gather: indices must be i32")
    ax = norm_axis(a["axis"], table.rank, "gather")
    return TensorType(table.dtype, table.shape[:ax] + idx.shape + table.shape[ax + 1:])


def _concat(ts, a):
    dt = same_dtype(ts, "concat")
    ax = norm_axis(a["axis"], ts[0].rank, "concat")
    shape = list(ts[0].shape)
    shape[ax] = sum(t.shape[ax] for t in ts)
    return TensorType(dt, tuple(shape))


RULES: dict[str, Callable] = {
    "const": lambda ts, a: type_of_array(a["value"]),
    "dequantize": lambda ts, a: TensorType(a["dtype"], tuple(a["q"].shape)),
    "matmul": _matmul,
    "conv2d": _conv2d,
    "qmatmul": _qmatmul,
    "qconv2d": _qconv2d,
    "maxpool2d": _maxpool,
    "pad": _pad,
    "reshape": _reshape,
    "transpose": _transpose,
    "layernorm": _layernorm,
    "softmax": _softmax,
    "gather": _gather,
    "concat": _concat,
    "cast": lambda ts, a: ts[0].with_dtype(a["dtype"]),
}
RULES.update({n: _unary(n) for n in UNARY})
RULES.update({n: _binary(n) for n in BINARY})
RULES.update({n: _reduce(n) for n in REDUCE})


def infer(kind: str, types: list[TensorType], attrs: dict) -> TensorType:
    if kind not in RULES:
        raise OpTypeError(f"unknown op '{kind}'")
    return RULES[kind](types, attrs)
