"""Compile-time host evaluation: constant folding and W8A8 calibration.

The reference runs both on the CPU with its op registry (mira/passes.py:26-38,
mira/quantize.py:73-92): calibration executes the float graph on sample inputs
to find each q-op input's peak |x|.  This module does the same for the rocm
target's compile step.  Its results only ever become constants or x_scale
attrs; it is never used to produce an output of RocmExecutable.run, whose
only compute path is the HIP library.

Float convolutions and matmuls here use BLAS-friendly loop orders (one GEMM
per kernel tap over NHWC rows), so calibration peaks can differ from the
reference's in the last bits; parity tests therefore feed one set of attrs to
both the rocm target and the golden model.
"""
from __future__ import annotations

import numpy as np

from .ops import conv_out, conv_params
from .types import NP_DTYPES


def _f32(a) -> np.ndarray:
    return np.asarray(a).astype(np.float32, copy=False)


def _native_or_f32(x: np.ndarray) -> np.ndarray:
    return x if x.dtype.kind == "i" else _f32(x)


def _gelu(x):
    return 0.5 * x * (1.0 + np.tanh(0.7978845608028654 * (x + 0.044715 * x ** 3)))


UNARY = {
    "relu": lambda x: np.maximum(x, 0), "gelu": _gelu, "sigmoid": lambda x: 1.0 / (1.0 + np.exp(-x)),
    "tanh": np.tanh, "exp": np.exp, "log": np.log, "sqrt": np.sqrt, "abs": np.abs, "neg": np.negative,
    "sign": np.sign,
}
BINARY = {
    "add": np.add, "sub": np.subtract, "mul": np.multiply, "div": np.divide, "pow": np.power,
    "maximum": np.maximum, "minimum": np.minimum, "greater": np.greater, "greater_equal": np.greater_equal,
    "equal": np.equal,
}


def _epilogue(acc: np.ndarray, xs: list, epilogue) -> np.ndarray:
    for fn, idx, swapped in epilogue:
        if idx is None:
            acc = UNARY[fn](acc)
        else:
            other = _f32(xs[idx])
            acc = BINARY[fn](other, acc) if swapped else BINARY[fn](acc, other)
    return acc


def _conv2d_f32(x: np.ndarray, w: np.ndarray, a: dict) -> np.ndarray:
    """NCHW x OIHW -> NCHW float32 convolution, one GEMM (or multiply) per kernel tap."""
    (sh, sw), (ph, pw), (dh, dw), g = conv_params(a)
    n, c, h, wd = x.shape
    o, cg, kh, kw = w.shape
    oh, ow = conv_out(h, kh, sh, ph, dh), conv_out(wd, kw, sw, pw, dw)
    xp = np.pad(_f32(x), ((0, 0), (0, 0), (ph, ph), (pw, pw))).transpose(0, 2, 3, 1)   # NHWC
    w = _f32(w)
    og = o // g
    if g == 1:
        # im2col: one [N*OH*OW, KH*KW*C] x [KH*KW*C, O] GEMM
        cols = np.empty((n, oh, ow, kh, kw, c), np.float32)
        for i in range(kh):
            for j in range(kw):
                cols[:, :, :, i, j, :] = xp[:, i * dh:i * dh + sh * (oh - 1) + 1:sh,
                                            j * dw:j * dw + sw * (ow - 1) + 1:sw, :]
        wm = w.transpose(2, 3, 1, 0).reshape(kh * kw * c, o)
        out = np.matmul(cols.reshape(n * oh * ow, -1), wm).reshape(n, oh, ow, o)
        return np.ascontiguousarray(out.transpose(0, 3, 1, 2))
    acc = np.zeros((n, oh, ow, o), np.float32)
    for i in range(kh):
        for j in range(kw):
            xt = xp[:, i * dh:i * dh + sh * (oh - 1) + 1:sh, j * dw:j * dw + sw * (ow - 1) + 1:sw, :]
            if g == 1:
                acc += np.matmul(xt.reshape(-1, c), w[:, :, i, j].T).reshape(n, oh, ow, o)
            elif cg == 1 and og == 1:
                acc += xt * w[:, 0, i, j]
            else:
                for gi in range(g):
                    xs = xt[..., gi * cg:(gi + 1) * cg].reshape(-1, cg)
                    acc[..., gi * og:(gi + 1) * og] += (xs @ w[gi * og:(gi + 1) * og, :, i, j].T).reshape(
                        n, oh, ow, og)
    return np.ascontiguousarray(acc.transpose(0, 3, 1, 2))


def evaluate(kind: str, xs: list, a: dict) -> np.ndarray:
    if kind == "const":
        return a["value"]
    if kind == "dequantize":
        q, scale, axis = a["q"], a["scale"], a["axis"]
        shape = [1] * q.ndim
        shape[axis] = -1
        return (q.astype(np.float32) * scale.reshape(shape)).astype(NP_DTYPES[a["dtype"]])
    if kind in UNARY:
        return UNARY[kind](_native_or_f32(xs[0])).astype(xs[0].dtype)
    if kind in BINARY:
        return BINARY[kind](_native_or_f32(xs[0]), _native_or_f32(xs[1])).astype(xs[0].dtype)
    if kind == "matmul":
        acc = np.matmul(_f32(xs[0]), _f32(xs[1]))
        return _epilogue(acc, xs, a.get("epilogue", ())).astype(xs[0].dtype)
    if kind == "conv2d":
        acc = _conv2d_f32(xs[0], xs[1], a)
        return _epilogue(acc, xs, a.get("epilogue", ())).astype(xs[0].dtype)
    if kind == "maxpool2d":
        k, s = a["size"], a["stride"]
        win = np.lib.stride_tricks.sliding_window_view(xs[0], (k, k), axis=(2, 3))[:, :, ::s, ::s]
        return win.max(axis=(-2, -1)).astype(xs[0].dtype)
    if kind == "pad":
        return np.pad(xs[0], a["pads"], constant_values=np.asarray(a.get("value", 0)).astype(xs[0].dtype))
    if kind in ("reduce_sum", "reduce_mean", "reduce_max"):
        f = {"reduce_sum": np.sum, "reduce_mean": np.mean, "reduce_max": np.max}[kind]
        return np.asarray(f(_native_or_f32(xs[0]), axis=tuple(a["axes"]), keepdims=a["keepdims"])).astype(
            xs[0].dtype)
    if kind == "reshape":
        return xs[0].reshape(a["shape"])
    if kind == "transpose":
        return np.ascontiguousarray(np.transpose(xs[0], a["perm"]))
    if kind == "softmax":
        x = _f32(xs[0])
        e = np.exp(x - x.max(axis=a["axis"], keepdims=True))
        return (e / e.sum(axis=a["axis"], keepdims=True)).astype(xs[0].dtype)
    if kind == "layernorm":
        x, g, b = (_f32(v) for v in xs)
        mu = x.mean(axis=-1, keepdims=True)
        var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
        return ((x - mu) / np.sqrt(var + a["eps"]) * g + b).astype(xs[0].dtype)
    if kind == "cast":
        return xs[0].astype(NP_DTYPES[a["dtype"]])
    if kind == "gather":
        return np.take(xs[0], xs[1], axis=a["axis"])
    if kind == "concat":
        return np.concatenate(xs, axis=a["axis"])
    # qmatmul/qconv2d are deliberately absent: folding and calibration run on the
    # float graph, before W8A8 rewriting, and int8 math only ever runs on the GPU.
    raise NotImplementedError(f"no compile-time evaluation for '{kind}'")


def peaks(g, feeds: list, watch: set) -> dict:
    """Largest |value| of each watched value over the calibration feeds (mira/quantize.py:73-92)."""
    peak = {v: 0.0 for v in watch}
    for feed in feeds:
        env = {}
        for v in g.inputs:
            if v.name not in feed:
                raise ValueError(f"calibration input is missing '{v.name}'")
            env[v] = np.asarray(feed[v.name]).astype(v.type.np_dtype)
        for op in g.ops:
            if op.is_control:
                raise ValueError("W8A8 quantization doesn't support programs with data-dependent control flow yet")
            env[op.result] = evaluate(op.kind, [env[x] for x in op.inputs], op.attrs)
            if op.result in peak:
                peak[op.result] = max(peak[op.result], float(np.abs(env[op.result].astype(np.float32)).max()))
        for v in g.inputs:
            if v in peak:
                peak[v] = max(peak[v], float(np.abs(env[v].astype(np.float32)).max()))
    return peak
