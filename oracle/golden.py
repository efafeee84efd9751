"""NumPy restatement of MIRA's `cpu` golden model for the W8A8 inference path.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import this module, and only to check GPU results
against (or, in bench.py, as the timed CPU baseline).  The rocm target never calls it:
its run path is the HIP library, and it fails loudly without it.

Every function restates one reference function; the docstring names the
reference file:line it follows (paths relative to the reference checkout).
How each is pinned (golden vectors, closed forms, brute force, invariants) is
in tests/test_oracle.py.  Functions whose exact output no such check fixes
say "parity unpinned" in their docstring.

Graph-level helpers walk any IR with the reference's data model
(`graph.inputs/ops/outputs`, `op.kind/inputs/attrs/result/results`), so they run
the rocm package's mirror graphs without importing it.
"""
from __future__ import annotations

from typing import Callable, Optional

import numpy as np

NP_DTYPES = {"f16": np.float16, "f32": np.float32, "i32": np.int32}


def f32(a) -> np.ndarray:
    """mira/ops.py:43-44."""
    return np.asarray(a).astype(np.float32, copy=False)


def _native_or_f32(x: np.ndarray) -> np.ndarray:
    """mira/ops.py:150-152: floats compute in f32, integers stay exact."""
    return x if x.dtype.kind == "i" else f32(x)


# ---------------------------------------------------------------- elementwise (mira/ops.py:94-172)

def _gelu(x):
    """mira/ops.py:94-96 (tanh approximation).  Pinned by float64 closed forms (gelu(1) =
    0.8411920 for the tanh form); its last bits are libm's tanh, so device results are
    compared within a tolerance."""
    return 0.5 * x * (1.0 + np.tanh(0.7978845608028654 * (x + 0.044715 * x ** 3)))


UNARY: dict[str, Callable] = {
    "relu": lambda x: np.maximum(x, 0),
    "gelu": _gelu,
    "sigmoid": lambda x: 1.0 / (1.0 + np.exp(-x)),
    "tanh": np.tanh,
    "exp": np.exp,
    "log": np.log,
    "sqrt": np.sqrt,
    "abs": np.abs,
    "neg": np.negative,
    "sign": np.sign,
}

BINARY: dict[str, Callable] = {
    "add": np.add,
    "sub": np.subtract,
    "mul": np.multiply,
    "div": np.divide,
    "pow": np.power,
    "maximum": np.maximum,
    "minimum": np.minimum,
    "greater": np.greater,
    "greater_equal": np.greater_equal,
    "equal": np.equal,
}


def unary(kind: str, x: np.ndarray) -> np.ndarray:
    """mira/ops.py:163-165."""
    return UNARY[kind](_native_or_f32(x)).astype(x.dtype)


def binary(kind: str, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """mira/ops.py:167-169."""
    return BINARY[kind](_native_or_f32(a), _native_or_f32(b)).astype(a.dtype)


def epilogue_ref(acc: np.ndarray, xs: list, epilogue) -> np.ndarray:
    """mira/ops.py:192-199: ordered steps (fn, operand index, swapped)."""
    for fn, idx, swapped in epilogue:
        if idx is None:
            acc = UNARY[fn](acc)
        else:
            other = f32(xs[idx])
            acc = BINARY[fn](other, acc) if swapped else BINARY[fn](acc, other)
    return acc


# ---------------------------------------------------------------- matmul / conv (mira/ops.py:217-279)

def matmul(xs: list, attrs: dict) -> np.ndarray:
    """mira/ops.py:217-219.  f32 BLAS order: bit parity unpinned; pinned to the rounding bound
    of any f32 summation order against a float64 brute force (tests/test_oracle.py)."""
    acc = np.matmul(f32(xs[0]), f32(xs[1]))
    return epilogue_ref(acc, xs, attrs.get("epilogue", ())).astype(xs[0].dtype)


def conv_params(a: dict):
    """mira/ops.py:229-231."""
    return tuple(a["stride"]), tuple(a["padding"]), tuple(a.get("dilation", (1, 1))), a.get("groups", 1)


def conv_out(size: int, k: int, stride: int, pad: int, dilation: int = 1) -> int:
    """mira/ops.py:225-226."""
    return (size + 2 * pad - dilation * (k - 1) - 1) // stride + 1


def _taps(x: np.ndarray, kh: int, kw: int, a: dict, oh: int, ow: int):
    """mira/ops.py:256-262: zero-pad, then a strided view per kernel tap (i, j)."""
    (sh, sw), (ph, pw), (dh, dw), _ = conv_params(a)
    xp = np.pad(x, ((0, 0), (0, 0), (ph, ph), (pw, pw)))
    for i in range(kh):
        for j in range(kw):
            yield i, j, xp[:, :, i * dh:i * dh + sh * (oh - 1) + 1:sh, j * dw:j * dw + sw * (ow - 1) + 1:sw]


def conv2d(xs: list, a: dict) -> np.ndarray:
    """mira/ops.py:265-276: one (grouped) einsum per tap, accumulated in f32 in (i, j) order.

    With groups == C and one output per group (depthwise) every einsum is one
    f32 multiply, so the result is fixed tap by tap; for groups == 1 the
    einsum's internal summation order is OpenBLAS's (parity unpinned for
    non-integer data)."""
    x, w = f32(xs[0]), f32(xs[1])
    g = a.get("groups", 1)
    n, c, h, wd = x.shape
    o, cg, kh, kw = w.shape
    (sh, sw), (ph, pw), (dh, dw), _ = conv_params(a)
    oh, ow = conv_out(h, kh, sh, ph, dh), conv_out(wd, kw, sw, pw, dw)
    acc = np.zeros((n, g, o // g, oh, ow), np.float32)
    wg = w.reshape(g, o // g, cg, kh, kw)
    for i, j, xt in _taps(x, kh, kw, a, oh, ow):
        acc += np.einsum("ngchw,goc->ngohw", xt.reshape(n, g, cg, oh, ow), wg[:, :, :, i, j], optimize=True)
    return epilogue_ref(acc.reshape(n, o, oh, ow), xs, a.get("epilogue", ())).astype(xs[0].dtype)


def maxpool2d(xs: list, a: dict) -> np.ndarray:
    """mira/ops.py:293-296."""
    k, s = a["size"], a["stride"]
    win = np.lib.stride_tricks.sliding_window_view(xs[0], (k, k), axis=(2, 3))[:, :, ::s, ::s]
    return win.max(axis=(-2, -1)).astype(xs[0].dtype)


def pad(xs: list, a: dict) -> np.ndarray:
    """mira/ops.py:469-470."""
    return np.pad(xs[0], a["pads"], constant_values=np.asarray(a.get("value", 0)).astype(xs[0].dtype))


def reduce(kind: str, xs: list, a: dict) -> np.ndarray:
    """mira/ops.py:318-343 (reduce_sum / reduce_mean / reduce_max via NumPy)."""
    f = {"reduce_sum": np.sum, "reduce_mean": np.mean, "reduce_max": np.max}[kind]
    out = f(_native_or_f32(xs[0]), axis=tuple(a["axes"]), keepdims=a["keepdims"])
    return np.asarray(out).astype(xs[0].dtype)


def softmax(xs: list, a: dict) -> np.ndarray:
    """mira/ops.py:310-313.  Pinned by closed forms (equal logits give fl32(1/n), a two-logit
    row its exact probabilities, no overflow for large logits); the last bits of exp are
    libm's, so device results are compared within a tolerance."""
    x = f32(xs[0])
    e = np.exp(x - x.max(axis=a["axis"], keepdims=True))
    return (e / e.sum(axis=a["axis"], keepdims=True)).astype(xs[0].dtype)


def layernorm(xs: list, a: dict) -> np.ndarray:
    """mira/ops.py:356-360.  Pinned bit for bit by a scalar restatement (pairwise means seeded
    with +0, float64 division by the count, one float32 operation per step) and by closed forms
    (constant rows give b, [a, -a] gives +-g + b, unit mean square with eps = 0)."""
    x, g, b = (f32(v) for v in xs)
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    return ((x - mu) / np.sqrt(var + a["eps"]) * g + b).astype(xs[0].dtype)


# ---------------------------------------------------------------- W8A8 (mira/ops.py:592-638, mira/quantize.py)

def quantize_array(w: np.ndarray, axis: int) -> tuple[np.ndarray, np.ndarray]:
    """mira/quantize.py:24-31: symmetric per-channel int8 weights."""
    reduce_ = tuple(i for i in range(w.ndim) if i != axis)
    amax = np.abs(w.astype(np.float32)).max(axis=reduce_)
    scale = np.where(amax > 0, amax / 127.0, 1.0).astype(np.float32)
    shape = [1] * w.ndim
    shape[axis] = -1
    q = np.clip(np.round(w.astype(np.float32) / scale.reshape(shape)), -127, 127).astype(np.int8)
    return q, scale


def quantize_activation(x: np.ndarray, scale: float) -> np.ndarray:
    """mira/ops.py:602-603: clip(round(f32(x) / f32(scale)), -127, 127), integer-valued float."""
    return np.clip(np.round(f32(x) / np.float32(scale)), -127, 127)


def qmatmul_acc(x: np.ndarray, a: dict) -> np.ndarray:
    """The int64 accumulator of mira/ops.py:617-618 (exact)."""
    xq = quantize_activation(x, a["x_scale"]).astype(np.int64)
    return np.matmul(xq, a["q"].astype(np.int64))


def qmatmul(xs: list, a: dict) -> np.ndarray:
    """mira/ops.py:616-620."""
    acc = qmatmul_acc(xs[0], a).astype(np.float64)
    y = (acc * (np.float64(a["x_scale"]) * a["w_scale"].astype(np.float64))).astype(np.float32)
    return epilogue_ref(y, xs, a.get("epilogue", ())).astype(NP_DTYPES[a["dtype"]])


def qconv2d_acc(x: np.ndarray, a: dict) -> np.ndarray:
    """The accumulator of mira/ops.py:631-632: per-tap f32 einsum sums of integer values.

    Equal to the exact integer convolution whenever every partial sum stays
    below 2**24 in magnitude (see qconv2d_certificate); beyond that it depends
    on OpenBLAS's summation order (parity unpinned)."""
    xq = quantize_activation(x, a["x_scale"]).astype(np.float64)
    return conv2d([xq, a["q"].astype(np.float64)], {**a, "epilogue": ()}).astype(np.float64)


def qconv2d(xs: list, a: dict) -> np.ndarray:
    """mira/ops.py:630-634."""
    acc = qconv2d_acc(xs[0], a)
    y = (acc * (np.float64(a["x_scale"]) * a["w_scale"].astype(np.float64)).reshape(1, -1, 1, 1)).astype(np.float32)
    return epilogue_ref(y, xs, a.get("epilogue", ())).astype(NP_DTYPES[a["dtype"]])


def qconv2d_certificate(x: np.ndarray, a: dict) -> float:
    """max over outputs of sum |xq| * |q|: the f32 accumulation of mira/ops.py:631-632 is
    exact (equals the integer convolution) when this is below 2**24."""
    xq = np.abs(quantize_activation(x, a["x_scale"])).astype(np.float64)
    aq = np.abs(a["q"].astype(np.float64))
    bound = conv2d([xq, aq], {**a, "epilogue": ()}).astype(np.float64)
    return float(bound.max()) if bound.size else 0.0


def dequantize(a: dict) -> np.ndarray:
    """mira/ops.py:581-586."""
    q, scale, axis = a["q"], a["scale"], a["axis"]
    shape = [1] * q.ndim
    shape[axis] = -1
    return (q.astype(np.float32) * scale.reshape(shape)).astype(NP_DTYPES[a["dtype"]])


# ---------------------------------------------------------------- op dispatch (mira/ops.py:704-709)

# ---------------------------------------------------------------- selection (mira/ops.py:426-458)

def _clamped_starts(start, shape, size) -> list:
    """mira/ops.py:538-539: each runtime start clamped so the window fits its axis."""
    return [int(min(max(int(b), 0), d - n)) for b, d, n in zip(np.asarray(start).ravel(), shape, size)]


def slice_(xs: list, a: dict) -> np.ndarray:
    """mira/ops.py:457-458: the box [begin, begin + size) of every axis, copied."""
    return xs[0][tuple(slice(b, b + n) for b, n in zip(a["begin"], a["size"]))].copy()


def where(xs: list, a: dict) -> np.ndarray:
    """mira/ops.py:432-433: a where cond is non-zero, else b, in a's dtype (broadcast)."""
    return np.where(xs[0] != 0, xs[1], xs[2]).astype(xs[1].dtype)


def evaluate(kind: str, xs: list, a: dict) -> np.ndarray:
    """mira/ops.py:708-709 for the ops the W8A8 configs use."""
    if kind == "const":
        return a["value"]
    if kind == "dequantize":
        return dequantize(a)
    if kind in UNARY:
        return unary(kind, xs[0])
    if kind in BINARY:
        return binary(kind, xs[0], xs[1])
    if kind == "matmul":
        return matmul(xs, a)
    if kind == "conv2d":
        return conv2d(xs, a)
    if kind == "qmatmul":
        return qmatmul(xs, a)
    if kind == "qconv2d":
        return qconv2d(xs, a)
    if kind == "maxpool2d":
        return maxpool2d(xs, a)
    if kind == "pad":
        return pad(xs, a)
    if kind in ("reduce_sum", "reduce_mean", "reduce_max"):
        return reduce(kind, xs, a)
    if kind == "reshape":
        return xs[0].reshape(a["shape"])                                  # mira/ops.py:385
    if kind == "transpose":
        return np.ascontiguousarray(np.transpose(xs[0], a["perm"]))       # mira/ops.py:375
    if kind == "softmax":
        return softmax(xs, a)
    if kind == "layernorm":
        return layernorm(xs, a)
    if kind == "cast":
        return xs[0].astype(NP_DTYPES[a["dtype"]])                        # mira/ops.py:405-406
    if kind == "gather":
        table, idx = xs                                                   # mira/ops.py:479-484
        return np.take(table, idx, axis=a["axis"])
    if kind == "concat":
        return np.concatenate(xs, axis=a["axis"])                         # mira/ops.py:402
    if kind == "slice":
        return slice_(xs, a)
    if kind == "where":
        return where(xs, a)
    if kind == "broadcast":
        return np.broadcast_to(xs[0], a["shape"]).copy()                  # mira/ops.py:443
    if kind == "dynamic_slice":                                           # mira/ops.py:551-554
        st = _clamped_starts(xs[1], xs[0].shape, a["size"])
        return xs[0][tuple(slice(b, b + n) for b, n in zip(st, a["size"]))].copy()
    if kind == "dynamic_update_slice":                                    # mira/ops.py:567-572
        st = _clamped_starts(xs[2], xs[0].shape, xs[1].shape)
        out = xs[0].copy()
        out[tuple(slice(b, b + n) for b, n in zip(st, xs[1].shape))] = xs[1]
        return out
    if kind == "sort":
        return np.sort(xs[0], axis=a["axis"])                             # mira/ops.py:419
    if kind == "cumprod":
        return np.cumprod(f32(xs[0]), axis=a["axis"]).astype(xs[0].dtype)  # mira/ops.py:420-421
    if kind in ("argmax", "argmin"):                                      # mira/ops.py:527-530
        f = np.argmax if kind == "argmax" else np.argmin
        return np.asarray(f(xs[0], axis=a["axis"], keepdims=a["keepdims"])).astype(np.int32)
    raise NotImplementedError(f"oracle has no semantics for '{kind}'")


# ---------------------------------------------------------------- graph execution (mira/backends/cpu.py:28-36)

class CPUExecutable:
    """mira/backends/cpu.py:18-51: ops in order; an if / while op runs its sub-graphs, here
    evaluated by the oracle itself."""

    def __init__(self, g):
        self.g = g

    def run(self, feeds: dict) -> dict:
        return dict(zip(self.g.outputs, self.run_list([feeds[v] for v in self.g.inputs])))

    def run_list(self, args: list) -> list:
        env = dict(zip(self.g.inputs, args))
        for op in self.g.ops:
            if op.is_control:
                env.update(zip(op.results, control(op, [env[v] for v in op.inputs])))
            else:
                env[op.result] = evaluate(op.kind, [env[v] for v in op.inputs], op.attrs)
        return [env[v] for v in self.g.outputs]

    def report(self) -> str:
        return f"cpu (oracle): {sum(op.kind not in ('const', 'dequantize') for op in self.g.ops)} ops"


def control(op, args: list) -> list:
    """mira/backends/cpu.py:38-51: `if` runs the branch its one-element condition picks on its
    captures; `while` runs cond then body on the state (plus each one's captures) until the
    condition is false, at most max_iters times."""
    if op.kind == "if":
        n = op.attrs["n_then"]
        taken = bool(np.asarray(args[0]).ravel()[0])
        sub = op.attrs["then"] if taken else op.attrs["else"]
        return CPUExecutable(sub).run_list(args[1:1 + n] if taken else args[1 + n:])
    ns, nc = op.attrs["n_state"], op.attrs["n_cond"]
    state, cond_caps, body_caps = list(args[:ns]), list(args[ns:ns + nc]), list(args[ns + nc:])
    cond, body = CPUExecutable(op.attrs["cond"]), CPUExecutable(op.attrs["body"])
    for _ in range(op.attrs["max_iters"]):
        if not bool(np.asarray(cond.run_list(state + cond_caps)[0]).ravel()[0]):
            return state
        state = body.run_list(state + body_caps)
    raise RuntimeError(f"while loop exceeded {op.attrs['max_iters']} iterations")


class CPUTarget:
    """mira/backends/cpu.py:56-66: the fallback target for segments the accelerator rejects."""
    name = "cpu"

    def check(self, op) -> Optional[str]:
        return None

    def compile(self, g, compile_sub=None) -> CPUExecutable:
        return CPUExecutable(g)


def run_graph(g, feeds: dict) -> list:
    """Evaluate a whole graph from {input name: array}; returns the outputs in order."""
    env = {}
    for v in g.inputs:
        env[v] = np.asarray(feeds[v.name]).astype(NP_DTYPES[v.type.dtype])
    out = CPUExecutable(g).run(env)
    return [out[v] for v in g.outputs]


# ---------------------------------------------------------------- calibration / rewrite (mira/quantize.py:73-143)

def calibrate(g, feeds: list, watch: set) -> dict:
    """mira/quantize.py:73-92: largest |value| of each watched value over the calibration feeds."""
    peak = {v: 0.0 for v in watch}
    for feed in feeds:
        env = {}
        for v in g.inputs:
            if v.name not in feed:
                raise ValueError(f"calibration input is missing '{v.name}'")
            env[v] = np.asarray(feed[v.name]).astype(NP_DTYPES[v.type.dtype])
        for op in g.ops:
            if op.kind in ("if", "while"):
                raise ValueError("W8A8 quantization doesn't support programs with data-dependent control flow yet")
            env[op.result] = evaluate(op.kind, [env[x] for x in op.inputs], op.attrs)
            if op.result in peak:
                peak[op.result] = max(peak[op.result], float(np.abs(env[op.result].astype(np.float32)).max()))
        for v in g.inputs:
            if v in peak:
                peak[v] = max(peak[v], float(np.abs(env[v].astype(np.float32)).max()))
    return peak


WEIGHT_ONLY_MIN_ELEMS = 1024     # mira/quantize.py:21


def weight_only_attrs(g) -> dict:
    """The `dequantize` attrs mira/quantize.py:46-68 (weight-only int8) would give each
    constant of g, keyed by const op (g itself is left untouched): constants of at least
    1024 elements whose every use is as a matmul [K, N] weight (axis 1; the same value
    not also the activation) or a conv [O, C, KH, KW] weight (axis 0), mira/quantize.py:34-43."""
    users: dict = {}
    for op in g.ops:
        for v in op.inputs:
            users.setdefault(v, []).append(op)
    out = {}
    for op in g.ops:
        if op.kind != "const" or int(np.prod(op.result.type.shape, dtype=np.int64)) < WEIGHT_ONLY_MIN_ELEMS:
            continue
        v, us = op.result, users.get(op.result, [])
        axis = None
        if us and v.type.rank == 2 and all(u.kind == "matmul" and u.inputs[1] is v and u.inputs[0] is not v
                                           for u in us):
            axis = 1
        elif us and v.type.rank == 4 and all(u.kind == "conv2d" and u.inputs[1] is v for u in us):
            axis = 0
        if axis is None:
            continue
        q, scale = quantize_array(op.attrs["value"], axis)
        out[op] = {"q": q, "scale": scale, "axis": axis, "dtype": v.type.dtype}
    return out


def w8a8_weight(op) -> Optional[tuple[np.ndarray, np.ndarray]]:
    """mira/quantize.py:95-115."""
    w = op.inputs[1].producer
    if w is None or w.kind not in ("const", "dequantize"):
        return None
    if op.kind == "matmul":
        if op.inputs[1].type.rank != 2 or op.inputs[0].type.rank < 2:
            return None
        axis = 1
    elif op.kind == "conv2d":
        if op.attrs.get("groups", 1) != 1:
            return None
        axis = 0
    else:
        return None
    if w.kind == "dequantize" and w.attrs["axis"] == axis:
        return w.attrs["q"], w.attrs["scale"]
    value = w.attrs["value"] if w.kind == "const" else None
    if value is None:
        return None
    return quantize_array(value, axis)


def w8a8_attrs(g, calibration: list) -> dict:
    """The attrs mira/quantize.py:118-137 would give each candidate op of g, keyed by op
    (the graph itself is left untouched)."""
    candidates = [op for op in g.ops if op.kind in ("matmul", "conv2d") and w8a8_weight(op) is not None]
    peak = calibrate(g, calibration, {op.inputs[0] for op in candidates})
    out = {}
    for op in candidates:
        q, w_scale = w8a8_weight(op)
        x_scale = peak[op.inputs[0]] / 127.0 or 1.0
        epi = tuple((fn, None if idx is None else idx - 1, sw) for fn, idx, sw in op.attrs.get("epilogue", ()))
        attrs = {k: v for k, v in op.attrs.items() if k != "epilogue"}
        attrs.update({"q": q, "w_scale": np.asarray(w_scale, np.float32), "x_scale": float(x_scale),
                      "dtype": op.result.type.dtype})
        if epi:
            attrs["epilogue"] = epi
        out[op] = attrs
    return out
