"""Host (NumPy) evaluation of float graphs for the harness.

Two uses, neither of which produces a result the rocm target returns:

* calibration (`lowering.calibrate`): a float forward pass that records the
  peak |x| of every q-op input, from which x_scale follows;
* `HostTarget`: the stand-in for MIRA's cpu target in the benchmark and the
  command-line driver: the fallback that runs the ops the rocm target rejects
  (the f32 attention, softmax, layernorm and gelu of the GPT decode step), and
  the `cpu` target that `run --check` compares with.  The parity tests use the
  oracle for that role instead.

Convolutions run as one im2col GEMM (grouped ones tap by tap), so float
results can differ from MIRA's per-tap einsum in the last bits; nothing here
is compared bit for bit.
"""
from __future__ import annotations

from typing import Optional

import numpy as np

from .graph import DTYPES, conv_out


def _f32(a) -> np.ndarray:
    return np.asarray(a).astype(np.float32, copy=False)


def _gelu(x):
    return 0.5 * x * (1.0 + np.tanh(0.7978845608028654 * (x + 0.044715 * x ** 3)))


def _num(a) -> np.ndarray:
    """Floats compute in f32; integers stay exact (mira/ops.py:150-152)."""
    a = np.asarray(a)
    return a if a.dtype.kind == "i" else _f32(a)


UNARY = {"relu": lambda x: np.maximum(x, 0), "gelu": _gelu, "sigmoid": lambda x: 1.0 / (1.0 + np.exp(-x)),
         "tanh": np.tanh, "exp": np.exp, "log": np.log, "neg": np.negative, "abs": np.abs, "sign": np.sign,
         "sqrt": np.sqrt}
BINARY = {"add": np.add, "sub": np.subtract, "mul": np.multiply, "div": np.divide, "pow": np.power,
          "maximum": np.maximum, "minimum": np.minimum, "greater": np.greater, "greater_equal": np.greater_equal,
          "equal": np.equal}
REDUCE = {"reduce_sum": np.sum, "reduce_mean": np.mean, "reduce_max": np.max}


def apply_epilogue(y: np.ndarray, operands: list, steps) -> np.ndarray:
    """Run epilogue steps (fn, operand index, swapped) on y in f32."""
    for fn, idx, swapped in steps:
        if idx is None:
            y = UNARY[fn](y)
        else:
            o = _f32(operands[idx])
            y = BINARY[fn](o, y) if swapped else BINARY[fn](y, o)
    return y


def conv2d_f32(x: np.ndarray, w: np.ndarray, a: dict, dt=np.float32) -> np.ndarray:
    """NCHW x OIHW -> NCHW convolution in `dt` (f64 for the integer accumulators of qconv2d,
    where any order is exact): im2col + one GEMM, or per tap for grouped convs."""
    (sh, sw), (ph, pw) = a["stride"], a["padding"]
    dh, dw = a.get("dilation", (1, 1))
    g = a.get("groups", 1)
    n, c, h, wd = x.shape
    o, cg, kh, kw = w.shape
    oh, ow = conv_out(h, kh, sh, ph, dh), conv_out(wd, kw, sw, pw, dw)
    xp = np.pad(np.asarray(x, dt), ((0, 0), (0, 0), (ph, ph), (pw, pw))).transpose(0, 2, 3, 1)
    w = np.asarray(w, dt)

    def tap(i, j):
        return xp[:, i * dh:i * dh + sh * (oh - 1) + 1:sh, j * dw:j * dw + sw * (ow - 1) + 1:sw, :]

    if g == 1:
        cols = np.empty((n, oh, ow, kh, kw, c), dt)
        for i in range(kh):
            for j in range(kw):
                cols[:, :, :, i, j, :] = tap(i, j)
        out = cols.reshape(n * oh * ow, -1) @ w.transpose(2, 3, 1, 0).reshape(kh * kw * c, o)
        return np.ascontiguousarray(out.reshape(n, oh, ow, o).transpose(0, 3, 1, 2))
    og = o // g
    acc = np.zeros((n, oh, ow, o), dt)
    for i in range(kh):
        for j in range(kw):
            xt = tap(i, j)
            if cg == 1 and og == 1:
                acc += xt * w[:, 0, i, j]
            else:
                for gi in range(g):
                    part = xt[..., gi * cg:(gi + 1) * cg].reshape(-1, cg) @ w[gi * og:(gi + 1) * og, :, i, j].T
                    acc[..., gi * og:(gi + 1) * og] += part.reshape(n, oh, ow, og)
    return np.ascontiguousarray(acc.transpose(0, 3, 1, 2))


def conv2d_taps_f32(x: np.ndarray, w: np.ndarray, a: dict) -> np.ndarray:
    """The f32 convolution as MIRA's golden model sums it (mira/ops.py:256-276): one grouped
    einsum per kernel tap over the padded input, added into an f32 accumulator in (i, j) tap
    order.  Float results (calibration peaks, the cpu fallback) then carry MIRA's roundings
    bit for bit, which one im2col product would not."""
    (sh, sw), (ph, pw) = a["stride"], a["padding"]
    dh, dw = a.get("dilation", (1, 1))
    g = a.get("groups", 1)
    x, w = _f32(x), _f32(w)
    n, c, h, wd = x.shape
    o, cg, kh, kw = w.shape
    oh, ow = conv_out(h, kh, sh, ph, dh), conv_out(wd, kw, sw, pw, dw)
    xp = np.pad(x, ((0, 0), (0, 0), (ph, ph), (pw, pw)))
    wg = w.reshape(g, o // g, cg, kh, kw)
    acc = np.zeros((n, g, o // g, oh, ow), np.float32)
    for i in range(kh):
        for j in range(kw):
            xt = xp[:, :, i * dh:i * dh + sh * (oh - 1) + 1:sh, j * dw:j * dw + sw * (ow - 1) + 1:sw]
            acc += np.einsum("ngchw,goc->ngohw", xt.reshape(n, g, cg, oh, ow), wg[:, :, :, i, j], optimize=True)
    return acc.reshape(n, o, oh, ow)


def quantize_activation(x: np.ndarray, x_scale: float) -> np.ndarray:
    """clip(rint(x / f32(x_scale)), +-127) in f32 arithmetic, as int64."""
    return np.clip(np.rint(_f32(x) / np.float32(x_scale)), -127, 127).astype(np.int64)


def _clamped_starts(start, shape, size) -> list:
    """Runtime slice starts, each clamped so the window stays inside its axis (mira/ops.py:538-539)."""
    return [int(min(max(int(b), 0), d - n)) for b, d, n in zip(np.asarray(start).ravel(), shape, size)]


def run_control(op, args: list, sub: dict) -> list:
    """An if / while op from host arrays (mira/backends/cpu.py:38-51); sub maps each sub-graph
    name to a callable from its input arrays to its output arrays."""
    if op.kind == "if":
        n = op.attrs["n_then"]
        if bool(np.asarray(args[0]).ravel()[0]):
            return sub["then"](args[1:1 + n])
        return sub["else"](args[1 + n:])
    ns, nc = op.attrs["n_state"], op.attrs["n_cond"]
    state, cond_caps, body_caps = list(args[:ns]), list(args[ns:ns + nc]), list(args[ns + nc:])
    for _ in range(op.attrs["max_iters"]):
        if not bool(np.asarray(sub["cond"](state + cond_caps)[0]).ravel()[0]):
            return state
        state = list(sub["body"](state + body_caps))
    raise RuntimeError(f"while loop exceeded {op.attrs['max_iters']} iterations")


def evaluate(kind: str, xs: list, a: dict) -> np.ndarray:
    if kind == "const":
        return a["value"]
    if kind == "dequantize":
        shape = [1] * a["q"].ndim
        shape[a["axis"]] = -1
        return (a["q"].astype(np.float32) * a["scale"].reshape(shape)).astype(DTYPES[a["dtype"]])
    dt = xs[0].dtype if xs else np.float32
    if kind in UNARY:
        return UNARY[kind](_num(xs[0])).astype(dt)
    if kind in BINARY:
        return BINARY[kind](_num(xs[0]), _num(xs[1])).astype(dt)
    if kind == "matmul":
        return apply_epilogue(_f32(xs[0]) @ _f32(xs[1]), xs, a.get("epilogue", ())).astype(dt)
    if kind == "conv2d":
        return apply_epilogue(conv2d_taps_f32(xs[0], xs[1], a), xs, a.get("epilogue", ())).astype(dt)
    if kind == "qmatmul":
        acc = quantize_activation(xs[0], a["x_scale"]) @ a["q"].astype(np.int64)
        y = (acc.astype(np.float64) * (np.float64(a["x_scale"]) * a["w_scale"].astype(np.float64))).astype(np.float32)
        return apply_epilogue(y, xs, a.get("epilogue", ())).astype(DTYPES[a["dtype"]])
    if kind == "qconv2d":
        # integer products summed in f64: exact while |sum| < 2^53 (127 * 127 * K is far below)
        acc = conv2d_f32(quantize_activation(xs[0], a["x_scale"]), a["q"], a, np.float64)
        scale = np.float64(a["x_scale"]) * a["w_scale"].astype(np.float64).reshape(1, -1, 1, 1)
        y = (acc * scale).astype(np.float32)
        return apply_epilogue(y, xs, a.get("epilogue", ())).astype(DTYPES[a["dtype"]])
    if kind == "maxpool2d":
        k, s = a["size"], a["stride"]
        win = np.lib.stride_tricks.sliding_window_view(xs[0], (k, k), axis=(2, 3))[:, :, ::s, ::s]
        return win.max(axis=(-2, -1)).astype(dt)
    if kind == "pad":
        return np.pad(xs[0], a["pads"], constant_values=np.asarray(a.get("value", 0)).astype(dt))
    if kind in REDUCE:
        return np.asarray(REDUCE[kind](_num(xs[0]), axis=tuple(a["axes"]), keepdims=a.get("keepdims", False))).astype(dt)
    if kind == "slice":
        return xs[0][tuple(slice(b, b + n) for b, n in zip(a["begin"], a["size"]))].copy()
    if kind == "gather":
        return np.take(xs[0], xs[1], axis=a["axis"])
    if kind == "where":
        return np.where(xs[0] != 0, xs[1], xs[2]).astype(xs[1].dtype)
    if kind == "broadcast":
        return np.broadcast_to(xs[0], a["shape"]).copy()
    if kind == "dynamic_slice":
        st = _clamped_starts(xs[1], xs[0].shape, a["size"])
        return xs[0][tuple(slice(b, b + n) for b, n in zip(st, a["size"]))].copy()
    if kind == "dynamic_update_slice":
        st = _clamped_starts(xs[2], xs[0].shape, xs[1].shape)
        out = xs[0].copy()
        out[tuple(slice(b, b + n) for b, n in zip(st, xs[1].shape))] = xs[1]
        return out
    if kind == "sort":
        return np.sort(xs[0], axis=a["axis"])
    if kind == "cumprod":
        return np.cumprod(_num(xs[0]), axis=a["axis"]).astype(dt)
    if kind in ("argmax", "argmin"):
        f = np.argmax if kind == "argmax" else np.argmin
        return np.asarray(f(xs[0], axis=a["axis"], keepdims=a.get("keepdims", False))).astype(np.int32)
    if kind == "reshape":
        return xs[0].reshape(a["shape"])
    if kind == "transpose":
        return np.ascontiguousarray(xs[0].transpose(a["perm"]))
    if kind == "concat":
        return np.concatenate(xs, axis=a["axis"])
    if kind == "softmax":
        x = _f32(xs[0])
        e = np.exp(x - x.max(axis=a["axis"], keepdims=True))
        return (e / e.sum(axis=a["axis"], keepdims=True)).astype(dt)
    if kind == "layernorm":
        x, gam, bet = (_f32(v) for v in xs)
        mu = x.mean(axis=-1, keepdims=True)
        var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
        return ((x - mu) / np.sqrt(var + a["eps"]) * gam + bet).astype(dt)
    if kind == "cast":
        return xs[0].astype(DTYPES[a["dtype"]])
    raise NotImplementedError(f"no host evaluation for '{kind}'")


def _sub_runner(graph, watch=None, peaks=None):
    return lambda arrays: [run(graph, dict(zip(graph.inputs, arrays)), watch, peaks)[v] for v in graph.outputs]


def run(g, feeds: dict, watch: Optional[set] = None, peaks: Optional[dict] = None, subs: Optional[dict] = None) -> dict:
    """Evaluate g from {input Value: array}; returns every value.  With `watch`, the running
    max |x| of each watched value is folded into `peaks`.  Control ops run their sub-graphs
    through `subs` ({(op, name): callable}) or, without it, evaluated here."""
    env = {v: np.asarray(feeds[v]).astype(v.type.np_dtype) for v in g.inputs}
    for op in g.ops:
        if op.is_control:
            sub = {n: subs[(op, n)] if subs else _sub_runner(sg, watch, peaks) for n, sg in op.subgraphs()}
            env.update(zip(op.results, run_control(op, [env[x] for x in op.inputs], sub)))
            continue
        env[op.result] = evaluate(op.kind, [env[x] for x in op.inputs], op.attrs)
    if watch:
        for v in watch:
            if v not in env:          # computed in another graph (a sub-graph's own run folds it)
                continue
            m = float(np.abs(_f32(env[v])).max()) if np.size(env[v]) else 0.0
            peaks[v] = max(peaks.get(v, 0.0), m)
    return env


class HostExecutable:
    """A host segment; its control ops' sub-graphs are compiled by `compile_sub` (the runner
    partitions them for the target, as MIRA's driver does, mira/compiler.py:83-96)."""

    def __init__(self, g, compile_sub=None):
        self.g = g
        self.sub = {}
        for op in g.ops:
            for name, sg in op.subgraphs():
                if compile_sub is None:
                    raise RuntimeError("control flow needs a sub-graph compiler")
                self.sub[(op, name)] = compile_sub(sg)

    def run(self, feeds: dict) -> dict:
        subs = {k: r.run_values for k, r in self.sub.items()}
        env = run(self.g, feeds, subs=subs)
        return {v: env[v] for v in self.g.outputs}

    def report(self) -> str:
        n = sum(op.is_control for op in self.g.ops)
        return f"host: {len(self.g.compute_ops())} ops evaluated with NumPy" + \
            (f" ({n} control-flow op(s))" if n else "")


class HostTarget:
    """The CPU fallback the benchmark gives the runner (MIRA's cpu target plays this role)."""
    name = "cpu"

    def check(self, op) -> Optional[str]:
        return None

    def compile(self, g, compile_sub=None) -> HostExecutable:
        return HostExecutable(g, compile_sub)
