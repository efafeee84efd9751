"""A small SSA graph for building and lowering the benchmark networks.

The rocm target reads graphs through a handful of attribute names -- the ones
MIRA's IR uses (mira/ir.py:34-154, mira/types.py:13-49) -- so any object with
them works: a MIRA graph in a MIRA checkout, or this module's graphs in the
tests and the benchmark.  Those names are the interface and are kept:

    value.type.dtype / .shape / .rank / .numel / .np_dtype, value.producer, value.name
    op.kind, op.inputs, op.attrs, op.results, op.result,
    op.is_const, op.is_constant_like, op.is_control
    graph.inputs, graph.ops, graph.outputs, graph.users(), graph.compute_ops()

Everything else here is this harness's own: a builder (`Graph.op`) whose
result types come from the small shape rules below, and a verifier.  Integer
(i32) values appear in index and mask arithmetic; comparisons give 1 / 0 in
their operands' dtype, as MIRA's do (mira/ops.py:134-140).

Control flow is structured as in MIRA (mira/ir.py:14-45, 160-183): an `if` op
owns a `then` and an `else` graph, a `while` op a `cond` and a `body` graph;
their inputs are the condition (if), the loop state (while), then the values
each sub-graph captures from enclosing graphs, and their results are the
branches' outputs / the final loop state.  The W8A8 rewrite rejects them, as
MIRA's does (mira/quantize.py:84-85); the runner drives them on the host.
"""
from __future__ import annotations

import itertools
from typing import Optional, Sequence

import numpy as np

DTYPES = {"f32": np.float32, "f16": np.float16, "i32": np.int32}
_next_id = itertools.count(1)


class TensorType:
    __slots__ = ("dtype", "shape")

    def __init__(self, dtype: str, shape: Sequence[int]):
        if dtype not in DTYPES:
            raise ValueError(f"unknown dtype {dtype!r}")
        self.dtype = dtype
        self.shape = tuple(int(d) for d in shape)

    rank = property(lambda self: len(self.shape))
    numel = property(lambda self: int(np.prod(self.shape, dtype=np.int64)))
    np_dtype = property(lambda self: DTYPES[self.dtype])
    is_float = property(lambda self: self.dtype in ("f32", "f16"))

    def __eq__(self, other) -> bool:
        return isinstance(other, TensorType) and (self.dtype, self.shape) == (other.dtype, other.shape)

    def __hash__(self) -> int:
        return hash((self.dtype, self.shape))

    def __repr__(self) -> str:
        return f"{self.dtype}{list(self.shape)}"


class Value:
    """One SSA value; identity is the key (values hash by id)."""
    __slots__ = ("type", "producer", "name", "id")

    def __init__(self, type_: TensorType, producer: Optional["Op"] = None, name: Optional[str] = None):
        self.type = type_
        self.producer = producer
        self.name = name
        self.id = next(_next_id)

    def __repr__(self) -> str:
        return f"%{self.name or self.id}"


class Op:
    __slots__ = ("kind", "inputs", "attrs", "results")

    def __init__(self, kind: str, inputs: list, attrs: dict, results: list):
        self.kind, self.inputs, self.attrs, self.results = kind, list(inputs), dict(attrs), list(results)

    @property
    def result(self) -> Value:
        return self.results[0]

    is_const = property(lambda self: self.kind == "const")
    is_constant_like = property(lambda self: self.kind in ("const", "dequantize"))
    is_control = property(lambda self: self.kind in ("if", "while"))

    def subgraphs(self) -> list:
        """(name, Graph) of a control op's sub-graphs, in MIRA's order."""
        names = ("then", "else") if self.kind == "if" else ("cond", "body") if self.kind == "while" else ()
        return [(n, self.attrs[n]) for n in names]

    def __repr__(self) -> str:
        res = ", ".join(map(repr, self.results))
        return f"{res} = {self.kind}({', '.join(map(repr, self.inputs))})"


# ---------------------------------------------------------------- shape rules

def conv_out(size: int, k: int, stride: int, pad: int, dilation: int = 1) -> int:
    """Output extent of a convolution / pooling window along one axis."""
    return (size + 2 * pad - dilation * (k - 1) - 1) // stride + 1


def _conv_shape(x: TensorType, w: TensorType, a: dict) -> tuple:
    (sh, sw), (ph, pw) = a["stride"], a["padding"]
    dh, dw = a.get("dilation", (1, 1))
    n, c, h, wd = x.shape
    o, cg, kh, kw = w.shape
    if cg * a.get("groups", 1) != c:
        raise ValueError(f"conv2d: {c} input channels vs weight {w}")
    return (n, o, conv_out(h, kh, sh, ph, dh), conv_out(wd, kw, sw, pw, dw))


def _matmul_shape(x: TensorType, w: TensorType) -> tuple:
    if x.shape[-1] != w.shape[-2]:
        raise ValueError(f"matmul: {x} @ {w}")
    batch = np.broadcast_shapes(x.shape[:-2], w.shape[:-2])
    return tuple(batch) + (x.shape[-2], w.shape[-1])


def _reduce_shape(x: TensorType, a: dict) -> tuple:
    axes = {ax % x.rank for ax in a["axes"]}
    if a.get("keepdims", False):
        return tuple(1 if i in axes else d for i, d in enumerate(x.shape))
    return tuple(d for i, d in enumerate(x.shape) if i not in axes)


ELEMENTWISE_UNARY = ("relu", "gelu", "sigmoid", "tanh", "exp", "log", "neg", "abs", "sign", "sqrt")
ELEMENTWISE_BINARY = ("add", "sub", "mul", "div", "pow", "maximum", "minimum", "greater", "greater_equal", "equal")


def _broadcast(*shapes) -> tuple:
    try:
        return tuple(np.broadcast_shapes(*shapes))
    except ValueError:
        raise ValueError(f"shapes {' and '.join(str(list(s)) for s in shapes)} do not broadcast") from None


def result_type(kind: str, ins: list, a: dict) -> TensorType:
    """The result type of an op the builders use (shape rules of this harness)."""
    t0 = ins[0] if ins else None
    if kind in ELEMENTWISE_UNARY or kind in ("softmax", "layernorm"):
        return t0
    if kind in ELEMENTWISE_BINARY:
        if t0.dtype != ins[1].dtype:
            raise ValueError(f"{kind}: operands {t0} and {ins[1]} differ in dtype")
        return TensorType(t0.dtype, _broadcast(t0.shape, ins[1].shape))
    if kind == "matmul":
        return TensorType(t0.dtype, _matmul_shape(t0, ins[1]))
    if kind == "conv2d":
        return TensorType(t0.dtype, _conv_shape(t0, ins[1], a))
    if kind == "maxpool2d":
        k, s = a["size"], a["stride"]
        n, c, h, w = t0.shape
        return TensorType(t0.dtype, (n, c, (h - k) // s + 1, (w - k) // s + 1))
    if kind == "pad":
        return TensorType(t0.dtype, tuple(d + lo + hi for d, (lo, hi) in zip(t0.shape, a["pads"])))
    if kind in ("reduce_mean", "reduce_sum", "reduce_max"):
        return TensorType(t0.dtype, _reduce_shape(t0, a))
    if kind == "slice":
        begin, size = tuple(a["begin"]), tuple(a["size"])
        if len(begin) != t0.rank or len(size) != t0.rank or \
                any(b < 0 or n < 0 or b + n > d for b, n, d in zip(begin, size, t0.shape)):
            raise ValueError(f"slice begin {list(begin)} size {list(size)} does not fit {t0}")
        return TensorType(t0.dtype, size)
    if kind == "gather":
        if ins[1].dtype != "i32":
            raise ValueError(f"gather: indices must be i32, got {ins[1]}")
        ax = a["axis"] % t0.rank
        return TensorType(t0.dtype, t0.shape[:ax] + ins[1].shape + t0.shape[ax + 1:])
    if kind == "where":
        if ins[1].dtype != ins[2].dtype:
            raise ValueError(f"where: {ins[1]} and {ins[2]} differ in dtype")
        return TensorType(ins[1].dtype, _broadcast(t0.shape, ins[1].shape, ins[2].shape))
    if kind in ("sort", "cumprod"):
        return t0
    if kind == "dynamic_slice":
        size = tuple(a["size"])
        if ins[1].dtype != "i32" or ins[1].shape != (t0.rank,) or len(size) != t0.rank or \
                any(n < 0 or n > d for n, d in zip(size, t0.shape)):
            raise ValueError(f"dynamic_slice: need start i32[{t0.rank}] and a size that fits {t0}")
        return TensorType(t0.dtype, size)
    if kind == "dynamic_update_slice":
        u, st = ins[1], ins[2]
        if u.dtype != t0.dtype or u.rank != t0.rank or any(n > d for n, d in zip(u.shape, t0.shape)) or \
                st.dtype != "i32" or st.shape != (t0.rank,):
            raise ValueError(f"dynamic_update_slice: update {u} at start {st} does not fit {t0}")
        return t0
    if kind in ("argmax", "argmin"):
        ax = a["axis"] % t0.rank
        keep = a.get("keepdims", False)
        return TensorType("i32", tuple(1 if i == ax else d for i, d in enumerate(t0.shape)) if keep else
                          tuple(d for i, d in enumerate(t0.shape) if i != ax))
    if kind == "broadcast":
        shape = tuple(a["shape"])
        if _broadcast(t0.shape, shape) != shape:
            raise ValueError(f"broadcast: {t0} does not broadcast to {list(shape)}")
        return TensorType(t0.dtype, shape)
    if kind == "reshape":
        shape = tuple(a["shape"])
        if int(np.prod(shape, dtype=np.int64)) != t0.numel:
            raise ValueError(f"reshape {t0} -> {list(shape)}")
        return TensorType(t0.dtype, shape)
    if kind == "transpose":
        return TensorType(t0.dtype, tuple(t0.shape[p] for p in a["perm"]))
    if kind == "concat":
        ax = a["axis"] % t0.rank
        return TensorType(t0.dtype, tuple(sum(t.shape[ax] for t in ins) if i == ax else d
                                          for i, d in enumerate(t0.shape)))
    if kind == "cast":
        return TensorType(a["dtype"], t0.shape)
    raise ValueError(f"no shape rule for '{kind}'")


# ---------------------------------------------------------------- graph

class Graph:
    def __init__(self, name: str):
        self.name = name
        self.inputs: list[Value] = []
        self.ops: list[Op] = []
        self.outputs: list[Value] = []

    def input(self, name: str, shape, dtype: str = "f32") -> Value:
        v = Value(TensorType(dtype, shape), name=name)
        self.inputs.append(v)
        return v

    def const(self, array) -> Value:
        a = np.asarray(array)
        dtype = {np.dtype(np.float32): "f32", np.dtype(np.float16): "f16", np.dtype(np.int32): "i32"}[a.dtype]
        return self.emit("const", [], {"value": a}, TensorType(dtype, a.shape))

    def op(self, kind: str, inputs: list, attrs: Optional[dict] = None) -> Value:
        """Append a float op whose result type follows from its inputs."""
        attrs = dict(attrs or {})
        return self.emit(kind, inputs, attrs, result_type(kind, [v.type for v in inputs], attrs))

    def add_control(self, kind: str, inputs: list, attrs: dict, types: list) -> list:
        """Append an if / while op with results of the given types; returns the results."""
        results = [Value(t) for t in types]
        op = Op(kind, inputs, attrs, results)
        for r in results:
            r.producer = op
        self.ops.append(op)
        check_control(op)
        return results

    def emit(self, kind: str, inputs: list, attrs: dict, rtype: TensorType) -> Value:
        """Append an op with an explicit result type."""
        v = Value(rtype)
        op = Op(kind, inputs, attrs, [v])
        v.producer = op
        self.ops.append(op)
        return v

    def users(self) -> dict:
        out: dict = {}
        for op in self.ops:
            for v in op.inputs:
                out.setdefault(v, []).append(op)
        return out

    def compute_ops(self) -> list:
        return [op for op in self.ops if not op.is_constant_like]

    def redirect(self, old: Value, new: Value) -> None:
        """Every use of `old` (op inputs and graph outputs) reads `new` instead."""
        for op in self.ops:
            op.inputs = [new if v is old else v for v in op.inputs]
        self.outputs = [new if v is old else v for v in self.outputs]

    def prune(self) -> None:
        """Drop ops none of whose results reach an output."""
        needed = set(self.outputs)
        keep = []
        for op in reversed(self.ops):
            if any(r in needed for r in op.results):
                keep.append(op)
                needed.update(op.inputs)
        self.ops = keep[::-1]

    def check(self) -> None:
        """Every input defined before use, every producer link consistent, every control op's
        sub-graphs matching its inputs and results (and checked themselves)."""
        seen = set(self.inputs)
        for op in self.ops:
            missing = [v for v in op.inputs if v not in seen]
            if missing:
                raise AssertionError(f"{op!r} reads {missing} before they are defined")
            for r in op.results:
                if r.producer is not op:
                    raise AssertionError(f"{r!r} has the wrong producer")
            if op.is_control:
                check_control(op)
                for _, sub in op.subgraphs():
                    sub.check()
            seen.update(op.results)
        if any(v not in seen for v in self.outputs):
            raise AssertionError("an output is never defined")

    def __str__(self) -> str:
        lines = [f"graph {self.name}({', '.join(f'{v!r}: {v.type}' for v in self.inputs)})"]
        for op in self.ops:
            extra = f" epilogue={list(op.attrs['epilogue'])}" if "epilogue" in op.attrs else ""
            lines.append(f"  {op!r} : {', '.join(str(r.type) for r in op.results)}{extra}")
            for name, sub in op.subgraphs():
                lines.append(f"    {name}: " + str(sub).replace("\n", "\n    "))
        lines.append("  return " + ", ".join(map(repr, self.outputs)))
        return "\n".join(lines)


def check_control(op: Op) -> None:
    """A control op's sub-graphs agree with its inputs and results (mira/ir.py:160-183)."""
    ins, outs = [v.type for v in op.inputs], [r.type for r in op.results]
    types = lambda vs: [v.type for v in vs]     # noqa: E731
    if op.kind == "if":
        n = op.attrs["n_then"]
        then, other = op.attrs["then"], op.attrs["else"]
        if op.inputs[0].type.numel != 1:
            raise AssertionError("if: the condition must have one element")
        if types(then.inputs) != ins[1:1 + n] or types(other.inputs) != ins[1 + n:]:
            raise AssertionError("if: branch inputs do not match the captures")
        if types(then.outputs) != outs or types(other.outputs) != outs:
            raise AssertionError("if: branch outputs do not match the results")
    else:
        ns, nc = op.attrs["n_state"], op.attrs["n_cond"]
        cond, body = op.attrs["cond"], op.attrs["body"]
        state = ins[:ns]
        if outs != state:
            raise AssertionError("while: results must match the loop state")
        if types(cond.inputs) != state + ins[ns:ns + nc] or len(cond.outputs) != 1 or \
                cond.outputs[0].type.numel != 1:
            raise AssertionError("while: bad condition graph signature")
        if types(body.inputs) != state + ins[ns + nc:] or types(body.outputs) != state:
            raise AssertionError("while: bad body graph signature")
