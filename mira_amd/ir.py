"""The IR data model the rocm target consumes (mirrors mira/ir.py:34-154).

A Graph is an SSA list of Ops; every Value is a graph input or the result of
exactly one op.  The rocm Target reads `op.kind`, `op.inputs`, `op.attrs` and
`op.result.type`, and segment graphs carry their constants as `const` ops,
exactly as the reference partitioner builds them (mira/partition.py:102-119),
so a reference Graph object can be handed to RocmTarget.compile unchanged.
"""
from __future__ import annotations

import itertools
from dataclasses import dataclass, field
from typing import Optional

import numpy as np

from . import ops as O
from .types import TensorType

_ids = itertools.count(1)


@dataclass(eq=False)
class Value:
    type: TensorType
    producer: Optional["Op"] = None
    name: Optional[str] = None
    id: int = field(default_factory=lambda: next(_ids))

    def __repr__(self) -> str:
        return f"%{self.name or self.id}"


@dataclass(eq=False)
class Op:
    kind: str
    inputs: list[Value]
    attrs: dict
    results: list[Value]

    @property
    def result(self) -> Value:
        return self.results[0]

    @property
    def is_const(self) -> bool:
        return self.kind == "const"

    @property
    def is_constant_like(self) -> bool:
        return self.kind in ("const", "dequantize")

    @property
    def is_control(self) -> bool:
        return self.kind in ("if", "while")

    def subgraphs(self) -> list[tuple[str, "Graph"]]:
        return [(k, v) for k, v in self.attrs.items() if isinstance(v, Graph)]


@dataclass(eq=False)
class Graph:
    name: str
    inputs: list[Value]
    ops: list[Op]
    outputs: list[Value]

    def add(self, kind: str, inputs: list[Value], attrs: Optional[dict] = None) -> Value:
        """Append an op, inferring its result type (raises ops.OpTypeError)."""
        attrs = attrs or {}
        v = Value(O.infer(kind, [x.type for x in inputs], attrs))
        op = Op(kind, list(inputs), attrs, [v])
        v.producer = op
        self.ops.append(op)
        return v

    def const(self, array: np.ndarray) -> Value:
        return self.add("const", [], {"value": np.asarray(array)})

    def input(self, name: str, shape, dtype: str = "f32") -> Value:
        v = Value(TensorType(dtype, tuple(shape)), name=name)
        self.inputs.append(v)
        return v

    def users(self) -> dict[Value, list[Op]]:
        uses: dict[Value, list[Op]] = {}
        for op in self.ops:
            for v in op.inputs:
                uses.setdefault(v, []).append(op)
        return uses

    def replace_uses(self, old: Value, new: Value) -> None:
        for op in self.ops:
            op.inputs = [new if v is old else v for v in op.inputs]
        self.outputs = [new if v is old else v for v in self.outputs]

    def compute_ops(self) -> list[Op]:
        return [op for op in self.ops if not op.is_constant_like]

    def verify(self) -> None:
        """SSA order and every result type still equal to its inferred type."""
        defined = set(self.inputs)
        for op in self.ops:
            for v in op.inputs:
                if v not in defined:
                    raise AssertionError(f"{op.kind} uses {v} before it is defined")
            if not op.is_control:
                expect = O.infer(op.kind, [v.type for v in op.inputs], op.attrs)
                if expect != op.result.type:
                    raise AssertionError(f"{op.kind} result type {op.result.type} != inferred {expect}")
            for r in op.results:
                if r.producer is not op:
                    raise AssertionError(f"{r} has wrong producer")
            defined.update(op.results)
        for v in self.outputs:
            if v not in defined:
                raise AssertionError(f"output {v} is not defined")

    def __str__(self) -> str:
        return format_graph(self)


def format_attr(k: str, v) -> str:
    if isinstance(v, np.ndarray):
        if v.size <= 4:
            return f"{k}={np.array2string(v.astype(np.float32).ravel(), precision=4, separator=',')}"
        dt = {"float16": "f16", "float32": "f32", "int8": "i8"}.get(v.dtype.name, v.dtype.name)
        return f"{k}=<{dt}[{', '.join(map(str, v.shape))}]>"
    if k == "epilogue":
        steps = [f"{fn}" if idx is None else f"{fn}(in{idx}{',swapped' if sw else ''})" for fn, idx, sw in v]
        return f"epilogue=[{' -> '.join(steps)}]"
    return f"{k}={v}"


def format_graph(g: Graph, annotate: Optional[dict] = None, indent: str = "") -> str:
    ins = ", ".join(f"{v!r}: {v.type}" for v in g.inputs)
    outs = ", ".join(str(v.type) for v in g.outputs)
    lines = [f"{indent}graph {g.name}({ins}) -> ({outs}) {{"]
    for op in g.ops:
        args = ", ".join(map(repr, op.inputs))
        attrs = ", ".join(format_attr(k, v) for k, v in op.attrs.items() if not isinstance(v, Graph))
        text = f"{', '.join(map(repr, op.results))} = {op.kind}({args})" + (f" {{{attrs}}}" if attrs else "")
        line = f"{indent}  {text:<60} : {', '.join(str(r.type) for r in op.results)}"
        if annotate and op in annotate:
            line += f"   @{annotate[op]}"
        lines.append(line)
    lines.append(f"{indent}  return " + ", ".join(map(repr, g.outputs)))
    lines.append(f"{indent}}}")
    return "\n".join(lines)
