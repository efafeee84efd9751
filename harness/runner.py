"""Split a graph between the rocm target and a CPU fallback, compile, run.

This is the harness's stand-in for MIRA's partitioner and driver
(mira/partition.py:70-120, mira/compiler.py:23-96), which do the same in a
deployment.  Only the behaviour the target depends on is kept: every op the
target's check() accepts runs there, the rest on the fallback target; a
target segment with no heavy op is handed to the fallback (transfers would
dominate); each segment is a graph of its own whose constants are ops inside
it; segments run in order, each taking host arrays in and giving host arrays
out.

The grouping is simpler than MIRA's list scheduler: ops stay in program order
and consecutive ops on one device form a segment.  A control op (if / while) runs
on the host segment that holds it; each of its sub-graphs is split and compiled the
same way, so the ops of a loop body run on the target (mira/partition.py:74-75,
mira/backends/cpu.py:18-51).
"""
from __future__ import annotations

import time
from typing import Optional

from .graph import Graph

HEAVY = {"matmul", "conv2d", "qmatmul", "qconv2d", "softmax", "layernorm", "maxpool2d", "while", "if"}


class Segment:
    def __init__(self, device: str, graph: Graph):
        self.device = device
        self.graph = graph
        self.executable = None


def _groups(ops: list, device: dict) -> list:
    out: list = []
    for op in ops:
        if out and out[-1][0] == device[op]:
            out[-1][1].append(op)
        else:
            out.append((device[op], [op]))
    return out


def split(g: Graph, target, cpu_name: str = "cpu") -> tuple:
    """(segments, reasons): reasons maps each op the target does not run to why."""
    compute = g.compute_ops()
    device, reasons = {}, {}
    for op in compute:
        why = target.check(op)
        device[op] = target.name if why is None else cpu_name
        if why is not None:
            reasons[op] = why
    while target.name != cpu_name:      # the cpu target keeps everything (mira/partition.py:77-87)
        light = [ops for dev, ops in _groups(compute, device) if dev == target.name
                 and not any(op.kind in HEAVY for op in ops)]
        if not light:
            break
        for ops in light:
            for op in ops:
                device[op] = cpu_name
                reasons[op] = "kept on the CPU: its segment has no heavy compute, transfers would dominate"
    users = g.users()
    consts = {op.result: op for op in g.ops if op.is_constant_like}
    segments = []
    for i, (dev, ops) in enumerate(_groups(compute, device)):
        s = Graph(f"{g.name}.{i}.{dev}")
        inside = {r for op in ops for r in op.results}
        used = [v for op in ops for v in op.inputs]
        s.ops = [consts[v] for v in dict.fromkeys(used) if v in consts] + ops
        s.inputs = [v for v in dict.fromkeys(used) if v not in inside and v not in consts]
        s.outputs = [r for r in dict.fromkeys(r for op in ops for r in op.results)
                     if r in g.outputs or any(u not in ops for u in users.get(r, []))]
        segments.append(Segment(dev, s))
    return segments, reasons


class Runner:
    """A graph split into segments, each compiled for its device."""

    def __init__(self, g: Graph, target, fallback=None):
        self.graph = g
        self.segments, self.reasons = split(g, target, getattr(fallback, "name", "cpu"))
        self.timings: list = []
        # outputs that are constants belong to no segment (a branch returning a literal)
        self.const_outputs = {op.result: op.attrs["value"] for op in g.ops
                              if op.kind == "const" and op.result in g.outputs}

        def compile_sub(sub: Graph) -> "Runner":       # if / while sub-graphs, split the same way
            return Runner(sub, target, fallback)

        for seg in self.segments:
            if seg.device == target.name:
                seg.executable = target.compile(seg.graph) if not any(op.is_control for op in seg.graph.ops) \
                    else target.compile(seg.graph, compile_sub)
            elif fallback is not None:
                seg.executable = fallback.compile(seg.graph, compile_sub)
            else:
                bad = sorted({f"{op.kind}: {self.reasons.get(op, '?')}" for op in seg.graph.compute_ops()})
                raise RuntimeError("these ops need a CPU fallback target and none was given: " + "; ".join(bad))

    @property
    def devices(self) -> list:
        return [s.device for s in self.segments]

    def run_env(self, feeds: dict) -> dict:
        env = {**self.const_outputs, **feeds}
        self.timings = []
        for seg in self.segments:
            t0 = time.perf_counter()
            env.update(seg.executable.run({v: env[v] for v in seg.graph.inputs}))
            self.timings.append((seg.device, time.perf_counter() - t0))
        return env

    def run_values(self, arrays: list) -> list:
        """Outputs in order from the inputs' arrays in order (how a control op runs a sub-graph)."""
        env = self.run_env(dict(zip(self.graph.inputs, arrays)))
        return [env[v] for v in self.graph.outputs]

    def run(self, feeds: dict) -> list:
        """Outputs in order from {input name: array}."""
        env = self.run_env({v: feeds[v.name] for v in self.graph.inputs})
        return [env[v] for v in self.graph.outputs]

    def placements(self) -> list:
        """(device, op kind) of every compute op, those of control ops' sub-graphs included."""
        out = []
        for seg in self.segments:
            out += [(seg.device, op.kind) for op in seg.graph.compute_ops()]
            for sub in getattr(seg.executable, "sub", {}).values():
                out += sub.placements()
        return out

    def summary_lines(self, indent: str = "  ") -> list:
        lines = []
        for i, seg in enumerate(self.segments):
            ins = ", ".join(f"{v!r}:{v.type}" for v in seg.graph.inputs)
            lines.append(f"{indent}[{i}] {seg.device:<8} {len(seg.graph.compute_ops()):3d} ops   inputs: {ins}")
            lines.append(f"{indent}    " + seg.executable.report().replace("\n", f"\n{indent}    "))
            for (op, name), sub in getattr(seg.executable, "sub", {}).items():
                lines.append(f"{indent}    {op.kind} {name}: {sub.graph.name}")
                lines += sub.summary_lines(indent + "      ")
        return lines

    def executables(self, device: Optional[str] = None) -> list:
        return [s.executable for s in self.segments if device is None or s.device == device]
