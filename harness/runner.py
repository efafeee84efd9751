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
and consecutive ops on one device form a segment.
"""
from __future__ import annotations

import time
from typing import Optional

from .graph import Graph

HEAVY = {"matmul", "conv2d", "qmatmul", "qconv2d", "softmax", "layernorm", "maxpool2d"}


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
    while True:
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
        for seg in self.segments:
            if seg.device == target.name:
                seg.executable = target.compile(seg.graph)
            elif fallback is not None:
                seg.executable = fallback.compile(seg.graph)
            else:
                bad = sorted({f"{op.kind}: {self.reasons.get(op, '?')}" for op in seg.graph.compute_ops()})
                raise RuntimeError("these ops need a CPU fallback target and none was given: " + "; ".join(bad))

    @property
    def devices(self) -> list:
        return [s.device for s in self.segments]

    def run_env(self, feeds: dict) -> dict:
        env = dict(feeds)
        self.timings = []
        for seg in self.segments:
            t0 = time.perf_counter()
            env.update(seg.executable.run({v: env[v] for v in seg.graph.inputs}))
            self.timings.append((seg.device, time.perf_counter() - t0))
        return env

    def run(self, feeds: dict) -> list:
        """Outputs in order from {input name: array}."""
        env = self.run_env({v: feeds[v.name] for v in self.graph.inputs})
        return [env[v] for v in self.graph.outputs]

    def executables(self, device: Optional[str] = None) -> list:
        return [s.executable for s in self.segments if device is None or s.device == device]
