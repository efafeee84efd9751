"""The back half of the MIRA driver for graphs that target rocm (mirrors
mira/compiler.py:23-161, 287-311): optimize -> W8A8 quantize -> partition ->
compile each segment -> run segment by segment.

Segments the rocm target rejects run on a CPU target object passed in as
`fallback` -- in a MIRA checkout that is mira.backends.cpu.CPUTarget, exactly
as in mira/compiler.py:91-95.  This package ships no CPU executor of its own:
with no fallback given, a graph that does not fit entirely on rocm is an error.
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Optional, Sequence, Union

import numpy as np

from . import ir, passes
from .partition import Placement, Segment, partition


def get_target(name: str, **options):
    """Registry branch a MIRA checkout adds to mira/backends/__init__.py:5-22."""
    if name == "rocm":
        from .target import RocmTarget
        return RocmTarget(device=options.get("device", 0), debug_acc=options.get("debug_acc", False))
    raise ValueError(f"unknown target '{name}' (this package provides: rocm)")


TARGETS = ["rocm"]


@dataclass
class GraphRunner:
    """mira/compiler.py:23-46: a graph split into segments, each compiled for its device."""
    graph: ir.Graph
    segments: list[Segment]
    placement: Placement
    target: str
    last_timings: list = field(default_factory=list)

    def run_env(self, feeds: dict) -> dict:
        env = dict(feeds)
        for op in self.graph.ops:
            if op.is_const and op.result in self.graph.outputs:
                env[op.result] = op.attrs["value"]
        self.last_timings = []
        for seg in self.segments:
            t0 = time.perf_counter()
            env.update(seg.executable.run({v: env[v] for v in seg.graph.inputs}))
            self.last_timings.append((seg.graph.name, time.perf_counter() - t0))
        return env

    def run_list(self, values: list) -> list:
        env = self.run_env(dict(zip(self.graph.inputs, values)))
        return [env[v] for v in self.graph.outputs]

    def annotations(self) -> dict:
        ann = {}
        for seg in self.segments:
            for op in seg.graph.compute_ops():
                where = seg.device
                if op in self.placement.reason:
                    where += f"  ({self.placement.reason[op]})"
                ann[op] = where
        return ann

    def summary_lines(self, indent: str = "  ") -> list[str]:
        lines = []
        for i, seg in enumerate(self.segments):
            n = len(seg.graph.compute_ops())
            ins = ", ".join(f"{v!r}:{v.type}" for v in seg.graph.inputs)
            lines.append(f"{indent}[{i}] {seg.device:<8} {n:3d} ops   inputs: {ins}")
            lines.append(f"{indent}    " + seg.executable.report().replace("\n", f"\n{indent}    "))
        return lines


def compile_graph(graph: ir.Graph, tgt, cost_model: bool = True, fallback=None) -> GraphRunner:
    """mira/compiler.py:83-96."""
    segments, placement = partition(graph, tgt, cost_model=cost_model)
    for seg in segments:
        if seg.device == tgt.name and tgt.name != "cpu":
            seg.executable = tgt.compile(seg.graph)
        elif fallback is not None:
            seg.executable = fallback.compile(seg.graph)
        else:
            bad = sorted({f"{op.kind}: {placement.reason.get(op, '?')}" for op in seg.graph.compute_ops()})
            raise RuntimeError("these ops need the CPU fallback target, and none was given: " + "; ".join(bad))
    return GraphRunner(graph, segments, placement, tgt.name)


@dataclass
class CompiledProgram:
    """mira/compiler.py:101-161."""
    target: str
    runner: GraphRunner
    pass_log: list = field(default_factory=list)
    compile_seconds: float = 0.0

    @property
    def graph(self) -> ir.Graph:
        return self.runner.graph

    @property
    def segments(self) -> list[Segment]:
        return self.runner.segments

    @property
    def placement(self) -> Placement:
        return self.runner.placement

    @property
    def last_timings(self) -> list:
        return self.runner.last_timings

    def run(self, inputs: dict) -> Union[np.ndarray, tuple]:
        missing = [v.name for v in self.graph.inputs if v.name not in inputs]
        if missing:
            raise ValueError(f"missing input(s): {', '.join(missing)}")
        feeds = {}
        for v in self.graph.inputs:
            arr = np.asarray(inputs[v.name])
            if tuple(arr.shape) != v.type.shape:
                raise ValueError(f"input '{v.name}' should have shape {list(v.type.shape)}, got {list(arr.shape)}")
            feeds[v] = arr.astype(v.type.np_dtype)
        env = self.runner.run_env(feeds)
        outs = [env[v] for v in self.graph.outputs]
        return outs[0] if len(outs) == 1 else tuple(outs)

    def placement_report(self) -> str:
        return ir.format_graph(self.graph, self.runner.annotations())

    def summary(self) -> str:
        head = f"target {self.target}: {len(self.segments)} segment(s), compiled in {self.compile_seconds:.2f}s"
        return "\n".join([head] + self.runner.summary_lines())


def default_calibration(graph: ir.Graph) -> list[dict]:
    """mira/compiler.py:302-305: four rng(0) standard-normal feeds."""
    rng = np.random.default_rng(0)
    return [{v.name: rng.standard_normal(v.type.shape).astype(v.type.np_dtype) for v in graph.inputs}
            for _ in range(4)]


def compile_ir(graph: ir.Graph, target: Union[str, object] = "rocm", *, optimize: bool = True, fuse: bool = True,
               precision: Optional[str] = None, cost_model: bool = True, quantize: Optional[str] = None,
               calibration: Optional[list] = None, peaks: Optional[Sequence[float]] = None, fallback=None,
               **target_options) -> CompiledProgram:
    """mira/compiler.py:287-311.  precision None keeps the f32 graph (bit-exact against the
    cpu target's f32 results); "f16" lowers it as the reference does for accelerator
    targets under its default "auto", and the rocm target then rounds every result to
    f16 exactly as the reference's ops do."""
    t0 = time.perf_counter()
    log = [("input", str(graph))]
    if optimize:
        passes.optimize(graph, fuse=fuse, log=log, precision=precision)
    elif precision == "f16":
        passes.to_f16(graph)
    if quantize == "w8a8":
        from .quantize import quantize_w8a8
        if calibration is None and peaks is None:
            calibration = default_calibration(graph)
        quantize_w8a8(graph, calibration, log=log, peaks=peaks)
    elif quantize:
        from .quantize import quantize_weights
        quantize_weights(graph, quantize, log=log)
    tgt = get_target(target, **target_options) if isinstance(target, str) else target
    runner = compile_graph(graph, tgt, cost_model, fallback=fallback)
    return CompiledProgram(tgt.name, runner, log, time.perf_counter() - t0)
