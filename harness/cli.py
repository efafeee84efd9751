"""Command-line driver for .mira programs and .onnx models: the counterpart of mira/cli.py's
run / emit / bench / check for the rocm target and its cpu reference.

    python -m harness.cli run   prog.mira -t rocm --quantize w8a8 --check
    python -m harness.cli emit  prog.mira --stage opt
    python -m harness.cli bench prog.mira --targets rocm,cpu
    python -m harness.cli check prog.mira

The compile steps follow mira/compiler.py:252-312: elaborate (or import the ONNX model),
precision "auto" -> f16 for every target but cpu, the optimizer's lowering, then W8A8
(calibrated on four batches of default_rng(0) normal inputs unless a calibration is given)
or int8 weight-only, then the split between the target and the cpu fallback.  Random
inputs are default_rng(seed + 1) normal (mira/cli.py:76-80); `run --check` compares every
output with the unquantized cpu run of the same program:
max|out - ref| / max|ref| < tol, tol 2e-2 by default (mira/cli.py:101-111).

The cpu target is the harness's NumPy evaluator (harness.hosteval.HostTarget).
"""
from __future__ import annotations

import argparse
import os
import sys
import time
from typing import Optional

import numpy as np

from harness import hosteval
from harness import lowering as LW
from harness import mira_lang
from harness import onnx_import
from harness.graph import Graph
from harness.runner import Runner

TARGETS = ["rocm", "cpu"]
STAGES = ["tokens", "ast", "ir", "opt", "partition"]


class CompileError(Exception):
    """A user-facing error: bad program text, shapes, flags."""


def _target(name: str):
    if name == "cpu":
        return hosteval.HostTarget()
    if name == "rocm":
        from mira_amd.target import RocmTarget
        return RocmTarget()
    raise CompileError(f"unknown target '{name}' (choose from {', '.join(TARGETS)})")


class Program:
    """A compiled program: the graph as lowered, its segments, timings of the last run."""

    def __init__(self, target: str, graph: Graph, ir_text: str, runner: Runner, seconds: float):
        self.target = target
        self.graph = graph
        self.ir_text = ir_text
        self.runner = runner
        self.compile_seconds = seconds

    @property
    def segments(self):
        return self.runner.segments

    @property
    def last_timings(self) -> list:
        return self.runner.timings

    def run(self, feeds: dict) -> list:
        return self.runner.run(feeds)

    def summary(self) -> str:
        lines = [f"target {self.target}: {len(self.segments)} segment(s), compiled in {self.compile_seconds:.2f}s"]
        return "\n".join(lines + self.runner.summary_lines())

    def placement_report(self) -> str:
        lines = []
        for op in self.graph.compute_ops():
            why = self.runner.reasons.get(op)
            dev = "cpu" if why is not None else self.target
            lines.append(f"{op.kind:<12} {str(op.result.type):<24} {dev}" + (f"   ({why})" if why else ""))
        return "\n".join(lines)


def load_graph(path: str, entry: str = "main", weights: Optional[dict] = None, dims: Optional[dict] = None,
               seed: Optional[int] = 0, input_shapes: Optional[dict] = None) -> Graph:
    """The float graph of a .mira program or a .onnx model."""
    if path.endswith(".onnx"):
        try:
            return onnx_import.load(path, input_shapes)
        except onnx_import.OnnxImportError as err:
            raise CompileError(str(err)) from None
    with open(path) as f:
        src = f.read()
    try:
        return mira_lang.elaborate(src, entry, weights, dims, seed, name=os.path.splitext(os.path.basename(path))[0])
    except mira_lang.MiraSyntaxError as err:
        raise CompileError(f"{path}: {err}") from None


def compile_graph(g: Graph, target: str, precision: Optional[str] = "auto", quantize: Optional[str] = None,
                  calibration: Optional[list] = None, started: Optional[float] = None) -> Program:
    """Lower a float graph for `target` (mira/compiler.py:287-312) and compile its segments."""
    t0 = started if started is not None else time.perf_counter()
    if precision == "auto":
        precision = None if target == "cpu" else "f16"
    ir_text = str(g)
    LW.prepare(g, precision=precision)
    if quantize == "w8a8":
        if calibration is None:
            rng = np.random.default_rng(0)
            calibration = [{v.name: rng.standard_normal(v.type.shape).astype(v.type.np_dtype) for v in g.inputs}
                           for _ in range(4)]
        try:
            LW.w8a8(g, calibration)
        except ValueError as err:
            raise CompileError(str(err)) from None
    elif quantize == "int8":
        LW.weight_only(g)
    elif quantize is not None:
        raise CompileError(f"unknown quantization '{quantize}' (int8, w8a8)")
    tgt = _target(target)
    runner = Runner(g, tgt, fallback=None if target == "cpu" else hosteval.HostTarget())
    return Program(target, g, ir_text, runner, time.perf_counter() - t0)


def compile_file(path: str, target: str = "cpu", *, entry: str = "main", weights: Optional[dict] = None,
                 dims: Optional[dict] = None, seed: Optional[int] = 0, precision: Optional[str] = "auto",
                 quantize: Optional[str] = None, calibration: Optional[list] = None,
                 input_shapes: Optional[dict] = None) -> Program:
    t0 = time.perf_counter()
    g = load_graph(path, entry, weights, dims, seed, input_shapes)
    return compile_graph(g, target, precision, quantize, calibration, started=t0)


# ---------------------------------------------------------------- what a command line asks for

def parse_bindings(items, flag: str, value) -> dict:
    """NAME=VALUE items of a repeatable flag (--dim B=32, --shape x=1,3,224,224) as a dict,
    each VALUE passed through `value`."""
    bound = {}
    for item in items or []:
        name, sep, text = item.partition("=")
        if not (name and sep and text):
            raise CompileError(f"{flag} takes NAME=VALUE items, not {item!r}")
        bound[name] = value(text)
    return bound


def _dims_tuple(text: str) -> tuple:
    return tuple(int(d) for d in text.split(",") if d.strip())


def read_arrays(path: Optional[str]) -> dict:
    """The arrays of an .npz file by name (no file: none)."""
    if not path:
        return {}
    with np.load(path, allow_pickle=False) as z:
        return dict(z.items())


def random_feeds(graph: Graph, given: dict, seed: int) -> dict:
    """Values for the graph inputs: the given ones, and standard-normal draws from one
    default_rng(seed + 1) stream for the others, in input order -- the inputs MIRA's driver
    makes up for a run (mira/cli.py:76-80), so the same flags feed the same values."""
    stream = np.random.default_rng(seed + 1)
    feeds = {}
    for v in graph.inputs:
        feeds[v.name] = given[v.name] if v.name in given else \
            stream.standard_normal(v.type.shape).astype(v.type.np_dtype)
    return feeds


def relative_error(out, ref) -> tuple:
    """(max|out - ref|, max|ref|, their ratio) with MIRA's 1e-12 guard on the peak."""
    a, b = np.asarray(out, np.float32), np.asarray(ref, np.float32)
    worst = float(np.abs(a - b).max()) if b.size else 0.0
    peak = float(np.abs(b).max()) if b.size else 0.0
    return worst, peak, worst / (peak + 1e-12)


def compare(outs: list, refs: list, tol: float) -> tuple:
    """Each output against its reference as max|out - ref| / max|ref| (the accuracy check of
    `run --check`, mira/cli.py:101-111): (every output under tol, one report line each)."""
    verdicts, lines = [], []
    for i, (out, ref) in enumerate(zip(outs, refs)):
        worst, peak, rel = relative_error(out, ref)
        verdicts.append(rel < tol)
        lines.append(f"output {i} vs the unquantized cpu run: |err| <= {worst:.3e}, {rel:.3e} of the peak "
                     f"{peak:.3e} (tol {tol:g})  {'PASS' if verdicts[-1] else 'FAIL'}")
    return all(verdicts), lines


class Invocation:
    """One command line resolved: the program file and the flags that shape its graph.
    Builds the program for a target, its unquantized cpu reference (once) and its feeds."""

    def __init__(self, args):
        self.path = args.file
        self.entry = args.entry
        self.seed = args.seed
        self.weights = read_arrays(args.weights)
        self.given = read_arrays(getattr(args, "inputs", None))
        self.dims = parse_bindings(args.dim, "--dim", int)
        self.shapes = parse_bindings(args.shape, "--shape", _dims_tuple)
        self.precision = args.precision
        self.quantize = args.quantize
        self._ref: Optional[Program] = None

    def program(self, target: str) -> Program:
        return compile_file(self.path, target, entry=self.entry, weights=self.weights, dims=self.dims,
                            seed=self.seed, precision=self.precision, quantize=self.quantize,
                            input_shapes=self.shapes)

    def reference(self) -> Program:
        """The same program on the cpu target in f32 without quantization."""
        if self._ref is None:
            self._ref = compile_file(self.path, "cpu", entry=self.entry, weights=self.weights, dims=self.dims,
                                     seed=self.seed, input_shapes=self.shapes)
        return self._ref

    def feeds(self, prog: Program) -> dict:
        return random_feeds(prog.graph, self.given, self.seed)


def _describe(i: int, out: np.ndarray) -> str:
    head = f"output {i}: {out.dtype}{list(out.shape)}"
    if out.size:
        head += f"  min {float(out.min()):.4g}  max {float(out.max()):.4g}  mean {float(out.mean()):.4g}"
    with np.printoptions(precision=4, suppress=True, threshold=12, edgeitems=3):
        return head + "\n" + np.array2string(out)


def _save(path: str, outs: list) -> None:
    if len(outs) == 1:
        np.save(path, outs[0])
    else:
        np.savez(path, **{f"output{i}": o for i, o in enumerate(outs)})


# ---------------------------------------------------------------- commands

def cmd_run(args) -> int:
    job = Invocation(args)
    prog = job.program(args.target)
    feeds = job.feeds(prog)
    outs = prog.run(feeds)
    print(prog.summary())
    seconds = [t for _, t in prog.last_timings]
    print(f"ran {len(seconds)} segment(s) in {sum(seconds) * 1e3:.2f} ms")
    for i, out in enumerate(outs):
        print(_describe(i, out))
    if args.save:
        _save(args.save, outs)
        print(f"saved to {args.save}")
    if not args.check or args.target == "cpu":
        return 0
    ok, lines = compare(outs, job.reference().run(feeds), args.tol)
    print("\n".join(lines))
    return 0 if ok else 1


def _format_dim(d) -> str:
    return f"({_format_dim(d[1])} {d[0]} {_format_dim(d[2])})" if isinstance(d, tuple) else str(d)


def _format_type(t) -> str:
    return f"{t.dtype}[{', '.join(_format_dim(d) for d in t.dims)}]" if t.dims else t.dtype


def _format_expr(e) -> str:
    kind = e[0]
    if kind == "num":
        return repr(e[1])
    if kind == "bool":
        return "true" if e[1] else "false"
    if kind in ("name", "dtype"):
        return e[1]
    if kind == "list":
        return "[" + ", ".join(_format_expr(x) for x in e[1]) + "]"
    if kind == "tuple":
        return "(" + ", ".join(_format_expr(x) for x in e[1]) + ("," if len(e[1]) == 1 else "") + ")"
    if kind == "neg":
        return f"-{_format_expr(e[1])}"
    if kind == "bin":
        return f"({_format_expr(e[2])} {e[1]} {_format_expr(e[3])})"
    if kind == "index":
        return f"{_format_expr(e[1])}[{_format_items(e[2])}]"
    _, name, args, kwargs, _ = e
    return f"{name}(" + ", ".join([_format_expr(a) for a in args] +
                                  [f"{k}={_format_expr(v)}" for k, v in kwargs.items()]) + ")"


def _format_items(items) -> str:
    def one(it):
        if it[0] == "at":
            return _format_expr(it[1])
        return "".join([_format_expr(it[1]) if it[1] is not None else "", ":",
                        _format_expr(it[2]) if it[2] is not None else ""])
    return ", ".join(one(it) for it in items)


def _format_block(body, indent: str) -> list:
    out = []
    for st in body:
        kind = st[0]
        if kind == "let":
            ann = f": {_format_type(st[2])}" if st[2] is not None else ""
            out.append(f"{indent}let {', '.join(st[1])}{ann} = {_format_expr(st[3])}")
        elif kind == "assign":
            out.append(f"{indent}{', '.join(st[1])} = {_format_expr(st[2])}")
        elif kind == "index_assign":
            out.append(f"{indent}{st[1]}[{_format_items(st[2])}] = {_format_expr(st[3])}")
        elif kind == "for":
            out.append(f"{indent}for {st[1]} in {_format_expr(st[2])}..{_format_expr(st[3])} {{")
            out += _format_block(st[4], indent + "  ") + [f"{indent}}}"]
        elif kind == "if":
            out.append(f"{indent}if {_format_expr(st[1])} {{")
            out += _format_block(st[2], indent + "  ")
            if st[3] is not None:
                out += [f"{indent}}} else {{"] + _format_block(st[3], indent + "  ")
            out.append(f"{indent}}}")
        elif kind == "while":
            out.append(f"{indent}while {_format_expr(st[1])} {{")
            out += _format_block(st[2], indent + "  ") + [f"{indent}}}"]
        else:
            out.append(f"{indent}return {', '.join(_format_expr(v) for v in st[1])}")
    return out


def format_module(fns: dict) -> str:
    """The parse tree of a program as fully parenthesized source."""
    out = []
    for fn in fns.values():
        params = ", ".join(("const " if p.const else "") + f"{p.name}: {_format_type(p.type)}" for p in fn.params)
        rets = ", ".join(_format_type(t) for t in fn.rets)
        out.append(f"fn {fn.name}({params}) -> {rets if len(fn.rets) == 1 else f'({rets})'} {{")
        out += _format_block(fn.body, "  ")
        out.append("}")
    return "\n".join(out)


def cmd_emit(args) -> int:
    if args.stage in ("tokens", "ast"):
        if args.file.endswith(".onnx"):
            raise CompileError(f"'{args.stage}' is a .mira source stage; ONNX models start at the 'ir' stage")
        with open(args.file) as f:
            src = f.read()
        try:
            if args.stage == "tokens":
                for t in mira_lang.tokenize(src):
                    print(f"{t.line:4d} {t.kind:<5} {t.text}")
            else:
                print(format_module(mira_lang.parse(src)))
        except mira_lang.MiraSyntaxError as err:
            raise CompileError(f"{args.file}: {err}") from None
        return 0
    prog = Invocation(args).program(args.target)
    if args.stage == "ir":
        print(prog.ir_text)
    elif args.stage == "opt":
        print(prog.graph)
    else:
        print(prog.placement_report())
        print()
        print(prog.summary())
    return 0


def _timed_runs(prog: Program, feeds: dict, n: int) -> np.ndarray:
    seconds = np.empty(n)
    for i in range(n):
        t0 = time.perf_counter()
        prog.run(feeds)
        seconds[i] = time.perf_counter() - t0
    return seconds


def cmd_bench(args) -> int:
    """Each target in turn: compile, one checked warm-up run, then `--iters` timed runs on the
    same feeds; the first output's error is against the unquantized cpu run."""
    job = Invocation(args)
    rows, feeds, ref = [], None, None
    for target in [t for t in args.targets.split(",") if t]:
        prog = job.program(target)
        feeds = feeds if feeds is not None else job.feeds(prog)
        first = prog.run(feeds)[0]
        ref = ref if ref is not None else job.reference().run(feeds)[0]
        rel = relative_error(first, ref)[2]
        t = _timed_runs(prog, feeds, args.iters) * 1e3
        rows.append((target, prog.compile_seconds, float(np.median(t)), float(t.min()), rel,
                     "+".join(s.device for s in prog.segments)))
    head = ("target", "compile s", "median ms", "best ms", "rel err", "segments")
    print("  ".join(f"{h:>10}" for h in head))
    for target, comp, med, best, rel, segs in rows:
        print(f"{target:>10}  {comp:>10.2f}  {med:>10.3f}  {best:>10.3f}  {rel:>10.2e}  {segs:>10}")
    return 0


def cmd_check(args) -> int:
    g = Invocation(args).program("cpu").graph
    sig = ", ".join(f"{v.name}: {v.type}" for v in g.inputs)
    print(f"ok: {args.file}  inputs ({sig}) -> {g.outputs[0].type}, {len(g.compute_ops())} ops")
    return 0


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="harness.cli", description="run .mira programs and .onnx models on rocm")
    sub = ap.add_subparsers(dest="cmd", required=True)

    def common(p):
        p.add_argument("file")
        p.add_argument("--target", "-t", default="cpu", choices=TARGETS)
        p.add_argument("--entry", default="main")
        p.add_argument("--weights", help=".npz with values for const parameters (default: random)")
        p.add_argument("--inputs", help=".npz with runtime inputs (default: random)")
        p.add_argument("--dim", action="append", help="bind a shape symbol of the entry function, e.g. --dim B=32")
        p.add_argument("--shape", action="append", metavar="NAME=D0,D1,...",
                       help="ONNX models: the shape of an input with symbolic dims")
        p.add_argument("--seed", type=int, default=0)
        p.add_argument("--precision", default="auto", choices=["auto", "f16", "none"])
        p.add_argument("--quantize", choices=["int8", "w8a8"],
                       help="int8: store large weights as int8; w8a8: also do the multiplies in int8")

    p = sub.add_parser("run", help="compile and run")
    common(p)
    p.add_argument("--check", action="store_true", help="compare against the cpu reference")
    p.add_argument("--tol", type=float, default=2e-2)
    p.add_argument("--save")
    p.set_defaults(fn=cmd_run)

    p = sub.add_parser("emit", help="print a compiler stage")
    common(p)
    p.add_argument("--stage", "-s", default="opt", choices=STAGES)
    p.set_defaults(fn=cmd_emit)

    p = sub.add_parser("bench", help="time targets")
    common(p)
    p.add_argument("--targets", default="rocm,cpu")
    p.add_argument("--iters", type=int, default=20)
    p.set_defaults(fn=cmd_bench)

    p = sub.add_parser("check", help="parse and type-check only")
    common(p)
    p.set_defaults(fn=cmd_check)

    args = ap.parse_args(argv)
    if getattr(args, "precision", None) == "none":
        args.precision = None
    try:
        return args.fn(args)
    except CompileError as err:
        print(f"error: {err}", file=sys.stderr)
        return 1


if __name__ == "__main__":
    sys.exit(main())
