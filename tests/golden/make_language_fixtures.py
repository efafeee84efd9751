"""Write golden fixtures from MIRA itself for this repository's language test programs.

Run in the build container only (the reference checkout is not on the GPU box):

    python tests/golden/make_language_fixtures.py [/root/reference]

The programs under tests/programs/{encoder_block,residual_loop,char_lm,selection}.mira use the
parts of MIRA's language beyond the CNN / MLP subset (compile-time int parameters, computed
dimensions, `for` and compile-time `if`, rebinding, comparisons and masks, `**`, indexing,
slicing and gathers, tuple returns, reductions, the selection builtins).  For each program
this compiles it with MIRA's own driver (mira/compiler.py:252-312) at fixed dims and seed 0:

* the elaborated graph (optimize=False) and the optimized f32 and f16 graphs, each constant
  recorded as a SHA-256 of its bytes;
* the W8A8 graphs (quantize="w8a8" with the two calibration feeds stored here), f32 and f16,
  with every array attr (q, w_scale, constants) as a SHA-256 and x_scale as a float;

and runs every compiled program with MIRA's cpu target on the stored feed.  Only these data
files travel; the reference never does.

The programs tests/programs/{fixed_point,greedy_lm,device_loop}.mira add runtime `if` / `while` (with
captures, indexed assignment and dynamic slices); MIRA's W8A8 rewrite rejects control flow, so
those have the f32 and f16 variants only, each also run on the feed with its float inputs
negated (the other branch of fixed_point's `if`).

Format (one .npz per program): "doc" is a JSON string (an if / while op's sub-graphs nest in
its attrs as {"graph": ...}); "feed:<name>" and "calib<i>:<name>" are inputs,
"out:<variant>:<k>" MIRA's k-th result of a variant (f32, f16, w8a8_f32, w8a8_f16, and f32neg /
f16neg for the negated feed).
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
PROGRAMS = os.path.join(ROOT, "tests", "programs")

# program, dims; integer inputs draw token ids below dims["V"] (or 8)
CASES = [("encoder_block", {"S": 16, "E": 32, "h": 4}),
         ("residual_loop", {"B": 8, "D": 16, "n": 5}),
         ("char_lm", {"B": 2, "T": 8, "V": 13, "D": 16, "F": 32, "L": 2}),
         ("selection", {"R": 6, "C": 5})]
# programs with runtime if / while (MIRA's W8A8 rejects control flow: f32 and f16 only); each
# also runs on the negated feed, which takes the other branch of fixed_point's if
CONTROL = [("fixed_point", {"N": 4, "M": 6, "tol": 1}),
           ("greedy_lm", {"P": 3, "V": 11, "T": 12, "D": 16, "F": 32, "L": 2}),
           ("device_loop", {"B": 8, "D": 32, "n": 5})]


def _jsonable(v):
    if hasattr(v, "ops") and hasattr(v, "outputs"):          # an if / while sub-graph
        return {"graph": graph_json(v)}
    if isinstance(v, np.ndarray):
        a = np.ascontiguousarray(v)
        return {"sha256": hashlib.sha256(a.tobytes()).hexdigest(), "shape": list(a.shape), "dtype": str(a.dtype)}
    if isinstance(v, (np.floating, np.integer)):
        v = v.item()
    if isinstance(v, tuple):
        return {"tuple": [_jsonable(x) for x in v]}
    if isinstance(v, list):
        return [_jsonable(x) for x in v]
    if isinstance(v, float) and not np.isfinite(v):
        return {"float": repr(v)}
    if v is None or isinstance(v, (bool, int, float, str)):
        return v
    raise TypeError(f"cannot serialise {type(v)}")


def graph_json(g) -> dict:
    ops = [{"kind": op.kind, "inputs": [v.id for v in op.inputs],
            "result": {"id": op.results[0].id, "dtype": op.results[0].type.dtype,
                       "shape": list(op.results[0].type.shape)},
            "results": [{"id": r.id, "dtype": r.type.dtype, "shape": list(r.type.shape)} for r in op.results],
            "attrs": {k: _jsonable(v) for k, v in op.attrs.items()}} for op in g.ops]
    return {"inputs": [{"id": v.id, "name": v.name, "dtype": v.type.dtype, "shape": list(v.type.shape)}
                       for v in g.inputs], "ops": ops, "outputs": [v.id for v in g.outputs]}


def draw(graph, seed: int, dims: dict) -> dict:
    rng = np.random.default_rng(seed)
    out = {}
    for v in graph.inputs:
        if v.type.dtype == "i32":
            out[v.name] = rng.integers(0, dims.get("V", 8), v.type.shape).astype(np.int32)
        else:
            out[v.name] = rng.standard_normal(v.type.shape).astype(v.type.np_dtype)
    return out


def main(ref: str) -> int:
    sys.path.insert(0, ref)
    import mira

    for name, dims in CASES:
        path = os.path.join(PROGRAMS, name + ".mira")
        elaborated = mira.compile_file(path, "cpu", dims=dims, optimize=False, precision=None).graph
        feed = draw(elaborated, 1, dims)
        calib = [draw(elaborated, s, dims) for s in (2, 3)]
        arrays = {f"feed:{k}": v for k, v in feed.items()}
        for i, c in enumerate(calib):
            arrays.update({f"calib{i}:{k}": v for k, v in c.items()})
        doc = {"program": f"tests/programs/{name}.mira", "dims": dims, "elaborated": graph_json(elaborated)}
        variants = {"f32": dict(precision=None), "f16": dict(precision="f16"),
                    "w8a8_f32": dict(precision=None, quantize="w8a8", calibration=calib),
                    "w8a8_f16": dict(precision="f16", quantize="w8a8", calibration=calib)}
        for tag, kw in variants.items():
            prog = mira.compile_file(path, "cpu", dims=dims, **kw)
            doc[tag] = graph_json(prog.graph)
            outs = prog.run(dict(feed))
            outs = outs if isinstance(outs, tuple) else (outs,)
            for k, o in enumerate(outs):
                arrays[f"out:{tag}:{k}"] = np.asarray(o)
        arrays["doc"] = np.asarray(json.dumps(doc))
        dst = os.path.join(HERE, f"mira_lang_{name}.npz")
        np.savez_compressed(dst, **arrays)
        print(f"wrote {dst}: {len(doc['f32']['ops'])} ops optimized, "
              f"{sum(op['kind'] == 'qmatmul' for op in doc['w8a8_f32']['ops'])} q-ops, "
              f"{os.path.getsize(dst) / 1024:.0f} KiB")
    for name, dims in CONTROL:
        path = os.path.join(PROGRAMS, name + ".mira")
        elaborated = mira.compile_file(path, "cpu", dims=dims, optimize=False, precision=None).graph
        feed = draw(elaborated, 1, dims)
        neg = {k: (-v if v.dtype.kind == "f" else v) for k, v in feed.items()}
        arrays = {f"feed:{k}": v for k, v in feed.items()}
        doc = {"program": f"tests/programs/{name}.mira", "dims": dims, "elaborated": graph_json(elaborated)}
        for tag, prec in (("f32", None), ("f16", "f16")):
            prog = mira.compile_file(path, "cpu", dims=dims, precision=prec)
            doc[tag] = graph_json(prog.graph)
            for suffix, f in (("", feed), ("neg", neg)):
                outs = prog.run(dict(f))
                outs = outs if isinstance(outs, tuple) else (outs,)
                for k, o in enumerate(outs):
                    arrays[f"out:{tag}{suffix}:{k}"] = np.asarray(o)
        arrays["doc"] = np.asarray(json.dumps(doc))
        dst = os.path.join(HERE, f"mira_lang_{name}.npz")
        np.savez_compressed(dst, **arrays)
        print(f"wrote {dst}: {len(doc['f32']['ops'])} ops optimized, {os.path.getsize(dst) / 1024:.0f} KiB")
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference"))
