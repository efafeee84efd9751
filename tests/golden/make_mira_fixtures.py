"""Write golden fixtures from MIRA itself for its own W8A8 programs.

Run in the build container only (the reference checkout is not on the GPU box):

    python tests/golden/make_mira_fixtures.py [/root/reference]

For each of the reference's two W8A8 programs (`examples/mlp.mira`,
`examples/cnn.mira`; the cases of its tests/test_control_dynamic_quant.py:202)
and each precision (f32 as the cpu target compiles it, and the f16 graph its
"auto" precision gives accelerator targets), this compiles the program with
MIRA's own driver exactly as tests/test_control_dynamic_quant.py:217-225 does:

    compile_file(path, "cpu", quantize="w8a8", calibration=[rng(2), rng(3)], precision=...)

and runs it on the feed rng(1) with MIRA's cpu target.  The fixture holds the
quantized graph MIRA produced (every op, its attrs: q, w_scale, x_scale,
epilogue steps, conv parameters, constants), the feed, MIRA's values of the
op results, and how MIRA's own partitioner splits that graph when the rocm
target is plugged in (which only calls RocmTarget.check, so it runs without a
GPU).  It also records the f32 float graph before quantization twice -- as
elaborated (random seed-0 weights, mira/elaborate.py:1114-1123) and after
MIRA's optimizer (epilogue fusion) -- with each constant as a SHA-256 of its
bytes, which pins how the test harness rebuilds these programs.  Only these data files travel; the reference never does.

Format (one .npz per program and precision): "graph" is a JSON string; every
array the JSON names as {"array": key} is stored under that key; "feed:<name>"
is an input, "value:<id>" the reference's result of the op whose result has
that id (graph outputs, and intermediate results of at most 65536 elements).
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))

# intermediate results larger than this are left out (the graph output is always kept)
MAX_VALUE_ELEMS = 65536

CASES = [("mlp", "examples/mlp.mira", "x", (64, 784)), ("cnn", "examples/cnn.mira", "img", (16, 1, 28, 28))]


def _attr_json(v, arrays: dict, key: str):
    if isinstance(v, np.ndarray):
        arrays[key] = v
        return {"array": key}
    if isinstance(v, (np.floating, np.integer)):
        arrays[key] = np.asarray(v)
        return {"array": key}
    if isinstance(v, tuple):
        return {"tuple": [_attr_json(x, arrays, f"{key}.{i}") for i, x in enumerate(v)]}
    if isinstance(v, list):
        return [_attr_json(x, arrays, f"{key}.{i}") for i, x in enumerate(v)]
    if isinstance(v, float) and not np.isfinite(v):
        return {"float": repr(v)}
    if v is None or isinstance(v, (bool, int, float, str)):
        return v
    raise TypeError(f"attr {key}: cannot serialise {type(v)}")


def _float_graph_json(g) -> dict:
    """A float graph's structure; constants appear as shape, dtype and a SHA-256 of their bytes."""
    ops = []
    for op in g.ops:
        attrs = {}
        for k, v in op.attrs.items():
            if op.kind == "const" and k == "value":
                a = np.ascontiguousarray(v)
                attrs[k] = {"sha256": hashlib.sha256(a.tobytes()).hexdigest(), "shape": list(a.shape),
                            "dtype": str(a.dtype)}
            else:
                attrs[k] = _attr_json(v, {}, k)
        ops.append({"kind": op.kind, "inputs": [v.id for v in op.inputs],
                    "result": {"id": op.result.id, "dtype": op.result.type.dtype, "shape": list(op.result.type.shape)},
                    "attrs": attrs})
    return {"inputs": [{"id": v.id, "name": v.name, "dtype": v.type.dtype, "shape": list(v.type.shape)}
                       for v in g.inputs], "ops": ops, "outputs": [v.id for v in g.outputs]}


def main(ref: str) -> int:
    sys.path.insert(0, ref)
    sys.path.insert(0, ROOT)
    import mira
    from mira import ops as O
    from mira.partition import partition
    from mira_amd.target import RocmTarget

    for name, path, inp, shape in CASES:
        calib = [{inp: np.random.default_rng(s).standard_normal(shape).astype(np.float32)} for s in (2, 3)]
        feed = np.random.default_rng(1).standard_normal(shape).astype(np.float32)
        # the float graph as elaborated (seed 0 weights), and after MIRA's optimizer (fold/simplify/
        # CSE/DCE, epilogue fusion), both f32
        elaborated = mira.compile_file(os.path.join(ref, path), "cpu", optimize=False, precision=None).graph
        optimized = mira.compile_file(os.path.join(ref, path), "cpu", precision=None).graph
        float_doc = {"elaborated": _float_graph_json(elaborated), "optimized": _float_graph_json(optimized)}
        for precision in (None, "f16"):
            prog = mira.compile_file(os.path.join(ref, path), "cpu", quantize="w8a8", calibration=calib,
                                     precision=precision)
            g = prog.graph
            arrays: dict = {"feed:" + inp: feed}
            env = {g.inputs[0]: feed.astype(g.inputs[0].type.np_dtype)}
            ops = []
            for i, op in enumerate(g.ops):
                env[op.result] = O.evaluate(op.kind, [env[v] for v in op.inputs], op.attrs)
                if op.result in g.outputs or np.size(env[op.result]) <= MAX_VALUE_ELEMS:
                    arrays[f"value:{op.result.id}"] = np.asarray(env[op.result])
                ops.append({"kind": op.kind, "inputs": [v.id for v in op.inputs],
                            "result": {"id": op.result.id, "dtype": op.result.type.dtype,
                                       "shape": list(op.result.type.shape)},
                            "attrs": {k: _attr_json(v, arrays, f"op{i}.{k}") for k, v in op.attrs.items()}})
            out = prog.run({inp: feed})
            assert np.array_equal(np.asarray(out), arrays[f"value:{g.outputs[0].id}"], equal_nan=True)
            segs, placement = partition(g, RocmTarget())
            doc = {
                "program": path, "precision": precision or "f32",
                "compile": f"compile_file({path!r}, 'cpu', quantize='w8a8', calibration=[rng(2), rng(3)], "
                           f"precision={precision!r}); feed rng(1)",
                "inputs": [{"id": v.id, "name": v.name, "dtype": v.type.dtype, "shape": list(v.type.shape)}
                           for v in g.inputs],
                "ops": ops,
                "outputs": [v.id for v in g.outputs],
                "partition_with_rocm": [{"device": s.device, "kinds": [op.kind for op in s.graph.ops
                                                                       if not op.is_constant_like]}
                                        for s in segs],
                "rocm_rejects": sorted({f"{op.kind}: {r}" for op, r in placement.reason.items()}),
            }
            doc["float_graphs"] = float_doc
            arrays["graph"] = np.asarray(json.dumps(doc))
            dst = os.path.join(HERE, f"mira_w8a8_{name}_{precision or 'f32'}.npz")
            np.savez_compressed(dst, **arrays)
            print(f"wrote {dst}: {len(ops)} ops, {sum(op['kind'] in ('qmatmul', 'qconv2d') for op in ops)} q-ops, "
                  f"partition {[s['device'] for s in doc['partition_with_rocm']]}, "
                  f"{os.path.getsize(dst) / 1024:.0f} KiB")
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference"))
