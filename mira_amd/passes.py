"""The graph passes that decide what a q-op's fused epilogue contains.

Mirrors the pass order of mira/passes.py:266-286 (fold/simplify/CSE/DCE to a
fixed point, then epilogue fusion) so that graphs reaching the rocm target
have the same op/epilogue structure the reference compiler gives them.  The
zero-bias removal in `simplify` matters: it is why a dense layer with an
all-zero constant bias reaches the target without an epilogue.
"""
from __future__ import annotations

import hashlib
from typing import Callable, Optional

import numpy as np

from . import ir

FOLD_LIMIT = 1 << 22   # largest result (elements) folded at compile time (mira/passes.py:17)


def _const_value(v: ir.Value) -> Optional[np.ndarray]:
    return v.producer.attrs["value"] if v.producer is not None and v.producer.is_const else None


def const_fold(g: ir.Graph) -> bool:
    """mira/passes.py:26-38: evaluate ops whose inputs are all constants."""
    from .hosteval import evaluate
    changed = False
    for op in g.ops:
        if op.is_const or op.is_control or not op.inputs or op.result.type.numel > FOLD_LIMIT:
            continue
        vals = [_const_value(v) for v in op.inputs]
        if any(v is None for v in vals):
            continue
        out = evaluate(op.kind, vals, op.attrs)
        op.kind, op.inputs, op.attrs = "const", [], {"value": np.asarray(out, dtype=op.result.type.np_dtype)}
        changed = True
    return changed


def _is_splat(v: ir.Value, x: float) -> bool:
    c = _const_value(v)
    return c is not None and bool(np.all(c == x))


def simplify(g: ir.Graph) -> bool:
    """mira/passes.py:48-100: x+0, x-0, x*1, x/1, identity reshapes/transposes/casts."""
    changed = False
    for op in list(g.ops):
        r = op.result
        ins = op.inputs
        new: Optional[ir.Value] = None
        if op.kind in ("add", "sub") and _is_splat(ins[1], 0) and ins[0].type == r.type:
            new = ins[0]
        elif op.kind == "add" and _is_splat(ins[0], 0) and ins[1].type == r.type:
            new = ins[1]
        elif op.kind in ("mul", "div", "pow") and _is_splat(ins[1], 1) and ins[0].type == r.type:
            new = ins[0]
        elif op.kind == "mul" and _is_splat(ins[0], 1) and ins[1].type == r.type:
            new = ins[1]
        elif op.kind == "neg" and ins[0].producer is not None and ins[0].producer.kind == "neg":
            new = ins[0].producer.inputs[0]
        elif op.kind == "transpose":
            perm = tuple(op.attrs["perm"])
            inner = ins[0].producer
            if perm == tuple(range(len(perm))):
                new = ins[0]
            elif inner is not None and inner.kind == "transpose":
                combined = tuple(inner.attrs["perm"][p] for p in perm)
                if combined == tuple(range(len(combined))):
                    new = inner.inputs[0]
                else:
                    op.inputs, op.attrs = [inner.inputs[0]], {"perm": combined}
                    changed = True
        elif op.kind == "reshape":
            inner = ins[0].producer
            if tuple(op.attrs["shape"]) == ins[0].type.shape:
                new = ins[0]
            elif inner is not None and inner.kind == "reshape":
                if inner.inputs[0].type.shape == r.type.shape:
                    new = inner.inputs[0]
                else:
                    op.inputs = [inner.inputs[0]]
                    changed = True
        elif op.kind == "cast":
            inner = ins[0].producer
            if ins[0].type.dtype == op.attrs["dtype"]:
                new = ins[0]
            elif (inner is not None and inner.kind == "cast" and inner.inputs[0].type == r.type
                  and inner.inputs[0].type.dtype == "f16"):
                new = inner.inputs[0]
        if new is not None and new is not r:
            g.replace_uses(r, new)
            changed = True
    return changed


def _digest(a: np.ndarray) -> tuple:
    return (a.dtype.str, a.shape, hashlib.sha1(np.ascontiguousarray(a).tobytes()).hexdigest())


def _key(op: ir.Op):
    if op.is_const:
        return ("const",) + _digest(op.attrs["value"])
    attrs = tuple(sorted((k, _digest(v) if isinstance(v, np.ndarray) else repr(v)) for k, v in op.attrs.items()))
    return (op.kind, tuple(v.id for v in op.inputs), attrs)


def cse(g: ir.Graph) -> bool:
    """mira/passes.py:116-132: identical ops on identical inputs are computed once."""
    seen: dict = {}
    changed = False
    for op in g.ops:
        if op.is_control:
            continue
        k = _key(op)
        prev = seen.get(k)
        if prev is not None and (not op.is_constant_like or all(
                np.array_equal(prev.attrs[a], op.attrs[a]) if isinstance(op.attrs[a], np.ndarray)
                else prev.attrs[a] == op.attrs[a] for a in op.attrs)):
            g.replace_uses(op.result, prev.result)
            changed = True
        else:
            seen[k] = op
    return changed


def dce(g: ir.Graph) -> bool:
    """mira/passes.py:135-146: drop ops whose results are never used."""
    live = set(g.outputs)
    kept = []
    for op in reversed(g.ops):
        if any(r in live for r in op.results):
            kept.append(op)
            live.update(op.inputs)
    kept.reverse()
    changed = len(kept) != len(g.ops)
    g.ops = kept
    return changed


FUSABLE_UNARY = {"relu", "gelu", "sigmoid", "tanh"}
FUSABLE_BINARY = {"add", "sub", "mul", "div", "maximum", "minimum"}


def fuse_epilogues(g: ir.Graph) -> bool:
    """mira/passes.py:155-201: fold the single elementwise consumer of a matmul/conv
    result (not a graph output) into that op's `epilogue`, repeatedly."""
    any_change = False
    while True:
        users = g.users()
        position = {op: i for i, op in enumerate(g.ops)}
        fused = False
        for op in g.ops:
            if op.kind not in ("matmul", "conv2d") or op.result in g.outputs:
                continue
            uses = users.get(op.result, [])
            if len(uses) != 1:
                continue
            u = uses[0]
            inputs = list(op.inputs)
            if u.kind in FUSABLE_UNARY:
                step = (u.kind, None, False)
            elif u.kind in FUSABLE_BINARY and u.result.type == op.result.type:
                lhs_is_acc = u.inputs[0] is op.result
                other = u.inputs[1] if lhs_is_acc else u.inputs[0]
                if other is op.result:
                    continue
                step = (u.kind, len(inputs), not lhs_is_acc)
                inputs.append(other)
            else:
                continue
            attrs = dict(op.attrs)
            attrs["epilogue"] = tuple(op.attrs.get("epilogue", ())) + (step,)
            new = ir.Op(op.kind, inputs, attrs, [u.result])
            u.result.producer = new
            g.ops[position[u]] = new
            g.ops.remove(op)
            fused = any_change = True
            break
        if not fused:
            return any_change


PIPELINE: list[tuple[str, Callable[[ir.Graph], bool]]] = [
    ("const-fold", const_fold),
    ("simplify", simplify),
    ("cse", cse),
    ("dce", dce),
]


def to_f16(g: ir.Graph) -> bool:
    """mira/passes.py:206-253 for graphs without control flow: every f32 value becomes f16
    (f32 constants are rounded to f16), a cast to f16 follows each f32 graph input and a
    cast back to f32 precedes each f32 graph output, and float<->float casts inside the
    graph disappear (casts to or from integers stay, aimed at f16)."""
    if all(op.result.type.dtype != "f32" for op in g.ops if op.results) and \
            all(v.type.dtype != "f32" for v in g.inputs):
        return False
    if any(op.is_control for op in g.ops):
        raise NotImplementedError("to_f16: graphs with control flow are not supported here")
    old_ops = g.ops
    g.ops = []
    remap: dict = {}
    for v in g.inputs:
        remap[v] = g.add("cast", [v], {"dtype": "f16"}) if v.type.dtype == "f32" else v
    for op in old_ops:
        if op.is_const:
            value = op.attrs["value"]
            remap[op.result] = g.const(value.astype(np.float16) if value.dtype.kind == "f" else value)
        elif op.kind == "cast":
            src = remap[op.inputs[0]]
            target = "f16" if op.attrs["dtype"] in ("f16", "f32") else op.attrs["dtype"]
            remap[op.result] = src if src.type.dtype == target else g.add("cast", [src], {"dtype": target})
        else:
            remap[op.result] = g.add(op.kind, [remap[v] for v in op.inputs], dict(op.attrs))
    outs = []
    for v in g.outputs:
        nv = remap[v]
        if v.type.dtype == "f32" and nv.type.dtype != "f32":
            nv = g.add("cast", [nv], {"dtype": "f32"})
        outs.append(nv)
    g.outputs = outs
    return True


def optimize(g: ir.Graph, fuse: bool = True, log: Optional[list] = None,
             precision: Optional[str] = None) -> ir.Graph:
    """mira/passes.py:266-286: optional f16 lowering, fold/simplify/CSE/DCE to a fixed
    point, then epilogue fusion."""
    def run(name: str, fn) -> bool:
        changed = fn(g)
        g.verify()
        if changed and log is not None:
            log.append((name, str(g)))
        return changed

    if precision == "f16":
        run("to-f16", to_f16)
    elif precision is not None:
        raise ValueError(f"precision={precision!r}: expected None (f32) or 'f16'")

    for _ in range(10):
        if not any([run(n, f) for n, f in PIPELINE]):
            break
    if fuse:
        run("fuse-epilogues", fuse_epilogues)
        run("dce", dce)
    return g
