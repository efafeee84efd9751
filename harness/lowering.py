"""Lowering of the harness's float graphs into the form the rocm target receives.

In a MIRA deployment MIRA's own compiler does all of this before the rocm
target sees a graph (mira/compiler.py:287-311): f16 lowering, simplification,
epilogue fusion, then the W8A8 (or weight-only int8) rewrite.  The tests and
the benchmark need the same graphs without MIRA, so this module produces
them.  What it must agree with MIRA on is the *result* -- which ops exist,
the epilogue step tuples, the q-op attrs -- and that is checked against
MIRA's own output for its programs (tests/golden, tests/test_mira_golden.py).
The attr names and the step tuple format are MIRA's interface:

    qmatmul / qconv2d attrs: q (int8), w_scale (f32 per output channel),
        x_scale (Python float), dtype, epilogue, and the conv's stride /
        padding / dilation / groups
    epilogue: ((fn, operand input index or None, swapped), ...)
    dequantize attrs: q, scale, axis, dtype

The arithmetic of the attrs follows MIRA's definitions:
    per-channel weights (mira/quantize.py:24-31)   scale = amax / 127 (1 when amax == 0),
                                                   q = clip(rint(w / scale), -127, 127)
    activation scale (mira/quantize.py:125-128)    x_scale = peak |x| / 127 (1.0 when the peak is 0)
"""
from __future__ import annotations

import hashlib
from typing import Optional, Sequence

import numpy as np

from . import hosteval
from .graph import Graph, Op, TensorType

FUSE_UNARY = ("relu", "gelu", "sigmoid", "tanh")
FUSE_BINARY = ("add", "sub", "mul", "div", "maximum", "minimum")
WEIGHT_ONLY_MIN = 1024        # smaller constants (biases, norms) stay float in the weight-only mode


# ---------------------------------------------------------------- weights

def quantize_array(w: np.ndarray, axis: int) -> tuple:
    """Symmetric per-channel int8 weights along `axis` (the output channel)."""
    wf = np.asarray(w).astype(np.float32)
    moved = np.moveaxis(wf, axis, 0)
    amax = np.abs(moved.reshape(moved.shape[0], -1)).max(axis=1)
    scale = np.where(amax > 0, amax / 127.0, 1.0).astype(np.float32)
    bshape = [1] * wf.ndim
    bshape[axis] = scale.size
    q = np.clip(np.round(wf / scale.reshape(bshape)), -127, 127).astype(np.int8)
    return q, scale


def _const_array(v) -> Optional[np.ndarray]:
    p = v.producer
    return p.attrs["value"] if p is not None and p.kind == "const" else None


# ---------------------------------------------------------------- float passes
# MIRA's optimizer (mira/passes.py:266-286): f16 lowering, then constant folding,
# simplification, common-subexpression and dead-code elimination to a fixed point, then
# epilogue fusion and a last dead-code pass.

FOLD_LIMIT = 1 << 22          # folded results above this many elements stay ops (mira/passes.py:17)


def const_fold(g: Graph) -> bool:
    """Ops whose inputs are all constants become constants (mira/passes.py:25-37)."""
    changed = False
    for op in g.ops:
        if op.kind == "const" or op.is_control or not op.inputs or op.result.type.numel > FOLD_LIMIT:
            continue
        vals = [_const_array(v) for v in op.inputs]
        if any(v is None for v in vals):
            continue
        out = hosteval.evaluate(op.kind, vals, op.attrs)
        op.kind, op.inputs, op.attrs = "const", [], {"value": np.asarray(out, dtype=op.result.type.np_dtype)}
        changed = True
    return changed


def _splat(v, x: float) -> bool:
    c = _const_array(v)
    return c is not None and bool(np.all(c == x))


def simplify(g: Graph) -> bool:
    """Peephole rewrites (mira/passes.py:47-102): x + 0, 0 + x, x - 0, x * 1, 1 * x, x / 1,
    x ** 1 (when the result keeps x's type), neg(neg x), identity and composed transposes,
    identity and chained reshapes, same-dtype casts and the exact f16 -> f32 -> f16 round trip."""
    changed = False
    for op in list(g.ops):
        r, ins, k = op.result, op.inputs, op.kind
        new = None
        if k in ("add", "sub") and _splat(ins[1], 0) and ins[0].type == r.type:
            new = ins[0]
        elif k == "add" and _splat(ins[0], 0) and ins[1].type == r.type:
            new = ins[1]
        elif k in ("mul", "div", "pow") and _splat(ins[1], 1) and ins[0].type == r.type:
            new = ins[0]
        elif k == "mul" and _splat(ins[0], 1) and ins[1].type == r.type:
            new = ins[1]
        elif k == "neg" and ins[0].producer is not None and ins[0].producer.kind == "neg":
            new = ins[0].producer.inputs[0]
        elif k == "transpose":
            perm, inner = tuple(op.attrs["perm"]), ins[0].producer
            ident = tuple(range(len(perm)))
            if perm == ident:
                new = ins[0]
            elif inner is not None and inner.kind == "transpose":
                both = tuple(inner.attrs["perm"][p] for p in perm)
                if both == ident:
                    new = inner.inputs[0]
                else:
                    op.inputs, op.attrs = [inner.inputs[0]], {"perm": both}
                    changed = True
        elif k == "reshape":
            inner = ins[0].producer
            if tuple(op.attrs["shape"]) == ins[0].type.shape:
                new = ins[0]
            elif inner is not None and inner.kind == "reshape":
                if inner.inputs[0].type.shape == r.type.shape:
                    new = inner.inputs[0]
                else:
                    op.inputs = [inner.inputs[0]]
                    changed = True
        elif k == "cast":
            inner = ins[0].producer
            if ins[0].type.dtype == op.attrs["dtype"]:
                new = ins[0]
            elif inner is not None and inner.kind == "cast" and inner.inputs[0].type == r.type \
                    and inner.inputs[0].type.dtype == "f16":
                new = inner.inputs[0]
        if new is not None and new is not r:
            g.redirect(r, new)
            changed = True
    return changed


def _op_key(op: Op) -> tuple:
    def digest(a):
        a = np.ascontiguousarray(a)
        return (a.dtype.str, a.shape, hashlib.sha1(a.tobytes()).hexdigest())
    if op.kind == "const":
        return ("const",) + digest(op.attrs["value"])
    attrs = tuple(sorted((k, digest(v) if isinstance(v, np.ndarray) else repr(v)) for k, v in op.attrs.items()))
    return (op.kind, tuple(v.id for v in op.inputs), attrs)


def cse(g: Graph) -> bool:
    """Identical ops on identical inputs computed once (mira/passes.py:116-130); constants match
    on their bytes, confirmed element for element."""
    seen: dict = {}
    changed = False
    for op in g.ops:
        if op.is_control:
            continue
        key = _op_key(op)
        prev = seen.get(key)
        if prev is not None and (op.kind != "const" or np.array_equal(prev.attrs["value"], op.attrs["value"])):
            g.redirect(op.result, prev.result)
            changed = True
        else:
            seen[key] = op
    return changed


def dce(g: Graph) -> bool:
    """Ops none of whose results reach an output are dropped (mira/passes.py:133-144)."""
    n = len(g.ops)
    g.prune()
    return len(g.ops) != n


def _absorb_step(g: Graph, op: Op, users: dict) -> bool:
    """Fold the single elementwise consumer of op's result into op's epilogue."""
    r = op.result
    if r in g.outputs or len(users.get(r, ())) != 1:
        return False
    u = users[r][0]
    if u.kind in FUSE_UNARY:
        step, extra = (u.kind, None, False), []
    elif u.kind in FUSE_BINARY and u.result.type == r.type:
        lhs, rhs = u.inputs
        if (lhs is r) == (rhs is r):
            return False
        other, swapped = (rhs, False) if lhs is r else (lhs, True)
        step, extra = (u.kind, len(op.inputs), swapped), [other]
    else:
        return False
    op.inputs += extra
    op.attrs["epilogue"] = tuple(op.attrs.get("epilogue", ())) + (step,)
    op.results = [u.result]
    u.result.producer = op
    # the fused op now sits where its consumer was, after everything the consumer read
    g.ops.remove(op)
    g.ops[g.ops.index(u)] = op
    return True


def fuse_epilogues(g: Graph) -> int:
    """Fold chains of single-use elementwise consumers of matmul/conv2d results into the
    producer's `epilogue`, always taking the earliest producer (in program order) that can
    absorb one more step -- the order decides, for a residual add of two conv results, which
    conv owns it."""
    n = 0
    while True:
        users = g.users()
        for op in g.ops:
            if op.kind in ("matmul", "conv2d") and _absorb_step(g, op, users):
                n += 1
                break
        else:
            return n


def lower_f16(g: Graph, keep_interface: bool = True) -> None:
    """MIRA's f16 precision (mira/passes.py:206-253): float constants are rounded to f16, every
    f32 result becomes f16, each f32 input is cast to f16 where it enters and each f32 output
    cast back to f32 where it leaves; casts between float types disappear and casts to or from
    integers stay, aimed at f16.  The sub-graphs of if / while ops are converted completely,
    inputs and outputs included (keep_interface=False), so loop state stays f16."""
    body, g.ops = g.ops, []
    out_dtypes = [v.type.dtype for v in g.outputs]
    sub: dict = {}
    for v in g.inputs:
        if v.type.dtype == "f32":
            if keep_interface:
                sub[v] = g.emit("cast", [v], {"dtype": "f16"}, TensorType("f16", v.type.shape))
            else:
                v.type = TensorType("f16", v.type.shape)
    for op in body:
        for _, sg in op.subgraphs():
            lower_f16(sg, keep_interface=False)
        op.inputs = [sub.get(x, x) for x in op.inputs]
        if op.kind == "const":
            a = op.attrs["value"]
            if a.dtype.kind == "f":
                op.attrs["value"] = a.astype(np.float16)
        elif op.kind == "cast":
            src = op.inputs[0]
            target = "f16" if op.attrs["dtype"] in ("f16", "f32") else op.attrs["dtype"]
            if src.type.dtype == target:
                sub[op.result] = src
                continue
            op.attrs = {**op.attrs, "dtype": target}
        for r in op.results:
            if r.type.dtype == "f32":
                r.type = TensorType("f16", r.type.shape)
        g.ops.append(op)
    outs = []
    for v, dt in zip(g.outputs, out_dtypes):
        v = sub.get(v, v)
        if keep_interface and dt == "f32" and v.type.dtype != "f32":
            v = g.emit("cast", [v], {"dtype": "f32"}, TensorType("f32", v.type.shape))
        outs.append(v)
    g.outputs = outs


def prepare(g: Graph, precision: Optional[str] = None) -> Graph:
    """The float graph as MIRA's optimizer leaves it (mira/passes.py:266-286): optional f16
    lowering, then const-fold / simplify / CSE / DCE to a fixed point (at most 10 rounds, each
    running all four), epilogue fusion, DCE."""
    if precision == "f16":
        lower_f16(g)
    elif precision is not None:
        raise ValueError(f"precision {precision!r}: None (f32) or 'f16'")
    for op in g.ops:                     # if / while sub-graphs first (mira/passes.py:276-278)
        for _, sg in op.subgraphs():
            prepare(sg)
    for _ in range(10):
        if not any([const_fold(g), simplify(g), cse(g), dce(g)]):
            break
    fuse_epilogues(g)
    dce(g)
    g.check()
    return g


# ---------------------------------------------------------------- W8A8

def _w8a8_weight(op: Op) -> Optional[tuple]:
    """(q, w_scale) when op is a W8A8 candidate: a matmul of a rank >= 2 activation with a
    constant rank-2 weight, or an ungrouped conv2d with a constant weight."""
    if op.kind == "matmul":
        axis = 1
        if op.inputs[1].type.rank != 2 or op.inputs[0].type.rank < 2:
            return None
    elif op.kind == "conv2d":
        axis = 0
        if op.attrs.get("groups", 1) != 1:
            return None
    else:
        return None
    p = op.inputs[1].producer
    if p is None:
        return None
    if p.kind == "dequantize":
        return (p.attrs["q"], p.attrs["scale"]) if p.attrs["axis"] == axis else None
    if p.kind == "const":
        return quantize_array(p.attrs["value"], axis)
    return None


def _graphs(g: Graph) -> list:
    """g and every if / while sub-graph inside it, outermost first."""
    out = [g]
    for op in g.ops:
        for _, sg in op.subgraphs():
            out += _graphs(sg)
    return out


def w8a8_candidates(g: Graph) -> list:
    """Candidates in program order; those inside an if / while sub-graph come at that op's place
    (sub-graphs in MIRA's order: then, else / cond, body)."""
    out = []
    for op in g.ops:
        if _w8a8_weight(op) is not None:
            out.append(op)
        for _, sg in op.subgraphs():
            out += w8a8_candidates(sg)
    return out


def calibrate(g: Graph, feeds: Sequence[dict]) -> list:
    """Peak |x| of each W8A8 candidate's activation over the calibration feeds ({input name:
    array}), one float per candidate in program order (so a same-shaped graph at another
    batch size can take them).  Candidates inside loop bodies and branches fold their peak over
    every iteration of every feed; one whose branch never runs keeps a peak of 0 (x_scale 1).
    MIRA's rewrite stops at control flow (mira/quantize.py:84-85); this one calibrates through it."""
    cands = w8a8_candidates(g)
    watch = {op.inputs[0] for op in cands}
    peaks: dict = {}
    for feed in feeds:
        hosteval.run(g, {v: feed[v.name] for v in g.inputs}, watch, peaks)
    return [peaks.get(op.inputs[0], 0.0) for op in cands]


def w8a8(g: Graph, calibration: Optional[Sequence[dict]] = None, peaks: Optional[Sequence[float]] = None) -> list:
    """Rewrite every candidate to qmatmul / qconv2d.  Returns the peaks used."""
    cands = w8a8_candidates(g)
    if peaks is None:
        peaks = calibrate(g, calibration)
    if len(peaks) != len(cands):
        raise ValueError(f"{len(peaks)} peaks for {len(cands)} W8A8 candidates")
    for op, peak in zip(cands, peaks):
        q, w_scale = _w8a8_weight(op)
        attrs = {k: v for k, v in op.attrs.items() if k != "epilogue"}
        attrs.update(q=q, w_scale=np.asarray(w_scale, np.float32), x_scale=float(peak / 127.0 or 1.0),
                     dtype=op.result.type.dtype)
        steps = tuple((fn, None if i is None else i - 1, sw) for fn, i, sw in op.attrs.get("epilogue", ()))
        if steps:
            attrs["epilogue"] = steps
        op.kind = "qmatmul" if op.kind == "matmul" else "qconv2d"
        op.inputs = [op.inputs[0]] + op.inputs[2:]
        op.attrs = attrs
    for sg in _graphs(g):
        sg.prune()
    g.check()
    return list(peaks)


# ---------------------------------------------------------------- weight-only int8

def weight_only(g: Graph) -> int:
    """Constants of at least WEIGHT_ONLY_MIN elements used only as matmul weights (rank 2,
    output axis 1, never also the activation) or conv weights (rank 4, axis 0) become
    `dequantize` constants.  Returns how many."""
    users = g.users()
    n = 0
    for op in g.ops:
        if op.kind != "const" or op.result.type.numel < WEIGHT_ONLY_MIN:
            continue
        v, us = op.result, users.get(op.result, [])
        axis = None
        if us and v.type.rank == 2 and all(u.kind == "matmul" and u.inputs[1] is v and u.inputs[0] is not v
                                           for u in us):
            axis = 1
        elif us and v.type.rank == 4 and all(u.kind == "conv2d" and u.inputs[1] is v for u in us):
            axis = 0
        if axis is None:
            continue
        q, scale = quantize_array(op.attrs["value"], axis)
        op.kind = "dequantize"
        op.attrs = {"q": q, "scale": scale, "axis": axis, "dtype": v.type.dtype}
        n += 1
    return n
