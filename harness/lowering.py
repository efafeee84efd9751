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

def drop_zero_terms(g: Graph) -> int:
    """x + 0, 0 + x and x - 0 with an all-zero constant disappear when the result has x's type
    (MIRA's simplify does this, mira/passes.py:56-57; it is why a dense layer with a zero bias
    reaches the target without an epilogue)."""
    n = 0
    for op in list(g.ops):
        if op.kind not in ("add", "sub"):
            continue
        a, b = op.inputs
        for keep, zero in ((a, b), (b, a)) if op.kind == "add" else ((a, b),):
            z = _const_array(zero)
            if z is not None and not np.any(z) and keep.type == op.result.type:
                g.redirect(op.result, keep)
                g.ops.remove(op)
                n += 1
                break
    g.prune()
    return n


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


def lower_f16(g: Graph) -> None:
    """MIRA's f16 precision (mira/passes.py:206-253) for a graph without casts: f32 constants
    are rounded to f16, every f32 result becomes f16, each f32 input is cast to f16 where it
    enters and each f32 output cast back to f32 where it leaves."""
    if any(op.kind == "cast" for op in g.ops):
        raise NotImplementedError("lower_f16: graphs with casts")
    body, g.ops = g.ops, []
    for v in g.inputs:
        if v.type.dtype == "f32":
            c = g.emit("cast", [v], {"dtype": "f16"}, TensorType("f16", v.type.shape))
            for op in body:
                op.inputs = [c if x is v else x for x in op.inputs]
    for op in body:
        if op.kind == "const" and op.attrs["value"].dtype == np.float32:
            op.attrs["value"] = op.attrs["value"].astype(np.float16)
        for r in op.results:
            if r.type.dtype == "f32":
                r.type = TensorType("f16", r.type.shape)
        g.ops.append(op)
    outs = []
    for v in g.outputs:
        outs.append(g.emit("cast", [v], {"dtype": "f32"}, TensorType("f32", v.type.shape))
                    if v.type.dtype == "f16" else v)
    g.outputs = outs


def prepare(g: Graph, precision: Optional[str] = None) -> Graph:
    """The float graph as MIRA's optimizer leaves it for these networks: optional f16
    lowering, zero-term removal, epilogue fusion."""
    if precision == "f16":
        lower_f16(g)
    elif precision is not None:
        raise ValueError(f"precision {precision!r}: None (f32) or 'f16'")
    drop_zero_terms(g)
    fuse_epilogues(g)
    g.prune()
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


def w8a8_candidates(g: Graph) -> list:
    return [op for op in g.ops if _w8a8_weight(op) is not None]


def calibrate(g: Graph, feeds: Sequence[dict]) -> list:
    """Peak |x| of each W8A8 candidate's activation over the calibration feeds ({input name:
    array}), one float per candidate in program order (so a same-shaped graph at another
    batch size can take them)."""
    cands = w8a8_candidates(g)
    watch = {op.inputs[0] for op in cands}
    peaks: dict = {}
    for feed in feeds:
        hosteval.run(g, {v: feed[v.name] for v in g.inputs}, watch, peaks)
    return [peaks[op.inputs[0]] for op in cands]


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
    g.prune()
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
