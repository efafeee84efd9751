"""Quantization rewrites whose results the rocm kernels consume.

Weight-only int8 (mira/quantize.py:21-68): large matmul/conv weight constants
become `dequantize` constants (int8 + per-output-channel scale).

W8A8: matmuls and ungrouped convs with constant weights become `qmatmul` /
`qconv2d`.

Follows mira/quantize.py:24-31 (weights) and :95-143 (calibration + rewrite):
  q, w_scale = per-output-channel symmetric int8 weights
  x_scale    = peak |x| over the calibration feeds / 127   (1.0 if the peak is 0)
  epilogue operand indices shift by -1 (the weight input is removed).
Activations feeding several q-ops share one peak, hence one x_scale and one
int8 tensor on the device.
"""
from __future__ import annotations

from typing import Optional, Sequence

import numpy as np

from . import ir
from .passes import dce


def quantize_array(w: np.ndarray, axis: int) -> tuple[np.ndarray, np.ndarray]:
    """mira/quantize.py:24-31: scale = amax/127 (1 for an all-zero channel), q = clip(round(w/scale))."""
    others = tuple(i for i in range(w.ndim) if i != axis)
    amax = np.abs(w.astype(np.float32)).max(axis=others)
    scale = np.where(amax > 0, amax / 127.0, 1.0).astype(np.float32)
    bshape = [1] * w.ndim
    bshape[axis] = -1
    q = np.clip(np.round(w.astype(np.float32) / scale.reshape(bshape)), -127, 127).astype(np.int8)
    return q, scale


MIN_ELEMS = 1024   # mira/quantize.py:21: smaller constants (biases, norms) stay f32


def _weight_axis(v: ir.Value, users: list) -> Optional[int]:
    """mira/quantize.py:34-43: the output-channel axis when every use of `v` is as a
    matmul weight ([K, N] -> 1) or a conv weight ([O, C, KH, KW] -> 0), else None."""
    if not users:
        return None
    if v.type.rank == 2 and all(u.kind == "matmul" and u.inputs[1] is v and u.inputs[0] is not v for u in users):
        return 1
    if v.type.rank == 4 and all(u.kind == "conv2d" and u.inputs[1] is v for u in users):
        return 0
    return None


def quantize_weights(g: ir.Graph, mode: str = "int8", log: Optional[list] = None) -> tuple[int, int]:
    """mira/quantize.py:46-68, the weight-only mode: each constant of at least
    MIN_ELEMS elements used only as matmul/conv weights becomes a `dequantize`
    constant (int8 q + one f32 scale per output channel).  Returns the weight
    bytes before and after."""
    if mode != "int8":
        raise ValueError(f"unknown quantization mode '{mode}' (supported: int8)")
    before = after = 0
    users = g.users()
    for op in g.ops:
        for _, sub in op.subgraphs():
            b, a = quantize_weights(sub, mode)
            before, after = before + b, after + a
        if not op.is_const or op.result.type.numel < MIN_ELEMS:
            continue
        axis = _weight_axis(op.result, users.get(op.result, []))
        if axis is None:
            continue
        w = op.attrs["value"]
        q, scale = quantize_array(w, axis)
        before += w.nbytes
        after += q.nbytes + scale.nbytes
        op.kind = "dequantize"
        op.attrs = {"q": q, "scale": scale, "axis": axis, "dtype": op.result.type.dtype}
    g.verify()
    if log is not None and before:
        log.append(("quantize-int8", f"// weights: {before / 2**20:.2f} MiB -> {after / 2**20:.2f} MiB\n{g}"))
    return before, after


def w8a8_weight(op: ir.Op) -> Optional[tuple[np.ndarray, np.ndarray]]:
    """mira/quantize.py:95-115: (int8 weights, scales) if `op` can compute in int8, else None."""
    w = op.inputs[1].producer
    if w is None or not w.is_constant_like:
        return None
    if op.kind == "matmul":
        if op.inputs[1].type.rank != 2 or op.inputs[0].type.rank < 2:
            return None
        axis = 1
    elif op.kind == "conv2d":
        if op.attrs.get("groups", 1) != 1:      # depthwise / grouped convs stay f32
            return None
        axis = 0
    else:
        return None
    if w.kind == "dequantize" and w.attrs["axis"] == axis:
        return w.attrs["q"], w.attrs["scale"]
    value = w.attrs["value"] if w.is_const else None
    if value is None:
        return None
    return quantize_array(value, axis)


def candidates(g: ir.Graph) -> list[ir.Op]:
    return [op for op in g.ops if op.kind in ("matmul", "conv2d") and w8a8_weight(op) is not None]


def calibration_peaks(g: ir.Graph, calibration: list[dict]) -> list[float]:
    """Peak |x| of each candidate's input, in candidate order (mira/quantize.py:73-92)."""
    from .hosteval import peaks
    cands = candidates(g)
    peak = peaks(g, calibration, {op.inputs[0] for op in cands})
    return [peak[op.inputs[0]] for op in cands]


def quantize_w8a8(g: ir.Graph, calibration: Optional[list[dict]] = None, log: Optional[list] = None,
                  peaks: Optional[Sequence[float]] = None) -> int:
    """mira/quantize.py:118-143.  `peaks` (one per candidate, in graph order) may be given
    instead of `calibration`: it lets a large-batch graph reuse the calibration of a
    small-batch twin built with the same weights."""
    cands = candidates(g)
    if peaks is None:
        if calibration is None:
            raise ValueError("quantize_w8a8 needs calibration feeds or peaks")
        peaks = calibration_peaks(g, calibration)
    if len(peaks) != len(cands):
        raise ValueError(f"{len(peaks)} peaks for {len(cands)} W8A8 candidates")
    for op, peak in zip(cands, peaks):
        q, w_scale = w8a8_weight(op)
        x_scale = float(peak) / 127.0 or 1.0
        epi = tuple((fn, None if idx is None else idx - 1, sw) for fn, idx, sw in op.attrs.get("epilogue", ()))
        attrs = {k: v for k, v in op.attrs.items() if k != "epilogue"}
        attrs.update({"q": q, "w_scale": np.asarray(w_scale, np.float32), "x_scale": float(x_scale),
                      "dtype": op.result.type.dtype})
        if epi:
            attrs["epilogue"] = epi
        op.kind = "qmatmul" if op.kind == "matmul" else "qconv2d"
        op.inputs = [op.inputs[0]] + op.inputs[2:]
        op.attrs = attrs
    dce(g)
    g.verify()
    if log is not None:
        log.append(("quantize-w8a8", f"// {len(cands)} ops now compute in int8\n{g}"))
    return len(cands)
