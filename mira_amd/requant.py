"""Integer requantization lines for int8-only epilogues, exact with a flag window.

A q-op whose only output is the int8 copy of its result computes, per output column c,

    q = clip(rint(f32(epilogue_c(f32(f64(acc) * scale_c)) / xs)), -127, 127)

(mira/ops.py:616-620 / 630-634 for the dequant, :192-199 for the epilogue, :602-603 for
the quantizer of the next op's input).  With only per-column or scalar epilogue operands
and non-decreasing steps (add, subtract a constant, multiply or divide by a positive
constant, maximum / minimum / relu, f16 rounding), q is a non-decreasing step function of
the int32 accumulator: over the accumulator range [-A, A] (A = K * 127 * 127) it is fixed
by its value lo at -A, its value hi at A, and the integer thresholds

    t_k = min{ acc : q(acc) >= k },   lo < k <= hi.

The kernels evaluate the integer line

    r = acc * M + C (int64),   q' = med3(r >> 32, lo, hi)

with per-column M (int32, >= 0) and C (int64).  The line's own thresholds are
t'_k = min{ acc : r >> 32 >= k }, and since both q and q' are non-decreasing,
q'(acc) = lo + #{k : acc >= t'_k} differs from q(acc) = lo + #{k : acc >= t_k} exactly on
the accumulators between t_k and t'_k for some k.  The f32 rounding of the golden chain
moves its thresholds off any straight line by a few hundredths of an accumulator step, so
a few such accumulators usually remain; each lies next to a crossing of the line, where
the low word of r is close to 0 mod 2^32.  The host enumerates them exactly and takes
h = 1 + the largest distance (min(r mod 2^32, 2^32 - r mod 2^32)) among them.  The stored
line is shifted by h, (M, C + h) with window w = 2h: the kernel takes (r + h) >> 32, which
equals r >> 32 wherever the low word of r is at least h from a multiple of 2^32, unless
(r + h) mod 2^32 < 2h (exactly the accumulators closer than h), and otherwise evaluates
the float chain.  So every output is exact, and the float chain runs only for
accumulators within h / M of a crossing of the line (none in columns the line fits
exactly, where h = 0).

This module computes the thresholds by binary search over the golden chain itself (NumPy
float32 / float64, the reference's operation order), fits M to minimise the spread of the
thresholds about the line (a convex problem in M, integer ternary search) and C to
satisfy as many of them as possible, then derives w from the exact mismatch set.
"""
from __future__ import annotations

from typing import Optional, Sequence

import numpy as np

# steps a line can carry: fn name -> whether it keeps q non-decreasing for a given operand
_MONOTONE = {"add", "sub", "mul", "div", "maximum", "minimum", "relu"}

# one per output column; the C ABI's mr_requant_line
LINE_DTYPE = np.dtype([("c", "<i8"), ("m", "<i4"), ("w", "<u4"), ("lo", "<i4"), ("hi", "<i4"), ("pad", "<i8")])
assert LINE_DTYPE.itemsize == 32

# columns whose mismatch set is larger than this take the float chain for the whole launch
MAX_MISMATCH = 4096
# the float chain runs for about w / 2^32 of a column's accumulators; lines whose windows
# send more than 1 in 1000 there on average (or 1 in 100 in one column) are not worth it
# (f16 results, whose rounding to f16 moves thresholds by tens of accumulators, land here)
MAX_MEAN_WINDOW = 1 << 22
MAX_WINDOW = 1 << 25


def _apply(fn: str, y: np.ndarray, o, swapped: bool) -> np.ndarray:
    """One epilogue step in float32, NumPy semantics (mira/ops.py:99-139)."""
    if fn == "relu":
        return np.maximum(y, np.float32(0))
    a, b = (o, y) if swapped else (y, o)
    with np.errstate(all="ignore"):
        if fn == "add":
            return np.add(a, b, dtype=np.float32)
        if fn == "sub":
            return np.subtract(a, b, dtype=np.float32)
        if fn == "mul":
            return np.multiply(a, b, dtype=np.float32)
        if fn == "div":
            return np.divide(a, b, dtype=np.float32)
        if fn == "maximum":
            return np.maximum(a, b).astype(np.float32)
        if fn == "minimum":
            return np.minimum(a, b).astype(np.float32)
    raise ValueError(fn)


def golden_q(acc: np.ndarray, scale: np.ndarray, steps: Sequence, f16: bool, xs: np.float32) -> np.ndarray:
    """The int8 result of the chain for accumulators acc[c, j] of column c (int64); steps
    are (fn, operand per column [C, 1] float32 or None, swapped).  NaN quantizes to -127,
    as the kernels' clamp does."""
    y = (acc.astype(np.float64) * scale[:, None]).astype(np.float32)
    for fn, o, sw in steps:
        y = _apply(fn, y, o, sw)
    if f16:
        with np.errstate(over="ignore"):
            y = y.astype(np.float16).astype(np.float32)
    with np.errstate(all="ignore"):
        t = np.rint(np.divide(y, np.float32(xs), dtype=np.float32))
    t = np.clip(t, -127, 127)
    return np.where(np.isnan(t), -127, t).astype(np.int64)


def _monotone(steps: Sequence) -> bool:
    for fn, o, sw in steps:
        if fn not in _MONOTONE:
            return False
        if fn == "relu":
            continue
        if not np.all(np.isfinite(o)):
            return False
        if fn == "sub" and sw:
            return False
        if fn == "mul" and np.any(o < 0):
            return False
        if fn == "div" and (sw or np.any(o <= 0)):
            return False
    return True


def _thresholds(scale, steps, f16, xs, A: int):
    """lo[c] = q(-A), hi[c] = q(A), and t[c, k + 127] for k in -126..127 (A + 1 where k is
    not reached in the range)."""
    C = scale.shape[0]
    ends = golden_q(np.array([[-A, A]] * C, np.int64), scale, steps, f16, xs)
    lo, hi = ends[:, 0], ends[:, 1]
    ks = np.arange(-126, 128, dtype=np.int64)
    # binary search for the least acc in [-A, A + 1) with q(acc) >= k (A + 1: none)
    left = np.full((C, ks.size), -A, np.int64)
    right = np.full((C, ks.size), A + 1, np.int64)
    while True:
        active = left < right
        if not active.any():
            break
        mid = (left + right) // 2
        q = golden_q(np.where(active, mid, 0), scale, steps, f16, xs)
        ok = q >= ks[None, :]
        right = np.where(active & ok, mid, right)
        left = np.where(active & ~ok, mid + 1, left)
    return lo, hi, left


def _best_slope(t: np.ndarray, valid: np.ndarray) -> np.ndarray:
    """Per column, the integer M in [0, 2^31) minimising the spread of d_k = k * 2^32 - t_k * M
    over the valid k, less M (the amount by which no C satisfies every threshold; <= 0: an
    exact line).  The spread is convex in M, so an integer ternary search finds it."""
    ks = (np.arange(-126, 128, dtype=np.int64) << 32)[None, :]
    big = np.int64(1) << 62

    def excess(M):
        d = ks - t * M[:, None]
        return np.where(valid, d, -big).max(axis=1) - np.where(valid, d, big).min(axis=1) - M

    lo = np.zeros(t.shape[0], np.int64)
    hi = np.full(t.shape[0], (1 << 31) - 1, np.int64)
    while True:
        open_ = hi - lo > 2
        if not open_.any():
            break
        m1 = lo + (hi - lo) // 3
        m2 = hi - (hi - lo) // 3
        left = excess(m1) <= excess(m2)
        hi = np.where(open_ & left, m2, hi)
        lo = np.where(open_ & ~left, m1, lo)
    best, best_e = lo.copy(), excess(lo)
    for off in (1, 2):
        m = np.minimum(lo + off, hi)
        e = excess(m)
        best = np.where(e < best_e, m, best)
        best_e = np.minimum(e, best_e)
    return best


def _best_offset(t: np.ndarray, v: np.ndarray, M: int) -> int:
    """The C meeting the most threshold conditions of one column: condition k holds for C
    in [d_k, d_k + M - 1]; the best C is one of the interval ends."""
    ks = np.arange(-126, 128, dtype=np.int64)[v]
    d = (ks << 32) - t[v] * M
    ends = np.concatenate([d, d + M - 1])
    cover = ((ends[:, None] >= d[None, :]) & (ends[:, None] <= d[None, :] + M - 1)).sum(axis=1)
    return int(ends[np.argmax(cover)])


def int8_lines(scale: np.ndarray, steps: Sequence, f16: bool, xs: float, k_real: int) -> Optional[np.ndarray]:
    """Lines (LINE_DTYPE, one per column) for an int8-only epilogue: with the kernels' flag
    window they reproduce its int8 output exactly for every accumulator in
    [-k_real * 127^2, k_real * 127^2].  None if the epilogue is not a non-decreasing
    per-column function or a line does not fit the kernels' integer ranges.

    scale: float64 [C], the combined dequant scale per column; steps: (fn, operand or None,
    swapped) with operands float32 of shape [C] (per column) or () (scalar); xs: the
    float32 scale of the int8 output."""
    scale = np.asarray(scale, np.float64)
    C = scale.shape[0]
    A = int(min(k_real * 127 * 127, (1 << 31) - 1))
    xs = np.float32(xs)
    cols = []
    for fn, o, sw in steps:
        if fn == "relu":
            cols.append((fn, None, False))
            continue
        o = np.asarray(o, np.float32)
        cols.append((fn, np.broadcast_to(o.reshape(-1) if o.size > 1 else o.reshape(1), (C,)).reshape(C, 1), bool(sw)))
    if not _monotone(cols) or not np.all(np.isfinite(scale)) or np.any(scale <= 0):
        return None
    if not (np.isfinite(xs) and xs > 0) or A * float(scale.max()) > 1e38:
        return None
    lo, hi, t = _thresholds(scale, cols, f16, xs, A)
    ks = np.arange(-126, 128, dtype=np.int64)
    valid = (ks[None, :] > lo[:, None]) & (ks[None, :] <= hi[:, None])
    M = _best_slope(t, valid)
    out = np.zeros(C, LINE_DTYPE)
    for c in range(C):
        v = valid[c]
        if not v.any():                      # constant column
            out[c] = (int(lo[c]) << 32, 0, 0, lo[c], hi[c], 0)
            continue
        m = int(M[c])
        cc = _best_offset(t[c], v, m)
        if m <= 0 or abs(cc) >= 1 << 62:
            return None
        # the line's thresholds t'_k = ceil((k * 2^32 - C) / M), and the accumulators
        # between t_k and t'_k, where the line and the chain disagree
        tp = -((cc - (ks[v] << 32)) // m)
        tk = t[c][v]
        a0 = np.clip(np.minimum(tk, tp), -A, A + 1)
        a1 = np.clip(np.maximum(tk, tp), -A, A + 1)
        n = int((a1 - a0).sum())
        if n > MAX_MISMATCH:
            return None
        h = 0
        if n:
            bad = np.concatenate([np.arange(x, y, dtype=np.int64) for x, y in zip(a0, a1) if y > x])
            low = (bad * m + cc) & 0xFFFFFFFF
            h = int(np.minimum(low, (1 << 32) - low).max()) + 1
            if 2 * h > MAX_WINDOW:
                return None
        out[c] = (cc + h, m, 2 * h, lo[c], hi[c], 0)
    if out["w"].astype(np.float64).mean() > MAX_MEAN_WINDOW:
        return None
    return out


def line_q(lines: np.ndarray, acc: np.ndarray) -> tuple:
    """What the kernels compute from the lines for accumulators acc[c, j] (int64): the
    clamped line value, and where the float chain replaces it."""
    r = acc * lines["m"].astype(np.int64)[:, None] + lines["c"][:, None]
    q = np.clip(r >> 32, lines["lo"].astype(np.int64)[:, None], lines["hi"].astype(np.int64)[:, None])
    flag = (r & 0xFFFFFFFF) < lines["w"].astype(np.int64)[:, None]
    return q, flag
