"""Integer requantization lines (mira_amd.requant) against the oracle's float chain.

The kernels take, for an int8-only epilogue, clamp((acc * m + c) >> 32, lo, hi) unless the
low word of acc * m + c is below the line's window w, where they evaluate the float chain.
These tests emulate exactly that and compare it with the oracle's dequant -> epilogue ->
quantize (oracle/golden.py, following mira/ops.py:602-603, 616-620, 192-199) at every
accumulator next to every threshold, at random accumulators and at the range ends.
"""
import numpy as np
import pytest

from mira_amd import requant
from oracle import golden as G


def _oracle_q(acc, scale, steps, f16, xs):
    """int8 result of the oracle's chain for acc[c, j] of column c."""
    y = (acc.astype(np.float64) * scale[:, None]).astype(np.float32)
    operands = [None]
    tuples = []
    for fn, o, sw in steps:
        if o is None:
            tuples.append((fn, None, sw))
        else:
            operands.append(np.asarray(o, np.float32).reshape(-1, 1) if np.ndim(o) else np.float32(o))
            tuples.append((fn, len(operands) - 1, sw))
    y = G.epilogue_ref(y, operands, tuple(tuples))
    if f16:
        y = y.astype(np.float16)
    q = G.quantize_activation(y.astype(np.float32), xs)
    return np.where(np.isnan(q), -127, q).astype(np.int64)


def _emulated(lines, acc, scale, steps, f16, xs):
    q, flag = requant.line_q(lines, acc)
    return np.where(flag, _oracle_q(acc, scale, steps, f16, xs), q), flag


def _probe_accs(lines, scale, steps, f16, xs, k_real, rng):
    """Accumulators at each threshold (from the oracle chain by bisection) +- 3, random ones
    of the whole range and of a typical range, and the range ends."""
    A = k_real * 127 * 127
    C = scale.size
    ks = np.arange(-126, 128)
    lo_ = np.full((C, ks.size), -A, np.int64)
    hi_ = np.full((C, ks.size), A + 1, np.int64)
    while (lo_ < hi_).any():
        mid = (lo_ + hi_) // 2
        ok = _oracle_q(np.clip(mid, -A, A), scale, steps, f16, xs) >= ks[None, :]
        hi_ = np.where((lo_ < hi_) & ok, mid, hi_)
        lo_ = np.where((lo_ < hi_) & ~ok, mid + 1, lo_)
    near = np.clip(lo_[:, :, None] + np.arange(-3, 4)[None, None, :], -A, A).reshape(C, -1)
    wide = rng.integers(-A, A + 1, (C, 3000))
    typical = rng.integers(-min(A, 200_000), min(A, 200_000) + 1, (C, 3000))
    ends = np.array([[-A, -A + 1, -1, 0, 1, A - 1, A]] * C, np.int64)
    return np.concatenate([near, wide, typical, ends], axis=1)


CASES = [
    # (fn steps, f16, columns, k_real, scale spread, bias spread)
    ("bias_relu", False, 64, 576, 1.0, 1.0),
    ("bias_relu", False, 96, 4608, 1.0, 3.0),
    ("bias", False, 80, 960, 1.0, 8.0),
    ("bias_relu6", False, 48, 144, 1.0, 1.0),
    ("bias_relu", True, 64, 1152, 1.0, 1.0),
    ("bias", True, 40, 64, 1.0, 1.0),
    ("bounds", False, 32, 300, 1.0, 1.0),
]


@pytest.mark.parametrize("kind,f16,C,k_real,sspread,bspread", CASES)
def test_lines_equal_the_oracle_chain(kind, f16, C, k_real, sspread, bspread):
    rng = np.random.default_rng(C * 31 + k_real)
    xs_in = np.float32(rng.uniform(0.005, 0.05))
    ws = (rng.uniform(0.2, 1.0, C) * sspread / 127 * 0.05).astype(np.float32)
    scale = np.float64(xs_in) * ws.astype(np.float64)
    bias = (rng.standard_normal(C) * bspread).astype(np.float32)
    if f16:
        bias = bias.astype(np.float16).astype(np.float32)
    if kind == "bias_relu":
        steps = [("add", bias, False), ("relu", None, False)]
    elif kind == "bias":
        steps = [("add", bias, False)]
    elif kind == "bias_relu6":
        steps = [("add", bias, False), ("maximum", np.float32(0), False), ("minimum", np.float32(6), False)]
    else:
        steps = [("maximum", np.float32(-0.75), False), ("minimum", np.float32(2.5), False)]
    # the next op's scale: the peak / 127 of results whose accumulators reach K * 20 * 20
    # (int8 activations and weights of typical magnitude 20)
    peak = float(np.abs(np.float64(k_real * 20 * 20) * scale).max())
    xs = np.float32(max(peak, 1e-3) / 127 * rng.uniform(0.3, 1.0))
    lines = requant.int8_lines(scale, steps, f16, xs, k_real)
    if f16 and lines is None:
        # f16 results round to f16 before the quantizer: its half-ulp (2^-12 relative) moves
        # the thresholds by tens of accumulators off any line, too many to window; the
        # float chain then runs (None is the documented answer)
        return
    assert lines is not None
    acc = _probe_accs(lines, scale, steps, f16, xs, k_real, rng)
    got, flag = _emulated(lines, acc, scale, steps, f16, xs)
    want = _oracle_q(acc, scale, steps, f16, xs)
    assert np.array_equal(got, want)
    # the window is small: the float chain runs for a tiny share of random accumulators
    A = k_real * 127 * 127
    _, rflag = requant.line_q(lines, rng.integers(-A, A + 1, (C, 20000)))
    assert rflag.mean() < 1e-3


def test_lines_have_windows_where_rounding_bends_the_thresholds():
    """Wide-range columns (K = 4608) put some thresholds off every straight line; those
    columns get a window, and the accumulators inside it are the ones the line misses."""
    rng = np.random.default_rng(5)
    C, k_real = 128, 4608
    scale = np.float64(0.02) * (rng.uniform(0.2, 1.0, C) / 127 * 0.05)
    bias = rng.standard_normal(C).astype(np.float32)
    steps = [("add", bias, False), ("relu", None, False)]
    xs = np.float32(0.05)
    lines = requant.int8_lines(scale, steps, False, xs, k_real)
    assert (lines["w"] > 0).any()
    acc = _probe_accs(lines, scale, steps, False, xs, k_real, rng)
    q, flag = requant.line_q(lines, acc)
    want = _oracle_q(acc, scale, steps, False, xs)
    missed = q != want
    assert missed.any() and not (missed & ~flag).any()


def test_constant_and_rejected_epilogues():
    scale = np.array([1e-4, 2e-4, 3e-4])
    # a bias far past the int8 range: constant columns (q = 127 or 0 for any accumulator)
    lines = requant.int8_lines(scale, [("add", np.float32([1e6, -1e6, 0.5]), False), ("relu", None, False)],
                               False, np.float32(0.01), 64)
    assert list(lines["m"][:2]) == [0, 0] and list(lines["lo"][:2]) == [127, 0] and lines["m"][2] > 0
    acc = np.array([[-520000, 0, 520000]] * 3, np.int64)
    q, flag = requant.line_q(lines, acc)
    assert list(q[0]) == [127] * 3 and list(q[1]) == [0] * 3 and not flag[:2].any()
    # steps that are not non-decreasing in the accumulator, or non-finite operands
    bad = [[("sub", np.float32(1), True)], [("mul", np.float32([1, -1, 1]), False)],
           [("div", np.float32(2), True)], [("add", np.float32([1, np.nan, 1]), False)],
           [("gelu", None, False)]]
    for steps in bad:
        assert requant.int8_lines(scale, steps, False, np.float32(0.01), 64) is None
    # a positive per-column multiply and a division by a positive constant are fine
    ok = [("mul", np.float32([0.5, 2, 0]), False), ("div", np.float32(3), False), ("add", np.float32(0.25), False)]
    lines = requant.int8_lines(scale, ok, False, np.float32(0.01), 64)
    rng = np.random.default_rng(2)
    acc = rng.integers(-64 * 127 * 127, 64 * 127 * 127, (3, 5000))
    got, _ = _emulated(lines, acc, scale, ok, False, np.float32(0.01))
    assert np.array_equal(got, _oracle_q(acc, scale, ok, False, np.float32(0.01)))


def test_line_layout_matches_the_c_struct():
    """mr_requant_line: int64 c, int32 m, uint32 w, int32 lo, int32 hi, 8 reserved bytes."""
    d = requant.LINE_DTYPE
    assert d.itemsize == 32
    assert [d.fields[f][1] for f in ("c", "m", "w", "lo", "hi")] == [0, 8, 12, 16, 20]


def test_lines_are_exact_or_absent_for_extreme_slopes():
    """A very small slope (one int8 step per ~10^5 accumulators) or a very large one is
    past the fixed-point line's precision or range: int8_lines then returns None (the
    float chain runs), and whatever it returns is exact."""
    rng = np.random.default_rng(11)
    for gain in (1e-6, 1e-5, 0.3, 3.0):
        C, k_real = 16, 4608
        scale = np.full(C, 1e-4) * rng.uniform(0.5, 1.0, C)
        steps = [("add", rng.standard_normal(C).astype(np.float32), False), ("relu", None, False)]
        xs = np.float32(float(scale.max()) / gain)
        lines = requant.int8_lines(scale, steps, False, xs, k_real)
        if lines is None:
            continue
        acc = _probe_accs(lines, scale, steps, False, xs, k_real, rng)
        got, _ = _emulated(lines, acc, scale, steps, False, xs)
        assert np.array_equal(got, _oracle_q(acc, scale, steps, False, xs))
