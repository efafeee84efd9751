"""Pin the oracle (oracle/golden.py) before the GPU parity tests compare against it.

The reference ships no golden vectors or known-answer tests for W8A8
(its only W8A8 tests are tolerance tests, tests/test_control_dynamic_quant.py:
192-236), so each function is pinned by its own invariant, by brute force on
tiny inputs, or by exact arithmetic:

  quantize_array       reference invariant |q*s - w| <= max(s)/2 (:192-197), amax -> +-127,
                       zero channel -> scale 1, half-even ties, axis brute force
  quantize_activation  exact rational division (fractions.Fraction) + half-even + clip
  qmatmul              Python-int dot products, Python-float dequant in the reference's order
  qconv2d              7-loop integer convolution (stride, padding, dilation), 2**24 certificate
  depthwise conv2d     scalar float32 tap loop in (i, j) order
  maxpool2d / pad      window brute force / closed form
  reduce_mean          NumPy's pairwise summation restated in scalar float32
  layernorm            scalar restatement (pairwise means, f64 divide, f32 steps); closed forms
  softmax              equal logits -> fl32(1/n), [0, ln 3] -> [1/4, 3/4], no overflow
  gelu/sigmoid/tanh    float64 closed forms, tanh-form gelu(1) = 0.8411920
  transpose / concat   index brute force
  epilogue_ref         operand order of every binary step, including swapped
  calibrate / attrs    hand-computed peaks on a two-layer graph
"""
from fractions import Fraction

import numpy as np
import pytest

from oracle import golden as G


def f32_round(fr: Fraction) -> np.float32:
    """Correctly rounded (half-even) float32 of an exact rational."""
    a = np.float32(float(fr))                  # within an ulp; fix up against the exact value
    best = a
    for cand in (np.nextafter(a, np.float32(-np.inf)), a, np.nextafter(a, np.float32(np.inf))):
        d, db = abs(Fraction(float(cand)) - fr), abs(Fraction(float(best)) - fr)
        if d < db or (d == db and int(np.float32(cand).view(np.int32)) % 2 == 0):
            best = cand
    return np.float32(best)


def round_half_even(fr: Fraction) -> int:
    fl = fr.numerator // fr.denominator
    rem = fr - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        return fl + 1
    return fl


# ---------------------------------------------------------------- quantize_array

def test_quantize_array_reference_invariant():
    w = np.random.default_rng(0).standard_normal((64, 32)).astype(np.float32)
    q, scale = G.quantize_array(w, axis=1)
    assert q.dtype == np.int8 and scale.shape == (32,)
    assert np.abs(q * scale - w).max() <= scale.max() / 2 + 1e-6


def test_quantize_array_axis_and_extremes_brute_force():
    rng = np.random.default_rng(1)
    w = rng.standard_normal((5, 3, 2, 2)).astype(np.float32)
    w[2] = 0.0                                                     # all-zero output channel
    q, scale = G.quantize_array(w, axis=0)
    for o in range(5):
        amax = max(abs(float(v)) for v in w[o].ravel())
        want = np.float32(amax / 127.0) if amax > 0 else np.float32(1.0)
        assert scale[o] == want
        if amax > 0:
            i = int(np.argmax(np.abs(w[o])))
            assert abs(int(q[o].ravel()[i])) == 127
        else:
            assert not q[o].any()


def test_quantize_array_half_even_ties():
    w = np.array([[0.5], [1.5], [2.5], [-0.5], [-2.5], [127.0]], np.float32)   # amax 127 -> scale 1
    q, scale = G.quantize_array(w, axis=1)
    assert scale[0] == 1.0
    assert q.ravel().tolist() == [0, 2, 2, 0, -2, 127]


# ---------------------------------------------------------------- quantize_activation

def _quant_exact(x: np.float32, s: float) -> int:
    s32 = np.float32(s)
    r = round_half_even(Fraction(float(f32_round(Fraction(float(x)) / Fraction(float(s32))))))
    return max(-127, min(127, r))


def test_quantize_activation_is_correctly_rounded_division():
    rng = np.random.default_rng(2)
    xs = (rng.standard_normal(3000) * 40).astype(np.float32)
    for s in (0.0371, 1 / 3, 0.7, 1.0):
        got = G.quantize_activation(xs, s)
        want = np.array([_quant_exact(x, s) for x in xs], np.float64)
        assert np.array_equal(got, want), s


def test_quantize_activation_reciprocal_would_differ():
    """A reciprocal-multiply quantizer disagrees somewhere on these inputs; the oracle must not."""
    rng = np.random.default_rng(3)
    s = np.float32(0.0371)
    xs = (rng.uniform(-4.7, 4.7, 200000)).astype(np.float32)
    recip = np.clip(np.round(xs * (np.float32(1) / s)), -127, 127)
    div = G.quantize_activation(xs, float(s))
    assert (recip != div).any()
    bad = np.nonzero(recip != div)[0][:50]
    assert all(div[i] == _quant_exact(xs[i], float(s)) for i in bad)


def test_quantize_activation_ties_and_clamps():
    x = np.array([0.5, 1.5, 2.5, -0.5, -1.5, 126.5, 127.5, 128.0, -500.0, 1e30, -1e30], np.float32)
    assert G.quantize_activation(x, 1.0).tolist() == [0, 2, 2, -0.0, -2, 126, 127, 127, -127, 127, -127]


def test_x_scale_is_rounded_to_f32_first():
    x = np.array([1.0], np.float32)
    s = 0.1 + 1e-12                     # differs from float32(0.1) only below f32 precision
    assert G.quantize_activation(x, s)[0] == G.quantize_activation(x, float(np.float32(s)))[0]


# ---------------------------------------------------------------- qmatmul

def test_qmatmul_brute_force():
    rng = np.random.default_rng(4)
    M, K, N = 3, 7, 5
    x = rng.standard_normal((M, K)).astype(np.float32)
    q = rng.integers(-127, 128, (K, N)).astype(np.int8)
    ws = rng.uniform(0.001, 0.05, N).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    xs = 0.021
    attrs = {"q": q, "w_scale": ws, "x_scale": xs, "dtype": "f32", "epilogue": (("add", 1, False), ("relu", None, False))}
    y = G.qmatmul([x, b], attrs)
    xq = [[_quant_exact(x[i, k], xs) for k in range(K)] for i in range(M)]
    for i in range(M):
        for j in range(N):
            acc = sum(xq[i][k] * int(q[k, j]) for k in range(K))
            v = np.float32(float(acc) * (float(xs) * float(ws[j])))
            v = np.float32(v + b[j])
            v = max(v, np.float32(0))
            assert y[i, j] == v
    assert np.array_equal(G.qmatmul_acc(x, attrs),
                          np.array([[sum(xq[i][k] * int(q[k, j]) for k in range(K)) for j in range(N)]
                                    for i in range(M)]))


def test_dequant_precision_matters():
    """Dequantizing in float32 instead of float64 (mira/ops.py:618) changes results on
    these values, so the brute-force check above would catch it."""
    rng = np.random.default_rng(5)
    acc = rng.integers(-2000000, 2000000, 5000)
    xs, ws = 0.0123456789, rng.uniform(0.001, 0.05, 5000).astype(np.float32)
    a = (acc.astype(np.float64) * (np.float64(xs) * ws.astype(np.float64))).astype(np.float32)
    b = acc.astype(np.float32) * (np.float32(xs) * ws)
    assert (a != b).any()
    x = rng.standard_normal((5000, 1)).astype(np.float32)
    attrs = {"q": np.ones((1, 1), np.int8), "w_scale": ws[:1], "x_scale": xs, "dtype": "f32"}
    y = G.qmatmul([x], attrs)
    acc1 = G.qmatmul_acc(x, attrs)
    assert np.array_equal(y, (acc1.astype(np.float64) * (np.float64(xs) * np.float64(ws[0]))).astype(np.float32))


# ---------------------------------------------------------------- qconv2d

def _int_conv(xq, q, stride, pad, dil):
    n, c, h, w = xq.shape
    o, _, kh, kw = q.shape
    oh = (h + 2 * pad[0] - dil[0] * (kh - 1) - 1) // stride[0] + 1
    ow = (w + 2 * pad[1] - dil[1] * (kw - 1) - 1) // stride[1] + 1
    out = np.zeros((n, o, oh, ow), np.int64)
    for b in range(n):
        for oc in range(o):
            for y in range(oh):
                for x in range(ow):
                    s = 0
                    for ic in range(c):
                        for i in range(kh):
                            for j in range(kw):
                                iy, ix = y * stride[0] - pad[0] + i * dil[0], x * stride[1] - pad[1] + j * dil[1]
                                if 0 <= iy < h and 0 <= ix < w:
                                    s += int(xq[b, ic, iy, ix]) * int(q[oc, ic, i, j])
                    out[b, oc, y, x] = s
    return out


@pytest.mark.parametrize("stride,pad,dil", [((1, 1), (1, 1), (1, 1)), ((2, 2), (1, 0), (1, 1)),
                                            ((1, 2), (2, 2), (2, 1))])
def test_qconv2d_brute_force(stride, pad, dil):
    rng = np.random.default_rng(6)
    x = rng.standard_normal((2, 3, 6, 7)).astype(np.float32)
    q = rng.integers(-127, 128, (4, 3, 3, 3)).astype(np.int8)
    ws = rng.uniform(0.001, 0.05, 4).astype(np.float32)
    xs = 0.03
    attrs = {"q": q, "w_scale": ws, "x_scale": xs, "dtype": "f32", "stride": stride, "padding": pad,
             "dilation": dil}
    xq = np.vectorize(lambda v: _quant_exact(np.float32(v), xs))(x)
    want_acc = _int_conv(xq, q, stride, pad, dil)
    assert np.array_equal(G.qconv2d_acc(x, attrs), want_acc.astype(np.float64))
    y = G.qconv2d([x], attrs)
    for oc in range(4):
        exp = np.array([np.float32(float(a) * (float(xs) * float(ws[oc]))) for a in want_acc[:, oc].ravel()])
        assert np.array_equal(y[:, oc].ravel(), exp)
    assert G.qconv2d_certificate(x, attrs) < 2 ** 24


def test_qconv2d_certificate_closed_form():
    x = np.full((1, 64, 5, 5), 10.0, np.float32)
    q = np.full((2, 64, 3, 3), 127, np.int8)
    attrs = {"q": q, "w_scale": np.ones(2, np.float32), "x_scale": 10.0 / 127, "dtype": "f32",
             "stride": (1, 1), "padding": (0, 0)}
    assert G.qconv2d_certificate(x, attrs) == 64 * 9 * 127 * 127


# ---------------------------------------------------------------- float ops

def test_depthwise_conv_is_tap_ordered_f32():
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((2, 5, 6, 6)) * 3).astype(np.float32)
    w = rng.standard_normal((5, 1, 3, 3)).astype(np.float32)
    a = {"stride": (2, 2), "padding": (1, 1), "groups": 5}
    y = G.conv2d([x, w], a)
    n, c, h, wd = x.shape
    oh = ow = 3
    for b in range(n):
        for ch in range(c):
            for oy in range(oh):
                for ox in range(ow):
                    acc = np.float32(0)
                    for i in range(3):
                        for j in range(3):
                            iy, ix = oy * 2 - 1 + i, ox * 2 - 1 + j
                            xv = x[b, ch, iy, ix] if 0 <= iy < h and 0 <= ix < wd else np.float32(0)
                            acc = np.float32(acc + np.float32(xv * w[ch, 0, i, j]))
                    assert y[b, ch, oy, ox] == acc


def test_maxpool_and_pad():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((2, 3, 7, 7)).astype(np.float32)
    p = G.pad([x], {"pads": ((0, 0), (0, 0), (1, 1), (1, 1)), "value": -np.inf})
    assert p.shape == (2, 3, 9, 9) and np.isneginf(p[:, :, 0]).all() and np.array_equal(p[:, :, 1:8, 1:8], x)
    y = G.maxpool2d([p], {"size": 3, "stride": 2})
    for b in range(2):
        for c in range(3):
            for i in range(4):
                for j in range(4):
                    assert y[b, c, i, j] == max(p[b, c, 2 * i + di, 2 * j + dj] for di in range(3) for dj in range(3))


def pairwise_f32(vals) -> np.float32:
    """NumPy's float32 pairwise sum (numpy/_core/src/umath/loops_utils.h.src), scalar restatement."""
    n = len(vals)
    if n < 8:
        r = np.float32(-0.0)
        for v in vals:
            r = np.float32(r + v)
        return r
    if n <= 128:
        r = [np.float32(v) for v in vals[:8]]
        i = 8
        while i < n - n % 8:
            for j in range(8):
                r[j] = np.float32(r[j] + vals[i + j])
            i += 8
        res = np.float32(np.float32(np.float32(r[0] + r[1]) + np.float32(r[2] + r[3]))
                         + np.float32(np.float32(r[4] + r[5]) + np.float32(r[6] + r[7])))
        for k in range(i, n):
            res = np.float32(res + vals[k])
        return res
    n2 = n // 2
    n2 -= n2 % 8
    return np.float32(pairwise_f32(vals[:n2]) + pairwise_f32(vals[n2:]))


@pytest.mark.parametrize("hw", [(1, 7), (7, 7), (8, 8), (14, 14), (56, 56)])
def test_reduce_mean_is_pairwise_then_f64_divide(hw):
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((2, 3) + hw) * 5).astype(np.float32)
    y = G.reduce("reduce_mean", [x], {"axes": (2, 3), "keepdims": True})
    n = hw[0] * hw[1]
    for b in range(2):
        for c in range(3):
            s = pairwise_f32(x[b, c].ravel().tolist())
            assert y[b, c, 0, 0] == np.float32(np.float64(s) / np.float64(n))


def _layernorm_scalar(x, g, b, eps) -> np.ndarray:
    """mira/ops.py:356-360 restated element by element: each mean is the pairwise sum seeded
    with +0, divided by the count in float64 (NumPy's mean divides by an intp count), and every
    other step is one float32 operation."""
    n = len(x)
    mu = np.float32(np.float64(np.float32(np.float32(0) + pairwise_f32(x))) / np.float64(n))
    sq = [np.float32(np.float32(v - mu) * np.float32(v - mu)) for v in x]
    var = np.float32(np.float64(np.float32(np.float32(0) + pairwise_f32(sq))) / np.float64(n))
    sd = np.sqrt(np.float32(var + np.float32(eps)))
    return np.array([np.float32(np.float32(np.float32(np.float32(v - mu) / sd) * gi) + bi)
                     for v, gi, bi in zip(x, g, b)], np.float32)


@pytest.mark.parametrize("d", [1, 3, 7, 8, 9, 64, 100, 128, 129, 300, 1029])
def test_layernorm_is_pairwise_mean_and_f32_steps(d):
    rng = np.random.default_rng(d)
    x = (rng.standard_normal((3, d)) * rng.uniform(0.1, 50) + rng.uniform(-20, 20)).astype(np.float32)
    g = rng.standard_normal(d).astype(np.float32)
    b = rng.standard_normal(d).astype(np.float32)
    y = G.layernorm([x, g, b], {"eps": 1e-5})
    for r in range(3):
        assert np.array_equal(y[r].view(np.uint32), _layernorm_scalar(x[r].tolist(), g, b, 1e-5).view(np.uint32))


def test_layernorm_closed_forms():
    g = np.float32([1.5, -2.0])
    b = np.float32([0.25, 3.0])
    # constant rows: x - mu == 0, so y == 0 * g + b == b exactly
    assert np.array_equal(G.layernorm([np.full((2, 2), 7.25, np.float32), g, b], {"eps": 1e-5}), np.stack([b, b]))
    # [a, -a]: mu = 0, var = a^2, y = +-a / sqrt(a^2 + eps) * g + b, which is +-g + b for large a
    y = G.layernorm([np.float32([[1000.0, -1000.0]]), g, b], {"eps": 1e-5})
    assert np.array_equal(y, np.float32([[1.75, 5.0]]))
    # biased variance (ddof 0): with g = 1, b = 0, eps = 0 the rows have mean 0 and mean square 1
    x = np.random.default_rng(1).standard_normal((4, 8)).astype(np.float32)
    y = G.layernorm([x, np.ones(8, np.float32), np.zeros(8, np.float32)], {"eps": 0.0}).astype(np.float64)
    assert np.abs(y.mean(axis=1)).max() < 1e-6 and np.abs((y ** 2).mean(axis=1) - 1).max() < 1e-5


def test_softmax_closed_forms():
    # equal logits: exp(0) = 1 each, so every probability is fl32(1 / n)
    for n in (1, 3, 273):
        assert np.array_equal(G.softmax([np.full((2, n), -4.5, np.float32)], {"axis": -1}),
                              np.full((2, n), np.float32(1) / np.float32(n), np.float32))
    # [0, d] -> [1, e^d] / (1 + e^d); the max is subtracted first, so large logits do not
    # overflow (d = 1.0986328125 ~ ln 3 is a multiple of 2^-10, so 1000 + d is exact in f32)
    d = 1.0986328125
    y = G.softmax([np.float32([[0.0, d], [1000.0, 1000.0 + d]])], {"axis": -1})
    assert np.abs(y - np.array([1.0, np.exp(d)]) / (1 + np.exp(d))).max() < 1e-6
    # the axis attribute selects the reduced axis
    x = np.random.default_rng(2).standard_normal((3, 5)).astype(np.float32)
    assert np.abs(G.softmax([x], {"axis": 0}).sum(axis=0) - 1).max() < 1e-6


def test_libm_unary_closed_forms():
    """gelu is the tanh form 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) (mira/ops.py:94-96)."""
    x = np.float32([0.0, 1.0, -1.0, 6.0, -6.0])
    gelu = G.unary("gelu", x).astype(np.float64)
    want = [0.5 * v * (1 + np.tanh(np.sqrt(2 / np.pi) * (v + 0.044715 * v ** 3))) for v in x.astype(np.float64)]
    assert np.abs(gelu - want).max() < 1e-6
    assert abs(gelu[1] - 0.8411920) < 1e-6                  # the tanh form at 1 (the erf form gives 0.8413447)
    assert np.array_equal(G.unary("sigmoid", np.float32([0.0])), np.float32([0.5]))
    assert np.array_equal(G.unary("tanh", np.float32([0.0, 20.0])), np.float32([0.0, 1.0]))


def test_transpose_and_concat_brute_force():
    x = np.arange(2 * 3 * 4 * 5, dtype=np.float32).reshape(2, 3, 4, 5)
    y = G.evaluate("transpose", [x], {"perm": (0, 2, 3, 1)})
    assert y.shape == (2, 4, 5, 3) and y.flags.c_contiguous
    for a, b_, c, d in np.ndindex(*y.shape):
        assert y[a, b_, c, d] == x[a, d, b_, c]
    p, q = x[:, :2], x[:, 2:] * -1
    z = G.evaluate("concat", [p, q], {"axis": 1})
    assert z.shape == x.shape
    for a, b_, c, d in np.ndindex(*z.shape):
        assert z[a, b_, c, d] == (x[a, b_, c, d] if b_ < 2 else -x[a, b_, c, d])


def test_slice_where_broadcast_gather_brute_force():
    """Element by element against index arithmetic written out: slice reads x[i + begin];
    where takes a where cond != 0 (negative and fractional conditions count as true) in a's
    dtype, broadcasting all three; broadcast repeats along the size-1 and new leading axes;
    gather takes rows of the table by i32 index along its axis, index shape in place."""
    x = np.arange(3 * 4 * 5, dtype=np.float32).reshape(3, 4, 5) - 7
    y = G.evaluate("slice", [x], {"begin": (1, 0, 2), "size": (2, 3, 3)})
    assert y.shape == (2, 3, 3)
    for i, j, k in np.ndindex(*y.shape):
        assert y[i, j, k] == x[i + 1, j, k + 2]
    cond = np.array([[0.0], [-0.5], [2.0]], np.float32)
    a = np.arange(3 * 4, dtype=np.int32).reshape(3, 4)
    b = np.int32(-1) * np.ones((1, 4), np.int32)
    w = G.evaluate("where", [cond, a, b], {})
    assert w.dtype == np.int32 and w.shape == (3, 4)
    for i, j in np.ndindex(3, 4):
        assert w[i, j] == (a[i, j] if cond[i, 0] != 0 else -1)
    r = G.evaluate("broadcast", [np.array([[1.0], [2.0]], np.float32)], {"shape": (3, 2, 4)})
    for i, j, k in np.ndindex(3, 2, 4):
        assert r[i, j, k] == j + 1
    idx = np.array([[2, 0], [1, 2]], np.int32)
    g = G.evaluate("gather", [x, idx], {"axis": 1})
    assert g.shape == (3, 2, 2, 5)
    for i, p, q, k in np.ndindex(*g.shape):
        assert g[i, p, q, k] == x[i, idx[p, q], k]
    # sort: ascending along its axis, the same multiset per row; cumprod: running f32
    # products left to right; argmax / argmin: the first index of the extreme value
    rows = np.array([[3.0, -1.0, 2.0, -1.0], [0.5, 4.0, 4.0, 0.25]], np.float32)
    srt = G.evaluate("sort", [rows], {"axis": 1})
    cum = G.evaluate("cumprod", [rows], {"axis": 1})
    for i in range(2):
        assert list(srt[i]) == sorted(rows[i].tolist())
        run = np.float32(1)
        for j in range(4):
            run = np.float32(run * rows[i, j])
            assert cum[i, j] == run
    am = G.evaluate("argmax", [rows], {"axis": 1, "keepdims": False})
    an = G.evaluate("argmin", [rows], {"axis": 1, "keepdims": True})
    assert am.dtype == np.int32 and list(am) == [0, 1] and an.shape == (2, 1) and list(an[:, 0]) == [1, 3]
    cmp = {"greater": lambda u, v: u > v, "greater_equal": lambda u, v: u >= v, "equal": lambda u, v: u == v}
    u = np.array([1, 2, 3], np.int32)
    v = np.array([[2], [3]], np.int32)
    for kind, f in cmp.items():
        m = G.evaluate(kind, [u, v], {})
        assert m.dtype == np.int32
        for i, j in np.ndindex(2, 3):
            assert m[i, j] == (1 if f(u[j], v[i, 0]) else 0)


@pytest.mark.parametrize("ashape,wshape", [((5, 7), (7, 3)), ((2, 3, 1, 64), (2, 3, 64, 273)),
                                           ((4, 1, 8, 32), (1, 3, 32, 16)), ((1, 1), (1, 1)), ((9, 300), (300, 2))])
def test_f32_matmul_within_its_rounding_bound(ashape, wshape):
    """oracle.matmul (mira/ops.py:217-219, NumPy/BLAS f32 order) against a float64 brute force
    of the same broadcast product, written as explicit loops over the batch and the output:
    every element within K * 2^-24 * (|a| @ |w|) plus one f32 ulp of the result, the bound
    for any summation order of K products in f32; a dropped term, a wrong operand index or a
    transposed operand misses it by far."""
    rng = np.random.default_rng(sum(ashape) + sum(wshape))
    a = rng.standard_normal(ashape).astype(np.float32)
    w = rng.standard_normal(wshape).astype(np.float32)
    got = G.matmul([a, w], {})
    K = ashape[-1]
    bshape = np.broadcast_shapes(ashape[:-2], wshape[:-2])
    ab = np.broadcast_to(a, bshape + ashape[-2:]).astype(np.float64)
    wb = np.broadcast_to(w, bshape + wshape[-2:]).astype(np.float64)
    want = np.zeros(bshape + (ashape[-2], wshape[-1]))
    mag = np.zeros_like(want)
    for idx in np.ndindex(*bshape) if bshape else [()]:
        for m in range(ashape[-2]):
            for n in range(wshape[-1]):
                terms = ab[idx + (m,)] * wb[idx + (slice(None), n)]
                want[idx + (m, n)] = terms.sum()
                mag[idx + (m, n)] = np.abs(terms).sum()
    assert got.shape == want.shape and got.dtype == np.float32
    bound = K * 2.0 ** -24 * mag + np.spacing(np.abs(got).astype(np.float32)).astype(np.float64)
    assert (np.abs(got.astype(np.float64) - want) <= bound).all()
    # the bound is not vacuous: the same product with its last K term dropped misses it
    if K > 1:
        dropped = np.matmul(a[..., :-1], w[..., :-1, :]).astype(np.float64)
        assert (np.abs(dropped - want) > bound).any()


def test_epilogue_operand_order():
    acc = np.array([5.0, -3.0], np.float32)
    other = np.array([2.0, 4.0], np.float32)
    for fn, want, want_sw in (("sub", [3, -7], [-3, 7]), ("div", [2.5, -0.75], [0.4, 4 / -3]),
                              ("maximum", [5, 4], [5, 4]), ("minimum", [2, -3], [2, -3])):
        assert np.array_equal(G.epilogue_ref(acc, [None, other], ((fn, 1, False),)), np.float32(want))
        assert np.array_equal(G.epilogue_ref(acc, [None, other], ((fn, 1, True),)), np.float32(want_sw))
    assert np.array_equal(G.epilogue_ref(np.float32([-1, 2]), [], (("relu", None, False),)), np.float32([0, 2]))


# ---------------------------------------------------------------- calibration and rewrite

def test_calibration_peaks_and_attrs():
    from harness.graph import Graph
    g = Graph("t")
    x = g.input("x", (4, 3))
    w1 = np.array([[1, -2], [0.5, 1], [-1, 0]], np.float32)
    w2 = np.array([[2], [-1]], np.float32)
    h = g.op("relu", [g.op("matmul", [x, g.const(w1)])])
    y = g.op("matmul", [h, g.const(w2)])
    g.outputs = [y]
    feeds = [{"x": np.array([[1, 2, 3]] * 4, np.float32)}, {"x": np.array([[-4, 0, 1]] * 4, np.float32)}]
    attrs = G.w8a8_attrs(g, feeds)
    ops = [op for op in g.ops if op.kind == "matmul"]
    assert attrs[ops[0]]["x_scale"] == 4.0 / 127
    hpk = max(np.maximum(np.array([1, 2, 3], np.float32) @ w1, 0).max(),
              np.maximum(np.array([-4, 0, 1], np.float32) @ w1, 0).max())
    assert attrs[ops[1]]["x_scale"] == float(hpk) / 127
    q, s = G.quantize_array(w1, 1)
    assert np.array_equal(attrs[ops[0]]["q"], q) and np.array_equal(attrs[ops[0]]["w_scale"], s)


def test_zero_peak_gives_unit_scale():
    from harness.graph import Graph
    g = Graph("t")
    x = g.input("x", (2, 3))
    g.outputs = [g.op("matmul", [x, g.const(np.ones((3, 2), np.float32))])]
    attrs = G.w8a8_attrs(g, [{"x": np.zeros((2, 3), np.float32)}])
    assert list(attrs.values())[0]["x_scale"] == 1.0
