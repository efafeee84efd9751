"""Seeded random sweeps of the int8 contractions and the f32 depthwise convolution against
the oracle, bit for bit: shapes no hand-picked case chose (odd channel counts, rectangular
kernels, unequal strides, padding up to past the kernel's half, dilation, row counts around
every tile and weight-stream boundary).  The contractions carry a column bias, a full
residual and ReLU, and the int32 accumulators, the f32 result and its int8 requantization
are checked; the depthwise cases carry bias + ReLU6 and check both outputs.

The geometries are drawn once from a fixed seed (at most ~25 M multiply-accumulates each, so
the oracle takes well under a second per case); their ids name the shape."""
import ctypes as C

import numpy as np
import pytest

from mira_amd import _lib as L
from mira_amd import pack
from oracle import golden as G

from conftest import bits_equal
from gpu_util import T, empty, epilogue, stream, sync
import test_gpu_kernels as K

pytestmark = pytest.mark.gpu

MAX_MACS = 25_000_000


def conv_cases(seed: int = 20261202, count: int = 100) -> list:
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        c = int(rng.choice([1, 2, 3, 4, 5, 8, 12, 16, 20, 24, 32, 40, 48, 64, 96, 128, 144, 160, 256]))
        if rng.random() < 0.7:
            kh = kw = int(rng.choice([1, 3, 5, 7]))
        else:
            kh, kw = (int(v) for v in rng.choice([(1, 3), (3, 1), (1, 7), (7, 1), (3, 5), (5, 3)]))
        sh = int(rng.choice([1, 2]))
        sw = sh if rng.random() < 0.7 else 3 - sh
        dh = 2 if kh > 1 and rng.random() < 0.2 else 1
        dw = 2 if kw > 1 and rng.random() < 0.2 else 1
        ph = int(rng.integers(0, (kh // 2) * dh + 2))
        pw = int(rng.integers(0, (kw // 2) * dw + 2))
        h, w = (int(v) for v in rng.integers(3, 41, 2))
        n = int(rng.integers(1, 4))
        o = int(rng.choice([1, 8, 16, 24, 32, 40, 64, 96, 100, 128, 160, 200, 256, 320]))
        oh, ow = G.conv_out(h, kh, sh, ph, dh), G.conv_out(w, kw, sw, pw, dw)
        if oh < 1 or ow < 1 or n * oh * ow * o * c * kh * kw > MAX_MACS:
            continue
        out.append((n, c, h, w, o, kh, kw, sh, sw, ph, pw, dh, dw))
    return out


def matmul_cases(seed: int = 20261203, count: int = 100) -> list:
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        m = int(rng.choice([1, 2, 3, 5, 8, 9, 16, 17, 63, 64, 65, 127, 128, 129, 255, 300, 513, 1000, 2049]))
        k = int(rng.choice([1, 3, 16, 31, 64, 65, 100, 128, 192, 255, 512, 777, 1024, 2000, 4096, 5000]))
        n = int(rng.choice([1, 5, 10, 16, 31, 32, 33, 64, 65, 96, 127, 128, 129, 250, 512, 1000, 1100]))
        if m * k * n > MAX_MACS:
            continue
        out.append((m, k, n))
    return out


def dwconv_cases(seed: int = 20261204, count: int = 60) -> list:
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        c = int(rng.choice([1, 3, 4, 6, 8, 12, 16, 24, 32, 40, 96, 144, 192, 384, 576, 960]))
        k = int(rng.choice([3, 3, 3, 5]))
        s = int(rng.choice([1, 2]))
        d = 2 if rng.random() < 0.15 else 1
        p = int(rng.choice([k // 2 * d, 0, 1]))
        h, w = (int(v) for v in rng.integers(3, 40, 2))
        n = int(rng.integers(1, 4))
        oh, ow = G.conv_out(h, k, s, p, d), G.conv_out(w, k, s, p, d)
        if oh < 1 or ow < 1 or n * oh * ow * c * k * k > MAX_MACS:
            continue
        out.append((n, c, h, w, k, s, p, d))
    return out


CONV = conv_cases()
MATMUL = matmul_cases()
DWCONV = dwconv_cases()


@pytest.mark.parametrize("case", CONV, ids=["n{}c{}_{}x{}_o{}_k{}x{}_s{}{}_p{}{}_d{}{}".format(*c) for c in CONV])
def test_qconv2d_sweep(lib, case):
    n, c, h, w, o, kh, kw, sh, sw, ph, pw, dh, dw = case
    torch = K._torch()
    rng = np.random.default_rng(abs(hash(case)) % (2 ** 32))
    x = rng.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = rng.standard_normal((o, c, kh, kw)).astype(np.float32)
    q, ws = G.quantize_array(wt, 0)
    xs = float(np.abs(x).max()) / 127
    oh, ow = G.conv_out(h, kh, sh, ph, dh), G.conv_out(w, kw, sw, pw, dw)
    bias = (rng.standard_normal((o, 1, 1)) * 0.1).astype(np.float32)
    res = rng.standard_normal((n, o, oh, ow)).astype(np.float32)
    attrs = {"q": q, "w_scale": ws, "x_scale": xs, "dtype": "f32", "stride": (sh, sw), "padding": (ph, pw),
             "dilation": (dh, dw), "epilogue": (("add", 1, False), ("add", 2, False), ("relu", None, False))}
    want_acc = G.qconv2d_acc(x, attrs)
    want = G.qconv2d([x, bias, res], attrs)
    next_xs = float(np.abs(want[np.isfinite(want)]).max()) / 127 or 1.0
    cp = pack.c_pad_for(c)
    xq = empty((n, h, w, cp), torch.int8)
    L.check(lib.mr_quantize_nchw_nhwc(T(x).data_ptr(), n, c, h, w, xq.data_ptr(), cp, xs, stream()), "q")
    bl = pack.pack_conv(q, cp)
    b = T(pack.device_weights(bl))
    scale = T(pack.combined_scale(xs, ws))
    g = L.ConvGeom(n=n, h=h, w=w, c=c, c_pad=cp, o=o, oh=oh, ow=ow, kh=kh, kw=kw, sh=sh, sw=sw, ph=ph, pw=pw,
                   dh=dh, dw=dw)
    M = n * oh * ow
    bias_t = T(bias.reshape(o))
    res_t = T(res.transpose(0, 2, 3, 1).reshape(M, o))
    acc = empty((M, o), torch.int32)
    y = empty((M, o), torch.float32)
    ocp = pack.c_pad_for(o)
    yq = empty((M, ocp), torch.int8)
    e = epilogue([("add", L.BC_COL, bias_t, 0, False), ("add", L.BC_FULL, res_t, o, False),
                  ("relu", 0, None, 0, False)], scale=scale, out_f32=y, ldo=o, out_i8=yq, ldq=ocp, xs=next_xs,
                 out_acc=acc, ldacc=o)
    print(f"qconv2d sweep {case}", flush=True)
    L.check(lib.mr_qconv2d(xq.data_ptr(), C.byref(g), b.data_ptr(), bl.shape[1], bl.shape[0], C.byref(e), stream()),
            "mr_qconv2d")
    sync()
    to_rows = lambda a: a.transpose(0, 2, 3, 1).reshape(M, o)
    assert np.array_equal(acc.cpu().numpy(), to_rows(want_acc).astype(np.int32))
    assert bits_equal(y.cpu().numpy(), to_rows(want))
    assert bits_equal(yq.cpu().numpy()[:, :o], to_rows(G.quantize_activation(want, next_xs)).astype(np.int8))


@pytest.mark.parametrize("case", MATMUL, ids=["M{}_K{}_N{}".format(*c) for c in MATMUL])
def test_qmatmul_sweep(lib, case):
    M, Kd, N = case
    rng = np.random.default_rng(M * 1_000_003 + Kd * 1009 + N)
    x = rng.standard_normal((M, Kd)).astype(np.float32)
    w = (rng.standard_normal((Kd, N)) / np.sqrt(Kd)).astype(np.float32)
    q, ws = G.quantize_array(w, 1)
    xs = float(np.abs(x).max()) / 127
    bias = rng.standard_normal(N).astype(np.float32) * 0.1
    res = rng.standard_normal((M, N)).astype(np.float32)
    attrs = {"q": q, "w_scale": ws, "x_scale": xs, "dtype": "f32",
             "epilogue": (("add", 1, False), ("add", 2, False), ("relu", None, False))}
    want_acc = G.qmatmul_acc(x, attrs)
    want = G.qmatmul([x, bias, res], attrs)
    next_xs = float(np.abs(want[np.isfinite(want)]).max()) / 127 or 1.0
    print(f"qmatmul sweep {case}", flush=True)
    acc, y, yq = K._run_qmatmul(lib, x, q, ws, xs, [("add", L.BC_COL, bias, False), ("add", L.BC_FULL, res, False),
                                                    ("relu", 0, None, False)], next_xs)
    assert np.array_equal(acc, want_acc.astype(np.int32))
    assert bits_equal(y, want)
    assert bits_equal(yq, G.quantize_activation(want, next_xs).astype(np.int8))


@pytest.mark.parametrize("case", DWCONV, ids=["n{}c{}_{}x{}_k{}_s{}_p{}_d{}".format(*c) for c in DWCONV])
def test_dwconv_sweep(lib, case):
    n, c, h, w, k, s, p, d = case
    torch = K._torch()
    rng = np.random.default_rng(abs(hash(case)) % (2 ** 32))
    x = (rng.standard_normal((n, c, h, w)) * 2).astype(np.float32)
    wt = rng.standard_normal((c, 1, k, k)).astype(np.float32)
    bias = (rng.standard_normal((c, 1, 1)) * 0.1).astype(np.float32)
    zero, six = np.array(0, np.float32), np.array(6, np.float32)
    attrs = {"stride": (s, s), "padding": (p, p), "dilation": (d, d), "groups": c,
             "epilogue": (("add", 2, False), ("maximum", 3, False), ("minimum", 4, False))}
    want = G.conv2d([x, wt, bias, zero, six], attrs)
    oh, ow = want.shape[2:]
    xs_next = float(want.max()) / 127 or 1.0
    xd = T(x.transpose(0, 2, 3, 1))
    wd = T(np.ascontiguousarray(wt[:, 0].transpose(1, 2, 0)))
    g = L.ConvGeom(n=n, h=h, w=w, c=c, c_pad=c, o=c, oh=oh, ow=ow, kh=k, kw=k, sh=s, sw=s, ph=p, pw=p, dh=d, dw=d)
    M = n * oh * ow
    y = empty((M, c), torch.float32)
    cp = pack.c_pad_for(c)
    yq = empty((M, cp), torch.int8)
    bt, zt, st = T(bias.reshape(c)), T(zero.reshape(1)), T(six.reshape(1))
    e = epilogue([("add", L.BC_COL, bt, 0, False), ("maximum", L.BC_SCALAR, zt, 0, False),
                  ("minimum", L.BC_SCALAR, st, 0, False)], out_f32=y, ldo=c, out_i8=yq, ldq=cp, xs=xs_next)
    print(f"dwconv sweep {case}", flush=True)
    L.check(lib.mr_dwconv2d_f32(xd.data_ptr(), C.byref(g), wd.data_ptr(), C.byref(e), stream()), "dw")
    sync()
    assert bits_equal(y.cpu().numpy(), want.transpose(0, 2, 3, 1).reshape(M, c))
    assert bits_equal(yq.cpu().numpy()[:, :c],
                      G.quantize_activation(want, xs_next).astype(np.int8).transpose(0, 2, 3, 1).reshape(M, c))
