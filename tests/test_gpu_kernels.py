"""Per-kernel parity of libmira_rocm.so against the oracle, through the C ABI.

int8 tensors and int32 accumulators must be bit-exact; f32 results are
compared bit for bit too (every epilogue step is a single IEEE operation), which
is stricter than the 1e-5 relative bound the W8A8 contract allows.
"""
import ctypes as C

import numpy as np
import pytest

from mira_amd import _lib as L
from mira_amd import pack
from oracle import golden as G

from conftest import bits_equal
from gpu_util import T, empty, epilogue, stream, sync

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


# ---------------------------------------------------------------- K1 quantize

@pytest.mark.parametrize("rows,cols,xs", [(513, 100, 0.0371), (1, 64, 1.0), (4096, 4096, 0.031), (7, 3, 0.5)])
def test_quantize_rows(lib, rows, cols, xs):
    torch = _torch()
    rng = np.random.default_rng(rows + cols)
    x = (rng.standard_normal((rows, cols)) * 3).astype(np.float32)
    x.ravel()[:6] = np.float32([0.5, 1.5, 2.5, -2.5, 1000, -1000]) * np.float32(xs)
    ldq = pack.row_stride_for(cols)
    q = empty((rows, ldq), torch.int8)
    L.check(lib.mr_quantize_rows(T(x).data_ptr(), rows, cols, cols, q.data_ptr(), ldq, xs, stream()), "q")
    sync()
    got = q.cpu().numpy()
    assert bits_equal(got[:, :cols], G.quantize_activation(x, xs).astype(np.int8))
    assert not got[:, cols:].any()


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("n,c,h,w,ties", [(3, 3, 21, 19, False), (2, 20, 5, 6, False), (1, 1, 28, 28, False),
                                           (2, 3, 8, 12, True), (2, 20, 6, 6, True), (3, 4, 7, 4, False)])
def test_quantize_nchw_nhwc(lib, n, c, h, w, ties, f16):
    """Both kernels: any pixel count, and four pixels per thread when h*w % 4 == 0; with f16,
    the input's f32 -> f16 cast fused in front (mr_quantize_f16_nchw_nhwc)."""
    torch = _torch()
    rng = np.random.default_rng(c + h)
    x = rng.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    if ties:    # values on and next to the half-way points of the int8 grid
        k = rng.integers(-140, 140, x.shape) + 0.5
        x = (k / 127).astype(np.float32)
        x.reshape(-1)[::3] = np.nextafter(x.reshape(-1)[::3], np.float32(np.inf))
    cp = pack.c_pad_for(c)
    q = empty((n, h, w, cp), torch.int8)
    xs = float(np.float32(1 / 127))
    fn = lib.mr_quantize_f16_nchw_nhwc if f16 else lib.mr_quantize_nchw_nhwc
    L.check(fn(T(x).data_ptr(), n, c, h, w, q.data_ptr(), cp, xs, stream()), "q")
    sync()
    got = q.cpu().numpy()
    want = G.quantize_activation(x.astype(np.float16) if f16 else x, xs).astype(np.int8).transpose(0, 2, 3, 1)
    assert bits_equal(got[..., :c], want) and not got[..., c:].any()


# ---------------------------------------------------------------- K2/K3 qmatmul

def _run_qmatmul(lib, x, q, ws, xs, steps_np, next_xs=None):
    """steps_np: (fn, mode, operand array or None, swapped). Returns (acc, y f32, y int8)."""
    torch = _torch()
    M, K = x.shape
    N = q.shape[1]
    lda = pack.row_stride_for(K)
    xq = empty((M, lda), torch.int8)
    L.check(lib.mr_quantize_rows(T(x).data_ptr(), M, K, K, xq.data_ptr(), lda, xs, stream()), "q")
    bl = pack.pack_matmul(q)
    b = T(pack.device_weights(bl))
    scale = T(pack.combined_scale(xs, ws))
    keep, steps = [], []
    for fn, mode, arr, sw in steps_np:
        if arr is None:
            steps.append((fn, mode, None, 0, sw))
            continue
        t = T(np.ascontiguousarray(arr, np.float32))
        keep.append(t)
        ld = N if mode == L.BC_FULL else (1 if mode == L.BC_ROW else 0)
        steps.append((fn, mode, t, ld, sw))
    acc = empty((M, N), torch.int32)
    y = empty((M, N), torch.float32)
    ldq = pack.row_stride_for(N)
    yq = empty((M, ldq), torch.int8) if next_xs else None
    e = epilogue(steps, scale=scale, out_f32=y, ldo=N, out_i8=yq, ldq=ldq, xs=next_xs or 1.0, out_acc=acc, ldacc=N)
    L.check(lib.mr_qmatmul(xq.data_ptr(), lda, b.data_ptr(), bl.shape[1], bl.shape[0], M, N, K, C.byref(e), stream()),
            "mr_qmatmul")
    sync()
    return acc.cpu().numpy(), y.cpu().numpy(), (yq.cpu().numpy()[:, :N] if yq is not None else None)


@pytest.mark.parametrize("M,K,N", [(256, 64, 10), (64, 784, 512), (300, 512, 1000), (1, 4096, 4096),
                                   (4096, 4096, 1000), (33, 128, 65), (70000, 64, 128),
                                   (49920, 160, 272),     # short K: 128x64 tiles, ragged K and N
                                   (6272, 960, 320),      # short K, under one 128x64 tile per CU: 64x32
                                   (25088, 384, 96),      # short K, under one 128x128 tile per CU: 64x32
                                   (25088, 64, 384),      # short K, N > 128: 128x64
                                   (3, 4096, 1000), (8, 512, 65), (2, 64, 64), (5, 192, 130),   # weight stream
                                   (2, 5000, 96), (1, 8192, 40),    # k_pad > 4096: lane groups per column pair
                                   (2, 1024, 3000),                 # weight stream, 8 columns per workgroup
                                   (96, 1024, 256), (40, 4000, 70),   # small grids: 64x32 tiles, 128-byte stages
                                   (600000, 48, 24)])                 # one K step on a huge grid: 128x32 tiles
def test_qmatmul_bias_relu_requant(lib, M, K, N):
    rng = np.random.default_rng(M * 7 + N)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((K, N)) / np.sqrt(K)).astype(np.float32)
    q, ws = G.quantize_array(w, 1)
    xs = float(np.abs(x).max()) / 127
    bias = rng.standard_normal(N).astype(np.float32) * 0.1
    attrs = {"q": q, "w_scale": ws, "x_scale": xs, "dtype": "f32",
             "epilogue": (("add", 1, False), ("relu", None, False))}
    want_acc = G.qmatmul_acc(x, attrs)
    want = G.qmatmul([x, bias], attrs)
    next_xs = float(np.abs(want[np.isfinite(want)]).max()) / 127 or 1.0
    acc, y, yq = _run_qmatmul(lib, x, q, ws, xs, [("add", L.BC_COL, bias, False), ("relu", 0, None, False)], next_xs)
    assert np.array_equal(acc, want_acc.astype(np.int32))
    assert bits_equal(y, want)
    assert bits_equal(yq, G.quantize_activation(want, next_xs).astype(np.int8))


@pytest.mark.parametrize("M,K,N,pad", [(1, 4096, 4096, 0), (1, 4096, 1000, 0), (3, 100, 77, 1), (8, 4096, 130, 0),
                                       (5, 1000, 33, 3), (2, 64, 2048, 0), (4, 4032, 3000, 4)])
def test_qmatmul_f32in_equals_quantize_then_qmatmul(lib, M, K, N, pad):
    """mr_qmatmul_f32in (the quantize inside the decode-shaped kernel) against the oracle and
    against mr_quantize_rows + mr_qmatmul, bit for bit; pad > 0 makes the rows' stride
    K + pad floats, so rows are not 16-byte aligned and the scalar loads run."""
    torch = _torch()
    rng = np.random.default_rng(M * 13 + N)
    ldx = K + pad
    xfull = rng.standard_normal((M, ldx)).astype(np.float32)
    x = np.ascontiguousarray(xfull[:, :K])
    w = (rng.standard_normal((K, N)) / np.sqrt(K)).astype(np.float32)
    q, ws = G.quantize_array(w, 1)
    xs = float(np.abs(x).max()) / 127
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    attrs = {"q": q, "w_scale": ws, "x_scale": xs, "dtype": "f32",
             "epilogue": (("add", 1, False), ("relu", None, False))}
    want_acc = G.qmatmul_acc(x, attrs)
    want = G.qmatmul([x, bias], attrs)
    next_xs = float(np.abs(want).max()) / 127 or 1.0
    acc_ref, y_ref, yq_ref = _run_qmatmul(lib, x, q, ws, xs, [("add", L.BC_COL, bias, False), ("relu", 0, None, False)],
                                          next_xs)
    bl = pack.pack_matmul(q)
    b = T(pack.device_weights(bl))
    scale = T(pack.combined_scale(xs, ws))
    bias_t = T(bias)
    acc = empty((M, N), torch.int32)
    y = empty((M, N), torch.float32)
    ldq = pack.row_stride_for(N)
    yq = empty((M, ldq), torch.int8)
    e = epilogue([("add", L.BC_COL, bias_t, 0, False), ("relu", 0, None, 0, False)], scale=scale, out_f32=y, ldo=N,
                 out_i8=yq, ldq=ldq, xs=next_xs, out_acc=acc, ldacc=N)
    xd = T(xfull)
    L.check(lib.mr_qmatmul_f32in(xd.data_ptr(), ldx, xs, b.data_ptr(), bl.shape[1], bl.shape[0], M, N, K, C.byref(e),
                                 stream()), "mr_qmatmul_f32in")
    sync()
    assert np.array_equal(acc.cpu().numpy(), want_acc.astype(np.int32))
    assert np.array_equal(acc.cpu().numpy(), acc_ref)
    assert bits_equal(y.cpu().numpy(), want) and bits_equal(y.cpu().numpy(), y_ref)
    assert bits_equal(yq.cpu().numpy()[:, :N], yq_ref)


def test_qmatmul_f32in_rejects(lib):
    torch = _torch()
    x = empty((16, 4096), torch.float32)
    b = empty((64, 4096), torch.int8)
    sc = empty((64,), torch.float64)
    y = empty((16, 64), torch.float32)
    e = epilogue(scale=sc, out_f32=y, ldo=64)
    assert lib.mr_qmatmul_f32in(x.data_ptr(), 4096, 0.1, b.data_ptr(), 4096, 64, 9, 64, 4096, C.byref(e),
                                stream()) == 3       # 9 rows: unsupported
    assert lib.mr_qmatmul_f32in(x.data_ptr(), 4160, 0.1, b.data_ptr(), 4160, 64, 1, 64, 4100, C.byref(e),
                                stream()) == 3       # k_pad past 4096 (nothing is launched)
    assert lib.mr_qmatmul_f32in(x.data_ptr(), 100, 0.1, b.data_ptr(), 4096, 64, 1, 64, 4096, C.byref(e),
                                stream()) == 1       # ldx < K
    assert lib.mr_qmatmul_f32in(x.data_ptr(), 4096, 0.0, b.data_ptr(), 4096, 64, 1, 64, 4096, C.byref(e),
                                stream()) == 1       # x_scale 0


@pytest.mark.parametrize("M", [200, 4])
def test_qmatmul_every_epilogue_step(lib, M):
    rng = np.random.default_rng(11)
    K, N = 96, 48
    x = rng.standard_normal((M, K)).astype(np.float32)
    q = rng.integers(-127, 128, (K, N)).astype(np.int8)
    ws = rng.uniform(0.001, 0.01, N).astype(np.float32)
    xs = 0.025
    full = rng.standard_normal((M, N)).astype(np.float32)
    row = rng.uniform(0.5, 2, (M, 1)).astype(np.float32)
    col = rng.uniform(0.5, 2, N).astype(np.float32)
    lo, hi = np.array(-0.5, np.float32), np.array(0.75, np.float32)
    epi = (("sub", 1, True), ("mul", 2, False), ("div", 3, True), ("add", 4, False), ("maximum", 5, False),
           ("minimum", 6, True))
    attrs = {"q": q, "w_scale": ws, "x_scale": xs, "dtype": "f32", "epilogue": epi}
    want = G.qmatmul([x, full, col, row, full, lo, hi], attrs)
    _, y, _ = _run_qmatmul(lib, x, q, ws, xs, [
        ("sub", L.BC_FULL, full, True), ("mul", L.BC_COL, col, False), ("div", L.BC_ROW, row, True),
        ("add", L.BC_FULL, full, False), ("maximum", L.BC_SCALAR, lo.reshape(1), False),
        ("minimum", L.BC_SCALAR, hi.reshape(1), True)])
    assert bits_equal(y, want)


@pytest.mark.parametrize("M,K", [(300, 80), (5, 80), (300, 16)])
def test_qmatmul_row_tail_past_k_is_not_read_as_data(lib, M, K):
    """lda < k_pad: the dense loader's K runs to k_pad, past each row's K bytes into the
    next row.  Those bytes are nonzero here; the packed weights are zero for k >= K (the
    packing contract), so the accumulators still equal the oracle's."""
    torch = _torch()
    rng = np.random.default_rng(M + K)
    N = 40
    xq = rng.integers(-127, 128, (M, K)).astype(np.int8)
    q = rng.integers(-127, 128, (K, N)).astype(np.int8)
    lda = pack.row_stride_for(K)
    bl = pack.pack_matmul(q)
    assert lda < bl.shape[1]
    rows = rng.integers(-127, 128, (M, lda)).astype(np.int8)      # bytes K..lda-1 nonzero
    rows[:, :K] = xq
    ws = np.full(N, 0.01, np.float32)
    attrs = {"q": q, "w_scale": ws, "x_scale": 1.0, "dtype": "f32", "epilogue": ()}
    want = G.qmatmul_acc(xq.astype(np.float32), attrs).astype(np.int32)
    acc = empty((M, N), torch.int32)
    y = empty((M, N), torch.float32)
    xd, bd, sc = T(rows), T(pack.device_weights(bl)), T(pack.combined_scale(1.0, ws))
    e = epilogue([], scale=sc, out_f32=y, ldo=N, out_acc=acc, ldacc=N)
    L.check(lib.mr_qmatmul(xd.data_ptr(), lda, bd.data_ptr(), bl.shape[1], bl.shape[0], M, N, K, C.byref(e),
                           stream()), "mr_qmatmul")
    sync()
    assert np.array_equal(acc.cpu().numpy(), want)


def test_qmatmul_rejects_bad_shapes(lib):
    torch = _torch()
    a = empty((4, 16), torch.int8)
    b = empty((32, 64), torch.int8)
    e = epilogue(out_f32=empty((4, 8), torch.float32), ldo=8, scale=T(np.ones(8)))
    assert lib.mr_qmatmul(a.data_ptr(), 15, b.data_ptr(), 64, 32, 4, 8, 16, C.byref(e), stream()) == 1
    assert b"lda" in lib.mr_last_error()
    assert lib.mr_qmatmul(a.data_ptr(), 16, b.data_ptr(), 60, 32, 4, 8, 16, C.byref(e), stream()) == 1


# ---------------------------------------------------------------- f16 results (values stored as f32)

def test_round_f16_matches_numpy(lib):
    """mr_round_f16_f32 == NumPy's astype(float16) back to f32: ties to even, f16
    subnormals, overflow to inf, signed zeros, inf and NaN."""
    torch = _torch()
    tiny = np.float32(2.0 ** -24)                  # smallest f16 subnormal
    special = np.array([0.0, -0.0, 1.0, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 65504.0, 65519.99, 65520.0, 7e4,
                        -7e4, tiny, tiny / 2, tiny * 0.5001, tiny * 1.5, 3.1e-5, 6.1e-5, np.inf, -np.inf, np.nan,
                        1e-30, -1e-30, 2049.0, 2051.0], np.float32)
    rng = np.random.default_rng(0)
    x = np.concatenate([special, rng.standard_normal(100_003).astype(np.float32) * 100,
                        rng.standard_normal(1000).astype(np.float32) * 1e-5])
    xd, y = T(x), empty(x.shape, torch.float32)
    L.check(lib.mr_round_f16_f32(xd.data_ptr(), x.size, y.data_ptr(), stream()), "round")
    L.check(lib.mr_round_f16_f32(xd.data_ptr(), x.size, xd.data_ptr(), stream()), "round in place")
    sync()
    want = x.astype(np.float16).astype(np.float32)
    assert bits_equal(y.cpu().numpy(), want) and bits_equal(xd.cpu().numpy(), want)


@pytest.mark.parametrize("M,K,N", [(300, 512, 1000), (4, 256, 96)])     # tiled and weight-stream kernels
def test_qmatmul_f16_result(lib, M, K, N):
    """A q-op of dtype f16 (mira/ops.py:620): the f32 epilogue result rounded to f16, and the
    int8 copy quantized from the rounded value; large outputs overflow to inf as in NumPy."""
    torch = _torch()
    rng = np.random.default_rng(M + N)
    x = (rng.standard_normal((M, K)) * 30).astype(np.float16).astype(np.float32)
    w = rng.standard_normal((K, N)).astype(np.float32)
    q, ws = G.quantize_array(w, 1)
    ws = ws * np.float32(40.0)                    # push some results past the f16 range
    xs = float(np.abs(x).max()) / 127
    bias = (rng.standard_normal(N) * 0.1).astype(np.float16)
    attrs = {"q": q, "w_scale": ws, "x_scale": xs, "dtype": "f16", "epilogue": (("add", 1, False),)}
    want = G.qmatmul([x.astype(np.float16), bias], attrs)
    assert want.dtype == np.float16 and np.isinf(want).any()
    lda = pack.row_stride_for(K)
    xq = empty((M, lda), torch.int8)
    L.check(lib.mr_quantize_rows(T(x).data_ptr(), M, K, K, xq.data_ptr(), lda, xs, stream()), "q")
    bl = pack.pack_matmul(q)
    b, scale, bt = T(pack.device_weights(bl)), T(pack.combined_scale(xs, ws)), T(bias.astype(np.float32))
    y = empty((M, N), torch.float32)
    ldq = pack.row_stride_for(N)
    yq = empty((M, ldq), torch.int8)
    e = epilogue([("add", L.BC_COL, bt, 0, False)], scale=scale, out_f32=y, ldo=N, out_i8=yq, ldq=ldq, xs=3.0)
    e.flags = L.EPI_OUT_F16
    L.check(lib.mr_qmatmul(xq.data_ptr(), lda, b.data_ptr(), bl.shape[1], bl.shape[0], M, N, K, C.byref(e), stream()),
            "mr_qmatmul")
    sync()
    assert bits_equal(y.cpu().numpy(), want.astype(np.float32))
    assert bits_equal(yq.cpu().numpy()[:, :N], G.quantize_activation(want, 3.0).astype(np.int8))


# ---------------------------------------------------------------- weight-only int8 matmul (f32 activations)

# The f32 sums run in another order than NumPy's BLAS, so parity is a tolerance:
# |got - want| <= W8_TOL * (|x| @ |W| + |epilogue operands|), want = the oracle's f32 matmul
# over the dequantized weight (mira/ops.py:217-219, 581-589).
W8_TOL = 1e-5


def _run_w8(lib, x, K, q, s, steps_np, next_xs=None, w16=False):
    """x: [M, ldx] f32 (columns >= K are ignored). Returns (y f32, y int8 or None)."""
    torch = _torch()
    M, ldx = x.shape
    N = q.shape[1]
    bl = pack.pack_matmul(q)
    b, ws, xd = T(pack.device_weights(bl)), T(s.astype(np.float32)), T(x)
    keep, steps = [], []
    for fn, mode, arr, sw in steps_np:
        if arr is None:
            steps.append((fn, mode, None, 0, sw))
            continue
        t = T(np.ascontiguousarray(arr, np.float32))
        keep.append(t)
        steps.append((fn, mode, t, N if mode == L.BC_FULL else (1 if mode == L.BC_ROW else 0), sw))
    y = empty((M, N), torch.float32)
    ldq = pack.row_stride_for(N)
    yq = empty((M, ldq), torch.int8) if next_xs else None
    e = epilogue(steps, out_f32=y, ldo=N, out_i8=yq, ldq=ldq, xs=next_xs or 1.0)
    L.check(lib.mr_w8_matmul_f32(xd.data_ptr(), ldx, b.data_ptr(), ws.data_ptr(), int(w16), bl.shape[1], bl.shape[0],
                                 M, N, K, C.byref(e), stream()), "mr_w8_matmul_f32")
    sync()
    return y.cpu().numpy(), (yq.cpu().numpy()[:, :N] if yq is not None else None)


@pytest.mark.parametrize("M,K,N,ldx", [(1, 4096, 4096, 4096), (1, 4096, 1000, 4096), (2, 784, 512, 784),
                                       (3, 100, 65, 100), (8, 512, 256, 520), (13, 256, 10, 257),
                                       (64, 784, 512, 784), (5, 33, 1, 33)])
def test_w8_matmul_bias_relu(lib, M, K, N, ldx):
    rng = np.random.default_rng(M * 31 + K + N)
    x = rng.standard_normal((M, ldx)).astype(np.float32)      # columns >= K are never read as data
    w = (rng.standard_normal((K, N)) / np.sqrt(K)).astype(np.float32)
    q, s = G.quantize_array(w, 1)
    deq = G.dequantize({"q": q, "scale": s, "axis": 1, "dtype": "f32"})
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    want = G.matmul([x[:, :K], deq, bias], {"epilogue": (("add", 2, False), ("relu", None, False))})
    y, yq = _run_w8(lib, x, K, q, s, [("add", L.BC_COL, bias, False), ("relu", 0, None, False)], next_xs=0.02)
    bound = np.abs(x[:, :K]).astype(np.float64) @ np.abs(deq).astype(np.float64) + np.abs(bias)
    assert np.all(np.abs(y.astype(np.float64) - want) <= W8_TOL * bound)
    assert (y >= 0).all()
    # the requantized copy is the reference's quantize_activation of the kernel's own f32 result
    assert bits_equal(yq, G.quantize_activation(y, 0.02).astype(np.int8))


@pytest.mark.parametrize("M,K,N,ldx", [(17, 64, 33, 64), (128, 784, 512, 784), (300, 1024, 1000, 1028),
                                       (1000, 256, 130, 256), (40, 33, 20, 36)])
def test_w8_matmul_tiled(lib, M, K, N, ldx):
    """More than 16 rows: 128 x 128 f32-MFMA tiles (ragged M, N and K tails; the last case,
    K % 4 != 0, takes the 8-row weight stream instead)."""
    rng = np.random.default_rng(M * 7 + K + N)
    x = rng.standard_normal((M, ldx)).astype(np.float32)
    x[:, K:] = np.inf                      # columns >= K must never be read as data
    w = (rng.standard_normal((K, N)) / np.sqrt(K)).astype(np.float32)
    q, s = G.quantize_array(w, 1)
    deq = G.dequantize({"q": q, "scale": s, "axis": 1, "dtype": "f32"})
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    want = G.matmul([x[:, :K], deq, bias], {"epilogue": (("add", 2, False), ("relu", None, False))})
    y, yq = _run_w8(lib, x, K, q, s, [("add", L.BC_COL, bias, False), ("relu", 0, None, False)], next_xs=0.02)
    bound = np.abs(x[:, :K]).astype(np.float64) @ np.abs(deq).astype(np.float64) + np.abs(bias)
    assert np.all(np.abs(y.astype(np.float64) - want) <= W8_TOL * bound)
    assert (y >= 0).all()
    assert bits_equal(yq, G.quantize_activation(y, 0.02).astype(np.int8))


def test_w8_matmul_tiled_f16_weights(lib):
    """The tiled kernel with an f16 dequantize: weights fl16(fl32(q * scale))."""
    rng = np.random.default_rng(81)
    M, K, N = 200, 512, 200
    x = rng.standard_normal((M, K)).astype(np.float16).astype(np.float32)
    q = rng.integers(-127, 128, (K, N)).astype(np.int8)
    s = rng.uniform(0.001, 0.01, N).astype(np.float32)
    deq = G.dequantize({"q": q, "scale": s, "axis": 1, "dtype": "f16"})
    want = G.matmul([x, deq.astype(np.float32)], {})
    y, _ = _run_w8(lib, x, K, q, s, [], w16=True)
    bound = np.abs(x).astype(np.float64) @ np.abs(deq.astype(np.float64))
    assert np.all(np.abs(y.astype(np.float64) - want) <= W8_TOL * bound)


@pytest.mark.parametrize("n,c,h,o,k,s,p,d,w16", [(2, 64, 14, 128, 3, 1, 1, 1, False), (2, 64, 15, 130, 3, 2, 1, 1, False),
                                                (3, 20, 9, 24, 1, 1, 0, 1, False), (2, 4, 17, 32, 3, 2, 1, 1, False),
                                                (2, 16, 11, 40, 3, 1, 2, 2, False), (1, 96, 7, 200, 1, 2, 0, 1, True)])
def test_w8_conv2d(lib, n, c, h, o, k, s, p, d, w16):
    """Weight-only int8 convolution (f32 conv2d over a dequantize weight, mira/ops.py:265-276,
    581-589) as an implicit GEMM on f32 MFMAs: within the f32-rounding bound of the matmul
    tests, every tap/stride/padding/dilation case and ragged pixel / channel counts."""
    torch = _torch()
    rng = np.random.default_rng(n * 100 + c + o + k)
    x = rng.standard_normal((n, c, h, h)).astype(np.float32)
    q = rng.integers(-127, 128, (o, c, k, k)).astype(np.int8)
    sc = rng.uniform(0.001, 0.01, o).astype(np.float32)
    deq = G.dequantize({"q": q, "scale": sc, "axis": 0, "dtype": "f16" if w16 else "f32"}).astype(np.float32)
    bias = (rng.standard_normal((o, 1, 1)) * 0.1).astype(np.float32)
    attrs = {"stride": (s, s), "padding": (p, p), "dilation": (d, d),
             "epilogue": (("add", 2, False), ("relu", None, False))}
    want = G.conv2d([x, deq, bias], attrs)
    oh = want.shape[2]
    M = n * oh * oh
    cp = pack.roundup(c, 16)
    bl = pack.pack_conv(q, cp)
    xd, b, ws, bt = T(x.transpose(0, 2, 3, 1)), T(pack.device_weights(bl)), T(sc), T(bias.reshape(o))
    y = empty((M, o), torch.float32)
    e = epilogue([("add", L.BC_COL, bt, 0, False), ("relu", 0, None, 0, False)], out_f32=y, ldo=o)
    g = L.ConvGeom(n=n, h=h, w=h, c=c, c_pad=cp, o=o, oh=oh, ow=oh, kh=k, kw=k, sh=s, sw=s, ph=p, pw=p, dh=d, dw=d)
    L.check(lib.mr_w8_conv2d_f32(xd.data_ptr(), C.byref(g), b.data_ptr(), ws.data_ptr(), int(w16), bl.shape[1],
                                 bl.shape[0], C.byref(e), stream()), "mr_w8_conv2d_f32")
    sync()
    got = y.cpu().numpy()
    to_nhwc = lambda a: a.transpose(0, 2, 3, 1).reshape(M, o)
    bound = to_nhwc(G.conv2d([np.abs(x).astype(np.float64), np.abs(deq).astype(np.float64)],
                             {"stride": (s, s), "padding": (p, p), "dilation": (d, d)})) + np.abs(bias.reshape(o))
    assert np.all(np.abs(got.astype(np.float64) - to_nhwc(want)) <= W8_TOL * bound)
    assert (got >= 0).all()


def test_w8_conv2d_rejects_bad_arguments(lib):
    torch = _torch()
    x = empty((1, 5, 5, 3), torch.float32)
    b = empty((64, 64), torch.int8)
    s = empty((8,), torch.float32)
    e = epilogue(out_f32=empty((25, 8), torch.float32), ldo=8)
    g = L.ConvGeom(n=1, h=5, w=5, c=3, c_pad=16, o=8, oh=5, ow=5, kh=1, kw=1, sh=1, sw=1, ph=0, pw=0, dh=1, dw=1)
    assert lib.mr_w8_conv2d_f32(x.data_ptr(), C.byref(g), b.data_ptr(), s.data_ptr(), 0, 64, 64, C.byref(e),
                                stream()) == 1
    assert b"multiple of 4" in lib.mr_last_error()


def test_w8_matmul_f16_weights(lib):
    """A dequantize of dtype f16 (mira/ops.py:584): the weights are fl16(fl32(q * scale)); with
    f16 activations and an f16 result rounded after the epilogue."""
    rng = np.random.default_rng(8)
    M, K, N = 3, 512, 200
    x = rng.standard_normal((M, K)).astype(np.float16)
    q = rng.integers(-127, 128, (K, N)).astype(np.int8)
    s = rng.uniform(0.001, 0.01, N).astype(np.float32)
    deq = G.dequantize({"q": q, "scale": s, "axis": 1, "dtype": "f16"})
    assert deq.dtype == np.float16
    bias = (rng.standard_normal(N) * 0.1).astype(np.float16)
    want = G.matmul([x, deq, bias], {"epilogue": (("add", 2, False),)})
    torch = _torch()
    bl = pack.pack_matmul(q)
    y = empty((M, N), torch.float32)
    bt = T(bias.astype(np.float32))
    e = epilogue([("add", L.BC_COL, bt, 0, False)], out_f32=y, ldo=N)
    e.flags = L.EPI_OUT_F16
    xd, bd, sd = T(x.astype(np.float32)), T(pack.device_weights(bl)), T(s)     # alive until the kernel ran
    L.check(lib.mr_w8_matmul_f32(xd.data_ptr(), K, bd.data_ptr(), sd.data_ptr(), 1, bl.shape[1], bl.shape[0], M, N, K,
                                 C.byref(e), stream()), "w8")
    sync()
    got = y.cpu().numpy()
    assert bits_equal(got, got.astype(np.float16).astype(np.float32))           # f16 values
    bound = np.abs(x.astype(np.float64)) @ np.abs(deq.astype(np.float64)) + np.abs(bias)
    # f32 summation order differences, then the f16 roundings may land one f16 ulp apart
    # (2^-10 relative, 2^-24 absolute for subnormals)
    assert np.all(np.abs(got - want.astype(np.float64)) <=
                  W8_TOL * bound + 2.0 ** -10 * np.abs(want.astype(np.float64)) + 2.0 ** -24)


def test_w8_matmul_row_blocks_and_operands(lib):
    """Row-indexed epilogue operands across several 8-row blocks (M = 21)."""
    rng = np.random.default_rng(5)
    M, K, N = 21, 192, 48
    x = rng.standard_normal((M, K)).astype(np.float32)
    q = rng.integers(-127, 128, (K, N)).astype(np.int8)
    s = rng.uniform(0.001, 0.01, N).astype(np.float32)
    deq = G.dequantize({"q": q, "scale": s, "axis": 1, "dtype": "f32"})
    full = rng.standard_normal((M, N)).astype(np.float32)
    row = rng.uniform(0.5, 2, (M, 1)).astype(np.float32)
    want = G.matmul([x, deq, full, row], {"epilogue": (("sub", 2, True), ("mul", 3, False))})
    y, _ = _run_w8(lib, x, K, q, s, [("sub", L.BC_FULL, full, True), ("mul", L.BC_ROW, row, False)])
    bound = (np.abs(x).astype(np.float64) @ np.abs(deq) + np.abs(full)) * row
    assert np.all(np.abs(y.astype(np.float64) - want) <= W8_TOL * bound)


def test_w8_matmul_rejects_bad_arguments(lib):
    torch = _torch()
    x = empty((4, 16), torch.float32)
    b = empty((32, 64), torch.int8)
    s = empty((8,), torch.float32)
    e = epilogue(out_f32=empty((4, 8), torch.float32), ldo=8)
    assert lib.mr_w8_matmul_f32(x.data_ptr(), 15, b.data_ptr(), s.data_ptr(), 0, 64, 32, 4, 8, 16, C.byref(e),
                                stream()) == 1
    assert b"ldx" in lib.mr_last_error()
    e2 = epilogue(out_f32=empty((4, 8), torch.float32), ldo=8, scale=s)
    assert lib.mr_w8_matmul_f32(x.data_ptr(), 16, b.data_ptr(), s.data_ptr(), 0, 64, 32, 4, 8, 16, C.byref(e2),
                                stream()) == 1


# ---------------------------------------------------------------- K2c qconv2d

CONV_CASES = [
    # n, c, h, w, o, k, stride, pad, dilation
    (2, 3, 32, 32, 64, 7, 2, 3, 1),       # ResNet stem layout (c_pad 4, 7 taps per row)
    (2, 3, 17, 19, 32, 3, 2, 1, 1),       # MobileNetV2 stem layout (3 taps per row)
    (2, 64, 14, 14, 64, 3, 1, 1, 1),
    (2, 64, 15, 15, 128, 3, 2, 1, 1),
    (2, 64, 14, 14, 128, 1, 2, 0, 1),     # downsample
    (1, 256, 7, 7, 512, 3, 1, 1, 1),
    (3, 24, 9, 9, 144, 1, 1, 0, 1),       # 1x1 as a dense GEMM, c_pad 32
    (2, 144, 28, 28, 24, 1, 1, 0, 1),     # 1x1 as a dense GEMM, c_pad 144: K tail past the row
    (2, 64, 14, 14, 384, 1, 1, 0, 1),     # 1x1 as a dense GEMM (a small grid: 64x32 tiles)
    (2, 16, 11, 11, 24, 3, 1, 2, 2),      # dilation 2
    (2, 1, 28, 28, 16, 3, 1, 1, 1),       # single channel (cnn.mira)
    # stride-1 convolutions read through the per-tile input patch
    (2, 64, 56, 56, 64, 3, 1, 1, 1),      # ResNet layer 1 (2 output rows per tile)
    (2, 128, 28, 28, 128, 3, 1, 1, 1),    # ResNet layer 2 (4 rows per tile, 8 chunks per pixel)
    (1, 256, 7, 7, 96, 3, 1, 1, 1),       # 16 chunks per pixel, 96 of 128 columns
    (3, 64, 20, 20, 40, 3, 1, 1, 1),      # last tile of each image 2 of 6 rows
    (2, 64, 11, 120, 96, 3, 1, 1, 1),     # one output row per tile (128-row tiles)
    (2, 64, 12, 12, 32, 5, 1, 2, 1),      # 5x5, pad 2
    (1, 64, 6, 9, 64, 3, 1, 0, 1),        # no padding
]


@pytest.mark.parametrize("n,c,h,w,o,k,s,p,d", CONV_CASES)
def test_qconv2d(lib, n, c, h, w, o, k, s, p, d):
    torch = _torch()
    rng = np.random.default_rng(n * 1000 + c * 10 + k)
    x = rng.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = rng.standard_normal((o, c, k, k)).astype(np.float32)
    q, ws = G.quantize_array(wt, 0)
    xs = float(np.abs(x).max()) / 127
    oh = G.conv_out(h, k, s, p, d)
    ow = G.conv_out(w, k, s, p, d)
    bias = (rng.standard_normal((o, 1, 1)) * 0.1).astype(np.float32)
    res = rng.standard_normal((n, o, oh, ow)).astype(np.float32)
    attrs = {"q": q, "w_scale": ws, "x_scale": xs, "dtype": "f32", "stride": (s, s), "padding": (p, p),
             "dilation": (d, d), "epilogue": (("add", 1, False), ("add", 2, False), ("relu", None, False))}
    assert G.qconv2d_certificate(x, attrs) < 2 ** 24
    want_acc = G.qconv2d_acc(x, attrs)
    want = G.qconv2d([x, bias, res], attrs)
    next_xs = float(np.abs(want[np.isfinite(want)]).max()) / 127 or 1.0
    cp = pack.c_pad_for(c)
    xq = empty((n, h, w, cp), torch.int8)
    L.check(lib.mr_quantize_nchw_nhwc(T(x).data_ptr(), n, c, h, w, xq.data_ptr(), cp, xs, stream()), "q")
    bl = pack.pack_conv(q, cp)
    b = T(pack.device_weights(bl))
    scale = T(pack.combined_scale(xs, ws))
    g = L.ConvGeom(n=n, h=h, w=w, c=c, c_pad=cp, o=o, oh=oh, ow=ow, kh=k, kw=k, sh=s, sw=s, ph=p, pw=p, dh=d, dw=d)
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
    L.check(lib.mr_qconv2d(xq.data_ptr(), C.byref(g), b.data_ptr(), bl.shape[1], bl.shape[0], C.byref(e), stream()),
            "mr_qconv2d")
    sync()
    to_nhwc = lambda a: a.transpose(0, 2, 3, 1).reshape(M, o)
    assert np.array_equal(acc.cpu().numpy(), to_nhwc(want_acc).astype(np.int32))
    assert bits_equal(y.cpu().numpy(), to_nhwc(want))
    assert bits_equal(yq.cpu().numpy()[:, :o], to_nhwc(G.quantize_activation(want, next_xs)).astype(np.int8))


# Epilogue forms the kernels compile straight-line code for (no int32
# accumulator output): each output kind and step combination on the conv
# loader modes that carry them, plus a form outside the list (fallback).
FORMS = {
    "relu_i8": ((("add", 1, False), ("relu", None, False)), False, True),
    "res_f32_i8": ((("add", 1, False), ("add", 2, False), ("relu", None, False)), True, True),
    "res_i8": ((("add", 1, False), ("add", 2, False), ("relu", None, False)), False, True),
    "res_f32": ((("add", 1, False), ("add", 2, False), ("relu", None, False)), True, False),
    "bias_f32": ((("add", 1, False),), True, False),
    "bias_relu6_f32": ((("add", 1, False), ("maximum", 3, False), ("minimum", 4, False)), True, False),
    "bias_f32_i8": ((("add", 1, False),), True, True),
    "bias_res_f32_i8": ((("add", 1, False), ("add", 2, False)), True, True),
    # MobileNet projections whose output no later residual reads: int8 only
    "bias_i8": ((("add", 1, False),), False, True),
    "bias_res_i8": ((("add", 1, False), ("add", 2, False)), False, True),
    # BatchNorm as MIRA's ONNX importer leaves it: a per-channel mul ahead of the bias
    "bn_relu_i8": ((("mul", 5, False), ("add", 1, False), ("relu", None, False)), False, True),
    "bn_res_f32_i8": ((("mul", 5, False), ("add", 1, False), ("add", 2, False), ("relu", None, False)), True, True),
    "bn_relu6_f32": ((("mul", 5, False), ("add", 1, False), ("maximum", 3, False), ("minimum", 4, False)), True,
                     False),
}
FORM_CONV_CASES = [
    (2, 64, 56, 56, 64, 3, 1, 1, 1),      # patch, 128x64 tiles
    (3, 64, 20, 20, 64, 3, 1, 1, 1),      # patch, last tile of each image 8 of 12 rows
    (2, 64, 7, 130, 64, 3, 1, 1, 1),      # patch, one 130-pixel row per tile
    (1, 64, 6, 9, 64, 3, 1, 0, 1),        # patch, no padding
    (2, 128, 28, 28, 128, 3, 1, 1, 1),    # patch, 128x128 tiles
    (1, 256, 7, 7, 96, 3, 1, 1, 1),       # patch, last column tile partial (run-time-flag rows)
    (2, 64, 15, 15, 128, 3, 2, 1, 1),     # stride 2, 64-channel loader
    (1, 256, 7, 7, 512, 3, 1, 1, 1),      # 128x256 tiles
    (2, 64, 14, 14, 128, 1, 2, 0, 1),     # downsample
    (2, 24, 14, 14, 144, 1, 1, 0, 1),     # 1x1 expansion as a dense GEMM (c_pad 32)
    (2, 96, 14, 14, 576, 1, 1, 0, 1),     # 1x1 expansion as a dense GEMM (c_pad 96)
    (2, 160, 7, 7, 960, 1, 1, 0, 1),      # 1x1 expansion as a dense GEMM, partial column tile
    (2, 3, 17, 17, 32, 3, 2, 1, 1),       # 3-channel stem, 4-channel loader
    (2, 32, 28, 28, 16, 1, 1, 0, 1),      # 1x1 projection to 16 channels (64x32 tiles)
    (2, 144, 14, 14, 24, 1, 1, 0, 1),     # 1x1 projection to 24 channels, K past one stage
    (2, 16, 28, 28, 96, 1, 1, 0, 1),      # 1x1 expansion 16 -> 96 as a dense GEMM: 96 of 128 tile columns
    (2, 64, 15, 15, 160, 3, 2, 1, 1),     # stride 2, 64-channel loader, 160 columns: last tile partial
    (4, 24, 56, 56, 144, 1, 1, 0, 1),     # 1x1 expansion, K in one step, large grid: 64x64 tiles, no ring
    (2, 16, 128, 128, 96, 1, 1, 0, 1),    # 1x1 expansion 16 -> 96, large grid: 128x128 tiles, no ring
    (1, 512, 7, 7, 512, 3, 1, 1, 1),      # batch-1 layer 4: a 16-tile grid, 64x32 tiles with 128-byte stages
    (1, 192, 9, 9, 96, 3, 2, 1, 1),       # small grid, c_pad 192: 64x32 tiles with 64-byte stages
    (42, 32, 112, 112, 16, 1, 1, 0, 1),   # 1x1 projection, one K step on over 32 64-row tiles per CU: 128x32
]


# forms of an f16 graph (results rounded to f16; operands are f16 values); _h16: the
# residual and the f32 result stored as IEEE halves, _h16r: only the residual
F16_FORMS = ["relu_i8_f16", "res_f32_i8_f16", "bias_f32_f16", "bias_relu6_f32_f16",
             "res_f32_i8_h16", "res_i8_h16", "res_f32_h16", "bias_f32_h16", "res_f32_i8_h16r", "res_f32_h16r",
             "bias_res_f32_i8_h16", "bn_res_f32_i8_h16"]


def _form_parts(form):
    """(base form, f16 graph, residual as halves, f32 result as halves)"""
    for suffix, res_h, out_h in (("_h16r", True, False), ("_h16", True, True), ("_f16", False, False)):
        if form.endswith(suffix):
            return form[:-len(suffix)], True, res_h, out_h
    return form, False, False, False


@pytest.mark.parametrize("form", list(FORMS) + F16_FORMS)
@pytest.mark.parametrize("n,c,h,w,o,k,s,p,d", FORM_CONV_CASES)
def test_qconv2d_epilogue_forms(lib, form, n, c, h, w, o, k, s, p, d):
    torch = _torch()
    base, f16, res_h16, out_h16 = _form_parts(form)
    steps, want_f32, want_i8 = FORMS[base]
    rng = np.random.default_rng(n * 1000 + c * 10 + k + 7)
    x = rng.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = rng.standard_normal((o, c, k, k)).astype(np.float32)
    q, ws = G.quantize_array(wt, 0)
    xs = float(np.abs(x).max()) / 127
    oh, ow = G.conv_out(h, k, s, p, d), G.conv_out(w, k, s, p, d)
    M = n * oh * ow
    bias = (rng.standard_normal((o, 1, 1)) * 0.1).astype(np.float32)
    res = rng.standard_normal((n, o, oh, ow)).astype(np.float32)
    zero, six = np.array(0, np.float32), np.array(6, np.float32)
    bn = rng.uniform(-1.5, 1.5, (o, 1, 1)).astype(np.float32)
    if f16:     # an f16 graph's tensors hold f16 values
        x, bias, res, bn = (a.astype(np.float16).astype(np.float32) for a in (x, bias, res, bn))
    attrs = {"q": q, "w_scale": ws, "x_scale": xs, "dtype": "f16" if f16 else "f32", "stride": (s, s),
             "padding": (p, p), "dilation": (d, d), "epilogue": steps}
    want = G.qconv2d([x, bias, res, zero, six, bn], attrs)
    next_xs = float(np.abs(want[np.isfinite(want)]).max()) / 127 or 1.0
    cp = pack.c_pad_for(c)
    xq = empty((n, h, w, cp), torch.int8)
    L.check(lib.mr_quantize_nchw_nhwc(T(x).data_ptr(), n, c, h, w, xq.data_ptr(), cp, xs, stream()), "q")
    bl = pack.pack_conv(q, cp)
    b = T(pack.device_weights(bl))
    scale = T(pack.combined_scale(xs, ws))
    g = L.ConvGeom(n=n, h=h, w=w, c=c, c_pad=cp, o=o, oh=oh, ow=ow, kh=k, kw=k, sh=s, sw=s, ph=p, pw=p, dh=d, dw=d)
    res_nhwc = res.transpose(0, 2, 3, 1).reshape(M, o)
    operands = {1: (L.BC_COL, T(bias.reshape(o)), 0),
                2: (L.BC_FULL, T(res_nhwc.astype(np.float16) if res_h16 else res_nhwc), o),
                3: (L.BC_SCALAR, T(zero.reshape(1)), 0), 4: (L.BC_SCALAR, T(six.reshape(1)), 0),
                5: (L.BC_COL, T(bn.reshape(o)), 0)}
    dev_steps = [(fn, 0, None, 0, sw) if idx is None else (fn, operands[idx][0], operands[idx][1], operands[idx][2], sw)
                 for fn, idx, sw in steps]
    y = empty((M, o), torch.float16 if out_h16 else torch.float32) if want_f32 else None
    ocp = pack.c_pad_for(o)
    yq = empty((M, ocp), torch.int8) if want_i8 else None
    e = epilogue(dev_steps, scale=scale, out_f32=y, ldo=o if want_f32 else 0, out_i8=yq, ldq=ocp if want_i8 else 0,
                 xs=next_xs)
    e.flags = (L.EPI_OUT_F16 if f16 else 0) | (L.EPI_OUT_H16 if out_h16 else 0) | (L.EPI_FULL_H16 if res_h16 else 0)
    L.check(lib.mr_qconv2d(xq.data_ptr(), C.byref(g), b.data_ptr(), bl.shape[1], bl.shape[0], C.byref(e), stream()),
            "mr_qconv2d")
    sync()
    to_nhwc = lambda a: a.transpose(0, 2, 3, 1).reshape(M, o)
    if want_f32:
        assert bits_equal(y.cpu().numpy().astype(np.float32), to_nhwc(want).astype(np.float32))
    if want_i8:
        assert bits_equal(yq.cpu().numpy()[:, :o], to_nhwc(G.quantize_activation(want, next_xs)).astype(np.int8))


def test_half_storage_flags_rejected_where_unsupported(lib):
    """Kernels without half-storage paths refuse the MR_EPI_*_H16 flags."""
    torch = _torch()
    x = empty((2, 8, 8, 16), torch.float32)
    wt = empty((9, 16), torch.float32)
    y = empty((128, 16), torch.float16)
    e = epilogue(out_f32=y, ldo=16)
    e.flags = L.EPI_OUT_H16
    g = L.ConvGeom(n=2, h=8, w=8, c=16, c_pad=16, o=16, oh=8, ow=8, kh=3, kw=3, sh=1, sw=1, ph=1, pw=1, dh=1, dw=1)
    assert lib.mr_dwconv2d_f32(x.data_ptr(), C.byref(g), wt.data_ptr(), C.byref(e), stream()) == 3
    assert "halves" in lib.mr_last_error().decode()


@pytest.mark.parametrize("form", ["relu_i8", "bias_f32", "res_f32_i8"])
@pytest.mark.parametrize("M,K,N", [(300, 512, 1000), (512, 256, 128), (64, 64, 10)])
def test_qmatmul_epilogue_forms(lib, form, M, K, N):
    torch = _torch()
    steps, want_f32, want_i8 = FORMS[form]
    rng = np.random.default_rng(M + N + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((K, N)) / np.sqrt(K)).astype(np.float32)
    q, ws = G.quantize_array(w, 1)
    xs = float(np.abs(x).max()) / 127
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    res = rng.standard_normal((M, N)).astype(np.float32)
    attrs = {"q": q, "w_scale": ws, "x_scale": xs, "dtype": "f32", "epilogue": steps}
    want = G.qmatmul([x, bias, res], attrs)
    next_xs = float(np.abs(want[np.isfinite(want)]).max()) / 127 or 1.0
    lda = pack.row_stride_for(K)
    xq = empty((M, lda), torch.int8)
    L.check(lib.mr_quantize_rows(T(x).data_ptr(), M, K, K, xq.data_ptr(), lda, xs, stream()), "q")
    bl = pack.pack_matmul(q)
    b = T(pack.device_weights(bl))
    bias_t, res_t = T(bias), T(res)
    dev_steps = [(fn, 0, None, 0, sw) if idx is None else
                 ((fn, L.BC_COL, bias_t, 0, sw) if idx == 1 else (fn, L.BC_FULL, res_t, N, sw))
                 for fn, idx, sw in steps]
    y = empty((M, N), torch.float32) if want_f32 else None
    ldq = pack.row_stride_for(N)
    yq = empty((M, ldq), torch.int8) if want_i8 else None
    sc = T(pack.combined_scale(xs, ws))        # named: kept alive until the kernel has run
    e = epilogue(dev_steps, scale=sc, out_f32=y, ldo=N if want_f32 else 0, out_i8=yq,
                 ldq=ldq if want_i8 else 0, xs=next_xs)
    L.check(lib.mr_qmatmul(xq.data_ptr(), lda, b.data_ptr(), bl.shape[1], bl.shape[0], M, N, K, C.byref(e), stream()),
            "mr_qmatmul")
    sync()
    if want_f32:
        assert bits_equal(y.cpu().numpy(), want)
    if want_i8:
        assert bits_equal(yq.cpu().numpy()[:, :N], G.quantize_activation(want, next_xs).astype(np.int8))


# ---------------------------------------------------------------- K4a depthwise, adjuncts

@pytest.mark.parametrize("n,c,h,s,k,form,ldo_pad", [
    (2, 32, 16, 1, 3, "relu6", 0),      # 3x3, 4-channel runs: vectorized kernel, 2 columns per thread
    (1, 8, 30, 1, 3, "relu6", 0),       # 4 columns per thread, last tile 2 of 4
    (2, 144, 15, 2, 3, "relu6", 0),     # stride 2, last column tile partial
    (1, 960, 7, 1, 3, "relu6", 0),      # 7 columns: one full and one partial tile
    (3, 24, 11, 1, 3, "relu6", 0),      # 11 output rows: the last row pair of a thread half past the map
    (1, 16, 17, 2, 3, "relu6", 0),      # stride 2, 9 output rows: the same at stride 2
    (2, 8, 13, 2, 3, "generic", 0),     # step interpreter epilogue (swapped subtract)
    (2, 16, 9, 1, 3, "relu6", 1),       # f32 rows not 16-byte aligned: element stores
    (1, 6, 9, 1, 3, "relu6", 0),        # 6 channels: per-element kernel
    (2, 8, 11, 1, 5, "relu6", 0),       # 5x5: per-element kernel
])
def test_dwconv_relu6(lib, n, c, h, s, k, form, ldo_pad):
    torch = _torch()
    rng = np.random.default_rng(c + k)
    x = (rng.standard_normal((n, c, h, h)) * 2).astype(np.float32)
    wt = rng.standard_normal((c, 1, k, k)).astype(np.float32)
    bias = (rng.standard_normal((c, 1, 1)) * 0.1).astype(np.float32)
    zero, six = np.array(0, np.float32), np.array(6, np.float32)
    p = k // 2
    steps = ((("add", 2, False), ("maximum", 3, False), ("minimum", 4, False)) if form == "relu6" else
             (("sub", 2, True), ("relu", None, False)))
    attrs = {"stride": (s, s), "padding": (p, p), "groups": c, "epilogue": steps}
    want = G.conv2d([x, wt, bias, zero, six], attrs)
    oh = want.shape[2]
    xs_next = float(want.max()) / 127 or 1.0
    xd = T(x.transpose(0, 2, 3, 1))
    wd = T(np.ascontiguousarray(wt[:, 0].transpose(1, 2, 0)))
    g = L.ConvGeom(n=n, h=h, w=h, c=c, c_pad=c, o=c, oh=oh, ow=oh, kh=k, kw=k, sh=s, sw=s, ph=p, pw=p, dh=1, dw=1)
    M = n * oh * oh
    ldo = c + ldo_pad
    y = empty((M, ldo), torch.float32)
    cp = pack.c_pad_for(c)
    yq = empty((M, cp), torch.int8)
    bt, zt, st = T(bias.reshape(c)), T(zero.reshape(1)), T(six.reshape(1))
    dev_steps = ([("add", L.BC_COL, bt, 0, False), ("maximum", L.BC_SCALAR, zt, 0, False),
                  ("minimum", L.BC_SCALAR, st, 0, False)] if form == "relu6" else
                 [("sub", L.BC_COL, bt, 0, True), ("relu", 0, None, 0, False)])
    e = epilogue(dev_steps, out_f32=y, ldo=ldo, out_i8=yq, ldq=cp, xs=xs_next)
    L.check(lib.mr_dwconv2d_f32(xd.data_ptr(), C.byref(g), wd.data_ptr(), C.byref(e), stream()), "dw")
    sync()
    assert bits_equal(y.cpu().numpy()[:, :c], want.transpose(0, 2, 3, 1).reshape(M, c))
    assert bits_equal(yq.cpu().numpy()[:, :c],
                      G.quantize_activation(want, xs_next).astype(np.int8).transpose(0, 2, 3, 1).reshape(M, c))


# ---------------------------------------------------------------- fused 1x1 expansion + 3x3 depthwise

def _expand_dw_case(lib, n, k, c, h, s, f32_out, seed, inf_bias=False, f16=False):
    """A MobileNet block's expansion (1x1 qconv2d, bias, ReLU6 -> f32) and depthwise
    conv (3x3, bias, ReLU6 -> int8 and optionally f32) as one mr_qconv1x1_dw3x3 launch.
    Returns (rc, got int8, got f32 or None, want int8, want f32)."""
    torch = _torch()
    rng = np.random.default_rng(seed)
    x = rng.uniform(-1, 1, (n, k, h, h)).astype(np.float32)
    we = rng.standard_normal((c, k, 1, 1)).astype(np.float32)
    q, ws = G.quantize_array(we, 0)
    xs = float(np.abs(x).max()) / 127
    be = (rng.standard_normal((c, 1, 1)) * 0.5).astype(np.float32)
    if inf_bias:    # channels whose expansion saturates: the exact (non-median) epilogue path
        be[3], be[5] = np.inf, -np.inf
    wd = (rng.standard_normal((c, 1, 3, 3)) * 0.5).astype(np.float32)
    bd = (rng.standard_normal((c, 1, 1)) * 0.5).astype(np.float32)
    if inf_bias:    # and depthwise outputs that saturate
        bd[6], bd[9] = np.inf, -np.inf
    zero, six = np.array(0, np.float32), np.array(6, np.float32)
    if f16:     # an f16 graph: f16 constants, both results rounded to f16
        be, wd, bd, zero, six = (a.astype(np.float16) for a in (be, wd, bd, zero, six))
    r6 = (("add", 1, False), ("maximum", 2, False), ("minimum", 3, False))
    ea = {"q": q, "w_scale": ws, "x_scale": xs, "dtype": "f16" if f16 else "f32", "stride": (1, 1),
          "padding": (0, 0), "epilogue": r6}
    want_e = G.qconv2d([x, be, zero, six], ea)
    da = {"stride": (s, s), "padding": (1, 1), "groups": c,
          "epilogue": (("add", 2, False), ("maximum", 3, False), ("minimum", 4, False))}
    want = G.conv2d([want_e, wd, bd, zero, six], da)
    assert want.dtype == (np.float16 if f16 else np.float32)
    be, wd, bd, zero, six = (np.asarray(a, np.float32) for a in (be, wd, bd, zero, six))
    oh = want.shape[2]
    next_xs = float(np.abs(want).max()) / 127 or 1.0
    want_q = G.quantize_activation(want, next_xs).astype(np.int8).transpose(0, 2, 3, 1).reshape(-1, c)
    cp = pack.c_pad_for(k)
    xq = empty((n, h, h, cp), torch.int8)
    L.check(lib.mr_quantize_nchw_nhwc(T(x).data_ptr(), n, k, h, h, xq.data_ptr(), cp, xs, stream()), "q")
    bl = pack.pack_conv(q, cp)
    b = T(pack.device_weights(bl))
    keep = [T(be.reshape(c)), T(zero.reshape(1)), T(six.reshape(1)), T(bd.reshape(c)),
            T(pack.combined_scale(xs, ws)), T(np.ascontiguousarray(wd[:, 0].transpose(1, 2, 0)))]
    bet, zt, st, bdt, scale, wdt = keep
    ee = epilogue([("add", L.BC_COL, bet, 0, False), ("maximum", L.BC_SCALAR, zt, 0, False),
                   ("minimum", L.BC_SCALAR, st, 0, False)], scale=scale)
    M = n * oh * oh
    ldq = pack.c_pad_for(c)
    yq = torch.full((M, ldq), 99, dtype=torch.int8, device="cuda")
    y = torch.full((M, c), float("nan"), dtype=torch.float32, device="cuda") if f32_out else None
    ed = epilogue([("add", L.BC_COL, bdt, 0, False), ("maximum", L.BC_SCALAR, zt, 0, False),
                   ("minimum", L.BC_SCALAR, st, 0, False)], out_f32=y, ldo=c, out_i8=yq, ldq=ldq, xs=next_xs)
    if f16:
        ee.flags = ed.flags = L.EPI_OUT_F16
    g = L.ConvGeom(n=n, h=h, w=h, c=c, c_pad=c, o=c, oh=oh, ow=oh, kh=3, kw=3, sh=s, sw=s, ph=1, pw=1, dh=1, dw=1)
    rc = lib.mr_qconv1x1_dw3x3(xq.data_ptr(), cp, b.data_ptr(), bl.shape[1], bl.shape[0], k, C.byref(ee), C.byref(g),
                               wdt.data_ptr(), C.byref(ed), stream())
    sync()
    got_q = yq.cpu().numpy()
    assert (got_q[:, c:] == 99).all()          # nothing written past the c channels
    got = y.cpu().numpy() if f32_out else None
    return rc, got_q[:, :c], got, want_q, want.astype(np.float32).transpose(0, 2, 3, 1).reshape(-1, c)


@pytest.mark.parametrize("n,k,c,h,s,f32_out", [
    (2, 16, 96, 112, 2, False),     # MobileNetV2 block 2 (k_pad 64, stride 2, 7x7 tiles)
    (2, 24, 144, 56, 1, False),     # 144 channels: a half-empty last 32-channel block; 14x14 tiles
    (2, 24, 144, 56, 2, True),      # with the f32 result too
    (1, 32, 192, 28, 1, False),
    (3, 64, 384, 14, 1, False),     # 12 channel blocks split over workgroups
    (2, 96, 576, 14, 2, False),     # k_pad 128
    (2, 160, 960, 7, 1, True),      # k_pad 192, one 7x7 tile per image
    (2, 40, 100, 17, 2, False),     # ragged: K 40 (row stride 48), 100 channels, odd image
    (1, 16, 36, 13, 1, False),      # partial tiles (13 = 7 + 6), 36 channels
    (2, 8, 32, 9, 1, True),         # K below one 16-byte chunk of the 16-byte row stride
])
def test_qconv1x1_dw3x3(lib, n, k, c, h, s, f32_out):
    rc, got_q, got, want_q, want = _expand_dw_case(lib, n, k, c, h, s, f32_out, n * 100 + k + c + h)
    assert rc == 0, lib.mr_last_error()
    assert bits_equal(got_q, want_q)
    if f32_out:
        assert bits_equal(got, want)


@pytest.mark.parametrize("n,k,c,h,s,f32_out", [(2, 16, 96, 56, 2, False), (2, 24, 144, 28, 1, True),
                                                (1, 160, 960, 7, 1, False)])
def test_qconv1x1_dw3x3_f16(lib, n, k, c, h, s, f32_out):
    """The f16 graph's pair: f16 constants, the expanded values and the depthwise results
    rounded to f16 after their epilogues (the f32 result holds those f16 values)."""
    rc, got_q, got, want_q, want = _expand_dw_case(lib, n, k, c, h, s, f32_out, n + k + c, f16=True)
    assert rc == 0, lib.mr_last_error()
    assert bits_equal(got_q, want_q)
    if f32_out:
        assert bits_equal(got, want)


@pytest.mark.parametrize("f32_out", [True, False])
def test_qconv1x1_dw3x3_infinite_bias(lib, f32_out):
    """A first channel block whose expansion and depthwise biases hold +inf and -inf takes
    the exact maximum/minimum epilogues (ReLU6 gives 6 and 0 there), the other blocks the
    median ones (the depthwise median only without an f32 result)."""
    rc, got_q, got, want_q, want = _expand_dw_case(lib, 2, 24, 96, 20, 1, f32_out, 5, inf_bias=True)
    assert rc == 0, lib.mr_last_error()
    assert bits_equal(got_q, want_q)
    if f32_out:
        assert bits_equal(got, want)


@pytest.mark.parametrize("n,cin,c,h,ss,s", [
    (2, 3, 32, 224, 2, 1),      # MobileNetV2's stem and first depthwise conv (14x14 tiles)
    (2, 3, 32, 30, 2, 1),       # partial tiles
    (1, 3, 16, 17, 2, 2),       # odd image, depthwise stride 2
    (2, 2, 48, 20, 1, 1),       # stride-1 stem, 2 channels, 48 outputs (a half-empty channel block)
])
def test_qstem3x3_dw3x3(lib, n, cin, c, h, ss, s):
    """The 3x3 stem (over an image stored 4 bytes per pixel) fused with the depthwise conv
    that reads its result: against the oracle's qconv2d and depthwise conv2d, bit for bit."""
    torch = _torch()
    rng = np.random.default_rng(n * 7 + c + h)
    x = rng.uniform(-1, 1, (n, cin, h, h)).astype(np.float32)
    we = rng.standard_normal((c, cin, 3, 3)).astype(np.float32)
    q, ws = G.quantize_array(we, 0)
    xs = float(np.abs(x).max()) / 127
    be = (rng.standard_normal((c, 1, 1)) * 0.5).astype(np.float32)
    wd = (rng.standard_normal((c, 1, 3, 3)) * 0.5).astype(np.float32)
    bd = (rng.standard_normal((c, 1, 1)) * 0.5).astype(np.float32)
    zero, six = np.array(0, np.float32), np.array(6, np.float32)
    r6 = (("add", 1, False), ("maximum", 2, False), ("minimum", 3, False))
    ea = {"q": q, "w_scale": ws, "x_scale": xs, "dtype": "f32", "stride": (ss, ss), "padding": (1, 1),
          "epilogue": r6}
    want_e = G.qconv2d([x, be, zero, six], ea)
    sh = want_e.shape[2]
    want = G.conv2d([want_e, wd, bd, zero, six], {"stride": (s, s), "padding": (1, 1), "groups": c,
                                                   "epilogue": (("add", 2, False), ("maximum", 3, False),
                                                                ("minimum", 4, False))})
    oh = want.shape[2]
    next_xs = float(np.abs(want).max()) / 127 or 1.0
    want_q = G.quantize_activation(want, next_xs).astype(np.int8).transpose(0, 2, 3, 1).reshape(-1, c)
    xq = empty((n, h, h, 4), torch.int8)
    L.check(lib.mr_quantize_nchw_nhwc(T(x).data_ptr(), n, cin, h, h, xq.data_ptr(), 4, xs, stream()), "q")
    bl = pack.pack_conv(q, 4)
    assert bl.shape[1] == 64
    b = T(pack.device_weights(bl))
    keep = [T(be.reshape(c)), T(zero.reshape(1)), T(six.reshape(1)), T(bd.reshape(c)),
            T(pack.combined_scale(xs, ws)), T(np.ascontiguousarray(wd[:, 0].transpose(1, 2, 0)))]
    bet, zt, st, bdt, scale, wdt = keep
    ee = epilogue([("add", L.BC_COL, bet, 0, False), ("maximum", L.BC_SCALAR, zt, 0, False),
                   ("minimum", L.BC_SCALAR, st, 0, False)], scale=scale)
    M = n * oh * oh
    ldq = pack.c_pad_for(c)
    yq = torch.full((M, ldq), 99, dtype=torch.int8, device="cuda")
    ed = epilogue([("add", L.BC_COL, bdt, 0, False), ("maximum", L.BC_SCALAR, zt, 0, False),
                   ("minimum", L.BC_SCALAR, st, 0, False)], out_i8=yq, ldq=ldq, xs=next_xs)
    sg = L.ConvGeom(n=n, h=h, w=h, c=cin, c_pad=4, o=c, oh=sh, ow=sh, kh=3, kw=3, sh=ss, sw=ss, ph=1, pw=1, dh=1,
                    dw=1)
    g = L.ConvGeom(n=n, h=sh, w=sh, c=c, c_pad=c, o=c, oh=oh, ow=oh, kh=3, kw=3, sh=s, sw=s, ph=1, pw=1, dh=1, dw=1)
    rc = lib.mr_qstem3x3_dw3x3(xq.data_ptr(), C.byref(sg), b.data_ptr(), bl.shape[1], bl.shape[0], C.byref(ee),
                               C.byref(g), wdt.data_ptr(), C.byref(ed), stream())
    sync()
    assert rc == 0, lib.mr_last_error()
    got = yq.cpu().numpy()
    assert (got[:, c:] == 99).all()
    assert bits_equal(got[:, :c], want_q)


def test_qconv1x1_dw3x3_rejects(lib):
    """Forms it has no kernel for return MR_EUNSUPPORTED (the target makes two launches);
    an expansion epilogue that stores its result is an argument error."""
    torch = _torch()
    x = empty((1, 8, 8, 256), torch.int8)
    b = empty((4, 64, 64), torch.int8)
    w = empty((9, 64), torch.float32)
    z, six, bias, sc = empty((1,), torch.float32), empty((1,), torch.float32), empty((64,), torch.float32), \
        empty((64,), torch.float64)
    r6 = [("add", L.BC_COL, bias, 0, False), ("maximum", L.BC_SCALAR, z, 0, False),
          ("minimum", L.BC_SCALAR, six, 0, False)]
    yq = empty((64, 64), torch.int8)
    g = L.ConvGeom(n=1, h=8, w=8, c=64, c_pad=64, o=64, oh=8, ow=8, kh=3, kw=3, sh=1, sw=1, ph=1, pw=1, dh=1, dw=1)
    ed = epilogue(r6, out_i8=yq, ldq=64, xs=0.1)

    def call(ee, k_pad=64, K=64, dw=ed):
        return lib.mr_qconv1x1_dw3x3(x.data_ptr(), 256, b.data_ptr(), k_pad, 64, K, C.byref(ee), C.byref(g),
                                     w.data_ptr(), C.byref(dw), stream())
    assert call(epilogue(r6, scale=sc), k_pad=256, K=256) == 3             # k_pad above 192
    assert call(epilogue(r6[:2], scale=sc)) == 3                          # ReLU without the upper bound
    f16 = epilogue(r6, scale=sc)
    f16.flags = L.EPI_OUT_F16
    assert call(f16) == 3                                       # f16 rounding on one convolution only
    assert call(epilogue(r6, scale=sc, out_i8=yq, ldq=64, xs=0.1)) == 1    # the expansion stores its result
    assert call(epilogue(r6, scale=sc), dw=epilogue(r6, out_f32=empty((64, 64), torch.float32), ldo=64)) == 1
    sync()


def test_maxpool_with_folded_pad(lib):
    torch = _torch()
    rng = np.random.default_rng(12)
    n, c, h = 2, 64, 112
    x = np.maximum(rng.standard_normal((n, c, h, h)), 0).astype(np.float32)
    p = G.pad([x], {"pads": ((0, 0), (0, 0), (1, 1), (1, 1)), "value": -np.inf})
    want = G.maxpool2d([p], {"size": 3, "stride": 2})
    oh = want.shape[2]
    xs = float(want.max()) / 127
    y = empty((n, oh, oh, c), torch.float32)
    yq = empty((n, oh, oh, c), torch.int8)
    L.check(lib.mr_maxpool2d_f32(T(x.transpose(0, 2, 3, 1)).data_ptr(), n, h, h, c, 3, 2, 1, 1, float("-inf"), oh, oh,
                                 y.data_ptr(), yq.data_ptr(), c, xs, stream()), "maxpool")
    sync()
    assert bits_equal(y.cpu().numpy(), want.transpose(0, 2, 3, 1))
    assert bits_equal(yq.cpu().numpy(), G.quantize_activation(want, xs).astype(np.int8).transpose(0, 2, 3, 1))


@pytest.mark.parametrize("hw", [(7, 7), (1, 5), (14, 14), (56, 56)])
@pytest.mark.parametrize("f16", [False, True])
def test_mean_hw(lib, hw, f16):
    """The mean over H*W in NumPy's order; with f16 (an f16 graph) its f16 rounding, and the
    int8 quantize of that rounded mean."""
    torch = _torch()
    rng = np.random.default_rng(hw[0])
    n, c = 3, 512
    x = (rng.standard_normal((n, c) + hw) * 4).astype(np.float32)
    if f16:
        x = x.astype(np.float16).astype(np.float32)
    want = G.reduce("reduce_mean", [x], {"axes": (2, 3), "keepdims": True}).reshape(n, c)
    if f16:
        want = want.astype(np.float16).astype(np.float32)
    xs = float(np.abs(want).max()) / 127
    y = empty((n, c), torch.float32)
    yq = empty((n, c), torch.int8)
    L.check(lib.mr_mean_hw_f32(T(x.transpose(0, 2, 3, 1)).data_ptr(), n, hw[0] * hw[1], c, y.data_ptr(),
                               yq.data_ptr(), c, xs, int(f16), stream()), "mean")
    sync()
    assert bits_equal(y.cpu().numpy(), want)
    assert bits_equal(yq.cpu().numpy(), G.quantize_activation(want, xs).astype(np.int8))


def test_pad_and_layouts(lib):
    torch = _torch()
    rng = np.random.default_rng(13)
    x = rng.standard_normal((2, 5, 7, 9)).astype(np.float32)
    xd = T(x)
    nhwc = empty((2, 7, 9, 5), torch.float32)
    back = empty((2, 5, 7, 9), torch.float32)
    L.check(lib.mr_nchw_to_nhwc_f32(xd.data_ptr(), 2, 5, 7, 9, nhwc.data_ptr(), stream()), "t")
    L.check(lib.mr_nhwc_to_nchw_f32(nhwc.data_ptr(), 2, 5, 7, 9, back.data_ptr(), stream()), "t")
    padded = empty((2, 7 + 3, 9 + 1, 5), torch.float32)
    L.check(lib.mr_pad_hw_f32(nhwc.data_ptr(), 2, 7, 9, 5, 1, 2, 0, 1, -7.5, padded.data_ptr(), stream()), "pad")
    sync()
    assert bits_equal(nhwc.cpu().numpy(), x.transpose(0, 2, 3, 1))
    assert bits_equal(back.cpu().numpy(), x)
    want = G.pad([x], {"pads": ((0, 0), (0, 0), (1, 2), (0, 1)), "value": -7.5}).transpose(0, 2, 3, 1)
    assert bits_equal(padded.cpu().numpy(), want)


@pytest.mark.parametrize("n,c,h,w,c_pad", [(2, 3, 7, 9, 4), (1, 3, 224, 224, 4), (3, 5, 4, 6, 8), (2, 1, 3, 3, 4)])
def test_nchw_to_nhwc_pad(lib, n, c, h, w, c_pad):
    """The channel-padded NHWC copy of a weight-only convolution's input: the channels in
    order, then zeros (NaN-filled output first, so every element is written)."""
    torch = _torch()
    x = np.random.default_rng(c * 31 + h).standard_normal((n, c, h, w)).astype(np.float32)
    y = torch.full((n, h, w, c_pad), float("nan"), dtype=torch.float32, device="cuda")
    L.check(lib.mr_nchw_to_nhwc_pad_f32(T(x).data_ptr(), n, c, h, w, y.data_ptr(), c_pad, stream()), "pad")
    sync()
    want = np.zeros((n, h, w, c_pad), np.float32)
    want[..., :c] = x.transpose(0, 2, 3, 1)
    assert bits_equal(y.cpu().numpy(), want)


def test_nchw_to_nhwc_pad_rejects(lib):
    """c_pad below c or not a multiple of 4 is an argument error, nothing launched."""
    torch = _torch()
    x = empty((1, 3, 4, 4), torch.float32)
    y = empty((1, 4, 4, 8), torch.float32)
    for c_pad in (2, 6):
        assert lib.mr_nchw_to_nhwc_pad_f32(x.data_ptr(), 1, 3, 4, 4, y.data_ptr(), c_pad, stream()) == 1


# ---------------------------------------------------------------- fused stem (conv -> pad -> maxpool)

@pytest.mark.parametrize("n,c,h,o,k,s,p,pool,pst,ppad,pval,neg", [
    (2, 3, 224, 64, 7, 2, 3, 3, 2, 1, float("-inf"), False),   # ResNet-18 stem
    (2, 3, 224, 64, 7, 2, 3, 3, 2, 1, float("-inf"), True),    # every accumulator negative
    (3, 3, 37, 32, 3, 2, 1, 3, 2, 1, float("-inf"), False),    # odd sizes, 3 taps per row
    (2, 1, 30, 16, 5, 1, 2, 2, 2, 0, 0.0, False),              # no pool padding
    (2, 4, 29, 48, 7, 2, 3, 3, 2, 1, 0.25, True),              # finite pad value
])
def test_qconv2d_maxpool(lib, n, c, h, o, k, s, p, pool, pst, ppad, pval, neg):
    torch = _torch()
    rng = np.random.default_rng(h + o)
    x = rng.uniform(-1, 1, (n, c, h, h)).astype(np.float32)
    wt = rng.standard_normal((o, c, k, k)).astype(np.float32)
    if neg:      # x > 0, w < 0: window maxima are negative, so the identity of max matters
        x, wt = np.abs(x) + 0.01, -np.abs(wt)
    q, ws = G.quantize_array(wt, 0)
    xs = float(np.abs(x).max()) / 127
    bias = (rng.standard_normal((o, 1, 1)) * 0.3).astype(np.float32)
    steps = (("add", 1, False),) if neg else (("add", 1, False), ("relu", None, False))
    attrs = {"q": q, "w_scale": ws, "x_scale": xs, "dtype": "f32", "stride": (s, s), "padding": (p, p),
             "epilogue": steps}
    conv = G.qconv2d([x, bias], attrs)
    padded = G.pad([conv], {"pads": ((0, 0), (0, 0), (ppad, ppad), (ppad, ppad)), "value": pval})
    want = G.maxpool2d([padded], {"size": pool, "stride": pst})
    oh = conv.shape[2]
    poh = want.shape[2]
    next_xs = float(np.abs(want[np.isfinite(want)]).max()) / 127
    cp = 4
    xq = empty((n, h, h, cp), torch.int8)
    L.check(lib.mr_quantize_nchw_nhwc(T(x).data_ptr(), n, c, h, h, xq.data_ptr(), cp, xs, stream()), "q")
    bl = pack.pack_conv(q, cp, min_rows=64)
    b = T(pack.device_weights(bl))
    scale = T(pack.combined_scale(xs, ws))
    g = L.ConvGeom(n=n, h=h, w=h, c=c, c_pad=cp, o=o, oh=oh, ow=oh, kh=k, kw=k, sh=s, sw=s, ph=p, pw=p, dh=1, dw=1)
    M = n * poh * poh
    y = empty((M, o), torch.float32)
    ocp = pack.c_pad_for(o)
    yq = empty((M, ocp), torch.int8)
    bt = T(bias.reshape(o))
    dev_steps = [("add", L.BC_COL, bt, 0, False)] + ([] if neg else [("relu", 0, None, 0, False)])
    e = epilogue(dev_steps, scale=scale, out_f32=y, ldo=o, out_i8=yq, ldq=ocp, xs=next_xs)
    L.check(lib.mr_qconv2d_maxpool(xq.data_ptr(), C.byref(g), b.data_ptr(), bl.shape[1], bl.shape[0], C.byref(e),
                                   pool, pst, ppad, ppad, pval, poh, poh, stream()), "mr_qconv2d_maxpool")
    sync()
    to_rows = lambda a: a.transpose(0, 2, 3, 1).reshape(M, o)
    assert bits_equal(y.cpu().numpy(), to_rows(want))
    assert bits_equal(yq.cpu().numpy()[:, :o], to_rows(G.quantize_activation(want, next_xs)).astype(np.int8))


@pytest.mark.parametrize("n,c,h,w,o,kw,sh,sw,pool,pval,f16,neg", [
    (2, 3, 224, 224, 64, 7, 2, 2, 3, float("-inf"), False, False),   # ResNet-18 stem from the f32 image
    (2, 3, 224, 224, 64, 7, 2, 2, 3, float("-inf"), True, False),    # f16 graph: quantize the f16 rounding
    (3, 1, 61, 45, 32, 7, 2, 2, 3, 0.25, False, True),               # odd sizes, finite pad, negative maxima
    (2, 4, 40, 38, 16, 6, 2, 2, 2, 0.0, False, False),               # 4 channels, 6 taps, 2x2 pool
    (2, 2, 23, 50, 64, 5, 1, 2, 3, float("-inf"), True, False),      # row stride 1, 5 taps
])
def test_qconv2d_maxpool_f32in(lib, n, c, h, w, o, kw, sh, sw, pool, pval, f16, neg):
    """The stem reading the f32 NCHW image (quantized per band into LDS) against the unfused
    quantize + mr_qconv2d_maxpool and against the oracle, bit for bit.  The image holds
    exact quantization ties, values far past the clip range and infinities."""
    torch = _torch()
    rng = np.random.default_rng(h * w + o)
    kh, ph, pw = 7, 3, kw // 2
    xs = 2.0 ** -6
    x = rng.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    flat = x.reshape(-1)
    picks = rng.choice(flat.size, 64, replace=False)
    flat[picks[:32]] = (rng.integers(-100, 100, 32) + 0.5) * xs       # ties: half to even
    flat[picks[32:48]] = rng.choice([-3.0, 5.0, np.inf, -np.inf], 16)  # clipped to +-127
    wt = rng.standard_normal((o, c, kh, kw)).astype(np.float32)
    if neg:
        x, wt = np.abs(x) + 0.01, -np.abs(wt)
    q, ws = G.quantize_array(wt, 0)
    bias = (rng.standard_normal((o, 1, 1)) * 0.3).astype(np.float32)
    steps = (("add", 1, False),) if neg else (("add", 1, False), ("relu", None, False))
    attrs = {"q": q, "w_scale": ws, "x_scale": xs, "dtype": "f32", "stride": (sh, sw), "padding": (ph, pw),
             "epilogue": steps}
    x_in = x.astype(np.float16).astype(np.float32) if f16 else x
    conv = G.qconv2d([x_in, bias], attrs)
    ppad = 1 if pool == 3 else 0
    padded = G.pad([conv], {"pads": ((0, 0), (0, 0), (ppad, ppad), (ppad, ppad)), "value": pval})
    want = G.maxpool2d([padded], {"size": pool, "stride": 2})
    oh, ow = conv.shape[2:]
    poh, pw_ = want.shape[2:]
    next_xs = float(np.abs(want[np.isfinite(want)]).max()) / 127
    cp = 4
    bl = pack.pack_conv(q, cp, min_rows=64)
    b = T(pack.device_weights(bl))
    scale = T(pack.combined_scale(xs, ws))
    g = L.ConvGeom(n=n, h=h, w=w, c=c, c_pad=cp, o=o, oh=oh, ow=ow, kh=kh, kw=kw, sh=sh, sw=sw, ph=ph, pw=pw, dh=1,
                   dw=1)
    M = n * poh * pw_
    ocp = pack.c_pad_for(o)
    bt = T(bias.reshape(o))
    dev_steps = [("add", L.BC_COL, bt, 0, False)] + ([] if neg else [("relu", 0, None, 0, False)])
    xd = T(x)
    outs = []
    for fused in (True, False):
        y, yq = empty((M, o), torch.float32), empty((M, ocp), torch.int8)
        e = epilogue(dev_steps, scale=scale, out_f32=y, ldo=o, out_i8=yq, ldq=ocp, xs=next_xs)
        print(f"f32in n={n} c={c} {h}x{w} o={o} kw={kw} stride=({sh},{sw}) pool={pool} f16={f16} fused={fused}",
              flush=True)
        if fused:
            L.check(lib.mr_qconv2d_maxpool_f32in(xd.data_ptr(), xs, int(f16), C.byref(g), b.data_ptr(), bl.shape[1],
                                                 bl.shape[0], C.byref(e), pool, 2, ppad, ppad, pval, poh, pw_,
                                                 stream()), "mr_qconv2d_maxpool_f32in")
        else:
            xq = empty((n, h, w, cp), torch.int8)
            quant = lib.mr_quantize_f16_nchw_nhwc if f16 else lib.mr_quantize_nchw_nhwc
            L.check(quant(xd.data_ptr(), n, c, h, w, xq.data_ptr(), cp, xs, stream()), "quantize")
            L.check(lib.mr_qconv2d_maxpool(xq.data_ptr(), C.byref(g), b.data_ptr(), bl.shape[1], bl.shape[0],
                                           C.byref(e), pool, 2, ppad, ppad, pval, poh, pw_, stream()),
                    "mr_qconv2d_maxpool")
        sync()
        outs.append((y.cpu().numpy(), yq.cpu().numpy()[:, :o]))
    to_rows = lambda a: a.transpose(0, 2, 3, 1).reshape(M, o)
    assert bits_equal(outs[0][0], outs[1][0]) and bits_equal(outs[0][1], outs[1][1])
    assert bits_equal(outs[0][0], to_rows(want))
    assert bits_equal(outs[0][1], to_rows(G.quantize_activation(want, next_xs)).astype(np.int8))


def test_qconv2d_maxpool_f32in_rejects(lib):
    """Shapes the f32-input stem has no kernel for answer MR_EUNSUPPORTED (3) before any launch."""
    g = L.ConvGeom(n=1, h=64, w=64, c=3, c_pad=4, o=64, oh=32, ow=32, kh=5, kw=5, sh=2, sw=2, ph=2, pw=2, dh=1, dw=1)
    e = epilogue(scale=T(np.ones(64)), out_f32=empty((16 * 16, 64), _torch().float32), ldo=64)
    x, b = T(np.zeros((1, 3, 64, 64), np.float32)), T(np.zeros((64, 192), np.int8))
    assert lib.mr_qconv2d_maxpool_f32in(x.data_ptr(), 0.1, 0, C.byref(g), b.data_ptr(), 192, 64, C.byref(e), 3, 2, 1,
                                        1, float("-inf"), 16, 16, stream()) == 3
    assert "7-row kernel" in lib.mr_last_error().decode()


@pytest.mark.parametrize("kind,shape", [("matmul", (300, 512, 256)), ("matmul", (4096, 1152, 128)),
                                        ("conv", (2, 64, 56, 56, 64, 3, 1, 1)),      # patch tiles
                                        ("conv", (2, 256, 14, 14, 512, 3, 1, 1)),    # 128x256 tiles
                                        ("conv", (4, 128, 28, 28, 256, 3, 2, 1))])   # stride 2
def test_int8_epilogue_ties(lib, kind, shape):
    """bias + ReLU -> int8 where every odd accumulator lands exactly on a rounding midpoint:
    power-of-two scales make y / next_xs = acc / 2 + integer, so the requant must round each
    of these exact ties half to even, as NumPy's rint does."""
    torch = _torch()
    rng = np.random.default_rng(sum(shape))
    xs, wsv, next_xs = 2.0 ** -5, np.float32(2.0 ** -7), 2.0 ** -11
    if kind == "matmul":
        M, K, N = shape
        xi = rng.integers(-1, 2, (M, K))
        q = rng.integers(-3, 4, (K, N)).astype(np.int8)
        o = N
    else:
        n, c, h, w, o, k, s, p = shape
        xi = rng.integers(-1, 2, (n, c, h, w))
        q = rng.integers(-3, 4, (o, c, k, k)).astype(np.int8)
    x = (xi * xs).astype(np.float32)
    ws = np.full(o, wsv, np.float32)
    bias = (rng.integers(-20, 20, o) * next_xs).astype(np.float32)
    steps = (("add", 1, False), ("relu", None, False))
    scale = T(pack.combined_scale(xs, ws))
    if kind == "matmul":
        attrs = {"q": q, "w_scale": ws, "x_scale": xs, "dtype": "f32", "epilogue": steps}
        want = G.qmatmul([x, bias], attrs)
        acc = G.qmatmul_acc(x, attrs)
        lda = pack.row_stride_for(K)
        xq = empty((M, lda), torch.int8)
        L.check(lib.mr_quantize_rows(T(x).data_ptr(), M, K, K, xq.data_ptr(), lda, xs, stream()), "q")
        bl = pack.pack_matmul(q)
        b = T(pack.device_weights(bl))
        ocp = pack.row_stride_for(o)
        rows = M
    else:
        attrs = {"q": q, "w_scale": ws, "x_scale": xs, "dtype": "f32", "stride": (s, s), "padding": (p, p),
                 "epilogue": steps}
        want = G.qconv2d([x, bias.reshape(o, 1, 1)], attrs)
        acc = G.qconv2d_acc(x, attrs)
        oh = ow = G.conv_out(h, k, s, p)
        rows = n * oh * ow
        want = want.transpose(0, 2, 3, 1).reshape(rows, o)
        acc = acc.transpose(0, 2, 3, 1).reshape(rows, o)
        cp = pack.c_pad_for(c)
        xq = empty((n, h, w, cp), torch.int8)
        L.check(lib.mr_quantize_nchw_nhwc(T(x).data_ptr(), n, c, h, w, xq.data_ptr(), cp, xs, stream()), "q")
        bl = pack.pack_conv(q, cp)
        b = T(pack.device_weights(bl))
        ocp = pack.c_pad_for(o)
    assert (np.abs(acc) < 2 ** 24).all()
    odd = (acc.astype(np.int64) % 2 != 0) & (want > 0) & (want < 127 * next_xs)
    assert odd.mean() > 0.15                      # plenty of exact ties in range
    yq = empty((rows, ocp), torch.int8)
    bd = T(bias)        # named: a temporary's memory could be reused before the kernel runs
    e = epilogue([("add", L.BC_COL, bd, 0, False), ("relu", 0, None, 0, False)], scale=scale, out_i8=yq,
                 ldq=ocp, xs=next_xs)
    if kind == "matmul":
        L.check(lib.mr_qmatmul(xq.data_ptr(), lda, b.data_ptr(), bl.shape[1], bl.shape[0], M, N, K, C.byref(e),
                               stream()), "mr_qmatmul")
    else:
        g = L.ConvGeom(n=n, h=h, w=w, c=c, c_pad=cp, o=o, oh=oh, ow=ow, kh=k, kw=k, sh=s, sw=s, ph=p, pw=p, dh=1,
                       dw=1)
        L.check(lib.mr_qconv2d(xq.data_ptr(), C.byref(g), b.data_ptr(), bl.shape[1], bl.shape[0], C.byref(e),
                               stream()), "mr_qconv2d")
    sync()
    assert bits_equal(yq.cpu().numpy()[:, :o], G.quantize_activation(want, next_xs).astype(np.int8))


# ---------------------------------------------------------------- standalone elementwise (device loops)

EW_SHAPES = [((4, 5), (4, 5)), ((4, 5), (5,)), ((3, 1, 5), (1, 4, 5)), ((), (2, 3)), ((2, 3, 4, 5), (1, 3, 1, 5)),
             ((7,), ()), ((1,), (6, 1)), ((33, 17), (33, 1))]


def _ew_strides(shape, full):
    pad = (1,) * (4 - len(shape)) + tuple(shape)
    st, acc = [0, 0, 0, 0], 1
    for d in range(3, -1, -1):
        st[d] = 0 if pad[d] == 1 else acc
        acc *= pad[d]
    return (C.c_int64 * 4)(*st)


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("fn", sorted(L.EW_FN))
def test_elementwise(fn, f16):
    """mr_elementwise_f32 against the oracle's elementwise op (mira/ops.py:163-169) bit for
    bit: every function, operands broadcast along any axes up to rank 4 (scalars included),
    NaN / +-inf / +-0 among the inputs, and the f16 rounding of an f16 op."""
    lib = L.load()
    rng = np.random.default_rng(L.EW_FN[fn] * 7 + f16)
    unary = fn in L.EW_UNARY
    special = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1.0, -1.0, 65504.0], np.float32)
    for ashape, bshape in EW_SHAPES:
        a = (rng.standard_normal(ashape) * 3).astype(np.float32)
        b = (rng.standard_normal(bshape) * 3).astype(np.float32)
        for x in (a, b):
            flat = x.reshape(-1)
            k = min(flat.size, special.size)
            flat[:k] = rng.permutation(special)[:k]
        if f16:
            a, b = a.astype(np.float16), b.astype(np.float16)
        full = tuple(ashape) if unary else tuple(np.broadcast_shapes(ashape, bshape))
        pad = (1,) * (4 - len(full)) + full
        y = empty(full, _torch().float32)
        at, bt = T(a.astype(np.float32)), T(b.astype(np.float32))
        print(f"elementwise {fn} f16={f16} {ashape} {bshape}", flush=True)
        L.check(lib.mr_elementwise_f32(L.EW_FN[fn], at.data_ptr(), _ew_strides(ashape, full),
                                       None if unary else bt.data_ptr(), None if unary else _ew_strides(bshape, full),
                                       y.data_ptr(), (C.c_int64 * 4)(*pad), int(f16), stream()), "mr_elementwise_f32")
        sync()
        want = G.evaluate(fn, [a] if unary else [a, b], {}).astype(np.float32)
        assert bits_equal(y.cpu().numpy(), want), (fn, ashape, bshape)


def test_elementwise_rejects():
    lib = L.load()
    x = empty((4,), _torch().float32)
    st = (C.c_int64 * 4)(0, 0, 0, 1)
    sh = (C.c_int64 * 4)(1, 1, 1, 4)
    assert lib.mr_elementwise_f32(99, x.data_ptr(), st, x.data_ptr(), st, x.data_ptr(), sh, 0, stream()) != 0
    assert lib.mr_elementwise_f32(L.EW_FN["add"], x.data_ptr(), st, None, None, x.data_ptr(), sh, 0, stream()) != 0
    assert lib.mr_elementwise_f32(L.EW_FN["neg"], None, st, None, None, x.data_ptr(), sh, 0, stream()) != 0


# ---------------------------------------------------------------- device-loop kernels (i32 held as bits)

def _bits(a: np.ndarray):
    """A 4-byte array as the float32 tensor holding its bits (how device loops store i32)."""
    return T(np.ascontiguousarray(a).view(np.float32))


def _unbits(t, dtype) -> np.ndarray:
    return t.cpu().numpy().view(dtype)


def test_elementwise_i32():
    """mr_elementwise_i32 against the oracle on int32 (NumPy wraps add / sub / mul / neg / abs
    at the int32 limits): every function but div, broadcast shapes, the extremes."""
    lib = L.load()
    rng = np.random.default_rng(21)
    edge = np.array([np.iinfo(np.int32).min, np.iinfo(np.int32).max, -1, 0, 1, 46341, -46341], np.int32)
    for fn in sorted(k for k in L.EW_FN if k != "div"):
        unary = fn in L.EW_UNARY
        for ashape, bshape in EW_SHAPES:
            a = rng.integers(-2**31, 2**31, ashape, dtype=np.int64).astype(np.int32)
            b = rng.integers(-50, 50, bshape, dtype=np.int64).astype(np.int32)
            for x in (a, b):
                flat = x.reshape(-1)
                flat[:min(flat.size, edge.size)] = edge[:min(flat.size, edge.size)]
            full = tuple(ashape) if unary else tuple(np.broadcast_shapes(ashape, bshape))
            pad = (1,) * (4 - len(full)) + full
            y = empty(full, _torch().float32)
            at, bt = _bits(a), _bits(b)
            print(f"elementwise_i32 {fn} {ashape} {bshape}", flush=True)
            L.check(lib.mr_elementwise_i32(L.EW_FN[fn], at.data_ptr(), _ew_strides(ashape, full),
                                           None if unary else bt.data_ptr(),
                                           None if unary else _ew_strides(bshape, full),
                                           y.data_ptr(), (C.c_int64 * 4)(*pad), stream()), "mr_elementwise_i32")
            sync()
            with np.errstate(over="ignore"):
                want = G.evaluate(fn, [a] if unary else [a, b], {})
            assert np.array_equal(_unbits(y, np.int32), want), (fn, ashape, bshape)


def test_cast_32():
    """mr_cast_32 against NumPy's astype: int32 -> f32 / f16 (one rounding), f32 / f16 ->
    int32 (toward zero; NaN, infinities and out-of-range values give INT_MIN on x86)."""
    lib = L.load()
    ints = np.array([0, 1, -1, 7, 2**24 + 1, -(2**24 + 3), 65519, 65520, 2**31 - 1, -2**31, 123456789], np.int32)
    floats = np.array([0.0, -0.0, 2.5, -2.5, 0.99, -0.99, 3e9, -3e9, 2147483520.0, -2147483648.0, np.nan, np.inf,
                       -np.inf, 65504.0, 1e-30], np.float32)
    for src, dst, x in (("i32", "f32", ints), ("i32", "f16", ints), ("f32", "i32", floats),
                        ("f16", "i32", floats.astype(np.float16))):
        y = empty(x.shape, _torch().float32)
        xt = _bits(x) if src == "i32" else T(x.astype(np.float32))
        print(f"cast {src} -> {dst}", flush=True)
        L.check(lib.mr_cast_32(xt.data_ptr(), x.size, L.DT[src], L.DT[dst], y.data_ptr(), stream()), "mr_cast_32")
        sync()
        with np.errstate(invalid="ignore"):
            want = G.evaluate("cast", [x], {"dtype": dst})
        got = _unbits(y, np.int32) if dst == "i32" else y.cpu().numpy()
        assert bits_equal(got, want.astype(np.int32 if dst == "i32" else np.float32)), (src, dst, got, want)


def test_gather_dynamic_slices_argmax_where():
    """mr_gather_rows_32 (negative indices from the end), mr_dynamic_slice_32 and
    mr_dynamic_update_slice_32 (starts out of range clamped, rank 1 to 3), mr_argmax_f32
    (ties to the first, the first NaN, rows longer than a wave) and mr_where_32 (f32 and
    i32 conditions, NaN and -0 among them, broadcast) against the oracle bit for bit."""
    lib = L.load()
    torch = _torch()
    rng = np.random.default_rng(31)
    table = rng.standard_normal((7, 5)).astype(np.float32)
    idx = np.array([[0, -1], [6, -7], [3, 3]], np.int32)
    y = empty((3, 2, 5), torch.float32)
    it = _bits(idx)
    tt = T(table)
    L.check(lib.mr_gather_rows_32(tt.data_ptr(), 7, 5, it.data_ptr(), idx.size, y.data_ptr(), stream()), "gather")
    sync()
    assert bits_equal(y.cpu().numpy(), G.evaluate("gather", [table, idx], {"axis": 0}))
    for shape, size, start in (((4, 6, 5), (2, 3, 5), (3, -2, 4)), ((4, 6, 5), (1, 6, 1), (0, 2, 9)),
                               ((12,), (1,), (11,)), ((12,), (3,), (-5,)), ((3, 8), (3, 2), (1, 7))):
        x = rng.standard_normal(shape).astype(np.float32)
        st = np.array(start, np.int32)
        pad = lambda s: (C.c_int64 * 4)(*((1,) * (4 - len(s)) + tuple(s)))      # noqa: E731
        xt, stt = T(x), _bits(st)
        ys = empty(size, torch.float32)
        print(f"dynamic slice {shape} {size} {start}", flush=True)
        L.check(lib.mr_dynamic_slice_32(xt.data_ptr(), pad(shape), stt.data_ptr(), len(shape), pad(size),
                                        ys.data_ptr(), stream()), "dynamic_slice")
        upd = rng.standard_normal(size).astype(np.float32)
        ut = T(upd)
        yu = empty(shape, torch.float32)
        L.check(lib.mr_dynamic_update_slice_32(xt.data_ptr(), pad(shape), ut.data_ptr(), pad(size), stt.data_ptr(),
                                               len(shape), yu.data_ptr(), stream()), "dynamic_update_slice")
        sync()
        assert bits_equal(ys.cpu().numpy(), G.evaluate("dynamic_slice", [x, st], {"size": size}))
        assert bits_equal(yu.cpu().numpy(), G.evaluate("dynamic_update_slice", [x, upd, st], {}))
    for rows, n in ((9, 33), (3, 70), (5, 1), (2, 200)):
        x = rng.integers(-3, 4, (rows, n)).astype(np.float32)     # many ties
        x[0, n // 2] = np.nan
        if rows > 1:
            x[1, :] = -np.inf
        if rows > 2 and n > 3:
            x[2, 3] = np.nan
            x[2, 1] = np.nan
        xt = T(x)
        ya = empty((rows,), torch.float32)
        print(f"argmax {rows}x{n}", flush=True)
        L.check(lib.mr_argmax_f32(xt.data_ptr(), rows, n, ya.data_ptr(), stream()), "argmax")
        sync()
        assert np.array_equal(_unbits(ya, np.int32), G.evaluate("argmax", [x], {"axis": 1, "keepdims": False}))
    cond_f = np.array([[0.0], [-0.0], [np.nan], [2.0]], np.float32)
    cond_i = np.array([[0], [np.iinfo(np.int32).min], [1], [0]], np.int32)
    a = rng.standard_normal((4, 3)).astype(np.float32)
    b = rng.standard_normal((1, 3)).astype(np.float32)
    for cond, cint in ((cond_f, 0), (cond_i, 1)):
        ct = _bits(cond) if cint else T(cond)
        at, bt = T(a), T(b)
        yw = empty((4, 3), torch.float32)
        L.check(lib.mr_where_32(ct.data_ptr(), cint, _ew_strides(cond.shape, (4, 3)), at.data_ptr(),
                                _ew_strides(a.shape, (4, 3)), bt.data_ptr(), _ew_strides(b.shape, (4, 3)),
                                yw.data_ptr(), (C.c_int64 * 4)(1, 1, 4, 3), stream()), "where")
        sync()
        assert bits_equal(yw.cpu().numpy(), G.evaluate("where", [cond, a, b], {}))
