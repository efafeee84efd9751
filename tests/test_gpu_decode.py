"""The float ops of a transformer decode step on rocm, through the C ABI and through the target.

layernorm, transpose and concat are bit-exact against the oracle (they are single IEEE
operations and copies).  softmax, the f32 batched matmul and the gelu/sigmoid/tanh epilogue
steps call libm or sum in another order than NumPy/BLAS; they run only in the target's
approx_f32 mode and are checked within the tolerances stated in each test.
"""
import ctypes as C

import numpy as np
import pytest

from harness import lowering as LW
from harness import models
from harness.runner import Runner
from mira_amd import _lib as L
from mira_amd import pack
from mira_amd.target import RocmTarget
from oracle import golden as G

from conftest import bits_equal
from gpu_util import T, empty, epilogue, oracle_env, stream, sync

T_ = T      # for tests whose parameters shadow T

pytestmark = pytest.mark.gpu

# f32 results of the approximate ops: |got - want| <= RTOL * |want| + ATOL * scale, where
# scale is the magnitude the result is computed from (see each test)
RTOL = 1e-5
ATOL = 1e-6


def _torch():
    import torch
    return torch


def _close(got, want, scale=1.0, rtol=RTOL, atol=ATOL):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert got.shape == want.shape
    err = np.abs(got - want) - (rtol * np.abs(want) + atol * np.asarray(scale, np.float64))
    assert err.max() <= 0, f"max excess {err.max():.3g}"


# ---------------------------------------------------------------- layernorm (bit-exact)

@pytest.mark.parametrize("rows,d", [(1, 64), (3, 1), (5, 7), (2, 8), (300, 100), (7, 128), (4, 129), (2, 768),
                                    (3, 1029), (1, 4096)])
@pytest.mark.parametrize("f16", [False, True])
def test_layernorm_bit_exact(lib, rows, d, f16):
    torch = _torch()
    rng = np.random.default_rng(rows * 1000 + d)
    x = (rng.standard_normal((rows, d)) * rng.uniform(0.05, 40) + rng.uniform(-10, 10)).astype(np.float32)
    if rows >= 3:
        x[1] = 2.5                              # constant row: variance 0
        x[2, : d // 2] *= 100 if f16 else 1e6   # wide dynamic range (f16 stays finite)
    g = rng.standard_normal(d).astype(np.float32)
    b = rng.standard_normal(d).astype(np.float32)
    if f16:
        x, g, b = (a.astype(np.float16).astype(np.float32) for a in (x, g, b))
    want = G.layernorm([x.astype(np.float16), g.astype(np.float16), b.astype(np.float16)] if f16 else [x, g, b],
                       {"eps": 1e-5}).astype(np.float32)
    xs = np.float32(0.0173)
    ld = pack.row_stride_for(d)
    y = empty((rows, d), torch.float32)
    yq = empty((rows, ld), torch.int8)
    xd, gd, bd = T(x), T(g), T(b)          # named: a temporary's memory could be reused before the kernel runs
    L.check(lib.mr_layernorm_f32(xd.data_ptr(), rows, d, gd.data_ptr(), bd.data_ptr(), 1e-5, int(f16),
                                 y.data_ptr(), yq.data_ptr(), ld, float(xs), stream()), "layernorm")
    sync()
    assert bits_equal(y.cpu().numpy(), want)
    assert bits_equal(yq.cpu().numpy()[:, :d], G.quantize_activation(want, xs).astype(np.int8))


@pytest.mark.parametrize("M,d,N,f16", [(1, 64, 192, False), (1, 64, 65, False), (3, 100, 256, False),
                                       (8, 128, 64, False), (2, 200, 96, False), (1, 1024, 300, False),
                                       (1, 64, 256, True), (5, 130, 40, True)])
def test_qmatmul_lnin(lib, M, d, N, f16):
    """mr_qmatmul_lnin (the layernorm inside the decode-shaped q-matmul) against the oracle's
    layernorm, quantize and q-matmul, bit for bit: rows of at most 128 elements (the lanes'
    pairwise sums) and longer ones (lane 0's recursion), f16 rounding of the normalised rows,
    a constant row (variance 0) and a wide one."""
    torch = _torch()
    rng = np.random.default_rng(M * 100 + d + N)
    x = (rng.standard_normal((M, d)) * rng.uniform(0.05, 40) + rng.uniform(-10, 10)).astype(np.float32)
    if M >= 3:
        x[1] = 2.5
        x[2, : d // 2] *= 100 if f16 else 1e6
    g = rng.standard_normal(d).astype(np.float32)
    b = rng.standard_normal(d).astype(np.float32)
    if f16:
        x, g, b = (a.astype(np.float16).astype(np.float32) for a in (x, g, b))
    y = G.layernorm([x.astype(np.float16), g.astype(np.float16), b.astype(np.float16)] if f16 else [x, g, b],
                    {"eps": 1e-5}).astype(np.float32)
    xs = float(np.abs(y).max()) / 127
    w = rng.standard_normal((d, N)).astype(np.float32)
    q, ws = G.quantize_array(w, 1)
    bias = rng.standard_normal(N).astype(np.float32)
    attrs = {"q": q, "w_scale": ws, "x_scale": xs, "dtype": "f32", "epilogue": (("add", 1, False),)}
    want = G.qmatmul([y, bias], attrs)
    want_acc = G.qmatmul_acc(y, attrs)
    bl = pack.pack_matmul(q)
    keep = [T(x), T(g), T(b), T(pack.device_weights(bl)), T(pack.combined_scale(xs, ws)), T(bias)]
    xd, gd, bd, bw, scale, bt = keep
    out = empty((M, N), torch.float32)
    acc = empty((M, N), torch.int32)
    e = epilogue([("add", L.BC_COL, bt, 0, False)], scale=scale, out_f32=out, ldo=N, out_acc=acc, ldacc=N)
    L.check(lib.mr_qmatmul_lnin(xd.data_ptr(), d, gd.data_ptr(), bd.data_ptr(), 1e-5, int(f16), xs, bw.data_ptr(),
                                bl.shape[1], bl.shape[0], M, N, d, C.byref(e), stream()), "mr_qmatmul_lnin")
    sync()
    assert np.array_equal(acc.cpu().numpy(), want_acc.astype(np.int32))
    assert bits_equal(out.cpu().numpy(), want)


def test_qmatmul_lnin_rejects(lib):
    """More than 8 rows or a row past 1024 elements: MR_EUNSUPPORTED (the caller keeps the
    layernorm launch); a row stride shorter than the row is an argument error."""
    torch = _torch()
    x = empty((16, 2048), torch.float32)
    g = empty((2048,), torch.float32)
    bw = empty((32, 2048), torch.int8)
    y = empty((16, 32), torch.float32)
    sc = empty((32,), torch.float64)
    e = epilogue(scale=sc, out_f32=y, ldo=32)
    call = lambda ldx, k_pad, M, K: lib.mr_qmatmul_lnin(x.data_ptr(), ldx, g.data_ptr(), g.data_ptr(), 1e-5, 0, 0.1,
                                                        bw.data_ptr(), k_pad, 32, M, 32, K, C.byref(e), stream())
    assert call(64, 64, 9, 64) == 3
    assert call(2048, 2048, 1, 2048) == 3
    assert call(32, 64, 1, 64) == 1
    sync()


def test_layernorm_int8_only_and_errors(lib):
    torch = _torch()
    x = np.random.default_rng(3).standard_normal((6, 48)).astype(np.float32)
    g, b = np.ones(48, np.float32), np.zeros(48, np.float32)
    yq = empty((6, 64), torch.int8)
    xd, gd, bd = T(x), T(g), T(b)
    L.check(lib.mr_layernorm_f32(xd.data_ptr(), 6, 48, gd.data_ptr(), bd.data_ptr(), 1e-5, 0, None, yq.data_ptr(), 64,
                                 0.05, stream()), "layernorm")
    sync()
    want = G.quantize_activation(G.layernorm([x, g, b], {"eps": 1e-5}), np.float32(0.05)).astype(np.int8)
    assert bits_equal(yq.cpu().numpy()[:, :48], want)
    assert lib.mr_layernorm_f32(xd.data_ptr(), 6, 48, gd.data_ptr(), bd.data_ptr(), 1e-5, 0, None, None, 0, 1.0,
                                stream()) == 1
    assert lib.mr_layernorm_f32(xd.data_ptr(), 6, 48, gd.data_ptr(), bd.data_ptr(), 1e-5, 0, None, yq.data_ptr(), 40,
                                0.05, stream()) == 1


# ---------------------------------------------------------------- transpose / concat (bit-exact)

@pytest.mark.parametrize("shape,perm", [((7,), (0,)), ((5, 9), (1, 0)), ((2, 273, 4, 16), (0, 2, 3, 1)),
                                        ((2, 273, 4, 16), (0, 2, 1, 3)), ((3, 1, 4, 5), (3, 0, 2, 1)),
                                        ((6, 5, 4), (2, 0, 1))])
def test_transpose_exact(lib, shape, perm):
    torch = _torch()
    x = np.random.default_rng(len(shape)).standard_normal(shape).astype(np.float32)
    want = G.evaluate("transpose", [x], {"perm": perm})
    y = empty(want.shape, torch.float32)
    r = len(shape)
    xd = T(x)
    L.check(lib.mr_transpose_f32(xd.data_ptr(), r, (C.c_int64 * r)(*shape), (C.c_int32 * r)(*perm), y.data_ptr(),
                                 stream()), "transpose")
    sync()
    assert bits_equal(y.cpu().numpy(), want)


@pytest.mark.parametrize("shapes,axis", [([(2, 272, 64), (2, 1, 64)], 1), ([(3, 4), (5, 4), (1, 4)], 0),
                                         ([(2, 3, 1), (2, 3, 6)], 2), ([(1, 0, 8), (1, 2, 8)], 1)])
def test_concat_exact(lib, shapes, axis):
    torch = _torch()
    rng = np.random.default_rng(11)
    xs = [rng.standard_normal(s).astype(np.float32) for s in shapes]
    want = G.evaluate("concat", xs, {"axis": axis})
    y = empty(want.shape, torch.float32)
    outer = int(np.prod(want.shape[:axis], dtype=np.int64))
    ld = int(np.prod(want.shape[axis:], dtype=np.int64))
    at = 0
    xd = [T(a) for a in xs]
    for a, t in zip(xs, xd):
        inner = int(np.prod(a.shape[axis:], dtype=np.int64))
        L.check(lib.mr_copy_rows_f32(t.data_ptr(), outer, inner, y.data_ptr(), ld, at, stream()), "concat")
        at += inner
    sync()
    assert bits_equal(y.cpu().numpy(), want)


# ---------------------------------------------------------------- softmax / bmm (approximate)

@pytest.mark.parametrize("rows,n", [(8, 273), (1, 1), (300, 65), (3, 1000), (2, 4097)])
def test_softmax_within_tolerance(lib, rows, n):
    """Probabilities within 1e-5 relative + 1e-6 absolute of NumPy's; rows sum to 1."""
    torch = _torch()
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((rows, n)) * 4).astype(np.float32)
    x[0, :: 3] = -10000.0                       # masked positions, as the decode mask writes them
    want = G.softmax([x], {"axis": -1})
    y = empty((rows, n), torch.float32)
    xd = T(x)
    L.check(lib.mr_softmax_f32(xd.data_ptr(), rows, n, 0, y.data_ptr(), stream()), "softmax")
    sync()
    got = y.cpu().numpy()
    _close(got, want)
    assert np.abs(got.astype(np.float64).sum(axis=1) - 1).max() < 1e-5


def _bstrides(shape, rs):
    nb = len(rs) - 2
    full = (1,) * (len(rs) - len(shape)) + tuple(shape)
    return [0 if full[i] == 1 else int(np.prod(full[i + 1:], dtype=np.int64)) for i in range(nb)]


@pytest.mark.parametrize("ashape,wshape", [((1, 4, 1, 16), (1, 4, 16, 273)), ((1, 4, 1, 273), (1, 4, 273, 16)),
                                           ((2, 3, 5, 7), (7, 9)), ((4, 1, 8, 32), (1, 3, 32, 16)),
                                           ((64, 128), (128, 96)), ((2, 1, 3, 2, 5, 6), (2, 2, 1, 2, 6, 4)),
                                           ((2, 1, 2, 3, 2, 5, 6), (2, 2, 1, 3, 2, 6, 4)),
                                           # decode-shaped rows: column blocks narrowed to 8 and 4
                                           ((1, 64), (64, 65)), ((1, 128), (128, 64)),
                                           ((1, 1000), (1000, 300)), ((1, 2, 1, 128), (1, 2, 128, 64))])
def test_bmm_f32_within_tolerance(lib, ashape, wshape):
    """a @ w with NumPy batch broadcasting and a scale+mask epilogue: every element within
    1e-5 of the float64 product's magnitude sum (|a| @ |w|), the bound for any f32 order, plus
    one f32 ulp of the result (masked entries are x - 10000, rounded at 10000's ulp)."""
    torch = _torch()
    rng = np.random.default_rng(len(ashape) * 10 + len(wshape))
    a = rng.standard_normal(ashape).astype(np.float32)
    w = rng.standard_normal(wshape).astype(np.float32)
    prod = np.matmul(a, w)
    rs = prod.shape
    nb = len(rs) - 2
    M, N, K = rs[-2], rs[-1], ashape[-1]
    scale = np.float32(0.25)
    mask = np.where(rng.random(N) < 0.3, -10000.0, 0.0).astype(np.float32)
    want = G.epilogue_ref(prod, [None, None, scale, mask], (("mul", 2, False), ("add", 3, False)))
    mag = np.matmul(np.abs(a).astype(np.float64), np.abs(w).astype(np.float64)) * 0.25
    y = empty((int(np.prod(rs[:-1])), N), torch.float32)
    st, mk = T(scale.reshape(1)), T(mask)
    e = epilogue([("mul", L.BC_SCALAR, st, 0, False), ("add", L.BC_COL, mk, 1, False)], out_f32=y, ldo=N)
    ad, wd = T(a), T(w)
    mk = (C.c_int64 * 4)(K, 1, N, 1)
    if nb > 4:
        with pytest.raises(L.RocmError):
            L.check(lib.mr_bmm_f32(ad.data_ptr(), wd.data_ptr(), nb, None, None, None, mk, M, N, K, C.byref(e),
                                   stream()), "bmm")
        return
    arr = lambda v: (C.c_int64 * max(nb, 1))(*v)
    L.check(lib.mr_bmm_f32(ad.data_ptr(), wd.data_ptr(), nb, arr(rs[:nb]), arr(_bstrides(ashape, rs)),
                           arr(_bstrides(wshape, rs)), mk, M, N, K, C.byref(e), stream()), "bmm")
    sync()
    _close(y.cpu().numpy().reshape(rs), want, scale=mag, rtol=2.0 ** -23, atol=1e-5)


@pytest.mark.parametrize("B,H,T,hd", [(1, 4, 273, 16), (3, 2, 40, 8), (2, 4, 300, 64)])
def test_bmm_f32_reads_transposed_operands_in_place(lib, B, H, T, hd):
    """The decode attention products with the cache read in place: scores = q @ keys^T and
    context = p @ values, where keys/values are [B, T, H*hd] rows and the matmul takes their
    transposed views through strides (short-K and long-K kernels)."""
    torch = _torch()
    rng = np.random.default_rng(T)
    D = H * hd
    q = rng.standard_normal((B, D)).astype(np.float32)
    keys = rng.standard_normal((B, T, D)).astype(np.float32)
    p = rng.random((B, H, 1, T)).astype(np.float32)
    q4 = q.reshape(B, 1, H, hd).transpose(0, 2, 1, 3)                   # [B, H, 1, hd]
    k4 = keys.reshape(B, T, H, hd).transpose(0, 2, 3, 1)                # [B, H, hd, T]
    v4 = keys.reshape(B, T, H, hd).transpose(0, 2, 1, 3)                # [B, H, T, hd]
    qd, kd, pd = T_(q), T_(keys), T_(p)
    arr = lambda v: (C.c_int64 * 2)(*v)
    for a_dev, a_np, sa, sam_sak, w_np, sw, swk_swn, (M, N, K) in [
            (qd, q4, (D, hd), (D, 1), k4, (T * D, hd), (1, D), (1, T, hd)),
            (pd, p, (H * T, T), (T, 1), v4, (T * D, hd), (D, 1), (1, hd, T))]:
        want = np.matmul(a_np.astype(np.float64), w_np.astype(np.float64))
        mag = np.matmul(np.abs(a_np).astype(np.float64), np.abs(w_np).astype(np.float64))
        y = empty((B * H, N), torch.float32)
        e = epilogue([], out_f32=y, ldo=N)
        mk = (C.c_int64 * 4)(*sam_sak, *swk_swn)
        L.check(lib.mr_bmm_f32(a_dev.data_ptr(), kd.data_ptr(), 2, arr((B, H)), arr(sa), arr(sw), mk, M, N, K,
                               C.byref(e), stream()), "bmm")
        sync()
        _close(y.cpu().numpy().reshape(want.shape), want, scale=mag, rtol=0, atol=1e-5)


# ---------------------------------------------------------------- libm epilogue steps (approximate)

@pytest.mark.parametrize("fn", ["gelu", "sigmoid", "tanh"])
@pytest.mark.parametrize("M,K,N", [(1, 256, 96), (300, 512, 256)])        # weight-stream and tiled kernels
def test_qmatmul_libm_epilogue(lib, fn, M, K, N):
    """The step after bias: within 1e-5 relative + 1e-6 absolute of NumPy's (gelu's absolute
    term scales with |x|, where 1 + tanh cancels)."""
    torch = _torch()
    rng = np.random.default_rng(M + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = rng.standard_normal((K, N)).astype(np.float32)
    q, ws = G.quantize_array(w, 1)
    bias = rng.standard_normal(N).astype(np.float32)
    xs = np.float32(np.abs(x).max() / 127)
    attrs = {"q": q, "w_scale": ws, "x_scale": float(xs), "dtype": "f32",
             "epilogue": (("add", 1, False), (fn, None, False))}
    want = G.qmatmul([x, bias], attrs)
    pre = G.qmatmul([x, bias], dict(attrs, epilogue=(("add", 1, False),)))
    xq = G.quantize_activation(x, xs).astype(np.int8)
    lda = pack.row_stride_for(K)
    xpad = np.zeros((M, lda), np.int8)
    xpad[:, :K] = xq
    bl = pack.pack_matmul(q)
    y = empty((M, N), torch.float32)
    sc, bd = T(pack.combined_scale(float(xs), ws)), T(bias)
    e = epilogue([("add", L.BC_COL, bd, 1, False), (fn, 0, None, 0, False)], scale=sc, out_f32=y, ldo=N)
    xd, bw = T(xpad), T(pack.device_weights(bl))
    L.check(lib.mr_qmatmul(xd.data_ptr(), lda, bw.data_ptr(), bl.shape[1], bl.shape[0], M, N, K, C.byref(e),
                           stream()), "qmatmul")
    sync()
    _close(y.cpu().numpy(), want, scale=np.maximum(np.abs(pre), 1.0))


# ---------------------------------------------------------------- the GPT decode step through the target

def _gpt_with_peaks(batch, peaks=None):
    """The quantized decode step at `batch`, calibrated on two seeded feeds of its own batch
    unless the peaks of another batch's calibration are given (the same attrs at any batch)."""
    cfg = models.GPTConfig()
    params = models.gpt_params(cfg, 0)
    g = LW.prepare(models.gpt_decode_step(cfg, batch, params))
    if peaks is None:
        calib = []
        for s in (2, 3):
            r = np.random.default_rng(s)
            toks = r.integers(0, cfg.V, (batch, cfg.T)).astype(np.int32)
            caches = [(r.standard_normal((batch, cfg.T, cfg.D)).astype(np.float32),
                       r.standard_normal((batch, cfg.T, cfg.D)).astype(np.float32)) for _ in range(cfg.L)]
            calib.append(models.gpt_step_feeds(cfg, params, toks, 16, caches))
        peaks = LW.calibrate(g, calib)
    LW.w8a8(g, peaks=peaks)
    return cfg, params, g, peaks


def _gpt(batch):
    cfg, params, g, _ = _gpt_with_peaks(batch)
    return cfg, params, g


def _step_feeds(cfg, params, batch, t, seed=9):
    r = np.random.default_rng(seed)
    toks = r.integers(0, cfg.V, (batch, cfg.T)).astype(np.int32)
    caches = [(r.standard_normal((batch, cfg.T, cfg.D)).astype(np.float32),
               r.standard_normal((batch, cfg.T, cfg.D)).astype(np.float32)) for _ in range(cfg.L)]
    return models.gpt_step_feeds(cfg, params, toks, t, caches)


def test_gpt_step_exact_mode_device_ops():
    """Default mode: layernorm, the head transposes and the cache concats join the W8A8
    projections on rocm (a layernorm that only rocm projections read runs inside their
    launches, mr_qmatmul_lnin; each layer's second one feeds the gelu projection on the CPU
    and keeps its own launch); the attention matmuls, softmax and the gelu projection stay
    on the CPU; every output bit-exact."""
    cfg, params, g = _gpt(2)
    feeds = _step_feeds(cfg, params, 2, 20)
    runner = Runner(g, RocmTarget(), fallback=G.CPUTarget())
    on_cpu = {op.kind for seg in runner.segments if seg.device == "cpu" for op in seg.graph.compute_ops()}
    assert on_cpu <= {"matmul", "softmax", "qmatmul", "transpose", "reshape", "concat"}, on_cpu
    kinds = {k for exe in runner.executables("rocm") for k in exe.kernel_counts}
    assert "concat" in kinds, kinds
    assert sum(exe.kernel_counts.get("layernorm", 0) for exe in runner.executables("rocm")) == cfg.L
    got = runner.run(feeds)
    want = G.run_graph(g, feeds)
    for a, b in zip(got, want):
        assert bits_equal(a, b)


def _flips(exe, g, env) -> int:
    """int32 accumulators of the rocm run that differ from the oracle's for the same graph
    inputs: each is an int8 activation that the two runs rounded to different steps."""
    acc = exe.accumulators()
    n = 0
    for op in g.compute_ops():
        if op.kind == "qmatmul":
            want = G.qmatmul_acc(env[op.inputs[0]], op.attrs).astype(np.int32)
            n += int((acc[op.result].reshape(want.shape) != want).sum())
    return n


@pytest.mark.parametrize("batch", [1, 2])
def test_gpt_step_approx_mode_one_segment(batch):
    """approx_f32: the whole step is one rocm segment.  Every approximate result (attention,
    softmax, gelu) is requantized to int8 before anything reads it, so the logits and the new
    key/value rows are bit-exact unless a requantization flipped (an accumulator differs);
    with no flip here they must be bit-exact."""
    cfg, params, g = _gpt(batch)
    feeds = _step_feeds(cfg, params, batch, 20)
    runner = Runner(g, RocmTarget(approx_f32=True, debug_acc=True), fallback=G.CPUTarget())
    assert runner.devices == ["rocm"]
    got = runner.run(feeds)
    env = oracle_env(g, feeds)
    flips = _flips(runner.executables("rocm")[0], g, env)
    for a, v in zip(got, g.outputs):
        assert bits_equal(a, env[v]) or flips > 0
    assert flips <= 2


def test_gpt_greedy_decode_256_tokens_approx_mode():
    """The configuration's decode (batch 1, seeded 16-token prompt, 256 new tokens, T = 272)
    with the whole step on rocm, teacher-forced: each step runs on the oracle's own feeds
    (its tokens and cache).  Every step's logits and key/value rows are bit-exact unless an
    int8 requantization flipped at that step; flips are rare (at most 1 step in 10), a flip
    step's logits stay within 5% of the largest logit, and the greedy tokens are the oracle's."""
    cfg, params, g = _gpt(1)
    prompt = np.random.default_rng(4).integers(0, cfg.V, (1, 16)).astype(np.int32)
    runner = Runner(g, RocmTarget(approx_f32=True, debug_acc=True), fallback=G.CPUTarget())
    assert runner.devices == ["rocm"]
    exe = runner.executables("rocm")[0]
    steps = []

    def run(feeds):
        got = runner.run(feeds)
        env = oracle_env(g, feeds)
        want = [env[v] for v in g.outputs]
        flips = _flips(exe, g, env)
        exact = all(bits_equal(a, b) for a, b in zip(got, want))
        err = float(np.abs(got[0] - want[0]).max() / max(np.abs(want[0]).max(), 1.0))
        steps.append((exact, flips, err, int(got[0].argmax()) == int(want[0].argmax())))
        return want

    models.gpt_decode(run, cfg, params, prompt, 256)
    assert len(steps) == 271
    print(f"steps with flips: {sum(f > 0 for _, f, _, _ in steps)}, max rel err {max(e for *_, e, _ in steps):.3g}")
    assert all(exact or flips > 0 for exact, flips, _, _ in steps)
    assert sum(flips > 0 for _, flips, _, _ in steps) <= 27
    assert max(err for _, _, err, _ in steps) <= 0.05
    assert all(same for *_, same in steps)


# ---------------------------------------------------------------- the decode loop resident on the device

@pytest.mark.parametrize("batch,new", [(1, 256), (2, 40)])
def test_device_decoder_matches_host_loop(batch, new):
    """harness.decode.DeviceDecoder (embedding, mask, cache writes and argmax on the device, no
    host synchronisation per token) gives the tokens and last logits of models.gpt_decode driven
    through the same executable, bit for bit; so does its HIP graph, replayed once per step with
    synchronisations and eager work between some replays."""
    import torch
    from harness.decode import DeviceDecoder
    cfg, params, g = _gpt(batch)
    prompt = np.random.default_rng(4).integers(0, cfg.V, (batch, 16)).astype(np.int32)
    runner = Runner(g, RocmTarget(approx_f32=True))
    want_tok, want_logits = models.gpt_decode(runner.run, cfg, params, prompt, new)
    dec = DeviceDecoder(runner, cfg, params, batch)
    got_tok = dec.decode(prompt, new)
    assert np.array_equal(got_tok, want_tok)
    assert bits_equal(dec.logits.cpu().numpy(), want_logits[-1])
    dec.capture()
    dec.reset(prompt)
    steps = 16 + new - 1
    for i in range(steps):
        dec.run_steps(1, use_graph=True)
        if i % 37 == 0:
            torch.cuda.synchronize()
            assert int(dec.t.item()) == i + 1
            _ = (dec.logits * 2).sum().item()          # eager work between replays
    graph_tok = dec.tokens[:, :16 + new].cpu().numpy()
    assert np.array_equal(graph_tok, want_tok)
    assert bits_equal(dec.logits.cpu().numpy(), want_logits[-1])
    # every step of the decode recorded as one graph: the whole loop is one launch
    dec.reset(prompt)
    dec.capture(steps)
    dec.reset(prompt)
    dec.run_steps(steps, use_graph=True)
    torch.cuda.synchronize()
    assert int(dec.t.item()) == steps and dec.graph_steps == steps
    assert np.array_equal(dec.tokens[:, :16 + new].cpu().numpy(), want_tok)
    assert bits_equal(dec.logits.cpu().numpy(), want_logits[-1])
    with pytest.raises(ValueError):
        dec.run_steps(steps - 1, use_graph=True)


# ---------------------------------------------------------------- batch 512: the decode that bench.py times

GPT512_ROWS = [0, 137, 317, 511]


def _flips_rows(exe, g, g_rows, env_rows, rows) -> int:
    """Accumulators of the checked rows of a batch run that differ from the oracle's run of
    those rows alone (g_rows: the same step at len(rows) rows, same attrs)."""
    acc = exe.accumulators()
    n = 0
    for op, op_r in zip(g.compute_ops(), g_rows.compute_ops()):
        if op.kind == "qmatmul":
            want = G.qmatmul_acc(env_rows[op_r.inputs[0]], op_r.attrs).astype(np.int32)
            got = acc[op.result].reshape(op.result.type.shape[0], -1)[rows]
            n += int((got != want.reshape(len(rows), -1)).sum())
    return n


def test_gpt_decode_batch512_approx_teacher_forced():
    """The batch-512 executable that bench.py's GPT decode times (approx_f32: the whole step
    on rocm), over all 271 steps, with rows 0, 137, 317 and 511 teacher-forced on the
    oracle: at each step those rows' feeds come from the oracle's own earlier outputs, and
    their logits and key/value rows are compared with the oracle's run of the same feeds.
    The flip accounting of the batch-1 test: a row-step is bit-exact unless an int8
    requantization flipped (an accumulator of those rows differs); flips are rare (at most
    1 step in 10); the logits stay within 5 % of the largest; a greedy token differs from
    the oracle's only at a flip step."""
    cfg, params, _, peaks = _gpt_with_peaks(2)
    _, _, g, _ = _gpt_with_peaks(512, peaks)
    _, _, g4, _ = _gpt_with_peaks(len(GPT512_ROWS), peaks)
    rows = GPT512_ROWS
    prompt = np.random.default_rng(5).integers(0, cfg.V, (512, 16)).astype(np.int32)
    runner = Runner(g, RocmTarget(approx_f32=True, debug_acc=True), fallback=G.CPUTarget())
    assert runner.devices == ["rocm"]
    exe = runner.executables("rocm")[0]
    steps = []

    def run(feeds):
        got = runner.run(feeds)
        sub = {k: (v if k == "mask" else v[rows]) for k, v in feeds.items()}
        env = oracle_env(g4, sub)
        want = [env[v] for v in g4.outputs]
        flips = _flips_rows(exe, g, g4, env, rows)
        exact = all(bits_equal(a[rows], b) for a, b in zip(got, want))
        err = float(np.abs(got[0][rows] - want[0]).max() / max(np.abs(want[0]).max(), 1.0))
        same = bool(np.array_equal(got[0][rows].argmax(1), want[0].argmax(1)))
        steps.append((exact, flips, err, same))
        forced = [a.copy() for a in got]
        for a, b in zip(forced, want):
            a[rows] = b                       # the checked rows continue from the oracle's outputs
        return forced

    print("batch 512 approx decode, teacher-forced rows", flush=True)
    models.gpt_decode(run, cfg, params, prompt, 256)
    assert len(steps) == 271
    n_flip = sum(f > 0 for _, f, _, _ in steps)
    print(f"steps with flips: {n_flip}, max rel err {max(e for *_, e, _ in steps):.3g}")
    assert all(exact or flips > 0 for exact, flips, _, _ in steps)
    assert n_flip <= 27
    assert max(err for _, _, err, _ in steps) <= 0.05
    assert all(same or flips > 0 for _, flips, _, same in steps)


def test_device_decoder_batch512_matches_host_loop():
    """DeviceDecoder at batch 512 -- the loop bench.py times -- against models.gpt_decode
    driven through the same executable: the same 272 tokens per row and the same logits at
    every one of the 271 steps, bit for bit, eager and replayed as a HIP graph."""
    import torch
    from harness.decode import DeviceDecoder
    cfg, params, _, peaks = _gpt_with_peaks(2)
    _, _, g, _ = _gpt_with_peaks(512, peaks)
    prompt = np.random.default_rng(5).integers(0, cfg.V, (512, 16)).astype(np.int32)
    runner = Runner(g, RocmTarget(approx_f32=True))
    assert runner.devices == ["rocm"]
    print("batch 512 host loop", flush=True)
    want_tok, want_logits = models.gpt_decode(runner.run, cfg, params, prompt, 256)
    dec = DeviceDecoder(runner, cfg, params, 512)
    dec.reset(prompt)
    logits = []
    for _ in range(271):
        dec.step()
        logits.append(dec.logits.clone())
    assert np.array_equal(dec.tokens.cpu().numpy(), want_tok)
    for t, (a, b) in enumerate(zip(logits, want_logits)):
        assert bits_equal(a.cpu().numpy(), b), f"step {t}"
    print("batch 512 graph replay", flush=True)
    dec.capture()
    dec.reset(prompt)
    for i in range(271):
        dec.run_steps(1, use_graph=True)
        if i % 50 == 0:
            torch.cuda.synchronize()
            assert int(dec.t.item()) == i + 1
    assert np.array_equal(dec.tokens.cpu().numpy(), want_tok)
    assert bits_equal(dec.logits.cpu().numpy(), want_logits[-1])


# ---------------------------------------------------------------- fused decode attention and the loop kernels

@pytest.mark.parametrize("B,H,hd,T", [(1, 4, 16, 272), (5, 4, 16, 40), (3, 2, 32, 0), (2, 2, 64, 700), (512, 4, 16, 272)])
def test_attention_decode_within_tolerance(lib, B, H, hd, T):
    """mr_attention_decode_f32 against the chain it replaces, in float64: scores of the query
    with the T cache keys and the new key, times the scale, plus the mask; softmax; the
    context.  Within 1e-5 of the float64 context's magnitude sum over the values; the int8 copy
    is the quantizer applied to the kernel's own f32 result."""
    torch = _torch()
    rng = np.random.default_rng(B * 7 + T)
    D = H * hd
    q = rng.standard_normal((B, D)).astype(np.float32)
    kc, vc = (rng.standard_normal((B, T, D)).astype(np.float32) for _ in range(2))
    kn, vn = (rng.standard_normal((B, D)).astype(np.float32) for _ in range(2))
    mask = np.where(rng.random(T + 1) < 0.3, -10000.0, 0.0).astype(np.float32)
    mask[T] = 0.0
    scale = np.float32(1.0 / np.sqrt(hd))
    keys = np.concatenate([kc, kn[:, None]], axis=1).astype(np.float64).reshape(B, T + 1, H, hd)
    vals = np.concatenate([vc, vn[:, None]], axis=1).astype(np.float64).reshape(B, T + 1, H, hd)
    s = np.einsum("bhd,bjhd->bhj", q.astype(np.float64).reshape(B, H, hd), keys) * scale + mask
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    want = np.einsum("bhj,bjhd->bhd", p, vals).reshape(B, D)
    mag = np.einsum("bhj,bjhd->bhd", p, np.abs(vals)).reshape(B, D)
    y = empty((B, D), torch.float32)
    ld8 = pack.row_stride_for(D)
    y8 = empty((B, ld8), torch.int8)
    xs = np.float32(np.abs(want).max() / 127)
    qd, kcd, vcd, knd, vnd, md = T_(q), T_(kc), T_(vc), T_(kn), T_(vn), T_(mask)
    L.check(lib.mr_attention_decode_f32(qd.data_ptr(), D, kcd.data_ptr() if T else None, vcd.data_ptr() if T else None,
                                        D, T * D, knd.data_ptr(), D, vnd.data_ptr(), D, md.data_ptr(), float(scale), B,
                                        H, hd, T, y.data_ptr(), D, y8.data_ptr(), ld8, float(xs), stream()), "attention")
    sync()
    got = y.cpu().numpy()
    _close(got, want, scale=mag, rtol=0, atol=1e-5)
    assert bits_equal(y8.cpu().numpy()[:, :D], G.quantize_activation(got, xs).astype(np.int8))


def test_attention_decode_rejects(lib):
    t = T_(np.zeros((4, 64), np.float32))
    args = lambda hd, T, ldq: (t.data_ptr(), ldq, t.data_ptr(), t.data_ptr(), 64, 64 * T, t.data_ptr(), 64,
                               t.data_ptr(), 64, t.data_ptr(), 1.0, 1, 64 // hd, hd, T, t.data_ptr(), 64, None, 0, 1.0,
                               stream())
    assert lib.mr_attention_decode_f32(*args(8, 3, 64)) == 1          # head width 8
    assert lib.mr_attention_decode_f32(*args(16, 1024, 64)) == 1      # 1025 keys
    assert lib.mr_attention_decode_f32(*args(16, 3, 62)) == 1         # query stride


def test_decode_embed_and_commit_exact(lib):
    """The loop-state kernels against NumPy: the embedding + position row (one f32 add), the
    mask row, the counter latch; then the cache row writes, NumPy's argmax (first maximum,
    a NaN first), the prompt kept while t + 1 < prompt_len, and the counter advance."""
    torch = _torch()
    rng = np.random.default_rng(3)
    B, T, D, V, P = 6, 20, 8, 11, 5
    emb = rng.standard_normal((V, D)).astype(np.float32)
    pos = rng.standard_normal((T, D)).astype(np.float32)
    tokens = rng.integers(0, V, (B, T)).astype(np.int32)
    caches = [rng.standard_normal((B, T, D)).astype(np.float32) for _ in range(3)]
    rows = [rng.standard_normal((B, D)).astype(np.float32) for _ in range(3)]
    logits = rng.standard_normal((B, V)).astype(np.float32)
    logits[1, [2, 7]] = 9.0                     # a tie: the first index wins
    logits[2, [4, 9]] = np.nan                  # NaNs: the first NaN wins
    logits[3, :] = -np.inf
    logits[4, 6] = np.inf
    tok_d, emb_d, pos_d = T_(tokens), T_(emb), T_(pos)
    cache_d = [T_(c) for c in caches]
    row_d = [T_(r) for r in rows]
    lg_d = T_(logits)
    h = empty((B, D), torch.float32)
    mask = empty((T + 1,), torch.float32)
    for t in (0, P - 2, P - 1, T - 2):
        state = T_(np.array([t, -1], np.int32))
        st = state.data_ptr()
        L.check(lib.mr_decode_embed(tok_d.data_ptr(), T, st, st + 4, emb_d.data_ptr(), V, pos_d.data_ptr(), T, D,
                                    h.data_ptr(), B, mask.data_ptr(), -10000.0, stream()), "embed")
        sync()
        assert bits_equal(h.cpu().numpy(), (emb[tokens[:, t]] + pos[t]).astype(np.float32))
        want_mask = np.full(T + 1, -10000.0, np.float32)
        want_mask[:t] = 0.0
        want_mask[T] = 0.0
        assert bits_equal(mask.cpu().numpy(), want_mask)
        assert list(state.cpu().numpy()) == [t, t]
        before = tok_d.cpu().numpy()
        rp = (C.c_void_p * 3)(*[r.data_ptr() for r in row_d])
        ld = (C.c_int64 * 3)(D, D, D)
        cp = (C.c_void_p * 3)(*[c.data_ptr() for c in cache_d])
        L.check(lib.mr_decode_commit(lg_d.data_ptr(), V, V, 3, rp, ld, cp, D, T * D, D, tok_d.data_ptr(), T, st,
                                     st + 4, P, T, B, stream()), "commit")
        sync()
        assert list(state.cpu().numpy()) == [t + 1, t]
        for c, r, cd in zip(caches, rows, cache_d):
            c[:, t] = r
            assert bits_equal(cd.cpu().numpy(), c)
        after = tok_d.cpu().numpy()
        want_tok = before.copy()
        if t + 1 >= P:
            want_tok[:, t + 1] = np.argmax(logits, axis=1)
        assert np.array_equal(after, want_tok)
    assert list(np.argmax(logits, axis=1)[1:5]) == [2, 4, 0, 6]


def test_gpt_step_approx_mode_fuses_attention():
    """approx_f32: each layer's attention (scores, scale, mask, softmax, context, and the cache
    concatenations) is one launch, which also writes the int8 input of the out projection, the
    query/key/value projections of a layer are one q-op launch, and each layernorm runs inside
    the launch of the projections that read it: 11 launches per step."""
    cfg, params, g = _gpt(2)
    exe = Runner(g, RocmTarget(approx_f32=True)).executables("rocm")[0]
    k = exe.kernel_counts
    assert k.get("attention") == cfg.L and not {"softmax", "bmm_f32", "concat", "quantize", "layernorm"} & set(k), k
    assert k["qmatmul"] == 4 * cfg.L + 1 and len(exe.launches) == 11
