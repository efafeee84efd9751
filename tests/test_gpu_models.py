"""End-to-end parity of the rocm target on the W8A8 configurations.

Each graph is lowered and W8A8-quantized once (harness.lowering); the same quantized
graph (the same attrs) then runs on the rocm target and on the oracle.  Every int32
accumulator and every output must match bit for bit.  Ops the rocm target rejects
(softmax, the f32 attention, layernorm and gelu of the GPT step) run on the oracle's
CPU target, as MIRA's partitioner would send them to its cpu target.

Full-size batches are checked through batch independence: chosen rows of the big run
must equal the oracle's results for those rows run on their own with the same attrs.
The rows are spread over the batch (and so over the tile grid), and include the
images an epilogue race once corrupted (7, 10, 12, 23, 53, 60, 78, 83, 130, 138, 162,
165, 180).
"""
import numpy as np
import pytest

from harness import lowering as LW
from harness import models
from harness.runner import Runner
from mira_amd.target import RocmTarget
from oracle import golden as G

from conftest import bits_equal
from gpu_util import oracle_env

pytestmark = pytest.mark.gpu

RACE_ROWS = [7, 10, 12, 23, 53, 60, 78, 83, 130, 138, 162, 165, 180]


def _gen(dist):
    return models.image_batch if dist == "uniform" else models.normal_batch


def _quantized(builder, batch, calib_seeds=(11, 12), dist="uniform", calib_batch=None, peaks=None,
               precision=None):
    """builder(batch, seed=0) lowered and W8A8-rewritten; calibration on a twin of
    calib_batch rows (same weights), or the given peaks."""
    g = LW.prepare(builder(batch=batch, seed=0), precision)
    if peaks is None:
        cb = calib_batch or batch
        twin = g if cb == batch else LW.prepare(builder(batch=cb, seed=0), precision)
        x = twin.inputs[0]
        peaks = LW.calibrate(twin, [{x.name: _gen(dist)(x.type.shape, s)} for s in calib_seeds])
    LW.w8a8(g, peaks=peaks)
    return g, peaks


def _compare(g, feeds, check_acc=True, fallback=True):
    runner = Runner(g, RocmTarget(debug_acc=True), fallback=G.CPUTarget() if fallback else None)
    got = runner.run(feeds)
    env = oracle_env(g, feeds)
    for v, out in zip(g.outputs, got):
        assert bits_equal(out, env[v]), f"output {v} differs: max abs {np.abs(out - env[v]).max()}"
    if check_acc:
        n_acc = 0
        for exe in runner.executables("rocm"):
            accs = exe.accumulators()
            for op in exe.g.ops:
                if op.kind == "qmatmul":
                    want = G.qmatmul_acc(env[op.inputs[0]], op.attrs)
                    want = want.reshape(-1, want.shape[-1])
                elif op.kind == "qconv2d":
                    x = env[op.inputs[0]]
                    assert G.qconv2d_certificate(x, op.attrs) < 2 ** 24
                    want = G.qconv2d_acc(x, op.attrs)
                    want = want.transpose(0, 2, 3, 1).reshape(-1, want.shape[1])
                else:
                    continue
                assert np.array_equal(accs[op.result], want.astype(np.int32)), f"{op.kind} accumulators differ"
                n_acc += 1
        assert n_acc > 0
    return runner


def _rows_match_small_run(builder, big, rows, dist, calib_seeds=(11, 12), runs=1):
    """The full batch on rocm (production path: fused stem, no debug copies); the chosen rows
    alone on the oracle with the same attrs.  With runs > 1 the executable runs again and
    every run must give the same bits."""
    g_big, peaks = _quantized(builder, big, calib_seeds, dist, calib_batch=2)
    x = _gen(dist)((big,) + g_big.inputs[0].type.shape[1:], 7)
    runner = Runner(g_big, RocmTarget())
    assert runner.devices == ["rocm"]
    outs = [runner.run({"x": x})[0] for _ in range(runs)]
    g_small, _ = _quantized(builder, len(rows), dist=dist, peaks=peaks)
    (want,) = G.run_graph(g_small, {"x": x[rows]})
    for out in outs:
        assert bits_equal(out[rows], want)
        assert np.isfinite(out).all()
        assert bits_equal(out, outs[0])


# ---------------------------------------------------------------- C1 and the reference's own programs

def test_c1_dense_256x64_to_10():
    """x f32[256,64] ~ N(0,1), w ~ N(0,0.1), b = 0; calibration on 8 seeded batches."""
    g, _ = _quantized(models.mlp_dense, 256, range(1, 9), "normal")
    ops = g.compute_ops()
    assert [op.kind for op in ops] == ["qmatmul"] and "epilogue" not in ops[0].attrs   # zero bias dropped
    _compare(g, {"x": models.normal_batch((256, 64), 100)}, fallback=False)


def test_mlp_mira_with_softmax_fallback():
    g, _ = _quantized(models.mlp_mira, 64, (2, 3), "normal")
    runner = _compare(g, {"x": models.normal_batch((64, 784), 1)})
    assert runner.devices == ["rocm", "cpu"]
    soft = next(op for op in g.compute_ops() if op.kind == "softmax")
    assert "softmax" in runner.reasons[soft]


def test_cnn_mira():
    g, _ = _quantized(models.cnn_mira, 16, (2, 3), "normal")
    _compare(g, {"img": models.normal_batch((16, 1, 28, 28), 1)})


# ---------------------------------------------------------------- C2 MLP-50M

def test_mlp50m_batch1_whole_network():
    """Batch 1 (the decode-shaped weight-streaming qmatmul), all four layers."""
    g, _ = _quantized(models.mlp_50m, 1, (2, 3), "normal", calib_batch=8)
    runner = _compare(g, {"x": models.normal_batch((1, 4096), 1)}, fallback=False)
    # the first layer quantizes the f32 input rows itself: four launches in all
    assert runner.executables("rocm")[0].kernel_counts == {"qmatmul": 4}


def test_mlp50m_batch8():
    g, _ = _quantized(models.mlp_50m, 8, (2, 3), "normal")
    _compare(g, {"x": models.normal_batch((8, 4096), 1)}, fallback=False)


def test_mlp50m_batch4096_rows():
    _rows_match_small_run(models.mlp_50m, 4096, [0, 1, 255, 256, 1234, 2047, 2048, 3333, 4095], "normal",
                          calib_seeds=(2, 3))


# ---------------------------------------------------------------- C3 ResNet-18

def test_resnet18_batch1():
    g, _ = _quantized(models.resnet18, 1)
    runner = _compare(g, {"x": models.image_batch((1, 3, 224, 224), 5)}, fallback=False)
    assert runner.devices == ["rocm"]


def test_resnet18_batch2():
    g, _ = _quantized(models.resnet18, 2)
    runner = _compare(g, {"x": models.image_batch((2, 3, 224, 224), 5)}, fallback=False)
    assert runner.devices == ["rocm"]


def test_resnet18_batch256_rows():
    """16 oracle rows of the batch-256 run, three runs of one executable bit-identical."""
    _rows_match_small_run(models.resnet18, 256, [0] + RACE_ROWS + [200, 255], "uniform", runs=3)


@pytest.mark.parametrize("bn_epilogue,precision", [(False, None), (True, None), (False, "f16")])
def test_resnet18_batch2_fused_stem(bn_epilogue, precision):
    """Without debug accumulators the stem conv, pad and max pool run as one kernel, also with
    the ONNX importer's BatchNorm mul (a positive per-channel constant keeps the epilogue
    monotone, so pooling the accumulators first is exact) and in the f16 graph (rounding to
    f16 is monotone too).  The image is the stem's only reader, so the stem quantizes it
    (from its f16 rounding in the f16 graph) from the f32 input: no input launch at all
    (f16 graphs still round the global average pool with round_f16 launches)."""
    def builder(batch, seed):
        return models.resnet18(batch=batch, seed=seed, bn_epilogue=bn_epilogue)
    g, _ = _quantized(builder, 2, precision=precision)
    runner = Runner(g, RocmTarget())
    exe = runner.executables("rocm")[0]
    assert exe.kernel_counts.get("qconv2d_maxpool") == 1 and "maxpool2d" not in exe.kernel_counts
    assert "input" not in exe.kernel_counts
    # in the f16 graph the stem's pooled output and the residual path are stored as halves
    halves = [d for d in exe.dv.values() if d.half]
    assert (len(halves) > 0) == (precision == "f16")
    assert all(str(d.f32.dtype) == "torch.float16" for d in halves)
    x = models.image_batch((2, 3, 224, 224), 5)
    (got,) = runner.run({"x": x})
    (want,) = G.run_graph(g, {"x": x})
    assert bits_equal(got, want)


# ---------------------------------------------------------------- C4 MobileNetV2

def test_mobilenet_v2_batch1():
    g, _ = _quantized(models.mobilenet_v2, 1, calib_batch=2)
    runner = _compare(g, {"x": models.image_batch((1, 3, 224, 224), 5)}, fallback=False)
    assert runner.devices == ["rocm"]


def test_mobilenet_v2_batch2():
    g, _ = _quantized(models.mobilenet_v2, 2)
    runner = _compare(g, {"x": models.image_batch((2, 3, 224, 224), 5)}, fallback=False)
    assert runner.devices == ["rocm"]


def test_mobilenet_v2_batch2_fused_expansions():
    """Production path (no debug accumulators): each of the 16 expansion 1x1 convolutions
    runs inside its depthwise convolution's launch (mr_qconv1x1_dw3x3), and so does the 3x3
    stem with the first block's depthwise convolution (mr_qstem3x3_dw3x3): no depthwise
    launch of its own is left; bit-exact."""
    g, _ = _quantized(models.mobilenet_v2, 2)
    runner = Runner(g, RocmTarget())
    exe = runner.executables("rocm")[0]
    assert exe.kernel_counts.get("expand_dw") == 17 and "dwconv2d" not in exe.kernel_counts, exe.kernel_counts
    x = models.image_batch((2, 3, 224, 224), 5)
    (got,) = runner.run({"x": x})
    (want,) = G.run_graph(g, {"x": x})
    assert bits_equal(got, want)


def test_mobilenet_v2_f16_batch2_fused_expansions():
    """MIRA's default precision on rocm (the f16 graph), production path: the same 17 fused
    launches with their f16 rounding, bit-exact against the oracle's f16 graph."""
    g, _ = _quantized(models.mobilenet_v2, 2, precision="f16")
    runner = Runner(g, RocmTarget())
    exe = runner.executables("rocm")[0]
    assert exe.kernel_counts.get("expand_dw") == 17 and "dwconv2d" not in exe.kernel_counts, exe.kernel_counts
    x = models.image_batch((2, 3, 224, 224), 5)
    (got,) = runner.run({"x": x})
    (want,) = G.run_graph(g, {"x": x})
    assert bits_equal(got, want)


def test_mobilenet_v2_batch128_rows():
    _rows_match_small_run(models.mobilenet_v2, 128, [0, 7, 10, 23, 53, 64, 100, 127], "uniform", runs=2)


# ---------------------------------------------------------------- other layouts and precisions

@pytest.mark.parametrize("builder", [models.resnet18, models.mobilenet_v2])
def test_onnx_layout_batch2(builder):
    """The CNNs as MIRA's ONNX importer lays them out: BatchNormalization as a per-channel mul +
    add after a bias-free conv (mira/frontends/onnx_import.py:423-431), fused into the conv
    epilogue.  Every op on rocm; accumulators and outputs bit-exact."""
    g, _ = _quantized(lambda batch, seed: builder(batch=batch, seed=seed, bn_epilogue=True), 2)
    assert any(op.attrs.get("epilogue", ())[:1] == (("mul", 1, False),) for op in g.compute_ops())
    runner = _compare(g, {"x": models.image_batch((2, 3, 224, 224), 5)}, fallback=False)
    assert runner.devices == ["rocm"]


def _imported(data: bytes, shape, seeds=(11, 12)):
    """An ONNX model read by harness/onnx_import.py, lowered and W8A8-rewritten with
    calibration on seeded uniform batches of its input shape."""
    from harness import onnx_import as OI
    g = LW.prepare(OI.import_model(data))
    LW.w8a8(g, peaks=LW.calibrate(g, [{"x": models.image_batch(shape, s)} for s in seeds]))
    return g


def test_onnx_import_resnet18_batch2():
    """A torchvision-layout ResNet-18 (torch modules, random weights) written as ONNX and read by
    this repository's importer: every op on rocm; accumulators and outputs bit-exact."""
    import torch_onnx_nets as N
    _, data = N.resnet18(2, seed=3)
    g = _imported(data, (2, 3, 224, 224))
    runner = _compare(g, {"x": models.image_batch((2, 3, 224, 224), 6)}, fallback=False)
    assert runner.devices == ["rocm"]


def test_onnx_import_mobilenet_v2_batch2():
    """A torchvision-layout MobileNetV2 written as ONNX and read by this repository's importer
    (as the reference imports torchvision's, tests/test_onnx.py:150-159): every op on rocm --
    the int8 pointwise and stem convs, the f32 depthwise convs, ReLU6, the residual adds, the
    average pool and the classifier; accumulators and outputs bit-exact."""
    import torch_onnx_nets as N
    _, data = N.mobilenet_v2(2, seed=3)
    g = _imported(data, (2, 3, 224, 224))
    runner = _compare(g, {"x": models.image_batch((2, 3, 224, 224), 6)}, fallback=False)
    assert runner.devices == ["rocm"]


@pytest.mark.parametrize("opset", [10, 13])
def test_onnx_import_edge_net(opset):
    """The importer's less common forms on rocm: an asymmetric pad before a 4-channel conv, a
    dilated depthwise conv, ReLU6 as Clip, a ceil-mode max pool, the Shape-Gather-Concat flatten,
    Gemm alpha/beta as epilogue steps."""
    import torch_onnx_nets as N
    _, data = N.edge_net(4, opset)
    g = _imported(data, (4, 3, 9, 9))
    runner = _compare(g, {"x": models.image_batch((4, 3, 9, 9), 6)}, fallback=False)
    assert runner.devices == ["rocm"]


@pytest.mark.parametrize("builder,shape,dist", [(models.resnet18, (2, 3, 224, 224), "uniform"),
                                                (models.mobilenet_v2, (2, 3, 224, 224), "uniform"),
                                                (models.mlp_50m, (8, 4096), "normal")])
def test_f16_graph(builder, shape, dist):
    """The reference's default precision for accelerator targets ("auto" -> f16,
    mira/compiler.py:293-294; lowering mira/passes.py:206-253): every op computes in f32 and
    rounds its result to f16 as the reference's ops do.  Every op on rocm (the interface
    casts included); accumulators and outputs bit-exact against the oracle on the same
    f16 graph."""
    g, _ = _quantized(builder, shape[0], dist=dist, precision="f16")
    assert sum(op.result.type.dtype == "f16" for op in g.compute_ops()) > 3
    runner = _compare(g, {"x": _gen(dist)(shape, 5)}, fallback=False)
    assert runner.devices == ["rocm"]


def test_f16_mlp_mira_with_softmax_fallback():
    g, _ = _quantized(models.mlp_mira, 64, (2, 3), "normal", precision="f16")
    runner = _compare(g, {"x": models.normal_batch((64, 784), 1)})
    assert "rocm" in runner.devices


# ---------------------------------------------------------------- C5 character-level GPT decode

def _gpt_quantized(batch, peaks=None):
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


def _gpt_runner(g, debug_acc=False):
    runner = Runner(g, RocmTarget(debug_acc=debug_acc), fallback=G.CPUTarget())
    assert "rocm" in runner.devices
    return runner


def test_gpt_decode_step_batch2():
    """One decode step: the W8A8 projections on rocm (weight-streaming kernel, M = 2), attention,
    softmax, layernorm and the gelu-fused projection on the cpu fallback; every accumulator and
    output bit-exact."""
    cfg, params, g, _ = _gpt_quantized(2)
    r = np.random.default_rng(9)
    toks = r.integers(0, cfg.V, (2, cfg.T)).astype(np.int32)
    caches = [(r.standard_normal((2, cfg.T, cfg.D)).astype(np.float32),
               r.standard_normal((2, cfg.T, cfg.D)).astype(np.float32)) for _ in range(cfg.L)]
    feeds = models.gpt_step_feeds(cfg, params, toks, 20, caches)
    runner = _compare(g, feeds)
    # the [b, 1, heads, d] head tensors are not images: they keep C order, no transposes
    assert not any(k in exe.kernel_counts for exe in runner.executables("rocm")
                   for k in ("nchw_to_nhwc", "nhwc_to_nchw"))
    gelu_q = [op for op in g.compute_ops() if op.kind == "qmatmul" and op.attrs.get("epilogue", ())
              and op.attrs["epilogue"][0][0] == "gelu"]
    assert len(gelu_q) == cfg.L and all("gelu" in runner.reasons[op] for op in gelu_q)


def test_gpt_greedy_decode_256_tokens_batch1():
    """The configuration's decode: batch 1, a seeded 16-token prompt of uniform token ids, 256
    generated tokens (context T = 272 = 16 + 256).  rocm and the oracle produce the same
    tokens and the same logits, bit for bit, at every one of the 271 steps."""
    cfg, params, g, _ = _gpt_quantized(1)
    prompt = np.random.default_rng(4).integers(0, cfg.V, (1, 16)).astype(np.int32)
    runner = _gpt_runner(g)
    got_tok, got_logits = models.gpt_decode(runner.run, cfg, params, prompt, 256)
    want_tok, want_logits = models.gpt_decode(lambda f: G.run_graph(g, f), cfg, params, prompt, 256)
    assert got_tok.shape == (1, 272) and np.array_equal(got_tok, want_tok)
    assert len(got_logits) == 271
    for a, b in zip(got_logits, want_logits):
        assert bits_equal(a, b)


# rows of the batch-512 decode checked against the oracle: both ends, and rows inside the
# first, middle and last 128-row blocks of the GPT step's kernels
GPT512_ROWS = [0, 137, 317, 511]


def test_gpt_greedy_decode_batch512_all_steps():
    """Batch 512, the configuration's whole decode: seeded 16-token prompts, 256 generated
    tokens (271 steps) with the q-ops on rocm.  Rows 0, 137, 317 and 511, decoded on their
    own by the oracle with the same attrs, give the same tokens and the same logits, bit for
    bit, at every step (the step's rows are independent)."""
    cfg, params, g2, peaks = _gpt_quantized(2)
    _, _, g, _ = _gpt_quantized(512, peaks=peaks)
    _, _, g4, _ = _gpt_quantized(len(GPT512_ROWS), peaks=peaks)
    prompt = np.random.default_rng(5).integers(0, cfg.V, (512, 16)).astype(np.int32)
    runner = _gpt_runner(g)
    print("batch 512 exact-mode decode, 271 steps", flush=True)
    got_tok, got_logits = models.gpt_decode(runner.run, cfg, params, prompt, 256)
    want_tok, want_logits = models.gpt_decode(lambda f: G.run_graph(g4, f), cfg, params, prompt[GPT512_ROWS], 256)
    assert got_tok.shape == (512, 272) and len(got_logits) == len(want_logits) == 271
    assert np.array_equal(got_tok[GPT512_ROWS], want_tok)
    for t, (a, b) in enumerate(zip(got_logits, want_logits)):
        assert bits_equal(a[GPT512_ROWS], b), f"step {t}"
    # the checked rows generate different tokens (each row follows its own prompt)
    assert len({tuple(r) for r in want_tok[:, 16:]}) > 1


# ---------------------------------------------------------------- weight-only int8 (decode-shaped f32 matmuls)
#
# quantize="int8" keeps activations in f32; the dequantized weights feed f32 matmuls that
# the rocm target runs as weight streams for up to 64 rows.  Their sums run in another
# order than BLAS's, so outputs match the oracle on the same quantized graph to within
# W8_MODEL_TOL of the output's peak magnitude (about ten f32 roundings of a K = 4096 dot
# product compounded over the layers), not bit for bit.

W8_MODEL_TOL = 1e-4


def _weight_only(g, precision=None):
    LW.prepare(g, precision)
    want = G.weight_only_attrs(g)
    LW.weight_only(g)
    for op, a in want.items():
        assert op.kind == "dequantize" and np.array_equal(op.attrs["q"], a["q"])
    return g


def _run_weight_only(g, feeds):
    runner = Runner(g, RocmTarget(), fallback=G.CPUTarget())
    got = runner.run(feeds)
    env = oracle_env(g, feeds)
    return runner, got, [env[v] for v in g.outputs]


def _w8_launches(runner) -> int:
    return sum(exe.kernel_counts.get("w8matmul", 0) for exe in runner.executables("rocm"))


@pytest.mark.parametrize("precision", [None, "f16"])
def test_weight_only_mlp50m_batch1(precision):
    """f32, and the f16 graph of MIRA's default precision: f16 weights (fl16(q * scale)),
    every result rounded to f16; f16 results may sit one f16 ulp apart where the f32 sums
    straddle a rounding boundary, hence the looser bound there."""
    g = _weight_only(models.mlp_50m(batch=1), precision)
    runner, (got,), (want,) = _run_weight_only(g, {"x": models.normal_batch((1, 4096), 3)})
    assert runner.devices == ["rocm"] and _w8_launches(runner) == 4
    tol = 1e-2 if precision else W8_MODEL_TOL
    assert np.abs(got - want).max() <= tol * np.abs(want).max()


def test_weight_only_mlp50m_batch4096():
    """The 4096-row weight-only MLP-50M on the f32-MFMA tiles, every row against the oracle."""
    g = _weight_only(models.mlp_50m(batch=4096))
    runner, (got,), (want,) = _run_weight_only(g, {"x": models.normal_batch((4096, 4096), 4)})
    assert runner.devices == ["rocm"] and _w8_launches(runner) == 4
    assert np.abs(got - want).max() <= W8_MODEL_TOL * np.abs(want).max()


@pytest.mark.parametrize("builder,convs,devices", [(models.resnet18, 20, ["rocm"]),
                                                    (models.mobilenet_v2, 33, ["cpu", "rocm"])])
def test_weight_only_cnn_batch2(builder, convs, devices):
    """Weight-only ResNet-18 and MobileNetV2: every dense convolution over a dequantize weight
    on rocm, ResNet-18's 3-channel stem through a channel-padded NHWC copy of the image (the
    two MobileNetV2 convolutions whose weights are under 1024 elements stay f32 and run on
    the CPU; depthwise weights are materialized in f32 and stay bit-exact), within f32
    rounding of the oracle compounded over the network."""
    g = _weight_only(builder(batch=2, seed=0))
    runner, (got,), (want,) = _run_weight_only(g, {"x": models.image_batch((2, 3, 224, 224), 7)})
    n = sum(exe.kernel_counts.get("w8conv2d", 0) for exe in runner.executables("rocm"))
    assert n == convs, n
    assert runner.devices[:2] == devices, runner.devices
    assert np.abs(got - want).max() <= W8_MODEL_TOL * np.abs(want).max()


def test_weight_only_stem_alone():
    """A lone 3-channel weight-only 7x7/2 convolution with a bias and relu: the padded copy
    and its zero weight channel against the oracle, at batch 1 and 3."""
    from harness.graph import Graph
    rng = np.random.default_rng(21)
    for n in (1, 3):
        g = Graph("stem")
        x = g.input("x", (n, 3, 61, 57))
        w = g.const(rng.standard_normal((16, 3, 7, 7)).astype(np.float32))
        b = g.const(rng.standard_normal((1, 16, 1, 1)).astype(np.float32))
        y = g.op("relu", [g.op("add", [g.op("conv2d", [x, w], {"stride": (2, 2), "padding": (3, 3)}), b])])
        g.outputs = [y]
        g = _weight_only(g)
        runner, (got,), (want,) = _run_weight_only(g, {"x": rng.standard_normal((n, 3, 61, 57)).astype(np.float32)})
        assert runner.devices == ["rocm"]
        assert sum(exe.kernel_counts.get("w8conv2d", 0) for exe in runner.executables("rocm")) == 1
        assert np.abs(got - want).max() <= W8_MODEL_TOL * np.abs(want).max()


def test_weight_only_mlp_mira_batch64():
    """The reference's own int8 check (its tests/test_control_dynamic_quant.py:178-189) with
    the three matmuls on rocm: within 0.05 of the f32 model, argmax agreement above 0.9."""
    x = np.random.default_rng(0).standard_normal((64, 784)).astype(np.float32)
    f32g = LW.prepare(models.mlp_mira(batch=64))
    (ref,) = G.run_graph(f32g, {"x": x})
    g = _weight_only(models.mlp_mira(batch=64))
    runner, (got,), (want,) = _run_weight_only(g, {"x": x})
    assert runner.devices == ["rocm", "cpu"] and _w8_launches(runner) == 3
    assert np.abs(got - want).max() <= 1e-5            # softmax probabilities
    assert np.abs(got - ref).max() < 0.05 and (got.argmax(1) == ref.argmax(1)).mean() > 0.9


def test_weight_only_gpt_decode_step_batch2():
    cfg = models.GPTConfig()
    params = models.gpt_params(cfg, 0)
    g = _weight_only(models.gpt_decode_step(cfg, 2, params))
    r = np.random.default_rng(9)
    toks = r.integers(0, cfg.V, (2, cfg.T)).astype(np.int32)
    caches = [(r.standard_normal((2, cfg.T, cfg.D)).astype(np.float32),
               r.standard_normal((2, cfg.T, cfg.D)).astype(np.float32)) for _ in range(cfg.L)]
    feeds = models.gpt_step_feeds(cfg, params, toks, 20, caches)
    runner, got, want = _run_weight_only(g, feeds)
    assert _w8_launches(runner) > 0
    for a, b in zip(got, want):
        assert np.abs(a - b).max() <= W8_MODEL_TOL * max(np.abs(b).max(), 1.0)
