"""Host-side logic on the CPU: the harness's lowering (against the oracle's
restatement of MIRA's rewrite), the split between the rocm target and the CPU
fallback, the target's check() decisions, weight packing, broadcast modes and
the requant arithmetic.  Structure tests follow the reference's own
(tests/test_passes.py:51-72, tests/test_backends.py:40-55)."""
import numpy as np
import pytest

from harness import lowering as LW
from harness import models
from harness.graph import Graph
from harness.runner import Runner, split
from mira_amd import _lib as L
from mira_amd import pack
from mira_amd.target import RocmTarget, _bcast_mode
from oracle import golden as G


def _dense_graph(bias_shape=(4,), relu=True, sub_from_bias=False):
    g = Graph("t")
    x = g.input("x", (8, 16))
    w = g.const(np.random.default_rng(0).standard_normal((16, 4)).astype(np.float32))
    b = g.const(np.random.default_rng(1).standard_normal(bias_shape).astype(np.float32))
    y = g.op("matmul", [x, w])
    y = g.op("sub", [b, y]) if sub_from_bias else g.op("add", [y, b])
    if relu:
        y = g.op("relu", [y])
    g.outputs = [y]
    return g


def test_fusion_builds_epilogue():
    g = _dense_graph()
    LW.prepare(g)
    (op,) = g.compute_ops()
    assert op.kind == "matmul" and [s[0] for s in op.attrs["epilogue"]] == ["add", "relu"]


def test_fusion_respects_operand_order():
    g = _dense_graph(bias_shape=(8, 4), relu=False, sub_from_bias=True)
    LW.prepare(g)
    (op,) = g.compute_ops()
    assert op.attrs["epilogue"][0][0] == "sub" and op.attrs["epilogue"][0][2] is True


def test_fusion_skips_multi_use_results():
    g = Graph("t")
    x = g.input("x", (8, 16))
    h = g.op("matmul", [x, g.const(np.ones((16, 16), np.float32))])
    g.outputs = [g.op("add", [g.op("relu", [h]), h])]
    LW.prepare(g)
    assert "epilogue" not in g.compute_ops()[0].attrs


def test_zero_bias_is_simplified_away():
    g = models.mlp_dense(batch=4)
    LW.prepare(g)
    (op,) = g.compute_ops()
    assert op.kind == "matmul" and "epilogue" not in op.attrs


@pytest.mark.parametrize("builder,shape", [(models.mlp_mira, (4, 784)), (models.cnn_mira, (4, 1, 28, 28))])
def test_quantizer_matches_oracle(builder, shape):
    g = builder(batch=shape[0])
    LW.prepare(g)
    calib = [{g.inputs[0].name: models.normal_batch(shape, s)} for s in (2, 3)]
    want = G.w8a8_attrs(g, calib)
    wanted = [(op.inputs[0], want[op]) for op in g.ops if op in want]
    LW.w8a8(g, calib)
    qops = [op for op in g.ops if op.kind in ("qmatmul", "qconv2d")]
    assert len(qops) == 3
    for op, (_x, a) in zip(qops, wanted):
        assert np.array_equal(op.attrs["q"], a["q"]) and np.array_equal(op.attrs["w_scale"], a["w_scale"])
        assert op.attrs["epilogue"] == a["epilogue"]
        assert abs(op.attrs["x_scale"] - a["x_scale"]) <= 1e-6 * a["x_scale"]   # BLAS order differs


def test_quantize_array_matches_oracle():
    w = np.random.default_rng(3).standard_normal((64, 3, 7, 7)).astype(np.float32)
    for axis in (0, 1):
        q1, s1 = LW.quantize_array(w.reshape(64, -1) if axis == 1 else w, axis)
        q2, s2 = G.quantize_array(w.reshape(64, -1) if axis == 1 else w, axis)
        assert np.array_equal(q1, q2) and np.array_equal(s1, s2)


def test_weight_only_rewrite_matches_oracle():
    """mira/quantize.py:46-68 on examples/mlp.mira: the reference's own test expects three
    dequantize constants (its tests/test_control_dynamic_quant.py:178-189); the biases stay
    f32; q, scale and axis equal the oracle's restatement."""
    g = models.mlp_mira(batch=4)
    LW.prepare(g)
    want = G.weight_only_attrs(g)
    assert LW.weight_only(g) == 3
    deq = [op for op in g.ops if op.kind == "dequantize"]
    assert len(deq) == 3 and set(deq) == set(want)
    for op in deq:
        a = want[op]
        assert np.array_equal(op.attrs["q"], a["q"]) and np.array_equal(op.attrs["scale"], a["scale"])
        assert op.attrs["axis"] == a["axis"] == 1 and op.attrs["dtype"] == "f32"
    assert [op.attrs["value"].shape for op in g.ops if op.kind == "const"] == [(512,), (256,), (10,)]


def test_weight_only_rules():
    """mira/quantize.py:34-43: conv weights get axis 0; a constant that is also an
    activation, feeds an elementwise op, or has fewer than 1024 elements stays f32."""
    rng = np.random.default_rng(0)
    conv = {"stride": (1, 1), "padding": (1, 1)}
    g = Graph("t")
    x = g.input("x", (2, 8, 6, 6))
    wc = g.const(rng.standard_normal((16, 8, 3, 3)).astype(np.float32))          # 1152 elements
    small = g.const(rng.standard_normal((8, 8, 3, 3)).astype(np.float32))       # 576 elements
    h = g.op("conv2d", [x, wc], conv)
    h = g.op("conv2d", [h, g.const(rng.standard_normal((8, 16, 3, 3)).astype(np.float32))], conv)
    y = g.input("y", (40, 40))
    sq = g.const(rng.standard_normal((40, 40)).astype(np.float32))
    m = g.op("matmul", [sq, sq])                                                # also the activation
    shared = g.const(rng.standard_normal((40, 40)).astype(np.float32))
    m2 = g.op("add", [g.op("matmul", [y, shared]), shared])                  # also an add operand
    g.outputs = [h, m, m2, g.op("conv2d", [x, small], conv)]
    want = G.weight_only_attrs(g)
    LW.weight_only(g)
    deq = {op for op in g.ops if op.kind == "dequantize"}
    assert deq == set(want)
    assert [op.attrs["axis"] for op in g.ops if op.kind == "dequantize"] == [0, 0]
    assert sq.producer.kind == shared.producer.kind == small.producer.kind == "const"


def test_to_f16_lowering():
    """mira/passes.py:206-253: a cast to f16 after each f32 input, f16 constants and results,
    a cast back to f32 before each f32 output."""
    g = Graph("t")
    x = g.input("x", (4, 16))
    w = g.const(np.full((16, 8), 0.1, np.float32))
    h = g.op("relu", [g.op("matmul", [x, w])])
    g.outputs = [g.op("add", [h, g.const(np.float32(1e-4))])]
    LW.lower_f16(g)
    g.check()
    ops = g.compute_ops()
    assert ops[0].kind == "cast" and ops[0].inputs[0] is x and ops[0].result.type.dtype == "f16"
    assert [op.kind for op in ops] == ["cast", "matmul", "relu", "add", "cast"]
    assert all(op.result.type.dtype == "f16" for op in ops[:-1])
    assert g.outputs[0].producer is ops[-1] and g.outputs[0].type.dtype == "f32"
    consts = [op.attrs["value"] for op in g.ops if op.is_const]
    assert all(c.dtype == np.float16 for c in consts)
    assert any(c.size == 1 and c.item() == np.float16(1e-4) for c in consts)


def test_check_decisions_weight_only():
    """Weight-only int8 matmuls run on rocm at any batch whose K is a multiple of 4 (f32-MFMA
    tiles above 16 rows); with K % 4 != 0 only up to 64 rows (the 8-row weight stream); matmuls
    whose weight is not a dequantize constant stay on the CPU."""
    t = RocmTarget()
    for batch in (4, 64, 65, 4096):
        g = models.mlp_mira(batch=batch)      # K = 784, 512, 256
        LW.prepare(g)
        LW.weight_only(g)
        mm = [op for op in g.compute_ops() if op.kind == "matmul"]
        assert len(mm) == 3
        assert all(t.check(op) is None for op in mm)
    from harness.graph import Graph
    for rows, ok in ((64, True), (65, False)):
        g = Graph("k33")
        x = g.input("x", (rows, 33))
        w = g.const(np.ones((33, 8), np.float32))
        y = g.op("matmul", [x, w])
        g.outputs = [y]
        w.producer.kind = "dequantize"
        w.producer.attrs = {"q": np.ones((33, 8), np.int8), "scale": np.ones(8, np.float32), "axis": 1, "dtype": "f32"}
        r = t.check(y.producer)
        assert (r is None) if ok else ("K % 4 == 0" in r)


def test_check_decisions_weight_only_stem():
    """A weight-only convolution whose channel count is not a multiple of 4 runs on rocm when
    it reads a graph input (the target makes a channel-padded NHWC copy) and stays on the CPU
    when another op produces its input."""
    from harness.graph import Graph
    t = RocmTarget()
    rng = np.random.default_rng(0)
    g = Graph("stem")
    x = g.input("x", (1, 3, 32, 32))
    y = g.op("conv2d", [x, g.const(rng.standard_normal((16, 3, 7, 7)).astype(np.float32))],
             {"stride": (2, 2), "padding": (3, 3)})
    z = g.op("conv2d", [g.op("relu", [x]), g.const(rng.standard_normal((16, 3, 7, 7)).astype(np.float32))],
             {"stride": (2, 2), "padding": (3, 3)})
    g.outputs = [y, z]
    LW.prepare(g)
    LW.weight_only(g)
    first, second = [op for op in g.compute_ops() if op.kind == "conv2d"]
    assert t.check(first) is None
    assert "graph input" in t.check(second)


def test_check_decisions():
    t = RocmTarget()
    g = models.mlp_mira(batch=4)
    LW.prepare(g)
    LW.w8a8(g, [{"x": models.normal_batch((4, 784), 2)}])
    reasons = {op.kind: t.check(op) for op in g.compute_ops()}
    assert reasons["qmatmul"] is None
    assert "softmax" in reasons["softmax"]
    gg = Graph("t")
    x = gg.input("x", (2, 3))
    m = gg.op("matmul", [x, gg.input("w", (3, 4))])
    assert "BLAS" in t.check(m.producer)
    gelu = _dense_graph(relu=False)
    y = gelu.op("gelu", [gelu.outputs[0]])
    gelu.outputs = [y]
    LW.prepare(gelu)
    LW.w8a8(gelu, [{"x": models.normal_batch((8, 16), 2)}])
    assert "not bit-reproducible" in t.check(gelu.compute_ops()[0])


def test_split_falls_back_and_requires_a_fallback_target():
    g = models.mlp_mira(batch=4)
    LW.prepare(g)
    LW.w8a8(g, [{"x": models.normal_batch((4, 784), 2)}])
    segs, reasons = split(g, RocmTarget())
    assert [s.device for s in segs] == ["rocm", "cpu"]
    soft = next(op for op in g.compute_ops() if op.kind == "softmax")
    assert "softmax" in reasons[soft]
    rocm, cpu = segs
    assert cpu.graph.inputs == rocm.graph.outputs and cpu.graph.outputs == g.outputs
    assert all(op.is_constant_like for op in rocm.graph.ops if op.result in {v for o in rocm.graph.ops
                                                                             for v in o.inputs[1:]})

    class NoCompile(RocmTarget):
        def compile(self, g):
            return object()
    with pytest.raises(RuntimeError, match="fallback"):
        Runner(g, NoCompile())


def test_light_segments_stay_on_cpu():
    g = Graph("t")
    x = g.input("x", (1, 4, 6, 6))
    y = g.op("pad", [x], {"pads": ((0, 0), (0, 0), (1, 1), (1, 1)), "value": 0.0})
    g.outputs = [y]
    segs, reasons = split(g, RocmTarget())
    assert [s.device for s in segs] == ["cpu"] and "heavy" in reasons[y.producer]


def test_pack_conv_layouts():
    rng = np.random.default_rng(4)
    q = rng.integers(-127, 128, (5, 3, 7, 7)).astype(np.int8)
    b = pack.pack_conv(q, 4)
    assert b.shape == (32, 256)
    for o in range(5):
        for kh in range(7):
            for kw in range(7):
                for c in range(3):
                    assert b[o, kh * 32 + kw * 4 + c] == q[o, c, kh, kw]
    assert not b[5:].any() and not b[:, 7 * 32:].any()
    q2 = rng.integers(-127, 128, (40, 24, 3, 3)).astype(np.int8)
    b2 = pack.pack_conv(q2, 32)
    assert b2.shape == (64, 320)
    assert b2[7, (2 * 3 + 1) * 32 + 5] == q2[7, 5, 2, 1] and b2[7, (2 * 3 + 1) * 32 + 30] == 0
    m = rng.integers(-127, 128, (100, 10)).astype(np.int8)
    bm = pack.pack_matmul(m)
    assert bm.shape == (32, 128) and np.array_equal(bm[:10, :100], m.T)
    # device byte order: byte k of row n at ((k // 64) * n_pad + n) * 64 + k % 64
    d = pack.device_weights(b2).reshape(-1)
    for n, k in ((0, 0), (7, 229), (63, 319), (40, 64), (13, 127)):
        assert d[((k // 64) * 64 + n) * 64 + k % 64] == b2[n, k]


def test_broadcast_modes():
    assert _bcast_mode((), (2, 8, 5, 5), True) == L.BC_SCALAR
    assert _bcast_mode((8, 1, 1), (2, 8, 5, 5), True) == L.BC_COL
    assert _bcast_mode((1, 8, 1, 1), (2, 8, 5, 5), True) == L.BC_COL
    assert _bcast_mode((2, 8, 5, 5), (2, 8, 5, 5), True) == L.BC_FULL
    assert _bcast_mode((2, 1, 5, 5), (2, 8, 5, 5), True) == L.BC_ROW
    assert _bcast_mode((5,), (2, 8, 5, 5), True) is None            # broadcasts along W, not channels
    assert _bcast_mode((4,), (8, 4), False) == L.BC_COL
    assert _bcast_mode((8, 1), (8, 4), False) == L.BC_ROW


def test_model_mac_counts():
    g = models.resnet18(batch=1)
    LW.prepare(g)
    LW.w8a8(g, peaks=[1.0] * 21)
    assert models.conv_macs(g) == 1_814_073_344
    g = models.mlp_50m(batch=1)
    n_params = sum(op.attrs["value"].size for op in g.ops if op.is_const)
    assert 54_000_000 < n_params < 54_500_000


def _quantize_by_division(y, xs):
    return np.clip(np.rint(np.float32(y) / np.float32(xs)), -127, 127)


def _quantize_by_f64_reciprocal(y, xs):
    """What the GEMM epilogues compute: f32(f64(y) * f64(1/f64(xs))), then rint and clip."""
    q = (y.astype(np.float64) * (1.0 / xs.astype(np.float64))).astype(np.float32)
    return q, np.clip(np.rint(q), -127, 127)


@np.errstate(over="ignore", divide="ignore", invalid="ignore")
def test_requant_reciprocal_is_exact():
    """The fused requant replaces the IEEE f32 division of mira/ops.py:602-603 by a
    multiply with a double-precision reciprocal.  For normal-range quotients the f32
    result is the correctly rounded quotient (no f32 midpoint is an exact quotient of
    two 24-bit significands, and the f64 error is far below the distance to one);
    subnormal quotients may differ in the last place but quantize to 0 either way."""
    rng = np.random.default_rng(0)
    n = 4_000_000
    y = (rng.standard_normal(n) * np.exp2(rng.integers(-30, 30, n))).astype(np.float32)
    xs = (rng.random(n) * np.exp2(rng.integers(-20, 20, n)) + 1e-30).astype(np.float32)
    q64, r64 = _quantize_by_f64_reciprocal(y, xs)
    q32 = y / xs
    normal = np.abs(q32) >= np.float32(2.0 ** -126)
    assert np.array_equal(q64[normal], q32[normal])
    assert np.array_equal(r64, _quantize_by_division(y, xs))
    # exact rint ties: y = (k + 1/2) * xs whenever that product is an f32
    k = rng.integers(-130, 130, n).astype(np.float64) + 0.5
    xs2 = rng.random(n).astype(np.float32) * np.float32(0.05) + np.float32(1e-3)
    y2 = (k * xs2.astype(np.float64)).astype(np.float32)
    exact = y2.astype(np.float64) == k * xs2.astype(np.float64)
    assert exact.sum() > 1000
    q64, r64 = _quantize_by_f64_reciprocal(y2[exact], xs2[exact])
    assert np.array_equal(r64, _quantize_by_division(y2[exact], xs2[exact]))
    assert np.array_equal(q64, np.float32(k[exact]))
    # extremes
    f = np.finfo(np.float32)
    ys = np.array([0.0, -0.0, f.max, -f.max, f.tiny, np.inf, -np.inf, 1e-45, 127.5, -127.5, 126.5], np.float32)
    for x in (np.float32(1e-30), np.float32(1.0), np.float32(3.0), f.max):
        xv = np.full(ys.shape, x, np.float32)
        _, r = _quantize_by_f64_reciprocal(ys, xv)
        assert np.array_equal(r, _quantize_by_division(ys, xv))


def test_gpt_decode_step_graph_and_placement():
    """The decode step verifies, W8A8 quantizes its 6 projections per layer plus the output
    projection, and the rocm target takes every projection except the gelu-fused ones (gelu's
    tanh is libm-dependent, so it stays with the cpu target as MIRA's partitioner would send it)."""
    cfg = models.GPTConfig()
    params = models.gpt_params(cfg, 0)
    g = models.gpt_decode_step(cfg, 2, params)
    LW.prepare(g)
    r = np.random.default_rng(2)
    toks = r.integers(0, cfg.V, (2, cfg.T)).astype(np.int32)
    caches = [(r.standard_normal((2, cfg.T, cfg.D)).astype(np.float32),
               r.standard_normal((2, cfg.T, cfg.D)).astype(np.float32)) for _ in range(cfg.L)]
    feeds = models.gpt_step_feeds(cfg, params, toks, 16, caches)
    LW.w8a8(g, [feeds])
    qops = [op for op in g.compute_ops() if op.kind == "qmatmul"]
    assert len(qops) == 6 * cfg.L + 1
    tgt = RocmTarget()
    rejected = [op for op in qops if tgt.check(op)]
    assert len(rejected) == cfg.L and all(op.attrs["epilogue"][0][0] == "gelu" for op in rejected)
    logits, *kv = G.run_graph(g, feeds)
    assert logits.shape == (2, cfg.V) and np.isfinite(logits).all() and len(kv) == 2 * cfg.L


def test_gpt_placement_by_mode():
    """Default mode: layernorm, the head transposes and the cache concats join the projections
    on rocm and the step splits into 9 segments; approx_f32: the whole step is one segment."""
    cfg = models.GPTConfig()
    params = models.gpt_params(cfg, 0)
    g = LW.prepare(models.gpt_decode_step(cfg, 1, params))
    r = np.random.default_rng(2)
    caches = [(r.standard_normal((1, cfg.T, cfg.D)).astype(np.float32),
               r.standard_normal((1, cfg.T, cfg.D)).astype(np.float32)) for _ in range(cfg.L)]
    LW.w8a8(g, [models.gpt_step_feeds(cfg, params, np.zeros((1, cfg.T), np.int32), 16, caches)])
    segs, reasons = split(g, RocmTarget())
    assert len(segs) == 9 and {op.kind for op in reasons} == {"matmul", "softmax", "qmatmul"}
    segs, reasons = split(g, RocmTarget(approx_f32=True))
    assert [s.device for s in segs] == ["rocm"] and not reasons


class _RecordingLib:
    """Stands in for libmira_rocm.so on the CPU: records the decode-loop calls, computes nothing."""

    def __init__(self):
        self.calls = []

    def __getattr__(self, name):
        def call(*args):
            self.calls.append((name, args))
            return 0
        return call


class _StepExecutable:
    """The device_input / device_output / launch surface of a step executable over CPU tensors."""

    def __init__(self, g):
        import torch
        self.g, self.dev, self.lib = g, torch.device("cpu"), _RecordingLib()
        self.inputs = {v: torch.zeros(v.type.shape, dtype=torch.float32) for v in g.inputs}
        self.outputs = {v: torch.zeros(v.type.shape, dtype=torch.float32) for v in g.outputs}

    def device_input(self, v):
        return self.inputs[v]

    def device_output(self, v):
        return self.outputs[v]

    def launch(self):
        self.lib.calls.append(("step", ()))


def test_decode_loop_host_protocol():
    """mira_amd.decode.DecodeLoop on the host side: each step queues the embed kernel, the
    step's launches and the commit kernel in that order, with the tables, the caches' layout,
    the counters and the prompt length; prompts are validated (shape, token range), and a step
    past the context raises instead of being queued."""
    from harness.decode import DeviceDecoder

    class FakeRunner:
        def __init__(self, g):
            self.graph, self.devices = g, ["rocm"]
            self.exe = _StepExecutable(g)

        def executables(self, device=None):
            return [self.exe]

    cfg = models.GPTConfig()
    params = models.gpt_params(cfg, 0)
    g = LW.prepare(models.gpt_decode_step(cfg, 2, params))
    runner = FakeRunner(g)
    dec = DeviceDecoder(runner, cfg, params, 2)
    calls = runner.exe.lib.calls
    prompt = np.random.default_rng(4).integers(0, cfg.V, (2, 16)).astype(np.int32)
    dec.reset(prompt)
    assert np.array_equal(dec.tokens[:, :16].numpy(), prompt) and not dec.tokens[:, 16:].any()
    dec.run_steps(3)
    assert [c[0] for c in calls] == ["mr_decode_embed", "step", "mr_decode_commit"] * 3
    emb = calls[0][1]
    assert emb[5] == cfg.V and emb[7] == cfg.T and emb[8] == cfg.D and emb[10] == 2 and emb[12] == -10000.0
    commit = calls[2][1]
    assert commit[2] == cfg.V and commit[3] == 2 * cfg.L and commit[9] == cfg.D and commit[14] == 16
    assert (commit[7], commit[8]) == (cfg.D, cfg.T * cfg.D)          # cache row and sequence strides
    assert commit[12] == emb[2] and commit[13] == emb[3] == emb[2] + 4   # the counter and its latch
    with pytest.raises(ValueError):
        dec.reset(np.full((2, 16), cfg.V, np.int32))                 # token id past the vocabulary
    with pytest.raises(ValueError):
        dec.reset(np.zeros((3, 16), np.int32))                       # another batch
    dec.reset(prompt)
    dec.steps_done = cfg.T - 1            # as after a full-context decode
    n = len(calls)
    with pytest.raises(RuntimeError):
        dec.step()
    assert len(calls) == n
    with pytest.raises(RuntimeError):
        dec.run_steps(1, use_graph=True)                             # no graph captured


def test_division_magic_is_exact():
    """The patch loader divides by launch constants d as umulhi(n, ceil(2^32 / d)), which the
    host allows only while n * d < 2^32: checked here for every d < 600 and n up to that
    bound's edge (all n below 4096, a sample above)."""
    rng = np.random.default_rng(0)
    for d in range(2, 600):
        m = ((1 << 32) + d - 1) // d
        nmax = (1 << 32) // d - 1
        n = np.concatenate([np.arange(min(nmax, 4096)), rng.integers(0, nmax, 4096), [nmax]]).astype(np.uint64)
        assert np.array_equal((n * np.uint64(m)) >> np.uint64(32), n // np.uint64(d))


def test_check_rejects_int8_operands_past_the_kernel_limits():
    """An int8 activation or packed weight of 2 GiB or more, or 2^31 pixels, stays on the CPU
    (the contraction kernels use 32-bit buffer offsets and int32 pixel indices) instead of
    failing at launch; the same shapes one size down run on rocm."""
    t = RocmTarget()

    from harness.graph import Op, TensorType, Value

    def q_op(kind, xshape, yshape, q, **conv):
        attrs = {"q": q, "w_scale": np.ones(q.shape[0 if conv else 1], np.float32), "x_scale": 1.0,
                 "dtype": "f32", "epilogue": (), **conv}
        return Op(kind, [Value(TensorType("f32", xshape))], attrs, [Value(TensorType("f32", yshape))])

    def qmm(rows, K, N):
        # the shapes only: an int8 weight of the right shape, with strides of 0 (no memory)
        q = np.lib.stride_tricks.as_strided(np.zeros(1, np.int8), (K, N), (0, 0))
        return q_op("qmatmul", (rows, K), (rows, N), q)

    def qconv(n, c, hw, o=8):
        return q_op("qconv2d", (n, c, hw, hw), (n, o, hw, hw), np.zeros((o, c, 3, 3), np.int8),
                    stride=(1, 1), padding=(1, 1), dilation=(1, 1), groups=1)

    assert t.check(qmm(2 ** 31 // 64 - 1, 64, 16)) is None
    assert "2 GiB" in t.check(qmm(2 ** 31 // 64, 64, 16))
    assert t.check(qmm(8, 133144, 16)) is None
    assert "overflow" in t.check(qmm(8, 133145, 16))        # K * 127^2 reaches 2^31
    assert t.check(qmm(16, 2 ** 17, 2 ** 14 - 32)) is None
    assert "weights of 2 GiB" in t.check(qmm(16, 2 ** 17, 2 ** 14))
    assert t.check(qconv(1024, 64, 180)) is None            # 2.12e9 bytes, under 2^31
    assert "2 GiB" in t.check(qconv(1024, 64, 200))
    assert "pixels" in t.check(qconv(2 ** 16, 4, 256))


def test_get_target_options():
    """The registry branch builds a RocmTarget from MIRA's keyword options (no GPU needed to
    build one) and rejects names it does not know."""
    from mira_amd import get_target
    t = get_target("rocm", approx_f32=True, graph_loops=False)
    assert (t.device, t.debug_acc, t.approx_f32, t.graph_loops) == (0, False, True, False)
    assert get_target("rocm").graph_loops
    with pytest.raises(ValueError, match="unknown rocm target options"):
        get_target("rocm", graph_loop=True)
    with pytest.raises(ValueError, match="unknown target"):
        get_target("npu-sim")
