"""Golden fixtures from MIRA itself (tests/golden, made by make_mira_fixtures.py with the
reference's own compiler): its W8A8 programs examples/mlp.mira and examples/cnn.mira,
compiled as tests/test_control_dynamic_quant.py:217-225 compiles them (calibration
rng(2), rng(3); feed rng(1)), in f32 and in the f16 graph of its "auto" precision.

CPU tests pin the harness (weights, epilogue fusion, W8A8 attrs) and the oracle (its
evaluation of MIRA's quantized graphs, its restatement of MIRA's rewrite) against
MIRA's output.  The GPU test runs MIRA's own quantized graphs -- MIRA's q, w_scale,
x_scale and epilogues -- on the rocm target and compares every stored value bit for
bit with MIRA's cpu target.
"""
import hashlib

import numpy as np
import pytest

from harness import lowering as LW
from harness import models
from harness.runner import Runner, split
from mira_amd.target import RocmTarget
from oracle import golden as G

from conftest import bits_equal
from mira_fixtures import CASES, Fixture

BUILDERS = {"mlp": (models.mlp_mira, "x", (64, 784)), "cnn": (models.cnn_mira, "img", (16, 1, 28, 28))}
_cache: dict = {}


def fixture(case: str) -> Fixture:
    if case not in _cache:
        _cache[case] = Fixture(case)
    return _cache[case]


def _sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _calib(name: str, shape: tuple) -> list:
    return [{name: np.random.default_rng(s).standard_normal(shape).astype(np.float32)} for s in (2, 3)]


def _harness_graph(prog: str, precision=None, quantize=True):
    builder, name, shape = BUILDERS[prog]
    g = builder(batch=shape[0], seed=0)
    LW.prepare(g, precision=precision)
    if quantize:
        LW.w8a8(g, _calib(name, shape))
    return g


# ---------------------------------------------------------------- harness vs MIRA (CPU)

@pytest.mark.parametrize("prog", ["mlp", "cnn"])
def test_builders_draw_mira_weights(prog):
    """The builders reproduce the weights MIRA's elaborator gives the program's const
    parameters (seed 0, mira/elaborate.py:196-213,1114-1123), byte for byte."""
    doc = fixture(f"{prog}_f32").float_graph("elaborated")
    want = [op["attrs"]["value"]["sha256"] for op in doc["ops"] if op["kind"] == "const"]
    builder, _, shape = BUILDERS[prog]
    g = builder(batch=shape[0], seed=0)
    got = [_sha(op.attrs["value"]) for op in g.ops if op.kind == "const"]
    assert got == want


@pytest.mark.parametrize("prog", ["mlp", "cnn"])
def test_lowering_matches_mira_optimizer(prog):
    """harness.lowering.prepare gives the compute ops, epilogue steps and operands that
    MIRA's optimizer (mira/passes.py:266-286) gives the same program."""
    doc = fixture(f"{prog}_f32").float_graph("optimized")
    const_sha = {op["result"]["id"]: op["attrs"]["value"]["sha256"] for op in doc["ops"] if op["kind"] == "const"}

    def norm(a):
        return {k: (tuple(tuple(s["tuple"]) for s in v["tuple"]) if k == "epilogue" else
                    tuple(v["tuple"]) if isinstance(v, dict) and "tuple" in v else v) for k, v in a.items()}
    want = [(op["kind"], tuple(op["result"]["shape"]), norm(op["attrs"]),
             tuple(const_sha.get(i, "value") for i in op["inputs"])) for op in doc["ops"] if op["kind"] != "const"]
    g = _harness_graph(prog, quantize=False)
    got = [(op.kind, op.result.type.shape, dict(op.attrs),
            tuple(_sha(v.producer.attrs["value"]) if v.producer is not None and v.producer.is_const else "value"
                  for v in op.inputs)) for op in g.compute_ops()]
    assert got == want


@pytest.mark.parametrize("case", CASES)
def test_w8a8_attrs_match_mira(case):
    """q and w_scale equal MIRA's bit for bit, the epilogue tuples and dtypes are MIRA's, and
    x_scale equals MIRA's (matmul activations: exactly; conv activations, whose calibration
    peaks come from another f32 summation order: to 1e-6 relative)."""
    fx = fixture(case)
    prog, prec = case.split("_")
    g = _harness_graph(prog, precision=None if prec == "f32" else "f16")
    got = [op for op in g.ops if op.kind in ("qmatmul", "qconv2d")]
    want = [op for op in fx.graph.ops if op.kind in ("qmatmul", "qconv2d")]
    assert [op.kind for op in got] == [op.kind for op in want]
    for a, b in zip(got, want):
        assert np.array_equal(a.attrs["q"], b.attrs["q"]) and a.attrs["q"].dtype == np.int8
        assert np.array_equal(a.attrs["w_scale"], b.attrs["w_scale"])
        assert a.attrs.get("epilogue", ()) == b.attrs.get("epilogue", ())
        assert a.attrs["dtype"] == b.attrs["dtype"] and a.result.type == b.result.type
        assert a.attrs["x_scale"] == b.attrs["x_scale"]


# ---------------------------------------------------------------- oracle vs MIRA (CPU)

@pytest.mark.parametrize("case", CASES)
def test_oracle_reproduces_mira_values(case):
    """The oracle's evaluation of MIRA's quantized graph equals MIRA's cpu target on every
    stored value, bit for bit (pins the oracle's q-op, epilogue, pooling, reshape, cast and
    softmax restatements on these programs)."""
    fx = fixture(case)
    env = {v: np.asarray(fx.feeds[v.name]) for v in fx.graph.inputs}
    for op in fx.graph.ops:
        env[op.result] = G.evaluate(op.kind, [env[x] for x in op.inputs], op.attrs)
    assert fx.values
    for v, want in fx.values.items():
        assert bits_equal(np.asarray(env[v]), want), f"{case}: {v.producer.kind} differs"


@pytest.mark.parametrize("prog", ["mlp", "cnn"])
def test_oracle_rewrite_matches_mira(prog):
    """The oracle's restatement of MIRA's calibration + W8A8 rewrite (w8a8_attrs, on the
    harness's float graph of the program) gives MIRA's attrs."""
    fx = fixture(f"{prog}_f32")
    _, name, shape = BUILDERS[prog]
    g = _harness_graph(prog, quantize=False)
    attrs = G.w8a8_attrs(g, _calib(name, shape))
    want = [op for op in fx.graph.ops if op.kind in ("qmatmul", "qconv2d")]
    got = [attrs[op] for op in g.ops if op in attrs]
    assert len(got) == len(want) == 3
    for a, b in zip(got, want):
        assert np.array_equal(a["q"], b.attrs["q"]) and np.array_equal(a["w_scale"], b.attrs["w_scale"])
        assert a.get("epilogue", ()) == b.attrs.get("epilogue", ())
        assert a["x_scale"] == b.attrs["x_scale"]


# ---------------------------------------------------------------- the split (CPU)

@pytest.mark.parametrize("case", CASES)
def test_split_matches_mira_partition(case):
    """The harness's split of MIRA's graph puts the same ops on rocm as MIRA's own
    partitioner (mira/partition.py:70-93) did with RocmTarget plugged in."""
    fx = fixture(case)
    segs, _ = split(fx.graph, RocmTarget())
    got = [{"device": s.device, "kinds": [op.kind for op in s.graph.compute_ops()]} for s in segs]
    assert got == fx.doc["partition_with_rocm"]


# ---------------------------------------------------------------- rocm vs MIRA (GPU)

@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES)
def test_rocm_runs_mira_programs(case):
    """MIRA's own quantized graph on the rocm target (softmax and the final cast on the
    oracle's cpu target, as MIRA's partitioner places them): outputs and every stored
    intermediate value equal MIRA's cpu target bit for bit; every int32 accumulator
    equals the oracle's."""
    fx = fixture(case)
    runner = Runner(fx.graph, RocmTarget(debug_acc=True), fallback=G.CPUTarget())
    assert runner.devices == ["rocm", "cpu"]
    env = runner.run_env({v: fx.feeds[v.name] for v in fx.graph.inputs})
    checked = 0
    for v, want in fx.values.items():
        if v in env:
            assert bits_equal(np.asarray(env[v]), want), f"{case}: {v.producer.kind} differs"
            checked += 1
    assert checked >= 2
    ref = {v: np.asarray(fx.feeds[v.name]) for v in fx.graph.inputs}
    for op in fx.graph.ops:
        ref[op.result] = G.evaluate(op.kind, [ref[x] for x in op.inputs], op.attrs)
    (exe,) = runner.executables("rocm")
    accs = exe.accumulators()
    for op in fx.graph.ops:
        if op.kind == "qmatmul":
            want = G.qmatmul_acc(ref[op.inputs[0]], op.attrs)
        elif op.kind == "qconv2d":
            assert G.qconv2d_certificate(ref[op.inputs[0]], op.attrs) < 2 ** 24
            want = G.qconv2d_acc(ref[op.inputs[0]], op.attrs).transpose(0, 2, 3, 1)
        else:
            continue
        assert np.array_equal(accs[op.result], want.reshape(-1, want.shape[-1]).astype(np.int32))
