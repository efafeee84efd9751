"""The .mira front end (harness/mira_lang.py) and the command-line driver (harness/cli.py).

The programs under tests/programs are this repository's own.  Two of them are written to
compute what MIRA's W8A8 example programs compute, so their elaborated graphs are checked
op for op -- kinds, wiring, shapes, attributes and the bytes of every seeded weight --
against the elaborated graphs MIRA itself wrote into the golden fixtures.  The third one
uses every builtin and operator form and is checked against the same computation written
in NumPy."""
import hashlib
import os
import re

import numpy as np
import pytest

from harness import cli
from harness import lowering as LW
from harness import mira_lang as ML
from harness import models
from oracle import golden as G

from conftest import bits_equal
from mira_fixtures import Fixture

PROGRAMS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "programs")
MLP = os.path.join(PROGRAMS, "affine_mlp.mira")
CNN = os.path.join(PROGRAMS, "conv_stages.mira")
BUILTINS = os.path.join(PROGRAMS, "builtins.mira")
# program, its dims, the builder that draws MIRA's example weights, input name and shape
CASES = {"mlp": (MLP, {"B": 64}, models.mlp_mira, "x", (64, 784)),
         "cnn": (CNN, {"N": 16}, models.cnn_mira, "img", (16, 1, 28, 28))}


def _read(path: str) -> str:
    with open(path) as f:
        return f.read()


def _sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _ours(g) -> tuple:
    ids = {v: ("input", v.name, tuple(v.type.shape)) for v in g.inputs}
    ops = []
    for i, op in enumerate(g.ops):
        ids[op.result] = i
        attrs = {k: _sha(v) if k == "value" else v for k, v in op.attrs.items()}
        ops.append((op.kind, tuple(ids[x] for x in op.inputs), tuple(op.result.type.shape), op.result.type.dtype,
                    attrs))
    return ops, [ids[v] for v in g.outputs]


def _mira(doc) -> tuple:
    def norm(v):
        if isinstance(v, dict) and "tuple" in v:
            return tuple(norm(x) for x in v["tuple"])
        return v["sha256"] if isinstance(v, dict) and "sha256" in v else v
    ids = {i["id"]: ("input", i["name"], tuple(i["shape"])) for i in doc["inputs"]}
    ops = []
    for i, op in enumerate(doc["ops"]):
        ids[op["result"]["id"]] = i
        ops.append((op["kind"], tuple(ids[x] for x in op["inputs"]), tuple(op["result"]["shape"]),
                    op["result"]["dtype"], {k: norm(v) for k, v in op["attrs"].items()}))
    return ops, [ids[v] for v in doc["outputs"]]


# ---------------------------------------------------------------- against MIRA's own elaboration

@pytest.mark.parametrize("case", ["mlp", "cnn"])
def test_elaborates_like_mira(case):
    """Generic helpers inlined with their shape symbols bound, `H / 2`-style return dims,
    the entry's const parameters drawn in declaration order from default_rng(0): the same
    graph MIRA's elaborator built for its example program, weights byte for byte."""
    path, dims, _, _, _ = CASES[case]
    g = ML.elaborate(_read(path), dims=dims)
    assert _ours(g) == _mira(Fixture(f"{case}_f32").float_graph("elaborated"))


@pytest.mark.parametrize("precision", [None, "f16"])
@pytest.mark.parametrize("case", ["mlp", "cnn"])
def test_driver_lowers_like_the_builders(case, precision):
    """compile_graph's lowering and W8A8 rewrite of the elaborated program give the same ops
    and attrs (q, w_scale, x_scale, epilogues) as the builders' graphs, which
    test_mira_golden pins against MIRA's quantized graphs; calibration rng(2), rng(3)."""
    path, dims, builder, name, shape = CASES[case]
    calib = [{name: np.random.default_rng(s).standard_normal(shape).astype(np.float32)} for s in (2, 3)]
    prog = cli.compile_graph(ML.elaborate(_read(path), dims=dims), "cpu", precision=precision, quantize="w8a8",
                             calibration=calib)
    built = LW.prepare(builder(batch=shape[0], seed=0), precision)
    LW.w8a8(built, calib)

    def key(g):
        """Compute ops in order; operands named by what they are (input, constant bytes, or
        the index of the compute op producing them), since constants may sit anywhere."""
        index = {op.result: i for i, op in enumerate(g.compute_ops())}

        def operand(v):
            if v in index:
                return index[v]
            return ("const", _sha(v.producer.attrs["value"])) if v.producer is not None else ("input", v.name)
        return [(op.kind, op.result.type.shape, op.result.type.dtype, [operand(v) for v in op.inputs],
                 sorted((k, _sha(v) if isinstance(v, np.ndarray) else v) for k, v in op.attrs.items()))
                for op in g.compute_ops()]
    assert key(prog.graph) == key(built)
    assert {op.kind for op in prog.graph.ops} >= ({"qmatmul"} if case == "mlp" else {"qmatmul", "qconv2d"})


# ---------------------------------------------------------------- builtins against NumPy

def _numpy_builtins(img, dk, w, s):
    n, c, h, wd = img.shape
    xp = np.pad(img, ((0, 0), (0, 0), (2, 2), (2, 2)))
    conv = np.zeros_like(img)
    for i in range(3):
        for j in range(3):
            conv += xp[:, :, 2 * i:2 * i + h, 2 * j:2 * j + wd] * dk[:, 0, i, j][None, :, None, None]
    d = img + conv
    p = d.reshape(n, c, h // 2, 2, wd // 2, 2).mean(axis=(3, 5))
    dp = np.pad(d, ((0, 0), (0, 0), (1, 1), (1, 1)), constant_values=-np.inf)
    q = np.empty_like(p)
    for a in range(h // 2):
        for b in range(wd // 2):
            q[:, :, a, b] = dp[:, :, 2 * a:2 * a + 3, 2 * b:2 * b + 3].max(axis=(2, 3))
    f = (p + q).reshape(n, -1)
    h0 = np.maximum(f @ w, 0.25) * s + 1.5
    hh = h0 - h0.mean(axis=1, keepdims=True)
    t = (1 / (1 + np.exp(-hh)) + np.tanh(hh) * 2 / 4).T
    u = np.minimum(np.abs(t), np.sqrt(np.exp(-t) + 1))
    e = np.exp(u - u.max(axis=0, keepdims=True))
    sm = e / e.sum(axis=0, keepdims=True)
    return np.maximum(u - u.mean(), 0) + sm.mean()


def test_builtins_match_numpy():
    """Dilated depthwise conv, avg / padded max pooling, reshape with symbol arithmetic,
    flatten, matmul, scalar operands on either side, unary minus, keepdims means,
    transpose's default perm, softmax over axis 0: the host evaluator and the oracle on
    the elaborated graph both agree with NumPy in f64 to f32 rounding."""
    rng = np.random.default_rng(4)
    weights = {"dk": rng.standard_normal((3, 1, 3, 3)).astype(np.float32),
               "w": (rng.standard_normal((48, 5)) / 7).astype(np.float32),
               "s": rng.uniform(0.5, 1.5, 5).astype(np.float32)}
    img = rng.standard_normal((2, 3, 8, 8)).astype(np.float32)
    want = _numpy_builtins(img.astype(np.float64), *(weights[k].astype(np.float64) for k in ("dk", "w", "s")))
    g = ML.elaborate(_read(BUILTINS), weights=weights, seed=None)
    (oracle_out,) = G.run_graph(g, {"img": img})
    np.testing.assert_allclose(oracle_out, want, rtol=2e-5, atol=1e-6)
    prog = cli.compile_graph(ML.elaborate(_read(BUILTINS), weights=weights, seed=None), "cpu")
    (host_out,) = prog.run({"img": img})
    np.testing.assert_allclose(host_out, want, rtol=2e-5, atol=1e-6)


def test_weights_given_seeded_and_f16():
    """Given weights replace the seeded draw for those parameters and take nothing from the
    generator, so the next parameter gets the draw the given one would have had
    (mira/elaborate.py:204-210); f16 parameters hold f16 constants."""
    src = ("fn main(x: f32[2, 3], const a: f32[3, 4], const b: f32[4], const c: f16[4]) -> f32[2, 4] {\n"
           "  return x @ a + b\n}\n")
    rng = np.random.default_rng(0)
    drawn = [models.mira_random_weight(rng, s) for s in ((3, 4), (4,), (4,))]
    g = ML.elaborate(src)
    consts = [op.attrs["value"] for op in g.ops if op.kind == "const"]
    assert all(np.array_equal(x, y.astype(x.dtype)) for x, y in zip(consts, drawn))
    assert consts[2].dtype == np.float16
    given = np.full((4,), 3.0, np.float32)
    consts2 = [op.attrs["value"] for op in ML.elaborate(src, weights={"b": given}).ops if op.kind == "const"]
    assert np.array_equal(consts2[1], given) and np.array_equal(consts2[0], consts[0])
    assert np.array_equal(consts2[2], drawn[1].astype(np.float16))


# ---------------------------------------------------------------- errors

ERRORS = [
    ("fn main(x: f32[2]) -> f32[2] {\n  return x +\n}\n", {}, "line 3"),
    ("fn main(x: f32[2]) -> f32[2] { return x $ x }", {}, "unexpected character"),
    ("fn main(x: f32[B, 3]) -> f32[B, 3] { return x }", {}, "'B' of the entry function needs a value"),
    ("fn f(a: f32[N], b: f32[N]) -> f32[N] { return a + b }\n"
     "fn main(x: f32[3], y: f32[4]) -> f32[3] { return f(x, y) }", {}, "N is already 3, got 4"),
    ("fn main(x: f32[4]) -> f32[5] { return x }", {}, "the result of 'main'"),
    ("fn half(v: f32[N]) -> f32[N / 2] { return v }\n"
     "fn main(x: f32[3]) -> f32[1] { return half(x) }", {}, "3 / 2 is not a whole number"),
    ("fn main(x: f32[2]) -> f32[2] { return frobnicate(x) }", {}, "unknown function 'frobnicate'"),
    ("fn f(v: f32[2]) -> f32[2] { return f(v) }\nfn main(x: f32[2]) -> f32[2] { return f(x) }", {},
     "recursive call to 'f'"),
    ("fn f(const v: f32[2]) -> f32[2] { return v }\nfn main(x: f32[2]) -> f32[2] { return f(x) }", {},
     "'const' is only allowed"),
    ("fn main(x: f32[2]) -> f32[2] { return y }", {}, "'y' is undefined"),
    ("fn main(x: f32[2]) -> f32[2] { return relu }", {}, "'relu' is a function"),
    ("fn main(x: f32[2, 2]) -> f32[2, 2] { return softmax(axis=0, x) }", {}, "positional argument after"),
    ("fn main(x: f32[2, 2]) -> f32[2, 2] { return softmax(x, dim=0) }", {}, "no argument 'dim'"),
    ("fn main(x: f32[2, 2]) -> f32[2, 1] { return mean(x, axis=1, keepdims=1) }", {}, "keepdims must be"),
    ("fn main(x: f32[2, 3]) -> f32[2, 3] { return x @ x }", {}, "matmul"),
    ("fn f(v: f32[2]) -> f32[2] { return v }\nfn main(x: f16[2]) -> f32[2] { return f(x) }", {}, "f16 != f32"),
    ("fn main(x: f32[2], const w: f32[2]) -> f32[2] { return x + w }", {"seed": None}, "no value for const"),
    ("fn main(x: f32[2], const w: f32[2]) -> f32[2] { return x + w }", {"weights": {"v": np.ones(2)}},
     "unknown const parameters: v"),
    ("fn main(x: f32[2], const w: f32[2]) -> f32[2] { return x + w }", {"weights": {"w": np.ones(3)}},
     "weight 'w' has shape [3]"),
    ("fn main(x: f32[6]) -> f32[4] { return reshape(x, [-1, 4]) }", {}, "cannot infer -1"),
    ("fn main(x: f32[2]) -> f32[2] { return x }\nfn main(x: f32[2]) -> f32[2] { return x }", {}, "defined twice"),
]


@pytest.mark.parametrize("src,kw,match", ERRORS, ids=[e[2] for e in ERRORS])
def test_errors(src, kw, match):
    with pytest.raises(ML.MiraSyntaxError, match=re.escape(match)):
        ML.elaborate(src, **kw)


# ---------------------------------------------------------------- the driver

def test_cli_check_and_emit(capsys):
    assert cli.main(["check", MLP, "--dim", "B=64"]) == 0
    assert "ok: " in capsys.readouterr().out
    for stage in ("tokens", "ir", "opt", "partition"):
        assert cli.main(["emit", CNN, "--dim", "N=2", "--stage", stage]) == 0
        assert capsys.readouterr().out.strip()
    # the parse tree printed as source parses back to the same tree (line numbers aside)
    assert cli.main(["emit", BUILTINS, "--stage", "ast"]) == 0
    printed = capsys.readouterr().out
    assert cli.format_module(ML.parse(printed)) == printed.strip()
    assert "(C * (H / 2)) * (W / 2)" in printed and "keepdims=true" in printed


def test_cli_run_save_weights_inputs(tmp_path, capsys):
    """--weights / --inputs from .npz, --save; the cpu target's W8A8 run of the CNN (host
    qconv2d / qmatmul) equals the oracle's evaluation of the same quantized graph."""
    rng = np.random.default_rng(9)
    wpath, xpath, out = tmp_path / "w.npz", tmp_path / "x.npz", tmp_path / "y.npy"
    np.savez(wpath, hb=np.linspace(-1, 1, 10).astype(np.float32))
    img = rng.standard_normal((4, 1, 28, 28)).astype(np.float32)
    np.savez(xpath, img=img)
    args = [CNN, "--dim", "N=4", "--weights", str(wpath), "--inputs", str(xpath), "--quantize", "w8a8"]
    assert cli.main(["run", *args, "--save", str(out)]) == 0
    assert "saved to" in capsys.readouterr().out
    got = np.load(out)
    prog = cli.compile_file(CNN, "cpu", dims={"N": 4}, weights={"hb": np.linspace(-1, 1, 10).astype(np.float32)},
                            quantize="w8a8")
    assert bits_equal(got, prog.run({"img": img})[0])
    assert bits_equal(got, G.run_graph(prog.graph, {"img": img})[0])
    assert {op.kind for op in prog.graph.ops} >= {"qconv2d", "qmatmul"}


def test_compare_outputs():
    """--check's measure: max|out - ref| / max|ref| against the tolerance, per output."""
    ref = np.array([[0.5, -2.0], [1.0, 0.0]], np.float32)
    ok, lines = cli.compare([ref + 0.039], [ref], 2e-2)
    assert ok and "PASS" in lines[0]
    ok, lines = cli.compare([ref, ref + np.float32(0.041)], [ref, ref], 2e-2)
    assert not ok and "PASS" in lines[0] and "FAIL" in lines[1] and "2.050e-02 of the peak" in lines[1]
    assert cli.relative_error(ref + 0.5, ref)[2] == pytest.approx(0.25)
    assert cli.relative_error(np.zeros(0), np.zeros(0)) == (0.0, 0.0, 0.0)


def test_random_feeds_follow_the_seed_rule():
    """Inputs not given are standard-normal draws of one default_rng(seed + 1) stream in input
    order; a given input takes no draw."""
    g = ML.elaborate(_read(MLP), dims={"B": 3})
    (x,) = g.inputs
    feeds = cli.random_feeds(g, {}, 4)
    assert np.array_equal(feeds[x.name], np.random.default_rng(5).standard_normal(x.type.shape).astype(np.float32))
    given = np.ones(x.type.shape, np.float32)
    assert cli.random_feeds(g, {x.name: given}, 4)[x.name] is given
    assert cli.parse_bindings(["B=3", "x=1,2"], "--dim", str) == {"B": "3", "x": "1,2"}
    with pytest.raises(cli.CompileError, match="NAME=VALUE"):
        cli.parse_bindings(["B"], "--dim", int)


def test_cli_bench_and_errors(tmp_path, capsys):
    assert cli.main(["bench", MLP, "--dim", "B=8", "--targets", "cpu", "--iters", "2"]) == 0
    assert "cpu" in capsys.readouterr().out
    bad = tmp_path / "bad.mira"
    bad.write_text("fn main(x: f32[2]) -> f32[2] {\n  return x @\n}\n")
    assert cli.main(["run", str(bad)]) == 1
    assert "line 3" in capsys.readouterr().err
    assert cli.main(["check", MLP]) == 1
    assert "'B' of the entry function needs a value" in capsys.readouterr().err


def test_cli_onnx_model(tmp_path, capsys):
    """.onnx files go through the importer; a symbolic batch is pinned with --shape."""
    import onnx_writer as W
    m = W.Model(13)
    x = m.input("x", ("n", 6))
    m.output(m.node("Relu", [m.node("Gemm", [x, m.init(np.eye(6, 3, dtype=np.float32))])]), ("n", 3))
    path = tmp_path / "tiny.onnx"
    path.write_bytes(m.bytes())
    assert cli.main(["check", str(path)]) == 1
    assert "symbolic" in capsys.readouterr().err
    assert cli.main(["check", str(path), "--shape", "x=5,6"]) == 0
    assert "x: f32[5, 6]" in capsys.readouterr().out


# ---------------------------------------------------------------- the rest of the language against MIRA

LANG = {"encoder_block": {"S": 16, "E": 32, "h": 4}, "residual_loop": {"B": 8, "D": 16, "n": 5},
        "char_lm": {"B": 2, "T": 8, "V": 13, "D": 16, "F": 32, "L": 2}, "selection": {"R": 6, "C": 5}}
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _lang_fixture(name: str):
    z = np.load(os.path.join(GOLDEN, f"mira_lang_{name}.npz"))
    doc = __import__("json").loads(str(z["doc"]))
    pick = lambda pre: {k.split(":", 1)[1]: z[k] for k in z.files if k.startswith(pre)}   # noqa: E731
    return doc, pick("feed:"), [pick("calib0:"), pick("calib1:")], z


def _norm_ours(v):
    if hasattr(v, "ops") and hasattr(v, "outputs"):
        return _graph_ours(v)
    if isinstance(v, np.ndarray):
        return _sha(v)
    if isinstance(v, (np.floating, np.integer)):
        return v.item()
    if isinstance(v, (tuple, list)):
        return type(v)(_norm_ours(x) for x in v)
    return v


def _norm_mira(v):
    if isinstance(v, dict):
        if "graph" in v:
            return _graph_mira(v["graph"])
        if "tuple" in v:
            return tuple(_norm_mira(x) for x in v["tuple"])
        if "sha256" in v:
            return v["sha256"]
        if "float" in v:
            return float(v["float"])
    if isinstance(v, list):
        return [_norm_mira(x) for x in v]
    return v


def _graph_ours(g) -> tuple:
    """(ops, outputs) with values named by position: inputs by (name, type), results by
    (op index, result index); sub-graphs nested the same way."""
    ids = {v: ("input", i, v.name, v.type.dtype, tuple(v.type.shape)) for i, v in enumerate(g.inputs)}
    ops = []
    for i, op in enumerate(g.ops):
        ids.update({r: (i, k) for k, r in enumerate(op.results)})
        ops.append((op.kind, tuple(ids[x] for x in op.inputs),
                    tuple((tuple(r.type.shape), r.type.dtype) for r in op.results),
                    {k: _norm_ours(v) for k, v in op.attrs.items()}))
    return ops, [ids[v] for v in g.outputs]


def _graph_mira(doc) -> tuple:
    ids = {v["id"]: ("input", i, v["name"], v["dtype"], tuple(v["shape"])) for i, v in enumerate(doc["inputs"])}
    ops = []
    for i, op in enumerate(doc["ops"]):
        results = op.get("results", [op["result"]])
        ids.update({r["id"]: (i, k) for k, r in enumerate(results)})
        ops.append((op["kind"], tuple(ids[x] for x in op["inputs"]),
                    tuple((tuple(r["shape"]), r["dtype"]) for r in results),
                    {k: _norm_mira(v) for k, v in op["attrs"].items()}))
    return ops, [ids[v] for v in doc["outputs"]]


def _same_graph(ours, theirs):
    (a, ao), (b, bo) = _graph_ours(ours), _graph_mira(theirs)
    assert len(a) == len(b), f"{len(a)} ops vs MIRA's {len(b)}"
    for i, (x, y) in enumerate(zip(a, b)):
        assert x == y, f"op {i}: {x} != MIRA's {y}"
    assert ao == bo


@pytest.mark.parametrize("name", sorted(LANG))
def test_language_elaborates_like_mira(name):
    """Compile-time ints and computed dims, for / if unrolled at elaboration, rebinding,
    comparisons (a < b as greater(b, a), != as 1 - equal), **, slices and integer subscripts
    (slice + reshape), i32 subscripts (gather), tuple returns and the selection builtins: the
    elaborated graph equals the one MIRA's elaborator builds from the same file, op for op,
    with every seeded constant byte for byte."""
    doc, *_ = _lang_fixture(name)
    g = ML.elaborate(_read(os.path.join(PROGRAMS, name + ".mira")), dims=LANG[name])
    _same_graph(g, doc["elaborated"])


@pytest.mark.parametrize("precision", [None, "f16"])
@pytest.mark.parametrize("name", sorted(LANG))
def test_language_optimizes_and_runs_like_mira(name, precision):
    """MIRA's optimizer (f16 lowering with integer casts kept, constant folding of the
    index arithmetic and masks, simplify, CSE of the per-layer masks, DCE, epilogue
    fusion) gives the same graph here, and both the host fallback and the oracle reproduce
    MIRA's results bit for bit on the same feed."""
    doc, feed, _, z = _lang_fixture(name)
    tag = "f16" if precision else "f32"
    prog = cli.compile_file(os.path.join(PROGRAMS, name + ".mira"), "cpu", dims=LANG[name], precision=precision)
    _same_graph(prog.graph, doc[tag])
    outs = prog.run(dict(feed))
    oracle_outs = G.run_graph(prog.graph, dict(feed))
    for k, (o, r) in enumerate(zip(outs, oracle_outs)):
        want = z[f"out:{tag}:{k}"]
        assert o.dtype == want.dtype and bits_equal(o, want), f"output {k} (host)"
        assert bits_equal(np.asarray(r), want), f"output {k} (oracle)"


@pytest.mark.parametrize("precision", [None, "f16"])
@pytest.mark.parametrize("name", sorted(LANG))
def test_language_w8a8_like_mira(name, precision):
    """The W8A8 rewrite of these programs on MIRA's calibration feeds: every q-op's q bytes,
    w_scale and x_scale, and every other op, equal MIRA's; the oracle's evaluation of the
    rewritten graph is MIRA's result bit for bit."""
    doc, feed, calib, z = _lang_fixture(name)
    tag = "w8a8_f16" if precision else "w8a8_f32"
    g = cli.load_graph(os.path.join(PROGRAMS, name + ".mira"), "main", None, LANG[name], 0, None)
    LW.prepare(g, precision=precision)
    LW.w8a8(g, calib)
    _same_graph(g, doc[tag])
    for k, r in enumerate(G.run_graph(g, dict(feed))):
        assert bits_equal(np.asarray(r), z[f"out:{tag}:{k}"]), f"output {k}"


CONTROL = {"fixed_point": {"N": 4, "M": 6, "tol": 1}, "greedy_lm": {"P": 3, "V": 11, "T": 12, "D": 16, "F": 32, "L": 2},
           "device_loop": {"B": 8, "D": 32, "n": 5}}


@pytest.mark.parametrize("name", sorted(CONTROL))
def test_control_flow_elaborates_like_mira(name):
    """Runtime if (both branches' changed variables as results, captures as inputs) and while
    (the assigned tensors as loop state, cond and body capturing what they read), indexed
    assignment as dynamic_update_slice with a start vector, dynamic_slice, token gathers:
    the elaborated graph and every nested sub-graph equal MIRA's."""
    doc, *_ = _lang_fixture(name)
    g = ML.elaborate(_read(os.path.join(PROGRAMS, name + ".mira")), dims=CONTROL[name])
    _same_graph(g, doc["elaborated"])


@pytest.mark.parametrize("precision", [None, "f16"])
@pytest.mark.parametrize("name", sorted(CONTROL))
def test_control_flow_optimizes_and_runs_like_mira(name, precision):
    """MIRA's optimizer on graphs with sub-graphs (each sub-graph optimized; f16 converts the
    loop state completely) gives the same graphs; the runner drives the if / while ops on the
    host and reproduces MIRA's results bit for bit, on the feed and on the negated feed (the
    other branch), as does the oracle."""
    doc, feed, _, z = _lang_fixture(name)
    tag = "f16" if precision else "f32"
    prog = cli.compile_file(os.path.join(PROGRAMS, name + ".mira"), "cpu", dims=CONTROL[name], precision=precision)
    _same_graph(prog.graph, doc[tag])
    neg = {k: (-v if v.dtype.kind == "f" else v) for k, v in feed.items()}
    for suffix, f in (("", feed), ("neg", neg)):
        outs = prog.run(dict(f))
        oracle_outs = G.run_graph(prog.graph, dict(f))
        for k, (o, r) in enumerate(zip(outs, oracle_outs)):
            want = z[f"out:{tag}{suffix}:{k}"]
            assert bits_equal(np.asarray(o), want), f"output {k} {suffix} (host)"
            assert bits_equal(np.asarray(r), want), f"output {k} {suffix} (oracle)"


def test_w8a8_calibrates_loop_bodies(monkeypatch):
    """Beyond MIRA (whose rewrite stops at control flow, mira/quantize.py:84-85): the matmuls
    inside the greedy decoder's while body are W8A8 candidates, each calibrated on the largest
    |activation| over every iteration of every calibration feed.  The peaks are checked against
    the oracle's own loop, instrumented to record every value of every iteration; the rewritten
    program then runs on the host exactly as the oracle evaluates it."""
    path = os.path.join(PROGRAMS, "greedy_lm.mira")
    dims = CONTROL["greedy_lm"]
    g = cli.load_graph(path, "main", None, dims, 0, None)
    LW.prepare(g)
    cands = LW.w8a8_candidates(g)
    (loop,) = [op for op in g.ops if op.kind == "while"]
    in_body = [op for op in cands if op in loop.attrs["body"].ops]
    assert len(in_body) == 2 * 6 + 1 and len(cands) == len(in_body)     # 6 per layer, 2 layers, the head
    rng = np.random.default_rng(5)
    calib = [{"prompt": rng.integers(0, dims["V"], dims["P"]).astype(np.int32)} for _ in range(2)]
    watch = {op.inputs[0] for op in cands}
    seen: dict = {}

    def run_list(self, args):
        env = dict(zip(self.g.inputs, args))
        for op in self.g.ops:
            if op.is_control:
                env.update(zip(op.results, G.control(op, [env[v] for v in op.inputs])))
            else:
                env[op.result] = G.evaluate(op.kind, [env[v] for v in op.inputs], op.attrs)
        for v in watch & env.keys():
            seen[v] = max(seen.get(v, 0.0), float(np.abs(env[v].astype(np.float32)).max()))
        return [env[v] for v in self.g.outputs]

    monkeypatch.setattr(G.CPUExecutable, "run_list", run_list)
    for feed in calib:
        G.run_graph(g, feed)
    monkeypatch.undo()
    assert LW.calibrate(g, calib) == [seen[op.inputs[0]] for op in cands]
    prog = cli.compile_file(path, "cpu", dims=dims, precision=None, quantize="w8a8", calibration=calib)
    body = next(o for o in prog.graph.ops if o.kind == "while").attrs["body"]
    kinds = [op.kind for op in body.ops]
    assert kinds.count("qmatmul") == 13 and "matmul" in kinds        # the attention's runtime products stay f32
    feed = {"prompt": np.array([3, 7, 1], np.int32)}
    (host,) = prog.run(feed)
    (oracle,) = G.run_graph(prog.graph, feed)
    assert bits_equal(host, oracle)


LANG_ERRORS = [
    ("fn main(x: f32[2]) -> f32[2] { let y = x\n let y = x\n return y }", {}, "'y' is already defined"),
    ("fn main(x: f32[2]) -> f32[2] { z = x\n return x }", {}, "undefined variable 'z'"),
    ("fn main(x: f32[2]) -> f32[2] { while x > 0 { x = x - 1 }\n return x }", {}, "must be a single value"),
    ("fn main(x: f32[2]) -> f32[2] { let k = 1\n if max(x) > 0 { k = 2 }\n return x * k }", {},
     "'k' is a compile-time value"),
    ("fn main(x: f32[2]) -> f32[2] { y[0] = 1\n return x }", {}, "undefined variable 'y'"),
    ("fn main(x: f32[2]) -> f32[2] { let t = zeros([], i32)\n while t < 3 { t = t + 1.5 }\n return x }", {},
     "does not mix with an i32 tensor"),
    ("fn main(x: f32[2]) -> f32[2] { return grad(sum(x), x) }", {}, "grad() is not supported"),
    ("fn main(x: f32[2]) -> f32[2] { return x[0:0] }", {}, "empty slice 0:0"),
    ("fn main(x: f32[2]) -> f32[2] { return x[2] }", {}, "index 2 is out of range"),
    ("fn main(x: f32[2]) -> f32[2] { return x[x] }", {}, "must be i32"),
    ("fn main(x: f32[2]) -> f32[2] { return x < x < x }", {}, "can't be chained"),
    ("fn main(x: f32[2], n: int) -> f32[2] { return x * n }", {}, "int parameter 'n'"),
    ("fn f(x: f32[2], n: int) -> f32[2] { return x * n }\nfn main(x: f32[2]) -> f32[2] { return f(x, 1.5) }",
     {}, "must be a whole number"),
    ("fn main(x: f32[2]) -> (f32[2], f32[2]) { return x }", {}, "returns 1 value(s)"),
    ("fn main(x: f32[2]) -> f32[2] { let a, b = x\n return a }", {}, "cannot unpack"),
    ("fn main(x: i32[2]) -> i32[2] { return x + 0.5 }", {}, "does not mix with an i32 tensor"),
]


@pytest.mark.parametrize("src,kw,match", LANG_ERRORS, ids=[e[2] for e in LANG_ERRORS])
def test_language_errors(src, kw, match):
    with pytest.raises(ML.MiraSyntaxError, match=re.escape(match)):
        ML.elaborate(src, **kw)


def test_emit_ast_round_trips():
    """`emit ast` prints every statement and expression form as source that parses back to
    the same tree (up to line numbers): formatting the re-parsed text gives the same text,
    and that text elaborates to the same graph."""
    for name in LANG:
        text = cli.format_module(ML.parse(_read(os.path.join(PROGRAMS, name + ".mira"))))
        assert cli.format_module(ML.parse(text)) == text, name
        _same_graph(ML.elaborate(text, dims=LANG[name]), _lang_fixture(name)[0]["elaborated"])


def test_device_loop_decisions():
    """Which while / if ops the rocm target runs on the device: the float-state loop once
    W8A8 has made its matmul a q-op (its body's standalone mul / add / greater and nested if
    accepted there, and only there), in f32 and f16; not while an f32 matmul (BLAS order,
    exact mode) or an op rocm lacks (reduce_max) remains; the greedy decoder, integer state
    and all, in the approximate mode."""
    from mira_amd.target import RocmTarget
    t = RocmTarget()
    dims = CONTROL["device_loop"]
    rng = np.random.default_rng(5)
    calib = [{"x": rng.standard_normal((dims["B"], dims["D"])).astype(np.float32)} for _ in range(2)]
    for precision in (None, "f16"):
        g = cli.load_graph(os.path.join(PROGRAMS, "device_loop.mira"), "main", None, dims, 0, None)
        LW.prepare(g, precision)
        loop = next(op for op in g.ops if op.kind == "while")
        assert "f32 matmul" in t.check(loop)
        LW.w8a8(g, calib)
        assert t.check(loop) is None
        body = [op for op in loop.attrs["body"].ops if op.kind != "const"]
        assert sorted({op.kind for op in body}) == ["add", "greater", "if", "mul", "qmatmul"]
        assert t.check(next(op for op in body if op.kind == "mul")) == "'mul' has no rocm kernel"
        assert t.check_in_loop(next(op for op in body if op.kind == "mul")) is None
    for name, blocker in (("fixed_point", "reduce_max"), ("greedy_lm", "f32 matmul")):
        g = cli.load_graph(os.path.join(PROGRAMS, name + ".mira"), "main", None, CONTROL[name], 0, None)
        LW.prepare(g)
        loop = next(op for op in g.ops if op.kind == "while")
        assert blocker in t.check(loop)
        if name == "greedy_lm":     # integer state, gathers, dynamic windows, argmax: all on rocm
            assert RocmTarget(approx_f32=True).check(loop) is None
