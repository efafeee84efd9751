""".mira programs through the command-line driver (harness/cli.py) on the rocm target.

The driver elaborates the program, lowers it as MIRA's compiler does (precision "auto"
is f16 for rocm), W8A8-quantizes it on its default calibration and splits it between
rocm and the host fallback (softmax stays on the host).  The output must equal the
oracle's evaluation of the same lowered graph bit for bit, and `run --check` must pass
against the unquantized cpu run, as MIRA's CLI checks it."""
import os

import numpy as np
import pytest

from harness import cli

from conftest import bits_equal
from gpu_util import oracle_env

pytestmark = pytest.mark.gpu

PROGRAMS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "programs")
CASES = [("affine_mlp.mira", {"B": 64}), ("conv_stages.mira", {"N": 16})]


@pytest.mark.parametrize("precision", ["auto", None])
@pytest.mark.parametrize("name,dims", CASES)
def test_program_bit_exact(name, dims, precision):
    prog = cli.compile_file(os.path.join(PROGRAMS, name), "rocm", dims=dims, precision=precision, quantize="w8a8")
    on_rocm = [op.kind for seg in prog.segments if seg.device == "rocm" for op in seg.graph.compute_ops()]
    assert "qmatmul" in on_rocm and ("qconv2d" in on_rocm) == name.startswith("conv")
    f16 = [op for op in prog.graph.compute_ops() if op.result.type.dtype == "f16"]
    assert bool(f16) == (precision == "auto")
    feeds = cli.random_feeds(prog.graph, {}, 0)
    print(f"{name} precision={precision}", flush=True)
    (got,) = prog.run(feeds)
    want = oracle_env(prog.graph, feeds)[prog.graph.outputs[0]]
    assert bits_equal(got, want), f"max abs {np.abs(got - want).max()}"


@pytest.mark.parametrize("name,dims", CASES)
def test_cli_run_check(name, dims, capsys):
    """--check at 3e-2, the tolerance of the reference's own W8A8 tests
    (tests/test_control_dynamic_quant.py:217-225): on the default calibration the MLP's
    W8A8 error is 0.021 (f32) / 0.023 (f16) of max|ref|, just above the CLI's 2e-2
    default, as it is for the reference itself with the same attrs."""
    dim = [f"{k}={v}" for k, v in dims.items()][0]
    assert cli.main(["run", os.path.join(PROGRAMS, name), "-t", "rocm", "--dim", dim, "--quantize", "w8a8",
                     "--check", "--tol", "3e-2"]) == 0
    out = capsys.readouterr().out
    assert "rocm" in out and "PASS" in out and "FAIL" not in out


def test_cli_run_weight_only(capsys):
    """--quantize int8 (weight-only): the matmuls on rocm, within --check's tolerance."""
    assert cli.main(["run", os.path.join(PROGRAMS, "affine_mlp.mira"), "-t", "rocm", "--dim", "B=8",
                     "--quantize", "int8", "--precision", "none", "--check"]) == 0
    assert "PASS" in capsys.readouterr().out


# ---------------------------------------------------------------- the rest of MIRA's language on rocm

LANG = {"encoder_block": {"S": 16, "E": 32, "h": 4}, "residual_loop": {"B": 8, "D": 16, "n": 5},
        "char_lm": {"B": 2, "T": 8, "V": 13, "D": 16, "F": 32, "L": 2}, "selection": {"R": 6, "C": 5}}
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("precision", ["auto", None])
@pytest.mark.parametrize("name", sorted(LANG))
def test_language_programs_on_rocm(name, precision):
    """Programs beyond the CNN / MLP subset (attention heads, unrolled loops, token gathers,
    masks, losses, selection builtins), W8A8-quantized on MIRA's calibration feeds: their
    q-matmuls (and layernorms) run on rocm, the rest on the host, and every result equals
    the oracle's evaluation of the same lowered graph and MIRA's own result bit for bit."""
    z = np.load(os.path.join(GOLDEN, f"mira_lang_{name}.npz"))
    pick = lambda pre: {k.split(":", 1)[1]: z[k] for k in z.files if k.startswith(pre)}   # noqa: E731
    feed, calib = pick("feed:"), [pick("calib0:"), pick("calib1:")]
    prog = cli.compile_file(os.path.join(PROGRAMS, name + ".mira"), "rocm", dims=LANG[name], precision=precision,
                            quantize="w8a8", calibration=calib)
    on_rocm = [op.kind for seg in prog.segments if seg.device == "rocm" for op in seg.graph.compute_ops()]
    assert "qmatmul" in on_rocm, on_rocm
    print(f"{name} precision={precision} rocm ops {len(on_rocm)}", flush=True)
    got = prog.run(dict(feed))
    env = oracle_env(prog.graph, dict(feed))
    tag = "w8a8_f16" if precision == "auto" else "w8a8_f32"
    for k, v in enumerate(prog.graph.outputs):
        assert bits_equal(got[k], env[v]), f"output {k} vs the oracle"
        assert bits_equal(got[k], z[f"out:{tag}:{k}"]), f"output {k} vs MIRA"


CONTROL = {"fixed_point": {"N": 4, "M": 6, "tol": 1}, "greedy_lm": {"P": 3, "V": 11, "T": 12, "D": 16, "F": 32, "L": 2},
           "device_loop": {"B": 8, "D": 32, "n": 5}}


@pytest.mark.parametrize("precision", ["auto", None])
@pytest.mark.parametrize("name", sorted(CONTROL))
def test_control_flow_programs_on_rocm(name, precision):
    """Runtime if / while programs compiled for rocm: the control ops run on the host (the
    rocm target does not take control flow, mira/partition.py:74-75) and their sub-graphs are
    split for rocm like any graph -- the greedy decoder's layernorms run on rocm inside every
    loop iteration -- and every result equals MIRA's, on the feed and on the negated feed."""
    z = np.load(os.path.join(GOLDEN, f"mira_lang_{name}.npz"))
    feed = {k.split(":", 1)[1]: z[k] for k in z.files if k.startswith("feed:")}
    prog = cli.compile_file(os.path.join(PROGRAMS, name + ".mira"), "rocm", dims=CONTROL[name], precision=precision)
    placed = prog.runner.placements()
    assert ("cpu", "while") in placed
    if name == "greedy_lm":
        assert ("rocm", "layernorm") in placed, placed
    tag = "f16" if precision == "auto" else "f32"
    for suffix, f in (("", feed), ("neg", {k: (-v if v.dtype.kind == "f" else v) for k, v in feed.items()})):
        print(f"{name} precision={precision} feed{suffix}", flush=True)
        got = prog.run(dict(f))
        for k, o in enumerate(got):
            assert bits_equal(np.asarray(o), z[f"out:{tag}{suffix}:{k}"]), f"output {k} {suffix} vs MIRA"


@pytest.mark.parametrize("precision", ["auto", None])
def test_w8a8_loop_body_on_rocm(precision):
    """The greedy decoder W8A8-quantized through its while loop (calibration folded over every
    iteration): 11 of its 13 loop-body q-matmuls and its layernorms run on rocm inside every
    iteration of the host-driven loop (the two whose epilogue is gelu, a libm call, stay on the
    host in the exact mode), and the decoded tokens equal the oracle's evaluation of the same
    quantized program."""
    dims = CONTROL["greedy_lm"]
    rng = np.random.default_rng(5)
    calib = [{"prompt": rng.integers(0, dims["V"], dims["P"]).astype(np.int32)} for _ in range(2)]
    prog = cli.compile_file(os.path.join(PROGRAMS, "greedy_lm.mira"), "rocm", dims=dims, precision=precision,
                            quantize="w8a8", calibration=calib)
    placed = prog.runner.placements()
    assert placed.count(("rocm", "qmatmul")) == 11 and placed.count(("cpu", "qmatmul")) == 2, placed
    assert ("rocm", "layernorm") in placed
    for prompt in ([3, 7, 1], [0, 10, 5]):
        feed = {"prompt": np.array(prompt, np.int32)}
        print(f"greedy_lm w8a8 precision={precision} prompt={prompt}", flush=True)
        (got,) = prog.run(dict(feed))
        want = oracle_env(prog.graph, feed)[prog.graph.outputs[0]]
        assert bits_equal(np.asarray(got), want), (got, want)


@pytest.mark.parametrize("precision", ["auto", None])
def test_device_loop_on_rocm(precision):
    """A while loop with float state, W8A8-quantized through the loop, runs on the device:
    the while op (and the if nested in its body) is a rocm op, its cond / body / branch
    sub-graphs nested rocm executables (the q-matmul, its fused epilogue, the standalone
    mul / add / greater on mr_elementwise_f32), the state in device buffers and one flag
    read back per iteration.  Both results equal the oracle's evaluation of the same
    quantized program bit for bit, on two feeds (state reset between runs)."""
    dims = CONTROL["device_loop"]
    rng = np.random.default_rng(5)
    calib = [{"x": rng.standard_normal((dims["B"], dims["D"])).astype(np.float32)} for _ in range(2)]
    prog = cli.compile_file(os.path.join(PROGRAMS, "device_loop.mira"), "rocm", dims=dims, precision=precision,
                            quantize="w8a8", calibration=calib)
    placed = prog.runner.placements()
    assert ("rocm", "while") in placed and not any(dev == "cpu" for dev, _ in placed), placed
    for seed in (1, 2):
        feed = {"x": np.random.default_rng(seed).standard_normal((dims["B"], dims["D"])).astype(np.float32)}
        print(f"device_loop precision={precision} seed={seed}", flush=True)
        got = prog.run(dict(feed))
        env = oracle_env(prog.graph, feed)
        for k, v in enumerate(prog.graph.outputs):
            assert bits_equal(np.asarray(got[k]), env[v]), f"output {k}"


def test_device_loop_iteration_limit():
    """A device while loop that would run past its max_iters raises after that many
    iterations (mira/backends/cpu.py:51), every kernel finishing normally: the limit is
    forced from the host on the compiled graph (5 iterations needed, 3 allowed)."""
    from harness import lowering as LW
    from harness.runner import Runner
    from mira_amd._lib import RocmError
    from mira_amd.target import RocmTarget
    dims = CONTROL["device_loop"]
    rng = np.random.default_rng(5)
    calib = [{"x": rng.standard_normal((dims["B"], dims["D"])).astype(np.float32)} for _ in range(2)]
    g = cli.load_graph(os.path.join(PROGRAMS, "device_loop.mira"), "main", None, dims, 0, None)
    LW.prepare(g)
    LW.w8a8(g, calib)
    next(op for op in g.ops if op.kind == "while").attrs["max_iters"] = 3
    runner = Runner(g, RocmTarget())
    assert runner.devices == ["rocm"]
    with pytest.raises(RocmError, match="exceeded 3 iterations"):
        runner.run({"x": calib[0]["x"]})


@pytest.mark.parametrize("graph_loops", [True, False])
@pytest.mark.parametrize("quantize", [None, "w8a8"])
@pytest.mark.parametrize("precision", [None, "f16"])
def test_greedy_decoder_device_loop(precision, quantize, graph_loops):
    """The greedy KV-cache decoder's while loop run on the device in the approximate mode:
    token buffer, step counter, embedding gathers, position and cache windows (dynamic
    slices and updates), masks, attention, argmax and the prompt-or-prediction where, all
    on rocm with the integer state held in device buffers.  The decoded tokens equal the
    oracle's (the attention's f32 products and softmax agree to f32 rounding, which moves no
    argmax here), for two prompts.  With graph_loops the condition and body steps are
    recorded as HIP graphs after the first iteration: every later iteration of both prompts
    is a replay, with the flag read back (a synchronisation) between replays."""
    from harness import hosteval, lowering as LW
    from harness.runner import Runner
    from mira_amd.target import RocmTarget
    dims = CONTROL["greedy_lm"]
    g = cli.load_graph(os.path.join(PROGRAMS, "greedy_lm.mira"), "main", None, dims, 0, None)
    LW.prepare(g, precision)
    if quantize:
        rng = np.random.default_rng(5)
        LW.w8a8(g, [{"prompt": rng.integers(0, dims["V"], dims["P"]).astype(np.int32)} for _ in range(2)])
    runner = Runner(g, RocmTarget(approx_f32=True, graph_loops=graph_loops), fallback=hosteval.HostTarget())
    placed = runner.placements()
    # the loop on rocm; before it, the prompt's write into the token buffer (an integer op
    # outside any loop) on the host
    assert placed == [("cpu", "dynamic_update_slice"), ("rocm", "while")], placed
    for prompt in ([3, 7, 1], [0, 10, 5]):
        feed = {"prompt": np.array(prompt, np.int32)}
        print(f"greedy_lm device loop precision={precision} quantize={quantize} graph_loops={graph_loops} "
              f"prompt={prompt}", flush=True)
        (got,) = runner.run(dict(feed))
        want = oracle_env(g, feed)[g.outputs[0]]
        assert np.array_equal(np.asarray(got), want), (got, want)
    import torch
    recorded = sum(isinstance(k, torch.cuda.CUDAGraph) for seg in runner.segments
                   for k in getattr(seg.executable, "keep", []))
    assert recorded == (2 if graph_loops else 0)


@pytest.mark.parametrize("quantize", [None, "w8a8"])
def test_greedy_decoder_host_loop_segments(quantize):
    """The same decoder with its loop driven from the host and the body split into rocm and
    cpu segments.  One rocm segment's attention matmul reads a key view whose transpose ran
    in a cpu segment: the rocm executable must treat that input as its own buffer rather than
    follow the transpose back into the other segment.  Tokens equal the oracle's."""
    from harness import hosteval, lowering as LW
    from harness.runner import Runner
    from mira_amd.target import RocmTarget

    class HostLoops(RocmTarget):
        def _check_control(self, op):
            return "loops driven from the host"

    dims = CONTROL["greedy_lm"]
    g = cli.load_graph(os.path.join(PROGRAMS, "greedy_lm.mira"), "main", None, dims, 0, None)
    LW.prepare(g)
    if quantize:
        rng = np.random.default_rng(5)
        LW.w8a8(g, [{"prompt": rng.integers(0, dims["V"], dims["P"]).astype(np.int32)} for _ in range(2)])
    runner = Runner(g, HostLoops(approx_f32=True), fallback=hosteval.HostTarget())
    assert ("cpu", "while") in runner.placements()
    for prompt in ([3, 7, 1], [0, 10, 5]):
        feed = {"prompt": np.array(prompt, np.int32)}
        print(f"greedy_lm host loop quantize={quantize} prompt={prompt}", flush=True)
        (got,) = runner.run(dict(feed))
        want = oracle_env(g, feed)[g.outputs[0]]
        assert np.array_equal(np.asarray(got), want), (got, want)
