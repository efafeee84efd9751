"""Benchmark: W8A8 ResNet-18 inference on one MI355X through the rocm target.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--batch 256] [--no-cpu-baseline]
    python bench.py --workload mlp50m|mlp50m-int8|mobilenetv2|mobilenetv2-f16 [--batch B] [--steps K] [--warmup W]
    python bench.py --per-launch [--workload W] [--batch B]

A step is one inference of the whole batch (all 20 int8 implicit-GEMM convs,
pooling, the fc layer) with the input already resident in HBM.  Prints ONE
JSON line on stdout; progress goes to stderr.

value      = int8 TOPS over the whole network: 2 * (conv + fc MACs) / step time
roofline   = the qconv2d kernels (the dominant kernel class): their algorithmic
             ops / their summed launch durations (HIP events around each launch
             on the stream they run on), against the 5.0 POPS int8 dense peak
cpu_baseline = the NumPy golden model (oracle/golden.py, the reference cpu
             target's algorithms) on a 2-image sample with the same attrs,
             timed on this host.
kernels    = every launch kind of the step: its summed launch durations and its
             algorithmic rate, int8 TOP/s against 5.0 POPS for the contractions,
             HBM GB/s against 8 TB/s for the rest.

--workload mlp50m / mobilenetv2 time the other W8A8 networks the same way and
print one JSON line with their per-kind breakdown (no cpu baseline): the 50M
MLP at batch 1 runs its four layers on the decode-shaped weight-streaming
qmatmul kernel, MobileNetV2 its 17 depthwise convolutions fused with the
convolutions before them (the expanded tensors never stored).  mlp50m-int8 is the same MLP in the
int8 weight-only mode (f32 activations, int8 weights dequantized in
registers), batch 1: four weight-streaming f32 matmul launches.
resnet18-onnx is ResNet-18 laid out as MIRA's ONNX importer emits it (BN as a
per-channel mul + add in each conv epilogue instead of folded weights);
resnet18-f16 and mobilenetv2-f16 are the f16 graphs (MIRA's default precision
for accelerator targets), every result rounded to f16.
gpt-decode times greedy decoding with the character-level GPT (default batch 1;
16-token prompt, --tokens generated): the whole loop resident on the GPU, one
HIP graph replay per step, in microseconds per token, beside the eager launch
loop and the bit-exact mode driven from the host.
greedy-loop times the same kind of decoder written as a MIRA program with a
runtime while loop, compiled whole for the device (approx_f32), in microseconds
per token, beside the eager loop, the host-driven loop and the host evaluator.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

# The CPU baseline's BLAS pool (set before NumPy loads it): the OpenMP thread count the
# environment gives, else every host CPU up to 16.
os.environ.setdefault("OPENBLAS_NUM_THREADS", os.environ.get("OMP_NUM_THREADS", str(min(os.cpu_count() or 1, 16))))

import numpy as np  # noqa: E402

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

INT8_PEAK_TOPS = 5000.0          # MI355X dense int8 MFMA peak (5.0 POPS)
HBM_PEAK_GBS = 8000.0            # MI355X HBM3E peak (8 TB/s)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def build(batch: int, seed: int = 0, peaks=None):
    """W8A8 ResNet-18 at `batch`, lowered as MIRA's compiler would; calibrated on two seeded
    2-image batches of a same-weight twin (or the given peaks)."""
    from harness import lowering as LW
    from harness import models
    g = LW.prepare(models.resnet18(batch=batch, seed=seed))
    if peaks is None:
        twin = LW.prepare(models.resnet18(batch=2, seed=seed))
        peaks = LW.calibrate(twin, [{"x": models.image_batch((2, 3, 224, 224), s)} for s in (11, 12)])
    LW.w8a8(g, peaks=peaks)
    return g, peaks


def build_workload(name: str, batch: int):
    """A W8A8 graph of another configuration, calibrated as the parity tests do it (or,
    for mlp50m-int8, the weight-only rewrite, which needs no calibration)."""
    from harness import lowering as LW
    from harness import models
    if name == "mlp50m-int8":
        g = LW.prepare(models.mlp_50m(batch=batch, seed=0))
        LW.weight_only(g)
        return g, models.normal_batch(g.inputs[0].type.shape, 7)
    if name == "mlp50m":
        builder, cb, seeds, gen = models.mlp_50m, 8, (2, 3), models.normal_batch
    elif name in ("mobilenetv2", "mobilenetv2-f16"):
        builder, cb, seeds, gen = models.mobilenet_v2, 2, (11, 12), models.image_batch
    elif name == "resnet18-onnx":
        def builder(batch, seed):
            return models.resnet18(batch=batch, seed=seed, bn_epilogue=True)
        cb, seeds, gen = 2, (11, 12), models.image_batch
    elif name == "resnet18-f16":
        builder, cb, seeds, gen = models.resnet18, 2, (11, 12), models.image_batch
    else:
        raise SystemExit(f"unknown workload {name!r}")
    precision = "f16" if name.endswith("-f16") else None
    g = LW.prepare(builder(batch=batch, seed=0), precision)
    twin = LW.prepare(builder(batch=cb, seed=0), precision)
    shape = twin.inputs[0].type.shape
    LW.w8a8(g, peaks=LW.calibrate(twin, [{"x": gen(shape, s)} for s in seeds]))
    return g, gen(g.inputs[0].type.shape, 7)


def single_segment(g):
    """Compile g on the rocm target; every op must run there (one segment)."""
    from harness.runner import Runner
    from mira_amd.target import RocmTarget
    runner = Runner(g, RocmTarget())
    if runner.devices != ["rocm"]:
        raise SystemExit(f"{g.name}: expected one rocm segment, got {runner.devices}")
    return runner.executables("rocm")[0]


def time_launches(exe, stream, reps: int = 3) -> dict:
    """Per-kind device time of one pass: HIP events around every launch on its stream."""
    import torch
    handle = stream.cuda_stream
    per_kind: dict[str, float] = {}
    for _ in range(reps):
        evs = []
        for name, fn in exe.launches:
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            fn(handle)
            b.record(stream)
            evs.append((name, a, b))
        torch.cuda.synchronize()
        for name, a, b in evs:
            per_kind[name] = per_kind.get(name, 0.0) + a.elapsed_time(b) / reps
    return per_kind


def kernel_breakdown(exe, per_kind: dict) -> dict:
    """Each launch kind against both rooflines: its algorithmic int8 ops in TOP/s against the
    MFMA peak and its algorithmic HBM bytes in GB/s against the HBM peak.  `bound` is the
    peak the kind is priced against: MFMA for the int8 contractions, HBM for everything
    else.  `launch_bounds` counts its launches by the side of the ridge point
    (5.0 POPS / 8 TB/s = 625 ops per byte) each one falls on, and `roofline_frac` is the sum
    over its launches of max(ops / MFMA peak, bytes / HBM peak) over the measured time."""
    ridge = INT8_PEAK_TOPS * 1e12 / (HBM_PEAK_GBS * 1e9)
    out = {}
    for name, ms in sorted(per_kind.items(), key=lambda kv: -kv[1]):
        cost = [(b, o) for k, b, o in exe.launch_cost if k == name]
        nbytes, nops = sum(b for b, _ in cost), sum(o for _, o in cost)
        sec = ms * 1e-3
        row = {"launches": len(cost), "ms": round(ms, 4)}
        if nops:
            row.update(tops=round(nops / sec / 1e12, 1), mfma_frac=round(nops / sec / 1e12 / INT8_PEAK_TOPS, 4))
        if nbytes:
            row.update(gbs=round(nbytes / sec / 1e9, 1), hbm_frac=round(nbytes / sec / 1e9 / HBM_PEAK_GBS, 4))
        if nops or nbytes:
            row["bound"] = "mfma" if nops else "hbm"
            row["launch_bounds"] = {"mfma": sum(1 for b, o in cost if b == 0 or o / b >= ridge),
                                    "hbm": sum(1 for b, o in cost if b and o / b < ridge)}
            roof = sum(max(o / (INT8_PEAK_TOPS * 1e12), b / (HBM_PEAK_GBS * 1e9)) for b, o in cost)
            row["roofline_frac"] = round(roof / sec, 4) if sec else None
        out[name] = row
    return out


def per_launch(args) -> int:
    """One row per launch of a step: its device time (HIP events around it, mean of 5 passes),
    algorithmic ops and bytes, and the fraction of its roofline time it reaches --
    roofline time = max(ops / 5.0 POPS, bytes / 8 TB/s)."""
    import torch
    from harness import models
    if args.workload == "resnet18":
        g, _ = build(args.batch)
        x = models.image_batch((args.batch, 3, 224, 224), 7)
    else:
        g, x = build_workload(args.workload, args.batch)
    exe = single_segment(g)
    exe.upload({g.inputs[0]: x})
    stream = torch.cuda.current_stream()
    handle = stream.cuda_stream
    for _ in range(3):
        exe.launch()
    torch.cuda.synchronize()
    reps = 5
    t = np.zeros(len(exe.launches))
    for _ in range(reps):
        evs = []
        for _name, fn in exe.launches:
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            fn(handle)
            b.record(stream)
            evs.append((a, b))
        torch.cuda.synchronize()
        t += np.array([a.elapsed_time(b) for a, b in evs]) * 1e3 / reps
    print(f"{'#':>3s} {'kind':16s} {'us':>8s} {'GOP':>8s} {'MB':>8s} {'TOP/s':>7s} {'TB/s':>6s} "
          f"{'ops/B':>6s} {'bound':>5s} {'roof us':>8s} {'frac':>6s}")
    for i, ((name, _fn), (_, nb, no)) in enumerate(zip(exe.launches, exe.launch_cost)):
        us = t[i]
        roof_mfma, roof_hbm = no / (INT8_PEAK_TOPS * 1e12) * 1e6, nb / (HBM_PEAK_GBS * 1e9) * 1e6
        roof = max(roof_mfma, roof_hbm)
        bound = "-" if roof == 0 else ("mfma" if roof_mfma >= roof_hbm else "hbm")
        print(f"{i:3d} {name:16s} {us:8.1f} {no / 1e9:8.2f} {nb / 1e6:8.1f} {no / us / 1e6 if us else 0:7.1f} "
              f"{nb / us / 1e6 if us else 0:6.2f} {no / nb if nb else 0:6.0f} {bound:>5s} {roof:8.1f} "
              f"{roof / us if us else 0:6.3f}")
    print(f"total {t.sum():.1f} us of launches; roofline {sum(max(o / 5e15, b / 8e12) for _, b, o in exe.launch_cost) * 1e6:.1f} us")
    return 0


def bench_workload(args) -> int:
    import torch
    g, x = build_workload(args.workload, args.batch)
    exe = single_segment(g)
    exe.upload({g.inputs[0]: x})
    stream = torch.cuda.current_stream()
    for _ in range(args.warmup):
        exe.launch()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(args.steps):
        exe.launch()
    stop.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / args.steps
    per_kind = time_launches(exe, stream)
    log(f"{args.workload} batch {args.batch}: {args.steps} steps, {ms:.4f} ms/step")
    graph_ms = graph_replay_ms(exe, stream, args.steps, args.warmup)
    log(f"{args.workload} batch {args.batch}: {graph_ms:.4f} ms/step replaying the step as one HIP graph")
    print(json.dumps({"workload": args.workload, "batch": args.batch, "steps": args.steps, "warmup": args.warmup,
                      "ms_per_step": round(ms, 4), "ms_per_step_graph": round(graph_ms, 4),
                      "dtype": "f32" if args.workload.endswith("-int8") else "int8",
                      "data": "synthetic",
                      "kernels": kernel_breakdown(exe, per_kind)}), flush=True)
    return 0


def graph_replay_ms(exe, stream, steps: int, warmup: int) -> float:
    """The step's launches recorded once as a HIP graph and replayed `steps` times (what a
    serving loop does at batch 1, where a step is a few launches of a few microseconds and
    the gaps between eager launches cost as much as the kernels).  Every replay recomputes
    the same outputs from the same resident inputs; after the timed replays the outputs
    must equal, bit for bit, those of the eager launches (the executable's kernels record
    no memset nodes)."""
    import torch
    eager = exe.download()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        exe.launch()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        graph.replay()
    stop.record(stream)
    torch.cuda.synchronize()
    replayed = exe.download()
    for k, v in eager.items():
        a, b = np.asarray(v), np.asarray(replayed[k])
        if a.shape != b.shape or a.tobytes() != b.tobytes():
            raise SystemExit(f"graph replay output {k} differs from the eager launches")
    return start.elapsed_time(stop) / steps


def bench_greedy_loop(args) -> int:
    """The greedy KV-cache decoder written in MIRA's language (tests/programs/greedy_lm.mira:
    one attention head, L=2, D=64, F=128, vocab 65, a 16-token prompt and a context of T=272),
    its runtime while loop compiled whole for rocm in approx_f32 mode: token buffer, counter,
    gathers, cache windows, attention and argmax run in device buffers, one flag read back per
    iteration.  Timed: the runner's whole run (prompt upload, the loop's T-1 iterations, the
    token download) with the condition and body steps replayed as HIP graphs, beside the same
    loop launched kernel by kernel, the loop driven from the host with its body split into
    rocm segments, and the host evaluator alone."""
    import torch
    from harness import cli, hosteval, lowering as LW
    from harness.runner import Runner
    from mira_amd.target import RocmTarget
    dims = {"P": 16, "V": 65, "T": 272, "D": 64, "F": 128, "L": 2}
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tests", "programs", "greedy_lm.mira")
    g = LW.prepare(cli.load_graph(path, "main", None, dims, 0, None))
    feed = {"prompt": np.random.default_rng(4).integers(0, dims["V"], dims["P"]).astype(np.int32)}
    iters = dims["T"] - 1

    class HostLoops(RocmTarget):
        def _check_control(self, op):
            return "loops driven from the host"

    def timed(runner, reps: int) -> tuple:
        runner.run(dict(feed))
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            (tok,) = runner.run(dict(feed))
        return (time.perf_counter() - t0) / reps, np.asarray(tok)

    graphs = Runner(g, RocmTarget(approx_f32=True), fallback=hosteval.HostTarget())
    eager = Runner(g, RocmTarget(approx_f32=True, graph_loops=False), fallback=hosteval.HostTarget())
    split = Runner(g, HostLoops(approx_f32=True), fallback=hosteval.HostTarget())
    host = Runner(g, hosteval.HostTarget())
    reps = max(args.steps // 4, 1)
    graph_s, tok = timed(graphs, reps)
    eager_s, tok_eager = timed(eager, reps)
    split_s, tok_split = timed(split, 1)
    host_s, tok_host = timed(host, 1)
    assert np.array_equal(tok, tok_eager) and np.array_equal(tok, tok_split), "rocm loop modes disagree"
    log(f"greedy loop: {1e6 * graph_s / iters:.1f} us/token (graphs), {1e6 * eager_s / iters:.1f} (eager), "
        f"{1e6 * split_s / iters:.1f} (host-driven), {1e6 * host_s / iters:.1f} (host evaluator)")
    print(json.dumps({
        "workload": "greedy-loop", "program": "tests/programs/greedy_lm.mira", "dims": dims,
        "placements": graphs.placements(), "iterations": iters, "seconds": round(graph_s, 6),
        "us_per_token": round(1e6 * graph_s / iters, 2),
        "eager_us_per_token": round(1e6 * eager_s / iters, 2),
        "host_driven_us_per_token": round(1e6 * split_s / iters, 2),
        "host_evaluator_us_per_token": round(1e6 * host_s / iters, 2),
        "tokens_equal_host_evaluator": bool(np.array_equal(tok, tok_host)),
        "mode": "approx_f32", "dtype": "f32", "data": "synthetic",
        "timed": f"wall clock of the runner's whole run, mean of {reps}, after one untimed run"}))
    return 0


def bench_gpt(args) -> int:
    """Greedy decoding with the character-level GPT (L=2, d=64, 4 heads, vocab 65, context
    T=272 = 16 + 256), W8A8 on the QKV/out/MLP/vocab projections: a seeded 16-token prompt per
    sequence, then `--tokens` generated tokens (16 + tokens - 1 decode steps).

    Timed (`us_per_token`): the whole decode resident on the GPU -- the step graph as one rocm
    executable in approx_f32 mode (softmax, the attention matmuls and gelu on the device) and
    the loop state (embedding row, mask, cache writes, argmax) kept in device memory by the
    library's decode-loop kernels (mira_amd.decode.DecodeLoop through harness.decode), each
    step replayed as one HIP graph; HIP events around
    all the steps, no host synchronisation inside.  Beside it: the same loop launched eagerly,
    and the bit-exact default mode driven from the host through the runner (softmax, the f32
    attention and the gelu projection on NumPy, host/device copies included)."""
    import torch
    from harness import lowering as LW
    from harness import models
    from harness.decode import DeviceDecoder
    from harness.hosteval import HostTarget
    from harness.runner import Runner
    from mira_amd.target import RocmTarget
    cfg = models.GPTConfig()
    params = models.gpt_params(cfg, 0)
    twin = LW.prepare(models.gpt_decode_step(cfg, 2, params))
    calib = []
    for s in (2, 3):
        r = np.random.default_rng(s)
        toks = r.integers(0, cfg.V, (2, cfg.T)).astype(np.int32)
        caches = [(r.standard_normal((2, cfg.T, cfg.D)).astype(np.float32),
                   r.standard_normal((2, cfg.T, cfg.D)).astype(np.float32)) for _ in range(cfg.L)]
        calib.append(models.gpt_step_feeds(cfg, params, toks, 16, caches))
    peaks = LW.calibrate(twin, calib)
    g = LW.prepare(models.gpt_decode_step(cfg, args.batch, params))
    LW.w8a8(g, peaks=peaks)
    prompt = np.random.default_rng(4).integers(0, cfg.V, (args.batch, 16)).astype(np.int32)
    new = min(args.tokens, cfg.T - 16)
    steps = 16 + new - 1
    stream = torch.cuda.current_stream()

    # the decode resident on the device: one executable, one graph replay per step
    dev_runner = Runner(g, RocmTarget(approx_f32=True))
    (exe,) = dev_runner.executables("rocm")
    dec = DeviceDecoder(dev_runner, cfg, params, args.batch)
    dec.reset(prompt)
    dec.capture()

    def timed_decode(use_graph: bool) -> tuple:
        dec.reset(prompt)
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        start.record(stream)
        dec.run_steps(steps, use_graph)
        stop.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(stop) * 1e-3, time.perf_counter() - t0, dec.tokens[:, :16 + new].cpu().numpy()

    for _ in range(max(args.warmup, 1)):
        timed_decode(True)
        timed_decode(False)
    graph_s, graph_wall, tok_graph = timed_decode(True)
    eager_s, eager_wall, tok_eager = timed_decode(False)
    assert np.array_equal(tok_graph, tok_eager), "graph and eager device decodes disagree"
    # the whole decode (every step) recorded as one graph: one launch for the loop
    dec.reset(prompt)
    dec.capture(steps)
    for _ in range(max(args.warmup, 1)):
        timed_decode(True)
    whole_s, _, tok_whole = timed_decode(True)
    assert np.array_equal(tok_whole, tok_eager), "the one-graph decode disagrees"
    log(f"gpt decode batch {args.batch} on the device: {new} tokens, {1e6 * graph_s / steps:.1f} us/step "
        f"(graph), {1e6 * eager_s / steps:.1f} us/step (eager launches)")
    kernels = {}
    for kind, row in kernel_breakdown(exe, time_launches(exe, stream)).items():
        kernels[kind] = {"launches": row["launches"], "ms": round(row["ms"], 4)}

    # the bit-exact default mode, driven from the host through the runner
    host_runner = Runner(g, RocmTarget(), fallback=HostTarget())
    models.gpt_decode(host_runner.run, cfg, params, prompt, 4)            # warm-up
    torch.cuda.synchronize()
    host_steps = min(steps, 16 + min(new, 64) - 1)
    t0 = time.perf_counter()
    tok_host, _ = models.gpt_decode(host_runner.run, cfg, params, prompt, host_steps - 15)
    host_s = time.perf_counter() - t0
    log(f"gpt decode batch {args.batch}, exact mode through the host: {1e6 * host_s / host_steps:.0f} us/step")

    print(json.dumps({
        "workload": "gpt-decode", "batch": args.batch, "prompt_tokens": 16, "generated_tokens": new,
        "decode_steps": steps, "seconds": round(graph_s, 6),
        "us_per_step": round(1e6 * graph_s / steps, 2),
        "us_per_token": round(1e6 * graph_s / (new * args.batch), 4),
        "tokens_per_s": round(new * args.batch / graph_s, 1),
        "mode": "approx_f32 (the attention and gelu on the device; W8A8 projections and layernorm bit-exact)",
        "eager_us_per_step": round(1e6 * eager_s / steps, 2),
        "one_graph_us_per_step": round(1e6 * whole_s / steps, 2),
        "graph_wall_us_per_step": round(1e6 * graph_wall / steps, 2),
        "exact_mode_host_loop_us_per_step": round(1e6 * host_s / host_steps, 1),
        "exact_mode_host_loop_steps": host_steps,
        "exact_mode_segments": host_runner.devices,
        "launches_per_step": len(exe.launches) + 2,          # the step, and the loop's embed and commit kernels
        "step_launches": len(exe.launches),
        "device_constant_bytes": exe.const_bytes,
        "dtype": "int8", "data": "synthetic",
        "timed": "HIP events around every decode step of the prompt and the generated tokens, the step "
                 "graph replayed once per step with the loop state on the device; inputs resident",
        "kernels": kernels}), flush=True)
    return 0


def _host_description() -> dict:
    """CPU model, logical CPUs, physical cores, the CPUs this process may run on, NumPy
    version and the BLAS library the baseline runs on."""
    model = "unknown"
    cores: set = set()
    phys = core = None
    try:
        for line in open("/proc/cpuinfo"):
            key, _, val = line.partition(":")
            key, val = key.strip(), val.strip()
            if key == "model name" and model == "unknown":
                model = val
            elif key == "physical id":
                phys = val
            elif key == "core id":
                core = val
            elif not key and core is not None:      # blank line: end of one logical CPU
                cores.add((phys, core))
                phys = core = None
        if core is not None:
            cores.add((phys, core))
    except OSError:
        pass
    try:
        allowed = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        allowed = None
    blas = []
    try:
        from threadpoolctl import threadpool_info
        blas = [{k: p.get(k) for k in ("internal_api", "version", "num_threads", "architecture")}
                for p in threadpool_info()]
    except Exception:
        pass
    return {"cpu_model": model, "logical_cpus": os.cpu_count(), "physical_cores": len(cores) or None,
            "cpus_allowed": allowed, "numpy": np.__version__, "blas": blas}


def cpu_baseline(peaks, macs_per_image: int, runs: int = 5) -> dict:
    """The golden model on a bounded 2-image sample of the same network and attrs: 1 warm-up,
    then the median of `runs` timed runs."""
    from oracle import golden as G
    from harness import models
    g, _ = build(2, peaks=peaks)
    x = models.image_batch((2, 3, 224, 224), 7)
    G.run_graph(g, {"x": x})
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        G.run_graph(g, {"x": x})
        times.append(time.perf_counter() - t0)
    t = float(np.median(times))
    host = _host_description()
    threads = max([b.get("num_threads") or 1 for b in host["blas"]] or [1])
    return {"value": round(2 * macs_per_image * 2 / t / 1e12, 6), "unit": "TOPS", "cores": int(threads),
            "kind": "port", "ms_per_image": round(t / 2 * 1e3, 2), "runs_s": [round(v, 3) for v in times],
            "host": host,
            "sample": f"2 images of the same W8A8 ResNet-18 (same attrs), NumPy golden model "
                      f"(int64 matmul, per-tap f32 einsum convs through BLAS with {threads} threads), "
                      f"median of {runs} after 1 warm-up"}


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "qconv2d_resnet18_b256_traffic.txt")


def measured_traffic(batch: int):
    """HBM bytes per qconv2d launch (FETCH_SIZE + WRITE_SIZE, copy-calibrated) from the
    committed counter summary of this workload, or None if there is none for this batch."""
    if batch != 256 or not os.path.exists(TRAFFIC_FILE):
        return None
    for line in open(TRAFFIC_FILE):
        if line.startswith("qconv2d_hbm_bytes_per_launch:"):
            return int(float(line.split(":")[1]))
    return None


def copy_calibration() -> int:
    """A plain 1 GiB device-to-device copy, 3 times: FETCH_SIZE / WRITE_SIZE read for it
    give the factor from counter units to bytes."""
    import torch
    n = 1 << 28
    x = torch.ones(n, device="cuda")
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    log(f"copied {4 * n} bytes x3")
    return 0


def blas_reference() -> int:
    """The vendor int8 GEMM (torch._int_mm, hipBLASLt) on the GEMM shapes of ResNet-18's 3x3
    convolutions at batch 256 (M = output pixels, K = 9 x input channels, N = output channels),
    already in im2col form, and on 8192^3: the reference the implicit-GEMM conv kernels are
    compared with.  HIP events around 20 calls after 3 warm-up calls."""
    import torch
    torch.manual_seed(0)
    shapes = [("layer1 3x3", 802816, 576, 64), ("layer2 3x3", 200704, 1152, 128),
              ("layer3 3x3", 50176, 2304, 256), ("layer4 3x3", 12544, 4608, 512), ("8192^3", 8192, 8192, 8192)]
    for name, M, K, N in shapes:
        a = torch.randint(-127, 127, (M, K), dtype=torch.int8, device="cuda")
        b = torch.randint(-127, 127, (N, K), dtype=torch.int8, device="cuda").t()
        for _ in range(3):
            torch._int_mm(a, b)
        st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        st.record()
        for _ in range(20):
            torch._int_mm(a, b)
        en.record()
        torch.cuda.synchronize()
        us = st.elapsed_time(en) * 1000 / 20
        log(f"{name:12s} M={M} K={K} N={N}: {us:8.1f} us {2 * M * N * K / us / 1e6:8.1f} TOP/s")
        del a, b
    return 0


def summarize_counters(d: str) -> int:
    """Summarize rocprofv3 --pmc CSV output of bench.py and of --copy-calibration.

    d/fetch, d/write: `rocprofv3 --pmc FETCH_SIZE|WRITE_SIZE --output-format csv -- python3 bench.py ...`
    d/cfetch, d/cwrite: the same counters over `python3 bench.py --copy-calibration`.
    Counters are KiB per dispatch; each is scaled by (bytes copied) / (what it reads for the copy)."""
    import csv
    import collections

    def rows(sub):
        p = os.path.join(d, sub, "run_counter_collection.csv")
        return list(csv.DictReader(open(p)))

    copy_kib = (4 << 28) / 1024
    ff = copy_kib / float(rows("cfetch")[-1]["Counter_Value"])
    wf = copy_kib / float(rows("cwrite")[-1]["Counter_Value"])
    per = collections.defaultdict(lambda: [0, 0.0, 0.0])
    for sub, fac, slot in (("fetch", ff, 1), ("write", wf, 2)):
        for r in rows(sub):
            k = r["Kernel_Name"]
            per[k][slot] += float(r["Counter_Value"]) * 1024 * fac
            if slot == 1:
                per[k][0] += 1
    print(f"copy calibration: FETCH_SIZE x{ff:.4f}, WRITE_SIZE x{wf:.4f} (1 GiB copy)")
    print(f"{'kernel':72s} {'launches':>8s} {'fetch MB/launch':>16s} {'write MB/launch':>16s}")
    conv_n, conv_b = 0, 0.0
    for k, (n, f, w) in sorted(per.items(), key=lambda kv: -(kv[1][1] + kv[1][2])):
        if "rocclr" in k or n == 0:
            continue
        print(f"{k[:72]:72s} {n:8d} {f / n / 1e6:16.2f} {w / n / 1e6:16.2f}")
        targs = k[k.find("<") + 1:k.find(">")].split(",") if "qgemm_kernel<" in k else []
        if len(targs) >= 6 and int(targs[5]) != 0:          # A operand mode 0 = dense matmul

            conv_n += n
            conv_b += f + w
    if conv_n:
        print(f"qconv2d_hbm_bytes_per_launch: {conv_b / conv_n:.0f}")
    return 0


def summarize_mfma(d: str) -> int:
    """MFMA utilisation per kernel from `rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE
    --output-format csv -d d/mfma -o run -- python3 bench.py ...`.

    SQ_VALU_MFMA_BUSY_CYCLES sums the cycles each of the 1024 SIMDs (256 CUs x 4) spent on
    MFMA work; GRBM_GUI_ACTIVE sums the busy cycles of the 8 XCDs.  Utilisation =
    (MFMA busy cycles per SIMD) / (kernel cycles) = MFMA_BUSY / (GUI_ACTIVE * 1024 / 8)."""
    import csv
    import collections
    rows = list(csv.DictReader(open(os.path.join(d, "mfma", "run_counter_collection.csv"))))
    per = collections.defaultdict(lambda: collections.defaultdict(float))
    disp = collections.defaultdict(set)
    for r in rows:
        k = r["Kernel_Name"]
        per[k][r["Counter_Name"]] += float(r["Counter_Value"])
        disp[k].add(r["Dispatch_Id"])
    print(f"{'kernel':72s} {'launches':>8s} {'MFMA busy':>10s}")
    conv_busy = conv_active = 0.0
    for k, c in sorted(per.items(), key=lambda kv: -kv[1].get("GRBM_GUI_ACTIVE", 0.0)):
        act = c.get("GRBM_GUI_ACTIVE", 0.0)
        if "rocclr" in k or act <= 0:
            continue
        util = c.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / (act * 1024 / 8)
        print(f"{k[:72]:72s} {len(disp[k]):8d} {100 * util:9.2f}%")
        targs = k[k.find("<") + 1:k.find(">")].split(",") if "qgemm_kernel<" in k else []
        if len(targs) >= 6 and int(targs[5]) != 0:
            conv_busy += c.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0)
            conv_active += act
    if conv_active:
        print(f"qconv2d_mfma_busy_fraction: {conv_busy / (conv_active * 1024 / 8):.4f}")
    return 0


SQ_PASS1 = ("SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_WAIT_INST_LDS SQ_WAIT_ANY SQ_ACTIVE_INST_LDS SQ_INSTS_LDS "
            "SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE")
SQ_PASS2 = ("SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU SQ_INSTS_SALU SQ_INSTS_MFMA SQ_WAIT_INST_ANY "
            "SQ_ACTIVE_INST_VALU SQ_LDS_DATA_FIFO_FULL SQ_INSTS_VMEM GRBM_GUI_ACTIVE")


def summarize_sq(d: str) -> int:
    """Per-kernel issue and wait counters from two rocprofv3 --pmc passes over the same command:
    d/sq1 = SQ_PASS1, d/sq2 = SQ_PASS2 (`--output-format csv -d d/sqN -o run`).

    mfma_busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE * 1024 / 8) (the 1024 SIMDs' MFMA-busy
    cycles over the 8 XCDs' active cycles); valu/salu/lds/vmem per mfma = instruction counts per
    MFMA instruction; wait_any, wait_lds, lds_active = fractions of SQ_WAVE_CYCLES (summed over
    resident waves); bank_conflict = SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE."""
    import csv
    import collections
    per = collections.defaultdict(lambda: collections.defaultdict(float))
    launches = collections.defaultdict(set)
    for sub in ("sq1", "sq2"):
        for r in csv.DictReader(open(os.path.join(d, sub, "run_counter_collection.csv"))):
            k = r["Kernel_Name"]
            per[k][r["Counter_Name"]] += float(r["Counter_Value"])
            launches[k].add((sub, r["Dispatch_Id"]))
    print(f"{'kernel':60s} {'n':>3s} {'mfma_busy':>9s} {'valu/mf':>7s} {'salu/mf':>7s} {'lds/mf':>6s} "
          f"{'vmem/mf':>7s} {'wait_any':>8s} {'wait_lds':>8s} {'lds_act':>7s} {'bankconf':>8s}")
    rows = sorted(per.items(), key=lambda kv: -kv[1].get("GRBM_GUI_ACTIVE", 0.0))
    for k, c in rows:
        if "rocclr" in k or c.get("GRBM_GUI_ACTIVE", 0) <= 0:
            continue
        n = len([x for x in launches[k] if x[0] == "sq2"])
        mf = c.get("SQ_INSTS_MFMA", 0.0)
        wc = c.get("SQ_WAVE_CYCLES", 0.0) or 1.0
        busy = c.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / (c["GRBM_GUI_ACTIVE"] * 1024 / 8)

        def per_mf(key):
            return f"{c.get(key, 0.0) / mf:7.2f}" if mf else "      -"
        name = k.replace("void ", "").replace("mr::", "")[:60]
        print(f"{name:60s} {n:3d} {busy:9.3f} {per_mf('SQ_INSTS_VALU')} {per_mf('SQ_INSTS_SALU')} "
              f"{per_mf('SQ_INSTS_LDS')[1:]} {per_mf('SQ_INSTS_VMEM')} {c.get('SQ_WAIT_ANY', 0) / wc:8.3f} "
              f"{c.get('SQ_WAIT_INST_LDS', 0) / wc:8.3f} {c.get('SQ_ACTIVE_INST_LDS', 0) / wc:7.3f} "
              f"{c.get('SQ_LDS_BANK_CONFLICT', 0) / max(1.0, c.get('SQ_LDS_IDX_ACTIVE', 0)):8.3f}")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=None,
                    help="default 256 (resnet18), 1 (mlp50m, mlp50m-int8), 128 (mobilenetv2)")
    ap.add_argument("--workload", default="resnet18",
                    choices=["resnet18", "resnet18-onnx", "resnet18-f16", "mlp50m", "mlp50m-int8", "mobilenetv2",
                             "mobilenetv2-f16",
                             "gpt-decode", "greedy-loop"])
    ap.add_argument("--tokens", type=int, default=256, help="gpt-decode: tokens generated per sequence")
    ap.add_argument("--per-launch", action="store_true", help="per-launch time against each launch's roofline")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true", help="run the plain copy used to scale counters")
    ap.add_argument("--blas-reference", action="store_true",
                    help="time hipBLASLt's int8 GEMM (torch._int_mm) on ResNet-18's conv GEMM shapes")
    ap.add_argument("--summarize-counters", metavar="DIR", help="summarize rocprofv3 --pmc CSV output in DIR")
    ap.add_argument("--summarize-mfma", metavar="DIR", help="MFMA utilisation from rocprofv3 --pmc CSV output in DIR/mfma")
    ap.add_argument("--summarize-sq", metavar="DIR", help="issue/wait/LDS counters from rocprofv3 --pmc output in "
                                                         "DIR/sq1 and DIR/sq2 (see SQ_PASS1, SQ_PASS2)")
    args = ap.parse_args()
    if args.summarize_counters:
        return summarize_counters(args.summarize_counters)
    if args.summarize_mfma:
        return summarize_mfma(args.summarize_mfma)
    if args.summarize_sq:
        return summarize_sq(args.summarize_sq)
    if args.blas_reference:
        return blas_reference()
    if args.copy_calibration:
        return copy_calibration()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the rocm target has no multi-GPU path (the batch would shard "
              "by data parallelism, one share per GPU). Run with --gpus 1.", file=sys.stderr)
        return 2
    if args.batch is None:
        args.batch = {"resnet18": 256, "resnet18-onnx": 256, "resnet18-f16": 256, "mlp50m": 1, "mlp50m-int8": 1,
                      "mobilenetv2": 128, "mobilenetv2-f16": 128, "gpt-decode": 1,
                      "greedy-loop": 1}[args.workload]
    if args.workload == "gpt-decode":
        return bench_gpt(args)
    if args.workload == "greedy-loop":
        return bench_greedy_loop(args)
    if args.per_launch:
        return per_launch(args)
    if args.workload != "resnet18":
        return bench_workload(args)

    import torch
    from harness import models

    t0 = time.perf_counter()
    g, peaks = build(args.batch)
    macs = models.conv_macs(g)
    exe = single_segment(g)
    log(f"compiled in {time.perf_counter() - t0:.1f}s: {exe.report()}")
    x = models.image_batch((args.batch, 3, 224, 224), 7)
    exe.upload({g.inputs[0]: x})
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream()
    for _ in range(args.warmup):
        exe.launch()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(args.steps):
        exe.launch()
    stop.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / args.steps
    log(f"{args.steps} steps: {ms:.3f} ms/step")

    # per-launch durations (events around every launch, same stream), 3 instrumented passes
    per_kind = time_launches(exe, stream)
    conv_ms = per_kind.get("qconv2d", 0.0)
    n_conv = exe.kernel_counts.get("qconv2d", 0)
    conv_cost = [(b, o) for name, b, o in exe.launch_cost if name == "qconv2d"]
    conv_tops = sum(o for _, o in conv_cost) / (conv_ms * 1e-3) / 1e12
    conv_alg_bytes = sum(b for b, _ in conv_cost) / max(1, len(conv_cost))
    log("per-kind ms/step: " + ", ".join(f"{k} {v:.3f}" for k, v in sorted(per_kind.items(), key=lambda kv: -kv[1])))

    # PCIe-inclusive: host f32 input in, host logits out (Executable.run), 3 runs, median
    feeds = {g.inputs[0]: x}
    io_ms = []
    for _ in range(3):
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        exe.run(feeds)
        io_ms.append(1e3 * (time.perf_counter() - t1))
    io_ms = float(np.median(io_ms))
    log(f"run() with host input/output copies: {io_ms:.3f} ms")

    tops = 2 * macs / (ms * 1e-3) / 1e12
    out = {
        "metric": "int8 TOPS (% of MFMA peak) + ms/inference, W8A8 ResNet-18 shape, 1 MI355X",
        "value": round(tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "ms_per_inference": round(ms / args.batch, 5),
        "ms_per_step_host_io": round(io_ms, 3),
        "pct_of_int8_peak": round(100 * tops / INT8_PEAK_TOPS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "resnet18_w8a8", "batch": args.batch, "input": f"f32[{args.batch},3,224,224] U(0,1)",
                   "weights": "random Kaiming-normal, BN folded", "int8_macs_per_image": macs // args.batch,
                   "calibration": "2 batches of 2 images U(0,1)"},
        "roofline": {"bound": "mfma", "kernel": "qconv2d implicit GEMM (19 convs; the stem conv runs fused with its max pool)",
                     "achieved": round(conv_tops, 2), "peak": INT8_PEAK_TOPS, "unit": "TOP/s",
                     "frac": round(conv_tops / INT8_PEAK_TOPS, 4), "traffic": measured_traffic(args.batch),
                     "traffic_source": "HBM bytes per qconv2d launch from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE "
                                       "(copy-calibrated) of this workload, committed in "
                                       "profiles/qconv2d_resnet18_b256_traffic.txt; not measured in this run",
                     "algorithmic_bytes_per_launch": int(conv_alg_bytes),
                     "launches_per_step": n_conv, "ms_per_step": round(conv_ms, 4),
                     "us_per_launch": round(1e3 * conv_ms / max(1, n_conv), 2),
                     "hbm_frac": round(conv_alg_bytes * n_conv / (conv_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "ops_per_byte": round(sum(o for _, o in conv_cost) / max(1, sum(b for b, _ in conv_cost)), 1)},
        "kernels": kernel_breakdown(exe, per_kind),
    }
    if not args.no_cpu_baseline:
        log("timing the CPU golden model on a 2-image sample ...")
        out["cpu_baseline"] = cpu_baseline(peaks, macs // args.batch)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
