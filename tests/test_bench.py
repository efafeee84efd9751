"""bench.py's host-side logic on the CPU: the one-GPU guard and the per-kind
roofline classification (no kernel runs)."""
import os
import subprocess
import sys
from types import SimpleNamespace

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_exits_with_a_message():
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert p.returncode == 2
    assert "one GPU" in p.stderr and p.stdout == ""


def test_kernel_breakdown_rooflines():
    # a contraction above the ridge (625 ops/byte), one below it, and a pure copy
    exe = SimpleNamespace(launch_cost=[("qconv2d", 10_000_000, 10_000_000_000),    # 1000 ops/B
                                       ("qconv2d", 10_000_000, 10_000_000_000),
                                       ("qmatmul", 4_000_000, 400_000_000),        # 100 ops/B
                                       ("input", 8_000_000, 0)])
    out = bench.kernel_breakdown(exe, {"qconv2d": 1.0, "qmatmul": 0.01, "input": 0.002})
    conv = out["qconv2d"]
    assert conv["launches"] == 2 and conv["bound"] == "mfma"
    assert abs(conv["tops"] - 20.0) < 1e-9                     # 2e10 ops in 1 ms
    assert abs(conv["mfma_frac"] - 20.0 / bench.INT8_PEAK_TOPS) < 1e-6
    assert abs(conv["gbs"] - 20.0) < 1e-9 and abs(conv["hbm_frac"] - 20.0 / bench.HBM_PEAK_GBS) < 1e-6
    assert conv["launch_bounds"] == {"mfma": 2, "hbm": 0}
    # priced against MFMA (a contraction) even though this launch sits below the ridge
    mm = out["qmatmul"]
    assert mm["bound"] == "mfma" and mm["launch_bounds"] == {"mfma": 0, "hbm": 1}
    assert abs(mm["roofline_frac"] - (4e6 / (bench.HBM_PEAK_GBS * 1e9)) / 1e-5) < 1e-9
    inp = out["input"]
    assert inp["bound"] == "hbm" and "tops" not in inp and abs(inp["gbs"] - 4000.0) < 1e-6
    # kinds come out slowest first
    assert list(out) == ["qconv2d", "qmatmul", "input"]
