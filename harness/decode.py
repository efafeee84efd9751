"""The GPT decode step's greedy loop on the device, for the tests and the benchmark.

`models.gpt_decode` drives one decode step per token through host arrays (feeds in, outputs
out, argmax on the host), as the reference's `generate` loop does (examples/gpt_text.mira).
DeviceDecoder runs the same loop with nothing on the host: it binds the library's
mira_amd.decode.DecodeLoop to the step graph of `models.gpt_decode_step` (its input and output
names) and to the model's embedding and position tables.  With RocmTarget(approx_f32=True)
every op of the step runs on the device, so a step is the loop's two state kernels around the
step executable's launches, and capture() records it as one HIP graph.  Tokens and logits are
the same as `models.gpt_decode` with the same executable.
"""
from __future__ import annotations

import numpy as np

from mira_amd.decode import DecodeLoop


class DeviceDecoder(DecodeLoop):
    def __init__(self, runner, cfg, params: dict, batch: int):
        """runner: a Runner of the step graph whose only segment is a rocm executable."""
        if runner.devices != ["rocm"]:
            raise ValueError(f"the decode step must be one rocm segment, not {runner.devices}")
        (exe,) = runner.executables("rocm")
        byname = {v.name: v for v in exe.g.inputs}
        if set(byname) != {"h", "mask"} | {f"{k}c{l}" for l in range(cfg.L) for k in "kv"}:
            raise ValueError("the executable must hold the whole decode step (inputs h, mask and every cache)")
        outs = runner.graph.outputs                 # logits, then k, v of every layer
        super().__init__(exe, byname["h"], byname["mask"],
                         [(byname[f"kc{l}"], byname[f"vc{l}"]) for l in range(cfg.L)],
                         outs[0], [(outs[1 + 2 * l], outs[2 + 2 * l]) for l in range(cfg.L)],
                         params["emb"], params["pos"])
        self.cfg = cfg
        assert self.B == batch and self.T == cfg.T

    def decode(self, prompt: np.ndarray, new_tokens: int, use_graph: bool = False) -> np.ndarray:
        return super().decode(prompt, new_tokens, use_graph).astype(np.int32)
