"""Greedy decoding with the decode step and the loop state resident on the GPU.

`models.gpt_decode` drives one decode step per token through host arrays (feeds in,
outputs out, argmax on the host), as the reference's `generate` loop does
(examples/gpt_text.mira).  DeviceDecoder runs the same loop with nothing on the
host: the step is one rocm executable (RocmTarget(approx_f32=True) places every op
of `models.gpt_decode_step` on the device); the embedding row, position row and
mask row, the key/value cache writes and the argmax are device tensor operations
on the same stream, indexed by a device step counter.  A step therefore issues no
host synchronisation, and `capture()` records it once as a HIP graph that each
later step replays with one launch.  Tokens and logits are the same as
`models.gpt_decode` with the same executable.
"""
from __future__ import annotations

import numpy as np


class DeviceDecoder:
    def __init__(self, runner, cfg, params: dict, batch: int):
        """runner: a Runner of the step graph whose only segment is a rocm executable."""
        import torch
        self.torch = torch
        if runner.devices != ["rocm"]:
            raise ValueError(f"the decode step must be one rocm segment, not {runner.devices}")
        (exe,) = runner.executables("rocm")
        self.exe, self.cfg, self.B = exe, cfg, batch
        byname = {v.name: v for v in exe.g.inputs}
        if set(byname) != {"h", "mask"} | {f"{k}c{l}" for l in range(cfg.L) for k in "kv"}:
            raise ValueError("the executable must hold the whole decode step (inputs h, mask and every cache)")
        dev = exe.dev
        self.h = exe.device_input(byname["h"])
        self.mask = exe.device_input(byname["mask"])
        self.kc = [exe.device_input(byname[f"kc{l}"]) for l in range(cfg.L)]
        self.vc = [exe.device_input(byname[f"vc{l}"]) for l in range(cfg.L)]
        outs = runner.graph.outputs                 # logits, then k, v of every layer
        self.logits = exe.device_output(outs[0])
        self.k = [exe.device_output(outs[1 + 2 * l]).reshape(batch, 1, cfg.D) for l in range(cfg.L)]
        self.v = [exe.device_output(outs[2 + 2 * l]).reshape(batch, 1, cfg.D) for l in range(cfg.L)]
        f32 = torch.float32
        self.emb = torch.from_numpy(np.ascontiguousarray(params["emb"], np.float32)).to(dev)
        self.pos = torch.from_numpy(np.ascontiguousarray(params["pos"], np.float32)).to(dev)
        T = cfg.T
        masks = np.full((T, T + 1), -10000.0, np.float32)      # row t: the mask of step t
        for t in range(T):
            masks[t, :t] = 0.0
        masks[:, T] = 0.0
        self.masks = torch.from_numpy(masks).to(dev)
        self.tokens = torch.zeros((batch, T), dtype=torch.int64, device=dev)
        self.t = torch.zeros(1, dtype=torch.int64, device=dev)
        self.prompt_len = torch.zeros(1, dtype=torch.int64, device=dev)
        self.steps_done = 0           # host copy of t: a step at t reads token t + 1, so t + 1 < T
        self.graph = None
        assert self.h.dtype == f32 and self.mask.numel() == T + 1

    def reset(self, prompt: np.ndarray) -> None:
        """Load the prompt, clear the caches and rewind the step counter."""
        B, P = prompt.shape
        assert B == self.B and P <= self.cfg.T
        self.tokens.zero_()
        self.tokens[:, :P] = self.torch.from_numpy(prompt.astype(np.int64)).to(self.tokens.device)
        for c in self.kc + self.vc:
            c.zero_()
        self.t.zero_()
        self.steps_done = 0
        self.prompt_len.fill_(P)

    def _advance(self) -> None:
        """Account for one step on the host before queueing it: every index a step at t uses
        (token t + 1, position t, mask row t, cache row t) must stay inside its buffer."""
        if self.steps_done + 1 >= self.cfg.T:
            raise RuntimeError(f"step {self.steps_done} would read token {self.steps_done + 1} of a "
                               f"{self.cfg.T}-token context")
        self.steps_done += 1

    def step(self) -> None:
        """One decode step at position t (models.gpt_step_feeds, the step graph, then the cache
        writes and the argmax of models.gpt_decode), all queued on the current stream."""
        self._advance()
        self._step_ops()

    def _step_ops(self) -> None:
        torch, B, t = self.torch, self.B, self.t
        tok = self.tokens.gather(1, t.expand(B, 1)).reshape(B)
        torch.add(self.emb.index_select(0, tok), self.pos.index_select(0, t), out=self.h)
        self.mask.view(1, -1).copy_(self.masks.index_select(0, t))
        self.exe.launch()
        for l in range(self.cfg.L):
            self.kc[l].index_copy_(1, t, self.k[l])
            self.vc[l].index_copy_(1, t, self.v[l])
        nxt = self.tokens.gather(1, (t + 1).expand(B, 1))
        best = torch.argmax(self.logits, dim=1, keepdim=True)
        self.tokens.scatter_(1, (t + 1).expand(B, 1), torch.where(t + 1 >= self.prompt_len, best, nxt))
        t.add_(1)

    def capture(self) -> None:
        """Record one step as a HIP graph (the loop state is rewound afterwards by reset())."""
        torch = self.torch
        self.t.zero_()                         # the warm-up step runs at position 0
        self.steps_done = 0
        side = torch.cuda.Stream(device=self.exe.dev)
        side.wait_stream(torch.cuda.current_stream(self.exe.dev))
        with torch.cuda.stream(side):
            self.step()                        # warm-up outside the capture (allocator, kernels)
        torch.cuda.current_stream(self.exe.dev).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._step_ops()                   # recorded, not run
        torch.cuda.synchronize(self.exe.dev)
        self.t.zero_()
        self.steps_done = 0

    def decode(self, prompt: np.ndarray, new_tokens: int, use_graph: bool = False) -> np.ndarray:
        """Greedy decode as models.gpt_decode does it; returns tokens [B, P + new_tokens].  The
        steps are queued without a host synchronisation; the tokens are read back at the end."""
        P = prompt.shape[1]
        total = P + new_tokens
        assert total <= self.cfg.T, "the step counter must stay inside the cache"
        self.reset(prompt)
        self.run_steps(total - 1, use_graph)
        return self.tokens[:, :total].cpu().numpy().astype(np.int32)

    def run_steps(self, n: int, use_graph: bool = False) -> None:
        if use_graph and self.graph is None:
            raise RuntimeError("capture() first")
        for _ in range(n):
            if use_graph:
                self._advance()
                self.graph.replay()
            else:
                self.step()
