"""Greedy decoding with the loop on the device: the rocm counterpart of the host-driven `while`
loop of a decode program (examples/gpt_text.mira:66-81, run by mira/backends/cpu.py:44-51).

A decode step is one compiled rocm executable of the loop body (inputs: the current token's
embedding row h, the attention mask and the key/value caches; outputs: the logits and each
layer's new key and value rows).  The loop state stays on the device and is updated by two
library kernels around the executable's launches, all on one stream:

    mr_decode_embed    h = emb[token t] + pos[t], the step's mask row, latch t
    <the step's kernels>
    mr_decode_commit   key/value rows -> cache row t, argmax -> token t + 1, t += 1

so a step needs no host synchronisation, and capture() records it as one HIP graph that each
later step replays with a single launch.  Nothing here computes with torch: torch only holds
the device buffers (tokens, counters, tables) and records the graph.
"""
from __future__ import annotations

import ctypes as C
from typing import Sequence

import numpy as np

from . import _lib as L


def _t():
    import torch
    return torch


class DecodeLoop:
    """Greedy decode over one step executable (mira_amd.target.RocmExecutable).

    exe        the compiled step (its inputs and outputs are the values named below)
    h, mask    step inputs: [B, D] input row, [..., T + 1] mask (0 for cache rows already written
               and for the step's own row, `neg` for the others)
    caches     [(key cache, value cache)] step inputs per layer, [B, T, D] each
    logits     step output [B, V]
    rows       [(new key row, new value row)] step outputs per layer, [B, D] each
    emb, pos   host arrays [V, D] and [T, D]: token and position tables
    """

    def __init__(self, exe, h, mask, caches: Sequence, logits, rows: Sequence, emb: np.ndarray, pos: np.ndarray,
                 neg: float = -10000.0):
        torch = _t()
        self.exe, self.lib = exe, exe.lib
        dev = exe.dev
        self.h = exe.device_input(h)
        self.mask = exe.device_input(mask)
        self.caches = [exe.device_input(c) for pair in caches for c in pair]
        self.logits = exe.device_output(logits)
        self.rows = [exe.device_output(r) for pair in rows for r in pair]
        self.B, self.D = self.h.shape
        self.V = int(emb.shape[0])
        self.T = int(pos.shape[0])
        if self.logits.shape != (self.B, self.V) or self.logits.stride(1) != 1:
            raise ValueError(f"logits {tuple(self.logits.shape)} are not [B, V] rows")
        if self.mask.numel() != self.T + 1 or not self.mask.is_contiguous() or not self.h.is_contiguous():
            raise ValueError("the mask must hold T + 1 values and h must be C order")
        if len(self.caches) != len(self.rows) or len(self.caches) > L.DECODE_MAX_CACHES:
            raise ValueError(f"{len(self.caches)} caches for {len(self.rows)} rows (at most {L.DECODE_MAX_CACHES})")
        for c, r in zip(self.caches, self.rows):
            if c.shape != (self.B, self.T, self.D) or c.stride() != self.caches[0].stride() or c.stride(2) != 1:
                raise ValueError("caches must be [B, T, D] with one layout")
            if r.shape != (self.B, self.D) or r.stride(1) != 1:
                raise ValueError("new key/value rows must be [B, D] rows")
        self.emb = torch.from_numpy(np.ascontiguousarray(emb, np.float32)).to(dev)
        self.pos = torch.from_numpy(np.ascontiguousarray(pos, np.float32)).to(dev)
        self.tokens = torch.zeros((self.B, self.T), dtype=torch.int32, device=dev)
        self.state = torch.zeros(2, dtype=torch.int32, device=dev)     # [t, t latched by the step's start]
        self.neg = float(neg)
        n = len(self.caches)
        self._rows = (C.c_void_p * max(n, 1))(*[r.data_ptr() for r in self.rows])
        self._ld_rows = (C.c_int64 * max(n, 1))(*[r.stride(0) for r in self.rows])
        self._caches = (C.c_void_p * max(n, 1))(*[c.data_ptr() for c in self.caches])
        self.prompt_len = 0
        self.steps_done = 0       # host copy of t: a step at t writes token t + 1, so t + 1 < T
        self.graph = None
        self.graph_steps = 0
        self._graph_prompt_len = None

    @property
    def t(self):
        """The device step counter (a view of the loop state)."""
        return self.state[0:1]

    def reset(self, prompt: np.ndarray) -> None:
        """Load the prompt [B, P] (token ids in [0, V)), clear the caches, rewind the counter."""
        torch = _t()
        prompt = np.asarray(prompt)
        B, P = prompt.shape
        if B != self.B or not 1 <= P <= self.T:
            raise ValueError(f"prompt {prompt.shape} for batch {self.B} and context {self.T}")
        if prompt.min() < 0 or prompt.max() >= self.V:
            raise ValueError(f"prompt token ids must lie in [0, {self.V})")
        self.tokens.zero_()
        self.tokens[:, :P] = torch.from_numpy(prompt.astype(np.int32)).to(self.tokens.device)
        for c in self.caches:
            c.zero_()
        self.state.zero_()
        self.steps_done = 0
        self.prompt_len = P

    def _advance(self) -> None:
        """Account for one step on the host before queueing it: the step at t reads position t
        and token t and writes token t + 1, which must stay inside the context."""
        if self.steps_done + 1 >= self.T:
            raise RuntimeError(f"step {self.steps_done} would write token {self.steps_done + 1} of a "
                               f"{self.T}-token context")
        self.steps_done += 1

    def _queue(self, stream: int) -> None:
        lib, st = self.lib, self.state.data_ptr()
        L.check(lib.mr_decode_embed(self.tokens.data_ptr(), self.T, st, st + 4, self.emb.data_ptr(), self.V,
                                    self.pos.data_ptr(), self.T, self.D, self.h.data_ptr(), self.B,
                                    self.mask.data_ptr(), self.neg, stream), "mr_decode_embed")
        self.exe.launch()
        c0 = self.caches[0] if self.caches else None
        L.check(lib.mr_decode_commit(self.logits.data_ptr(), self.logits.stride(0), self.V, len(self.caches),
                                     self._rows, self._ld_rows, self._caches,
                                     c0.stride(1) if c0 is not None else self.D,
                                     c0.stride(0) if c0 is not None else self.T * self.D, self.D,
                                     self.tokens.data_ptr(), self.T, st, st + 4, self.prompt_len, self.T, self.B,
                                     stream), "mr_decode_commit")

    def _stream(self) -> int:
        dev = self.exe.dev
        return _t().cuda.current_stream(dev).cuda_stream if getattr(dev, "type", "cuda") == "cuda" else 0

    def step(self) -> None:
        """One decode step, queued on the current stream."""
        self._advance()
        self._queue(self._stream())

    def capture(self, steps: int = 1) -> None:
        """Record `steps` consecutive decode steps as one HIP graph for the current prompt length
        (every step reads its position from the device counter, so the same launches repeat).
        With steps = prompt length + new tokens - 1 the whole greedy decode is one graph launch:
        the loop of examples/gpt_text.mira:66-81 runs on the device from start to end.  A
        warm-up step runs first, outside the capture; the state is rewound afterwards, so
        reset() must load a prompt before the graph is replayed."""
        torch = _t()
        if not 1 <= steps < self.T:
            raise ValueError(f"{steps} steps do not fit a {self.T}-token context")
        dev = self.exe.dev
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        self.state.zero_()                     # the warm-up step runs at position 0
        self.steps_done = 0
        with torch.cuda.stream(side):
            self.step()                        # warm-up outside the capture
        torch.cuda.current_stream(dev).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            stream = torch.cuda.current_stream(dev).cuda_stream
            for _ in range(steps):
                self._queue(stream)            # recorded, not run
        torch.cuda.synchronize(dev)
        self._graph_prompt_len = self.prompt_len
        self.graph_steps = steps
        self.state.zero_()
        self.steps_done = 0

    def run_steps(self, n: int, use_graph: bool = False) -> None:
        """n more decode steps: queued eagerly, or as replays of the captured graph (n must be a
        multiple of its step count)."""
        if use_graph:
            if self.graph is None or self._graph_prompt_len != self.prompt_len:
                raise RuntimeError("capture() first (for this prompt length)")
            if n % self.graph_steps:
                raise ValueError(f"{n} steps are not whole replays of a {self.graph_steps}-step graph")
            for _ in range(n // self.graph_steps):
                for _ in range(self.graph_steps):
                    self._advance()
                self.graph.replay()
            return
        for _ in range(n):
            self._advance()
            self._queue(self._stream())

    def decode(self, prompt: np.ndarray, new_tokens: int, use_graph: bool = False) -> np.ndarray:
        """Greedy decode: the prompt [B, P], then new_tokens argmax tokens; returns [B, P + new]."""
        P = np.asarray(prompt).shape[1]
        if P + new_tokens > self.T:
            raise ValueError(f"{P} + {new_tokens} tokens do not fit a {self.T}-token context")
        self.reset(prompt)
        self.run_steps(P + new_tokens - 1, use_graph)
        return self.tokens[:, :P + new_tokens].cpu().numpy()
