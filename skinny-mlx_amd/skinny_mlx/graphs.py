"""Decode steps captured as HIP graphs.

A verify or decode step is a few hundred small launches (norms, matmuls, attention, the
recurrence, argmax); issued one by one from Python they cost more host time than the GPU spends
on them. Every kernel on the path takes its sequence position from device memory and advances
it with a kernel of its own (cache.PromptCache.advance), so one captured step replays correctly
at any position. What a capture cannot record is the host-side bookkeeping: the per-layer KV
lengths and the tracked device length, and the recorded-token count of a recording (verify)
pass. `CapturedStep` undoes that bookkeeping after capturing (no kernel ran) and redoes it
after every replay.

Rules for the captured function: device work only on torch's current stream, inputs and
outputs in tensors that stay alive (the object holds the returned outputs), no host->device
copies of Python data, and no memset nodes (torch's `fill_`/`zero_` launch fill kernels).
"""

from __future__ import annotations

import gc

import torch

from .cache import PromptCache


class CapturedStep:
    """`fn()` — forwards that advance `cache` by `tokens` positions in total — captured once.

    Calling the object replays it: it first makes the cache's device length current (outside
    the graph, only if it is stale), replays, then updates the host bookkeeping exactly as the
    eager forwards would have. `recorded`, when given, is the token count a recording pass
    leaves for the rollback check. Returns whatever `fn` returned at capture (static tensors,
    overwritten by each replay)."""

    def __init__(self, fn, cache: PromptCache, tokens: int, recorded: int | None = None):
        self.cache, self.tokens, self.recorded = cache, tokens, recorded
        cache.begin_step(tokens)  # device length current, so the capture records no write of it
        saved = cache.host_state()
        self.graph = torch.cuda.CUDAGraph()
        # No cyclic garbage collection while capturing: a graph in an unreachable cycle (a
        # dropped cache and the step kept on it) destroyed mid-capture is a HIP error, and
        # torch aborts the process on it. Collection resumes when the capture is over.
        gc_was_on = gc.isenabled()
        gc.disable()
        try:
            with torch.cuda.graph(self.graph):
                self.out = fn()
        finally:
            if gc_was_on:
                gc.enable()
        cache.restore_host_state(saved)

    def __call__(self):
        cache = self.cache
        cache.begin_step(self.tokens)
        self.graph.replay()
        cache.end_step(self.tokens)
        if self.recorded is not None and cache.shared.gdn is not None:
            cache.shared.gdn.recorded = self.recorded
        return self.out
