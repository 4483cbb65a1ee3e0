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

import contextlib
import gc
import weakref

import torch

from .cache import PromptCache


@contextlib.contextmanager
def no_cyclic_gc():
    """No cyclic garbage collection inside the block. A capture runs under it: a graph that the
    collector destroys in the middle of another capture (one left in an unreachable reference
    cycle) is a HIP error, and torch aborts the process on it."""
    was_on = gc.isenabled()
    gc.disable()
    try:
        yield
    finally:
        if was_on:
            gc.enable()


def capture_graph(fn):
    """(graph, fn's result) for `fn` captured on torch's current stream with no cyclic
    collection during the capture."""
    graph = torch.cuda.CUDAGraph()
    with no_cyclic_gc():
        with torch.cuda.graph(graph):
            out = fn()
    return graph, out


class CapturedStep:
    """`fn()` — forwards that advance `cache` by `tokens` positions in total — captured once.

    Calling the object replays it: it first makes the cache's device length current (outside
    the graph, only if it is stale), replays, then updates the host bookkeeping exactly as the
    eager forwards would have. `recorded`, when given, is the token count a recording pass
    leaves for the rollback check. Returns whatever `fn` returned at capture (static tensors,
    overwritten by each replay).

    `weak_cache=True` holds the cache by a weak reference, for a step the cache itself keeps:
    the pair then forms no reference cycle, so a dropped cache frees its graph by reference
    counting (`fn` must not hold the cache strongly either)."""

    def __init__(self, fn, cache: PromptCache, tokens: int, recorded: int | None = None, weak_cache: bool = False):
        self._cache = weakref.ref(cache) if weak_cache else (lambda c=cache: c)
        self.tokens, self.recorded = tokens, recorded
        cache.begin_step(tokens)  # device length current, so the capture records no write of it
        saved = cache.host_state()
        self.graph, self.out = capture_graph(fn)
        cache.restore_host_state(saved)

    @property
    def cache(self) -> PromptCache:
        cache = self._cache()
        if cache is None:
            raise RuntimeError("the cache of this captured step is gone")
        return cache

    def __call__(self):
        cache = self.cache
        cache.begin_step(self.tokens)
        self.graph.replay()
        cache.end_step(self.tokens)
        if self.recorded is not None and cache.shared.gdn is not None:
            cache.shared.gdn.recorded = self.recorded
        return self.out
