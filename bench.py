"""Benchmark of the flat-cost speculative-verify path on one MI355X.

Default run (`python bench.py`): prints ONE JSON line.

  step     one pass of the W4 g64 projection stack of a 36-layer hidden-2560 decoder at M=8
           tokens: per layer fused QKV (2560->6144), o_proj (4096->2560), fused gate+up
           (2560->19456), down (9728->2560), plus the lm_head (2560->151936) — 145 skinny
           qmm launches, 2.26 GB of weights, replayed as one HIP graph. Inputs are resident in
           HBM before timing; the stack (2.26 GB) is far larger than the 256 MB Infinity Cache.
  value    algorithmic bytes of the step (packs + scales + biases + activations in + out)
           divided by the measured step time, in GB/s.
  roofline the dominant kernel (fused gate+up shape, 36 launches per step) timed with HIP
           events on the launch stream over back-to-back launches.
  cpu_baseline  the oracle's dequant+matmul (numpy, fp64) on the config-0 matmul, a bounded
           sample timed on the host cores.

Options: --gpus N (only 1 is supported: this path runs on one GPU), --steps K, --warmup W, --m M.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "skinny-mlx_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, AMD public spec
HIDDEN, HEADS_Q, HEADS_KV, HEAD_DIM, FFN, VOCAB, LAYERS = 2560, 32, 8, 128, 9728, 151936, 36
# (K, N) of the projection stack per layer, then the head.
LAYER_SHAPES = [(HIDDEN, (HEADS_Q + 2 * HEADS_KV) * HEAD_DIM), (HEADS_Q * HEAD_DIM, HIDDEN), (HIDDEN, 2 * FFN),
                (FFN, HIDDEN)]
HEAD_SHAPE = (HIDDEN, VOCAB)


def qmm_bytes(m: int, k: int, n: int) -> int:
    """Algorithmic bytes of one call: packs + scales + biases + x in + y out."""
    return n * k // 2 + 4 * n * (k // 64) + 2 * m * k + 2 * m * n


def parse_args(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--m", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    return ap.parse_args(argv)


class Stack:
    """The 36-layer projection stack (+ head) as relaid W4 weights with static I/O buffers."""

    def __init__(self, m: int, dev, seed: int = 0):
        import torch

        from skinny_mlx import qmm as Q

        g = torch.Generator(device=dev).manual_seed(seed)
        self.m = m
        self.calls = []
        self.bytes = 0
        xs = {}
        for li in range(LAYERS):
            for k, n in LAYER_SHAPES:
                self._add(Q, g, dev, xs, k, n, m, tag=(k, n))
        self._add(Q, g, dev, xs, *HEAD_SHAPE, m, tag=HEAD_SHAPE)
        torch.cuda.synchronize()

    def _add(self, Q, g, dev, xs, k, n, m, tag):
        import torch

        w, s, b = Q.random_w4g64(n, k, generator=g, device=dev)
        wf = Q.repack_for_skinny(w, s, b)
        del w
        if k not in xs:
            xs[k] = torch.randn((m, k), generator=g, device=dev).to(torch.bfloat16)
        y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        self.calls.append((tag, xs[k], wf, s, b, y))
        self.bytes += qmm_bytes(m, k, n)

    def run(self, select=None):
        from skinny_mlx.qmm import skinny_qmm

        for tag, x, wf, s, b, y in self.calls:
            if select is None or tag == select:
                skinny_qmm(x, wf, s, b, out=y)


def capture(fn):
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # one eager pass outside capture (first-call work happens here)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    torch.cuda.synchronize()
    return graph


def time_graph(graph, steps: int, warmup: int):
    """(ms per replay from HIP events on the replay stream, wall ms per replay)."""
    import torch

    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return e0.elapsed_time(e1) / steps, wall


def cpu_baseline(seconds: float):
    """The oracle's dequant+matmul (numpy fp64) on the config-0 matmul, repeated ~`seconds`."""
    import numpy as np
    import torch

    from oracle import w4
    from skinny_mlx.qmm import random_w4g64

    m, k, n = 8, 2560, 9728
    g = torch.Generator().manual_seed(0)
    w, s, b = random_w4g64(n, k, generator=g)
    x = torch.randn((m, k), generator=g).to(torch.bfloat16)
    bits = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16)
    xb, wb, sb, bb = bits(x), w.numpy().view(np.uint32), bits(s), bits(b)
    w4.qmm(xb, wb, sb, bb)  # warm-up
    reps, t0 = 0, time.perf_counter()
    while True:
        w4.qmm(xb, wb, sb, bb)
        reps += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt = (time.perf_counter() - t0) / reps
    cores = _blas_threads()
    return {"value": round(qmm_bytes(m, k, n) / dt / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
            "ms_per_call": round(dt * 1e3, 2),
            "sample": f"oracle dequant+matmul (numpy fp64) of one M=8 K=2560 N=9728 W4 g64 matmul, "
                      f"{reps} calls in {seconds:.0f} s on {os.cpu_count()} host cores"}


def _blas_threads() -> int:
    try:
        from threadpoolctl import threadpool_info

        n = [i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"]
        return int(max(n)) if n else 1
    except Exception:  # noqa: BLE001
        return 1


def main(argv=None) -> int:
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported; this path runs on exactly one GPU "
              "(see DESIGN.md for how it would shard).", file=sys.stderr)
        return 2
    import torch

    from skinny_mlx import qmm as Q

    dev = torch.device("cuda:0")
    m = args.m
    stack = Stack(m, dev)
    graph = capture(stack.run)
    ms, wall_ms = time_graph(graph, args.steps, args.warmup)
    gbs = stack.bytes / (ms * 1e-3) / 1e9

    # dominant kernel: the fused gate+up shape, 36 back-to-back launches per replay
    dom_k, dom_n = LAYER_SHAPES[2]
    dom_graph = capture(lambda: stack.run(select=(dom_k, dom_n)))
    dom_ms, _ = time_graph(dom_graph, max(args.steps, 20), args.warmup)
    dom_us = dom_ms * 1e3 / LAYERS
    dom_bytes = qmm_bytes(m, dom_k, dom_n)
    dom_gbs = dom_bytes / (dom_us * 1e-6) / 1e9

    per_shape = {}
    for k, n in LAYER_SHAPES + [HEAD_SHAPE]:
        gr = capture(lambda k=k, n=n: stack.run(select=(k, n)))
        count = LAYERS if (k, n) != HEAD_SHAPE else 1
        reps = max(args.steps, 20) if count > 1 else max(args.steps, 200)
        sms, _ = time_graph(gr, reps, args.warmup)
        us = sms * 1e3 / count
        per_shape[f"{k}x{n}"] = {"us": round(us, 3), "GB/s": round(qmm_bytes(m, k, n) / (us * 1e-6) / 1e9, 1),
                                 "tile": list(Q.config_for(m, k, n))}
        del gr

    out = {
        "metric": "W4 qmm HBM GB/s + verify-step cost vs M=1 at M=8; spec-decode tok/s at 1 GPU",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "wall_ms_per_step": round(wall_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"W4A16 g64 projection stack of a 36-layer hidden-2560 decoder at M={m} "
                               "(per layer fused QKV 2560x6144, o 4096x2560, fused gate+up 2560x19456, "
                               "down 9728x2560; plus lm_head 2560x151936), one HIP graph of 145 skinny qmm launches",
                   "tokens_per_step": m, "bytes_per_step": stack.bytes},
        "roofline": {"bound": "hbm", "achieved": round(dom_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": f"skinny qmm M={m} K={dom_k} N={dom_n}", "us_per_launch": round(dom_us, 3),
                     "bytes_per_launch": dom_bytes},
        "stack_frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
        "per_shape": per_shape,
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
