"""Benchmark of the flat-cost speculative-verify path on one MI355X.

Default run (`python bench.py`): prints ONE JSON line.

  value     the W4 g64 projection stack of a 36-layer hidden-2560 decoder at M=8 tokens: per
            layer fused QKV (2560->6144), o_proj (4096->2560), fused gate+up (2560->19456),
            down (9728->2560), plus the lm_head (2560->151936) — 145 skinny qmm launches over
            2.29 GB of weights, replayed as one HIP graph with everything resident in HBM (far
            beyond the 256 MB Infinity Cache). The launches are independent (the reference's
            protocol evaluates the list of matmuls in one mx.eval): the graph spreads them over
            --streams streams (4), balanced by bytes, and its outputs are checked
            bitwise against the same launches as one dependent chain (`stack_chain`: each launch
            waits for the one before, as in a decoder step). value = algorithmic bytes of the
            step (packs + scales + biases + activations in + out) / measured step time, in GB/s.
  stack_sweep  the same stack at every M in 1, 2, 3, 4, 6, 8, 12, 16 (the reference's protocol,
            qmm.py:189-198), both forms, with each (K, N) shape timed per M as a chain of its
            launches (bench/model_matmuls.py:25-44).
  config0   the single matmul M=8, K=2560, N=9728 over 64 distinct weight sets, back to back in
            one HIP graph: us per launch, GB/s, fraction of 8 TB/s.
  roofline  the dominant kernel (the fused gate+up shape, 36 launches per step), timed with HIP
            events on the launch stream over back-to-back launches of its 36 weight sets;
            roofline.ceiling.stream_read: a streaming read of the same sizes as single launches and
            back to back in a graph (bench/hw_roofline.py:3-11), the achievable fraction at each size;
            roofline.attention: the fused attention (chunk kernel + merge) over 2048 cached tokens,
            36 layers' caches in one graph per M, against the same-size (8 MiB) read ceiling.
  verify_step  a random-init 36-layer dense decoder (hidden 2560, GQA 32q/8kv x 128, SwiGLU 9728,
            W4 g64 linears, vocab 151936) with 2048 cached tokens: one captured forward of M
            tokens for M in {1, 2, 4, 6, 8, 12, 16}, its ms and the cost relative to M = 1; beside it
            the same curve with the unpatched kernels on the fused projections ("fuse") and for the
            unpatched model ("stock"), the columns of bench/step_cost_curve.py:50-57.
  spec_decode  the hybrid model (3 Gated-DeltaNet layers per attention layer), 256-token uniform
            random prompt, 512 generated tokens: greedy tok/s, and speculative tok/s with the
            random-init MTP head (K = 2, 3, 4; random weights draft almost nothing acceptable),
            and with a replay drafter that proposes the model's own greedy continuation (the
            acceptance upper bound; K = 3), and at the reference's measured acceptance
            (`mtp_at_reference_acceptance_k*`: the MTP head's chain and update run as usual, its
            proposals replaced by the greedy continuation, each position right with probability
            0.827, which reproduces the reference's 2.51 / 3.05 / 3.47 tokens per step at K = 2 /
            3 / 4, docs/flatspec-design.md:65-66). Every greedy run is checked token for token against
            greedy decoding. At temperature 1: plain sampled decoding, and speculative decoding with
            rejection sampling (MTP K = 3). `tok_s` is end to end (the reference's protocol: prompt,
            graph captures and decode); `decode_tok_s` the decode loop alone.
  tree_decode  the same model and prompt with a 16-node draft tree (branching 4, 2, 1) verified
            in one tree-masked M=16 forward per step: tok/s and tokens/step with the MTP head's
            top-k tree and with a replay tree (greedy continuation along a second-ranked branch),
            the per-phase ms of a step, and the captured tree verify forward vs an M=1 forward.
  cpu_baseline  the config-0 matmul in torch fp32 on the host cores (mlx, whose CPU quantized
            matmul the reference would time, is not installed): dequantise + matmul per call (value)
            and the matmul alone on pre-dequantised weights, with the thread count and CPU model.

Options: --gpus N (only 1: this path runs on one GPU), --steps K, --warmup W, --m M,
--no-model (qmm stack only), --stack-only, --streams S, --no-cpu, --cpu-seconds S, --spec-tokens N,
--verify-only M (just the captured M-token verify forward, K replays over a synthetic 2048-token
cache: a clean trace for profiling; --verify-preset hybrid-36 and --verify-tree select the model
and a draft tree).
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
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "qmm_gate_up_m8_traffic.json")
MFMA_FILE = os.path.join(ROOT, "profiles", "qmm_gate_up_m8_mfma.json")
L2_FILE = os.path.join(ROOT, "profiles", "qmm_gate_up_m8_l2_requests.json")
# per-dispatch counters of the gate|up forms the decoder step runs (the SwiGLU epilogue; for one
# token with the RMSNorm formed inside): HBM traffic and L2 requests per launch, keyed by form
DECODER_COUNTERS_FILE = os.path.join(ROOT, "profiles", "qmm_gate_up_decoder_forms_counters.json")
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16


def qmm_bytes(m: int, k: int, n: int) -> int:
    """Algorithmic bytes of one call: packs + scales + biases + x in + y out."""
    return n * k // 2 + 4 * n * (k // 64) + 2 * m * k + 2 * m * n


FOLD_NORMS = None  # --separate-norms: False (every RMSNorm its own launch); None: Model.fold_norms as built


def parse_args(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--m", type=int, default=8)
    ap.add_argument("--no-model", action="store_true", help="only the qmm stack")
    ap.add_argument("--stack-only", action="store_true",
                    help="only the qmm stack at --m (no M sweep, config 0, ceiling, model or CPU legs): the command "
                         "behind the stack's kernel summary")
    ap.add_argument("--streams", type=int, default=4,
                    help="streams the stack's independent launches are spread over inside its graph (1: the "
                         "launches as one dependent chain only)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--spec-tokens", type=int, default=512)
    ap.add_argument("--verify-only", type=int, default=0, metavar="M",
                    help="only the captured M-token verify forward, over a synthetic 2048-token cache (for profiling)")
    ap.add_argument("--verify-preset", default="dense-36", help="model of --verify-only (dense-36 or hybrid-36)")
    ap.add_argument("--verify-tree", action="store_true", help="--verify-only as a draft tree (branching 4, 2, 1)")
    ap.add_argument("--spec-only", type=int, default=0, metavar="K",
                    help="only speculative decoding with the MTP head at the reference's acceptance, K drafts, on "
                         "the hybrid decoder (--spec-tokens tokens): the command behind the decode loop's kernel "
                         "summary")
    ap.add_argument("--separate-norms", action="store_true",
                    help="every RMSNorm as its own launch, also in one-token forwards (Model.fold_norms off; "
                         "the same bits)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="for rocprofv3 --pmc: one launch of the dominant qmm on each of its 36 weight sets, "
                         "then a 64 MiB device copy and a 64 MiB streaming read as calibration kernels")
    return ap.parse_args(argv)


def traffic_probe(args, dev) -> None:
    """Kernels whose hardware counters (FETCH_SIZE, WRITE_SIZE, L2 requests) give the dominant
    kernels' traffic: 36 launches each (2 passes) on distinct weight sets of the M x 2560 x 19456
    qmm (the projection stack's form), then of the decoder's own gate|up forms (DecoderGateUp:
    SwiGLU at M, and the one-token norm-in SwiGLU), then the calibration kernels of known
    traffic."""
    import torch

    from skinny_mlx import _lib
    from skinny_mlx import qmm as Q

    k, n = LAYER_SHAPES[2]
    g = torch.Generator(device=dev).manual_seed(0)
    ws = [Q.repack_for_skinny(*Q.random_w4g64(n, k, generator=g, device=dev)) for _ in range(LAYERS)]
    x = torch.randn((args.m, k), generator=g, device=dev).to(torch.bfloat16)
    y = torch.empty((args.m, n), dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()
    for _ in range(2):
        for w in ws:
            Q.skinny_qmm(x, w, out=y)
    torch.cuda.synchronize()
    del ws
    dec = DecoderGateUp(dev)
    for form, m in DecoderGateUp.FORMS:
        for _ in range(2):
            dec.run(form, m)
    torch.cuda.synchronize()
    del dec
    src = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    red = torch.empty(1024, dtype=torch.float32, device=dev)
    _lib.check(_lib.lib().skinny_stream_read(src.data_ptr(), src.numel(), red.data_ptr(), 1024, _lib.stream_of(src)),
               "stream_read")
    torch.cuda.synchronize()
    print(json.dumps({"traffic_probe": {"qmm": [args.m, k, n], "launches": 2 * LAYERS,
                                        "algorithmic_bytes_per_launch": qmm_bytes(args.m, k, n),
                                        "decoder_forms": {f"{form} M={m}": DecoderGateUp.bytes(form, m)
                                                          for form, m in DecoderGateUp.FORMS},
                                        "calibration_bytes": 64 << 20}}), flush=True)


class DecoderGateUp:
    """The fused gate|up projection (2560 -> 2 x 9728) in the forms the decoder step launches, on
    36 distinct weight sets (one per layer, 1 GB in all, past the Infinity Cache):
      * "swiglu": skinny_glu(x, w, swiglu=True), the verify step's form (from two tokens on, the
        tile's four K groups in one wave);
      * "normin_swiglu": skinny_glu_normin of a kernels.NormIn, the one-token step's form: the
        RMSNorm of h + the down projection's three fp32 slices formed inside the launch."""

    FORMS = (("swiglu", 8), ("normin_swiglu", 1))
    K, F = HIDDEN, FFN

    def __init__(self, dev):
        import torch

        from skinny_mlx import qmm as Q

        g = torch.Generator(device=dev).manual_seed(3)
        self.dev, self.g = dev, g
        self.ws = []
        for _ in range(LAYERS):
            w, s, b = Q.random_w4g64(2 * self.F, self.K, generator=g, device=dev)
            self.ws.append(Q.repack_gate_up(w, s, b))
            del w, s, b
        self.norm_w = (torch.randn(self.K, generator=g, device=dev) * 0.1 + 1).to(torch.bfloat16)
        self.io = {}

    @classmethod
    def bytes(cls, form: str, m: int) -> int:
        """Algorithmic bytes of one launch: packs + scales + biases, the input rows, the SwiGLU
        output [M, F]; the norm-in form reads h [M, K] bf16, three fp32 slices [3, M, K] and the
        norm weight instead of X, and writes the new residual rows [M, K]."""
        k, n = cls.K, 2 * cls.F
        w = n * k // 2 + 4 * n * (k // 64)
        if form == "swiglu":
            return w + 2 * m * k + 2 * m * cls.F
        return w + 2 * m * k + 3 * 4 * m * k + 2 * k + 2 * m * cls.F + 2 * m * k

    def _io(self, form: str, m: int):
        import torch

        from skinny_mlx import kernels as Kn

        key = (form, m)
        if key not in self.io:
            y = torch.empty((m, self.F), dtype=torch.bfloat16, device=self.dev)
            h = torch.randn((m, self.K), generator=self.g, device=self.dev).to(torch.bfloat16)
            if form == "swiglu":
                self.io[key] = (h, y)
            else:
                parts = torch.randn((3, m, self.K), generator=self.g, device=self.dev) * 0.1
                h_out = torch.empty_like(h)
                self.io[key] = (Kn.NormIn(h, Kn.PartialSum(parts), self.norm_w, 1e-6, h_out), y)
        return self.io[key]

    def run(self, form: str, m: int) -> None:
        from skinny_mlx import qmm as Q

        x, y = self._io(form, m)
        for w in self.ws:
            if form == "swiglu":
                Q.skinny_glu(x, w, swiglu=True, out=y)
            else:
                Q.skinny_glu_normin(x, w, out=y)


def decoder_roofline(args, dev) -> dict:
    """The gate|up launches as the decoder step runs them (DecoderGateUp), each form as one graph of
    36 launches on distinct weight sets: us per launch from HIP events on the replay stream,
    algorithmic GB/s against the 8 TB/s peak, and the per-dispatch HBM traffic and L2 request
    counters of the same kernels where profiles/ holds them."""
    dec = DecoderGateUp(dev)
    counters = {}
    if os.path.exists(DECODER_COUNTERS_FILE):
        with open(DECODER_COUNTERS_FILE) as f:
            counters = json.load(f).get("forms", {})
    out = {}
    for form, m in DecoderGateUp.FORMS:
        graph = capture(lambda form=form, m=m: dec.run(form, m))
        best = min(time_replays(graph.replay, max(args.steps, 20), args.warmup)[0] for _ in range(3))
        del graph
        us = best * 1e3 / LAYERS
        nbytes = DecoderGateUp.bytes(form, m)
        gbs = nbytes / (us * 1e-6) / 1e9
        rec = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
               "frac": round(gbs / HBM_PEAK_GBS, 4), "us_per_launch": round(us, 3), "bytes_per_launch": nbytes,
               "m": m, "traffic": None}
        c = counters.get(f"{form} M={m}")
        if c:
            rec["traffic"] = c.get("hbm_bytes_per_launch")
            rec["kernel"] = c.get("kernel")
            for key in ("l2_request_bytes_per_launch", "l2_miss_bytes_per_launch", "traffic_over_algorithmic",
                        "l2_requests_over_algorithmic"):
                if key in c:
                    rec[key] = c[key]
        out[f"{form} M={m}"] = rec
    del dec
    return {"workload": "fused gate|up 2560 -> 2 x 9728 as the decoder step launches it: SwiGLU at M=8 (the verify "
                        "step's dominant launch) and the one-token norm-in form; 36 distinct weight sets in one HIP "
                        "graph per form", "forms": out}


class Stack:
    """The 36-layer projection stack (+ head) as packed W4 weights, built once; static bf16 input
    and output buffers per token count M."""

    def __init__(self, dev, seed: int = 0):
        import torch

        from skinny_mlx import qmm as Q

        g = torch.Generator(device=dev).manual_seed(seed)
        self.dev = dev
        self.weights = []  # (tag (K, N), packed, scales, biases)
        for _ in range(LAYERS):
            for k, n in LAYER_SHAPES:
                self.weights.append(((k, n),) + self._weight(Q, g, dev, k, n))
        self.weights.append((HEAD_SHAPE,) + self._weight(Q, g, dev, *HEAD_SHAPE))
        self.g = g
        self.io = {}
        torch.cuda.synchronize()

    @staticmethod
    def _weight(Q, g, dev, k, n):
        w, s, b = Q.random_w4g64(n, k, generator=g, device=dev)
        return Q.repack_for_skinny(w, s, b), s, b

    def buffers(self, m: int):
        import torch

        if m not in self.io:
            xs = {k: torch.randn((m, k), generator=self.g, device=self.dev).to(torch.bfloat16)
                  for k in {t[0] for t, *_ in self.weights}}
            ys = [torch.empty((m, t[1]), dtype=torch.bfloat16, device=self.dev) for t, *_ in self.weights]
            self.io[m] = (xs, ys)
        return self.io[m]

    def bytes(self, m: int, select=None) -> int:
        return sum(qmm_bytes(m, *t) for t, *_ in self.weights if select is None or t == select)

    def run(self, m: int, select=None):
        from skinny_mlx.qmm import skinny_qmm

        xs, ys = self.buffers(m)
        for (tag, wf, s, b), y in zip(self.weights, ys):
            if select is None or tag == select:
                skinny_qmm(xs[tag[0]], wf, s, b, out=y)

    def lanes(self, streams: int) -> list[int]:
        """Stream index of each launch when the launches are spread over `streams` streams: the
        largest launches first, each to the stream with the fewest bytes so far (split-K calls
        keep a workspace per stream, so any shape may go on any stream). Measured at M=8 over 4
        streams: 3414-3422 GB/s, against 3311-3353 GB/s with one (K, N) shape per stream."""
        import heapq

        sizes = [qmm_bytes(8, k, n) for (k, n), *_ in self.weights]
        load = [(0, s) for s in range(streams)]
        lanes = [0] * len(sizes)
        for i in sorted(range(len(sizes)), key=lambda i: (-sizes[i], i)):
            used, s = heapq.heappop(load)
            lanes[i] = s
            heapq.heappush(load, (used + sizes[i], s))
        return lanes

    def run_concurrent(self, m: int, streams) -> None:
        """The stack as a batch of independent launches: spread over `streams` (forked from the
        current stream and joined back to it), so no launch waits for one on another stream."""
        import torch

        from skinny_mlx.qmm import skinny_qmm

        xs, ys = self.buffers(m)
        main = torch.cuda.current_stream()
        for st in streams:
            st.wait_stream(main)
        for (tag, wf, s, b), y, lane in zip(self.weights, ys, self.lanes(len(streams))):
            with torch.cuda.stream(streams[lane]):
                skinny_qmm(xs[tag[0]], wf, s, b, out=y)
        for st in streams:
            main.wait_stream(st)


def capture(fn):
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # one eager pass outside capture (first-call work happens here)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    from skinny_mlx.graphs import capture_graph

    graph, _ = capture_graph(fn)
    torch.cuda.synchronize()
    return graph


def time_replays(replay, steps: int, warmup: int):
    """(ms per replay from HIP events on the replay stream, wall ms per replay)."""
    import torch

    for _ in range(warmup):
        replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        replay()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return e0.elapsed_time(e1) / steps, wall


STACK_MS = (1, 2, 3, 4, 6, 8, 12, 16)  # the reference's stack protocol (qmm.py:189-198)


def qmm_stack(args, dev):
    """The stack at every M of STACK_MS and each (K, N) shape per M (one graph of its 36 launches,
    or the head's one): algorithmic GB/s and fraction of the 8 TB/s peak. The stack is one HIP
    graph of 145 launches per M, timed twice: as a batch of independent launches spread over
    `args.streams` streams (the reference's protocol evaluates the list of independent matmuls in
    one mx.eval, qmm.py:195-197; nothing orders them), and as one dependent chain on one stream
    (each launch waits for the one before, as the matmuls of a decoder step do). The batch's
    outputs are checked bitwise against the chain's. Returns the M = args.m stack numbers (the
    batch's), its roofline record and the sweep."""
    import torch

    from skinny_mlx import qmm as Q

    stack = Stack(dev)
    sweep = {}
    main = None
    dom = None
    streams = [torch.cuda.Stream() for _ in range(args.streams)] if args.streams > 1 else None
    for m in ((args.m,) if args.stack_only else sorted(set(STACK_MS) | {args.m})):
        nbytes = stack.bytes(m)
        graph = capture(lambda m=m: stack.run(m))
        serial_ms, serial_wall_ms = time_replays(graph.replay, args.steps, args.warmup)
        del graph
        serial = {"ms": round(serial_ms, 4), "GB/s": round(nbytes / (serial_ms * 1e-3) / 1e9, 1),
                  "frac": round(nbytes / (serial_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        if streams:
            chain = [y.clone() for y in stack.buffers(m)[1]]
            graph = capture(lambda m=m: stack.run_concurrent(m, streams))
            for y in stack.buffers(m)[1]:
                y.zero_()
            graph.replay()
            torch.cuda.synchronize()
            if not all(torch.equal(a, b) for a, b in zip(chain, stack.buffers(m)[1])):
                raise RuntimeError(f"stack at M={m}: the batch of independent launches differs from the chain")
            del chain
            ms, wall_ms = time_replays(graph.replay, args.steps, args.warmup)
            del graph
        else:
            ms, wall_ms = serial_ms, serial_wall_ms
        gbs = nbytes / (ms * 1e-3) / 1e9
        per_shape = {}
        for k, n in LAYER_SHAPES + [HEAD_SHAPE]:
            gr = capture(lambda k=k, n=n, m=m: stack.run(m, select=(k, n)))
            count = LAYERS if (k, n) != HEAD_SHAPE else 1
            reps = max(args.steps, 20) if count > 1 else max(args.steps, 200)
            sms, _ = time_replays(gr.replay, reps, args.warmup)
            del gr
            us = sms * 1e3 / count
            sgbs = qmm_bytes(m, k, n) / (us * 1e-6) / 1e9
            splits, tile = Q._plain_config(k, n)
            per_shape[f"{k}x{n}"] = {"us": round(us, 3), "GB/s": round(sgbs, 1), "frac": round(sgbs / HBM_PEAK_GBS, 4),
                                     "tile": list(tile.as_tuple()), "splits": splits}
            if m == args.m and (k, n) == LAYER_SHAPES[2]:
                dom = (k, n, us)
        sweep[m] = {"ms": round(ms, 4), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                    "chain": serial, "per_shape": per_shape}
        if m == args.m:
            main = (gbs, ms, wall_ms, per_shape)
    if 1 in sweep:
        m1, c1 = sweep[1]["ms"], sweep[1]["chain"]["ms"]
        for m, rec in sweep.items():
            rec["cost_vs_m1"] = round(rec["ms"] / m1, 3)
            rec["chain"]["cost_vs_m1"] = round(rec["chain"]["ms"] / c1, 3)
    gbs, ms, wall_ms, per_shape = main
    m = args.m
    dk, dn, dus = dom
    dbytes = qmm_bytes(m, dk, dn)
    dgbs = dbytes / (dus * 1e-6) / 1e9
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            rec = json.load(f)
        if rec.get("m") == m and rec.get("shape") == [dk, dn]:
            traffic = rec.get("hbm_bytes_per_launch")
    roofline = {"bound": "hbm", "achieved": round(dgbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(dgbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                "kernel": f"skinny qmm M={m} K={dk} N={dn}", "us_per_launch": round(dus, 3),
                "bytes_per_launch": dbytes}
    if os.path.exists(L2_FILE):
        # bytes of L2 requests per launch of the same kernel (per-dispatch counters, 128 B per request)
        with open(L2_FILE) as f:
            rec = json.load(f)
        if rec.get("m") == m and rec.get("shape") == [dk, dn]:
            roofline["l2_request_bytes"] = rec["l2_request_bytes_per_launch"]
            roofline["l2_miss_bytes"] = rec["l2_miss_bytes_per_launch"]
    if os.path.exists(MFMA_FILE):
        # MFMA use of the same launch: per-dispatch counters (rocprofv3 --pmc) over the live duration
        with open(MFMA_FILE) as f:
            rec = json.load(f)
        if rec.get("m") == m and rec.get("shape") == [dk, dn]:
            sec = dus * 1e-6
            roofline["mfma"] = {
                "executed_tflops": round(rec["executed_flop_per_dispatch"] / sec / 1e12, 1),
                "algorithmic_tflops": round(rec["algorithmic_flop_per_dispatch"] / sec / 1e12, 1),
                "peak_tflops": MFMA_BF16_PEAK_TFLOPS,
                "busy_frac": round(rec["sq_valu_mfma_busy_cycles_per_dispatch"]
                                   / (rec["simds"] * rec["clock_mhz"] * 1e6 * sec), 4)}
    del stack
    return gbs, ms, wall_ms, roofline, per_shape, sweep[args.m]["chain"], sweep


def library_gemm_shapes(dev, m: int, per_shape: dict, min_bytes: int = 768 << 20, reps: int = 20):
    """The stack's shapes at m tokens as the model run unquantised computes them: bf16 weights
    (the W4 weights dequantised once) times bf16 rows by torch's GEMM, enough distinct weight sets
    per shape (at least `min_bytes`, past the Infinity Cache) back to back in one graph. Per shape:
    µs per call, GB/s of bf16 weight bytes (+ rows in and out) and the skinny kernel's speed-up in
    time (`per_shape`: the skinny stack's record at the same m)."""
    import torch

    from skinny_mlx import kernels as K
    from skinny_mlx import qmm as Q

    out = {}
    g = torch.Generator(device=dev).manual_seed(11)
    for k, n in LAYER_SHAPES + [HEAD_SHAPE]:
        wbytes = 2 * n * k
        sets = max(2, -(-min_bytes // wbytes))
        w, s, b = Q.random_w4g64(n, k, generator=torch.Generator(device=dev).manual_seed(k + n), device=dev)
        wd = K.dequant(w, s, b).to(torch.bfloat16)
        del w, s, b
        ws = [wd] + [wd.clone() for _ in range(sets - 1)]
        x = torch.randn((m, k), generator=g, device=dev).to(torch.bfloat16)

        def run(ws=ws, x=x):
            return [torch.nn.functional.linear(x, wi) for wi in ws]

        run()  # the library's first-call set-up, which a capture does not permit
        torch.cuda.synchronize()
        graph = capture(run)
        t_ms = min(time_replays(graph.replay, reps, 3)[0] for _ in range(2))
        del graph, ws, wd
        torch.cuda.empty_cache()
        us = t_ms * 1e3 / sets
        nbytes = wbytes + 2 * m * k + 2 * m * n
        gbs = nbytes / (us * 1e-6) / 1e9
        rec = {"us": round(us, 3), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4), "weight_sets": sets}
        sk = per_shape.get(f"{k}x{n}")
        if sk:
            rec["skinny_speedup"] = round(us / sk["us"], 3)
        out[f"{k}x{n}"] = rec
    return {"workload": f"each stack shape at M={m} with bf16 weights (the W4 weights dequantised once) and "
                        "torch's bf16 GEMM, distinct weight sets back to back in one HIP graph: the model run "
                        "unquantised", "per_shape": out}


CONFIG0 = (8, 2560, 9728)  # M, K, N of the single-matmul headline shape


def qmm_config0(args, dev, sets: int = 64):
    """The single W4A16 matmul M=8, K=2560, N=9728 over `sets` distinct weight sets (64 x 14.2 MB,
    far beyond the 256 MB Infinity Cache), back to back in one HIP graph: us per launch."""
    import torch

    from skinny_mlx import qmm as Q

    m, k, n = CONFIG0
    g = torch.Generator(device=dev).manual_seed(1)
    ws = []
    for _ in range(sets):
        w, s, b = Q.random_w4g64(n, k, generator=g, device=dev)
        ws.append((Q.repack_for_skinny(w, s, b), s, b))
        del w
    x = torch.randn((m, k), generator=g, device=dev).to(torch.bfloat16)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)

    def run():
        for wf, s, b in ws:
            Q.skinny_qmm(x, wf, s, b, out=y)

    graph = capture(run)
    best = min(time_replays(graph.replay, max(args.steps, 20), args.warmup)[0] for _ in range(3))
    del graph, ws
    torch.cuda.empty_cache()
    us = best * 1e3 / sets
    gbs = qmm_bytes(m, k, n) / (us * 1e-6) / 1e9
    return {"workload": f"one W4A16 g64 matmul M={m} K={k} N={n} (bf16 in/out, fp32 accumulate), {sets} distinct "
                        "weight sets back to back in one HIP graph", "us": round(us, 3), "GB/s": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": qmm_bytes(m, k, n), "weight_sets": sets,
            "tile": list(Q.config_for(m, k, n))}


STREAM_FORMS = [("stride", g, 4) for g in (1024, 2048, 4096, 8192)] + [
    ("chunk", g, l) for g in (256, 512, 1024, 2048) for l in (4, 8, 16)]


def stream_ceiling(dev, sizes=(5_898_240, 8_388_608, 14_204_928, 28_368_896, 221_000_000, 1 << 30), forms=STREAM_FORMS):
    """The streaming-read ceiling at the qmm launches' sizes, the reference's hw_roofline protocol
    (bench/hw_roofline.py:3-11): skinny_stream_read (a grid-stride read, four 16-byte loads in flight
    per thread) and skinny_stream_read_chunked (a contiguous chunk per workgroup, 4, 8 or 16 loads in
    flight), reduced so the loads cannot be elided; the best form and grid per size (8 MiB: one
    attention layer's K and V at 2048 cached tokens, what its chunk kernel reads). Each size reads
    enough distinct buffers (>= 1 GB in all) that no launch hits the Infinity Cache. `single`: one
    launch at a time between HIP events; `graph`: the launches back to back in one HIP graph."""
    import torch

    from skinny_mlx import _lib

    L = _lib.lib()
    out = []
    red = torch.empty(max(g for _, g, _ in forms), dtype=torch.float32, device=dev)
    for size in sizes:
        size16 = (size + 4095) // 4096 * 4096
        count = max(2, -(-(1 << 30) // size16))
        buf = torch.empty(count * size16, dtype=torch.uint8, device=dev)
        buf.fill_(1)
        stream = torch.cuda.current_stream()
        best = {"single": None, "graph": None}
        for form, grid, loads in forms:
            def launch(i, form=form, grid=grid, loads=loads):
                if form == "stride":
                    rc = L.skinny_stream_read(buf.data_ptr() + i * size16, size, red.data_ptr(), grid, _lib.stream_of(buf))
                else:
                    rc = L.skinny_stream_read_chunked(buf.data_ptr() + i * size16, size, red.data_ptr(), grid, loads,
                                                      _lib.stream_of(buf))
                _lib.check(rc, "stream_read")
            for i in range(count):
                launch(i)
            torch.cuda.synchronize()
            evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(count)]
            for i, (e0, e1) in enumerate(evs):
                e0.record(stream)
                launch(i)
                e1.record(stream)
            torch.cuda.synchronize()
            single = sum(e0.elapsed_time(e1) for e0, e1 in evs) / count * 1e3
            graph = capture(lambda: [launch(i) for i in range(count)])
            g_ms = min(time_replays(graph.replay, 5, 2)[0] for _ in range(2))
            del graph
            graph_us = g_ms * 1e3 / count
            for key, us in (("single", single), ("graph", graph_us)):
                if best[key] is None or us < best[key][0]:
                    best[key] = (us, f"{form} grid={grid} loads={loads}")
        del buf
        torch.cuda.empty_cache()
        rec = {"bytes": size, "buffers": count}
        for key, (us, form) in best.items():
            gbs = size / (us * 1e-6) / 1e9
            rec[key] = {"us": round(us, 3), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4), "form": form}
        out.append(rec)
    return out


def attention_roofline(dev, ceiling, ms=(1, 8, 16), layers: int = 36, length: int = 2048, reps: int = 20):
    """The attention of the 36-layer dense decoder (skinny_attention_fused_bf16: the chunk kernel
    and the merge) over 2048 cached tokens: one graph of 36 launches, each on its own layer's KV
    cache (600 MB in all, past the Infinity Cache), per M. Algorithmic bytes per layer: the cached
    keys and values it reads, 2 x 8 heads x 2048 x 128 bf16 = 8 MiB; beside them the streaming-read
    ceiling of the same size (`ceiling`: its stream_ceiling record)."""
    import torch

    from skinny_mlx import kernels as K

    Hq, Hkv, D, maxlen = 32, 8, 128, 4096
    g = torch.Generator(device=dev).manual_seed(5)
    kcs = [torch.randn((Hkv, maxlen, D), generator=g, device=dev).to(torch.bfloat16) for _ in range(layers)]
    vts = [torch.randn((Hkv, D, maxlen), generator=g, device=dev).to(torch.bfloat16) for _ in range(layers)]
    qn = (torch.randn(D, generator=g, device=dev) * 0.1 + 1).to(torch.bfloat16)
    kn = (torch.randn(D, generator=g, device=dev) * 0.1 + 1).to(torch.bfloat16)
    table = K.rope_table(1e6, maxlen, dev)
    ws = K.attn_workspace(Hkv, maxlen, dev)
    pos = torch.tensor([length], dtype=torch.int32, device=dev)
    kv_bytes = 2 * Hkv * length * D * 2
    per_m = {}
    for m in ms:
        qkv = torch.randn((m, (Hq + 2 * Hkv) * D), generator=g, device=dev).to(torch.bfloat16)

        def run(qkv=qkv):
            for kc, vt in zip(kcs, vts):
                K.attention_fused(qkv, Hq, Hkv, D, qn, kn, 1e-6, table, pos, kc, vt, D ** -0.5, ws)

        graph = capture(run)
        t_ms = min(time_replays(graph.replay, reps, 3)[0] for _ in range(2))
        del graph
        us = t_ms * 1e3 / layers
        gbs = kv_bytes / (us * 1e-6) / 1e9
        per_m[m] = {"us_per_layer": round(us, 3), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                    "of_graph_read_ceiling": round(ceiling["graph"]["us"] / us, 3)}
    del kcs, vts
    torch.cuda.empty_cache()
    return {"workload": f"fused attention (chunk kernel + merge) of 36 layers, Hq=32 Hkv=8 D=128, {length} cached "
                        "tokens, each layer its own cache; one HIP graph per M",
            "kv_bytes_per_layer": kv_bytes, "read_ceiling_same_size": ceiling, "per_m": per_m,
            "per_context_m8": attention_contexts(dev)}


def attention_contexts(dev, lengths=(2048, 8192, 32768), m: int = 8, min_bytes: int = 768 << 20, reps: int = 20):
    """The same fused attention at M = m over longer contexts: per length, enough layer caches (each
    sized to the context) to read at least `min_bytes` per replay, past the Infinity Cache, in one
    graph. µs per layer and GB/s of KV read: where the launch stops being latency-bound."""
    import torch

    from skinny_mlx import kernels as K

    Hq, Hkv, D = 32, 8, 128
    g = torch.Generator(device=dev).manual_seed(6)
    qn = (torch.randn(D, generator=g, device=dev) * 0.1 + 1).to(torch.bfloat16)
    kn = (torch.randn(D, generator=g, device=dev) * 0.1 + 1).to(torch.bfloat16)
    qkv = torch.randn((m, (Hq + 2 * Hkv) * D), generator=g, device=dev).to(torch.bfloat16)
    out = {}
    for length in lengths:
        maxlen = -(-(length + m) // 128) * 128
        kv_bytes = 2 * Hkv * length * D * 2
        layers = max(2, -(-min_bytes // kv_bytes))
        kcs = [torch.randn((Hkv, maxlen, D), generator=g, device=dev).to(torch.bfloat16) for _ in range(layers)]
        vts = [torch.randn((Hkv, D, maxlen), generator=g, device=dev).to(torch.bfloat16) for _ in range(layers)]
        table = K.rope_table(1e6, maxlen, dev)
        ws = K.attn_workspace(Hkv, maxlen, dev)
        pos = torch.tensor([length], dtype=torch.int32, device=dev)

        def run(kcs=kcs, vts=vts, table=table, ws=ws, pos=pos):
            for kc, vt in zip(kcs, vts):
                K.attention_fused(qkv, Hq, Hkv, D, qn, kn, 1e-6, table, pos, kc, vt, D ** -0.5, ws)

        graph = capture(run)
        t_ms = min(time_replays(graph.replay, reps, 3)[0] for _ in range(2))
        del graph, kcs, vts, ws, table
        torch.cuda.empty_cache()
        us = t_ms * 1e3 / layers
        gbs = kv_bytes / (us * 1e-6) / 1e9
        out[length] = {"us_per_layer": round(us, 3), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                       "layers": layers}
    return out


def _synthetic_context(model, cache, length: int, g) -> None:
    """Fill `cache` as if `length` tokens had been decoded: random K/V rows and GDN states (the
    verify kernels' cost does not depend on the values), without running the prefill passes."""
    import torch

    from skinny_mlx.cache import KVCache

    sh = cache.shared
    sh.k_all.copy_((torch.randn(sh.k_all.shape, generator=g) * 0.5).to(torch.bfloat16))
    sh.vt_all.copy_((torch.randn(sh.vt_all.shape, generator=g) * 0.5).to(torch.bfloat16))
    if sh.gdn is not None:
        sh.gdn.state.copy_(torch.randn(sh.gdn.state.shape, generator=g) * 0.01)
        sh.gdn.conv.copy_(torch.randn(sh.gdn.conv.shape, generator=g).to(torch.bfloat16))
    for c in cache:
        if isinstance(c, KVCache):
            c.offset = length


VERIFY_MS = (1, 2, 4, 6, 8, 12, 16)  # the reference's step-cost protocol (bench/step_cost_curve.py:25)


def dense_bf16(model) -> None:
    """Every W4 linear of an unpatched model as a bf16 linear: its weights dequantised once
    (q*s + b in fp32, rounded to bf16) and multiplied by torch's bf16 GEMM on each call."""
    import torch

    from skinny_mlx import kernels as K
    from skinny_mlx.model import QuantizedLinear

    for mod in model.modules():
        if isinstance(mod, QuantizedLinear):
            wd = K.dequant(mod.weight, mod.scales, mod.biases).to(torch.bfloat16)
            mod.forward = lambda x, wd=wd: torch.nn.functional.linear(x.value() if isinstance(x, K.NormIn) else x, wd)


def verify_curve(dev, reps: int = 30, m_list=VERIFY_MS, preset: str = "dense-36", tree: bool = False,
                 synthetic: bool = False, mode: str = "skinny", context: int = 2048):
    """Captured forward of M tokens with `context` cached tokens (a draft tree of M nodes, branching
    4, 2, 1, with `tree`). `synthetic` fills the cache directly instead of running the prompt.
    `mode`: "skinny" the patched model; "fuse" the patched model with every projection on the
    unpatched kernels (SKINNY_RANGE off, fused projections kept: the reference's "+fuse" column);
    "stock" the unpatched model (fp32 dequantise + fp32 GEMM per linear, the "mlx" column);
    "bf16" the unpatched model with every linear's weights dequantised once to bf16 and multiplied
    by torch's bf16 GEMM (the model run unquantised: four times the weight bytes)."""
    import torch

    from skinny_mlx import patch as P
    from skinny_mlx.cache import KVCache, make_prompt_cache
    from skinny_mlx.graphs import CapturedStep
    from skinny_mlx.model import build_model
    from skinny_mlx.patch import patch_model
    from skinny_mlx.rollback import HybridRollback
    from skinny_mlx.spec import forward
    from skinny_mlx.tree import DraftTree

    model = build_model(preset)
    if mode == "bf16":
        dense_bf16(model)
    elif mode != "stock":
        patch_model(model)
    if FOLD_NORMS is not None:
        model.fold_norms = FOLD_NORMS
    saved_range = P.SKINNY_RANGE
    if mode == "fuse":
        P.SKINNY_RANGE = (99, 99)
    g = torch.Generator().manual_seed(0)
    cache = make_prompt_cache(model)
    if synthetic:
        _synthetic_context(model, cache, context, g)
    else:
        model(torch.randint(0, model.args.vocab_size, (context,), generator=g).tolist(), cache)
    torch.cuda.synchronize()
    rb = HybridRollback.for_model(model)
    ms = {}
    for m in m_list:
        ids = torch.randint(0, model.args.vocab_size, (m,), generator=g).to(torch.int32).to(dev)
        if tree:
            dt = DraftTree.from_branching((4, 2, 1), m, dev)
            rb.record()
            step = CapturedStep(lambda ids=ids, dt=dt: forward(model, ids, cache, dt), cache, m, recorded=m)
            model.recorder.recording = False
        else:
            if mode != "skinny":
                # one eager pass first: the torch GEMMs of the unpatched linears do first-call work
                # (hipBLASLt set-up) that a capture does not permit
                forward(model, ids, cache)
                for c in cache:
                    if isinstance(c, KVCache):
                        c.trim(m)
            step = CapturedStep(lambda ids=ids: forward(model, ids, cache), cache, m)

        def once(step=step, m=m):
            step()
            for c in cache:
                if isinstance(c, KVCache):
                    c.trim(m)  # stay at `context` cached tokens

        best = min(time_replays(once, reps, 5)[0] for _ in range(3))
        ms[m] = round(best, 4)
        del step
    P.SKINNY_RANGE = saved_range
    a = model.args
    layers = (f"{sum(a.is_linear(i) for i in range(a.num_hidden_layers))} Gated-DeltaNet + "
              f"{sum(not a.is_linear(i) for i in range(a.num_hidden_layers))} attention layers"
              if a.full_attention_interval else f"{a.num_hidden_layers} layers")
    heads = (f"GQA {a.num_attention_heads}q/{a.num_key_value_heads}kv x {a.head_dim}"
             + (f", RoPE over {a.rotary_dim} dims" if a.rotary_dim != a.head_dim else "")
             + (", sigmoid output gate" if a.attn_output_gate else ""))
    del model, cache
    torch.cuda.empty_cache()
    return {"workload": f"{preset} decoder ({layers}, hidden {a.hidden_size}, {heads}, SwiGLU {a.intermediate_size}, "
                        f"vocab {a.vocab_size}, W4 g64 linears), {context} cached tokens; one captured forward of M tokens"
                        + (" as a draft tree (branching 4, 2, 1)" if tree else "") + f"; {mode} linears",
            "ms": ms, "cost_vs_m1": {m: round(v / ms[1], 3) for m, v in ms.items()} if 1 in ms else None,
            "m8_over_m1": round(ms[8] / ms[1], 3) if 1 in ms and 8 in ms else None}


# The reference's step-cost table (README.md:16-21: Qwen3.5-4B 4-bit, 512-token context, Apple M4
# Max, the patched model's pipelined step), beside the same M on a random-init model of that shape.
QWEN35_MS = (1, 6, 8, 16)
REFERENCE_QWEN35_STEP = {"ms": {1: 8.70, 6: 13.18, 8: 14.80, 16: 29.22}, "cost_vs_m1_at_8": 1.70,
                         "hardware": "Apple M4 Max, MLX 0.32.1", "source": "README.md:16-21"}


# The reference's measured acceptance of its MTP head (tokens per verify step at K = 1..4: 1.93 /
# 2.51 / 3.05 / 3.47, docs/flatspec-design.md:65-66) is matched, for K = 2..4, by drafts that are
# each right with one probability p per position, independently: 1 + p + ... + p^K gives
# 2.51 / 3.07 / 3.54 at p = 0.827.
REFERENCE_DRAFT_P = 0.827


def calibrated_drafts(ref: list[int], p: float, vocab: int, seed: int = 0):
    """int32 [len(ref)]: the draft of every position of the greedy continuation `ref`, its own
    token with probability p (seeded, independent per position), else the next token id, which
    greedy verification always rejects."""
    import torch

    truth = torch.tensor(ref, dtype=torch.int64)
    keep = torch.rand(len(ref), generator=torch.Generator().manual_seed(seed)) < p
    return torch.where(keep, truth, (truth + 1) % vocab).to(torch.int32)


def calibrated_drafter(model, head, ref: list[int], p: float):
    """The MTP head at a given per-position acceptance p: each step runs the head's draft chain and
    its update as MTPDrafter does, so drafting costs what the head costs, then the proposals are
    replaced by calibrated_drafts of the greedy continuation `ref` at the positions they stand for
    (the on-device loop's token count). Tokens per step then follow 1 + p + ... + p^K, and the
    output is still greedy's."""
    import torch

    from skinny_mlx.spec import MTPDrafter

    class CalibratedDrafter(MTPDrafter):
        def __init__(self):
            super().__init__(model, head)
            self.table = calibrated_drafts(ref, p, model.args.vocab_size).to(model.device)

        def draft_into(self, toks, emitted):
            super().draft_into(toks, emitted)
            at = emitted.long() + torch.arange(toks.shape[0], device=toks.device)
            toks.copy_(self.table.index_select(0, at.clamp_(max=self.table.shape[0] - 1)))

    return CalibratedDrafter()


def spec_profile(dev, k: int, n_tokens: int) -> dict:
    """Speculative decoding alone on the hybrid decoder, the MTP head at the reference's acceptance,
    K drafts: the on-device loop, timed (its decode loop is the roctx range "skinny:decode_loop",
    which bounds a rocprofv3 --marker-trace kernel trace), then the host loop's profile mode for the
    time per phase (draft, verify, rollback, drafter update)."""
    import torch

    from skinny_mlx.model import build_model
    from skinny_mlx.mtp import load_mtp_head
    from skinny_mlx.patch import patch_model
    from skinny_mlx.spec import greedy, speculative

    model = build_model("hybrid-36")
    patch_model(model)
    head = load_mtp_head(model)
    prompt = torch.randint(0, model.args.vocab_size, (256,), generator=torch.Generator().manual_seed(0)).tolist()
    ref = greedy(model, prompt, n_tokens + 16)
    speculative(model, prompt, 32, calibrated_drafter(model, head, ref, REFERENCE_DRAFT_P), k)  # warm-up
    torch.cuda.synchronize()
    st = {}
    t = time.perf_counter()
    got = speculative(model, prompt, n_tokens, calibrated_drafter(model, head, ref, REFERENCE_DRAFT_P), k, st)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t
    pst = {}
    got2 = speculative(model, prompt, n_tokens, calibrated_drafter(model, head, ref, REFERENCE_DRAFT_P), k, pst,
                       profile=True)
    return {"workload": f"36-layer hybrid decoder, 256-token random prompt, {n_tokens} generated tokens, MTP K={k} "
                        f"at the reference's acceptance (p = {REFERENCE_DRAFT_P})",
            "tok_s": round(n_tokens / dt, 1), "decode_tok_s": st["decode_tok_s"], "steps": st["steps"],
            "tokens_per_step": round(st["tokens_per_step"], 3), "identical_to_greedy": got == ref[:n_tokens],
            "host_loop_ms_per_step": pst["ms_per_step"], "host_loop_identical_to_greedy": got2 == ref[:n_tokens]}


def spec_decode(dev, n_tokens: int):
    import torch

    from skinny_mlx.model import build_model
    from skinny_mlx.mtp import load_mtp_head
    from skinny_mlx.patch import patch_model
    from skinny_mlx.spec import MTPDrafter, greedy, speculative

    class ReplayDrafter:
        """Proposes the model's own greedy continuation (every draft accepted): from the host
        list, or in speculative's on-device loop by indexing the continuation at the device
        token count."""

        device_draft = True

        def __init__(self, ref):
            self.ref = ref
            self.ref_dev = torch.tensor(ref, dtype=torch.int64, device=dev)

        def begin(self, prompt, h, first):
            self.pos = 1

        def draft(self, k):
            return self.ref[self.pos:self.pos + k]

        def update(self, h_kept, new_tokens):
            self.pos += len(new_tokens)

        def device_caches(self):
            return []

        def device_start(self):
            pass

        def draft_into(self, toks, emitted):
            at = emitted.long() + torch.arange(toks.shape[0], device=dev)
            toks.copy_(self.ref_dev.index_select(0, at.clamp_(max=len(self.ref) - 1)))

        def commit(self, pred, h, result):
            pass

        def device_finish(self):
            pass

    model = build_model("hybrid-36")
    patch_model(model)
    if FOLD_NORMS is not None:
        model.fold_norms = FOLD_NORMS
    head = load_mtp_head(model)
    g = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, model.args.vocab_size, (256,), generator=g).tolist()

    def timed(fn, warmup=None):
        """(fn(), wall seconds); `warmup` (a short run of the same configuration) first, untimed,
        so that first-use costs of kernels and libraries stay out of the timed run."""
        if warmup is not None:
            warmup()
        torch.cuda.synchronize()
        t = time.perf_counter()
        out = fn()
        torch.cuda.synchronize()
        return out, time.perf_counter() - t

    greedy(model, prompt, 8)  # warm-up
    gst = {}
    ref, t_g = timed(lambda: greedy(model, prompt, n_tokens, stats=gst))
    _progress(f"greedy: {n_tokens / t_g:.1f} tok/s")
    res = {"workload": f"36-layer hybrid decoder (27 Gated-DeltaNet + 9 attention layers), 256-token random "
                       f"prompt, {n_tokens} generated tokens, greedy",
           "greedy_tok_s": round(n_tokens / t_g, 1), "greedy_decode_tok_s": gst["decode_tok_s"]}
    for k in (2, 3, 4):
        st = {}
        got, t = timed(lambda: speculative(model, prompt, n_tokens, MTPDrafter(model, head), k, st),
                       lambda: speculative(model, prompt, 16, MTPDrafter(model, head), k))
        res[f"mtp_k{k}"] = {"tok_s": round(n_tokens / t, 1), "decode_tok_s": st["decode_tok_s"],
                            "tokens_per_step": round(st["tokens_per_step"], 3), "identical_to_greedy": got == ref}
    full = greedy(model, prompt, n_tokens + 8)
    st = {}
    got, t = timed(lambda: speculative(model, prompt, n_tokens, ReplayDrafter(full), 3, st),
                   lambda: speculative(model, prompt, 16, ReplayDrafter(full), 3))
    res["replay_k3"] = {"tok_s": round(n_tokens / t, 1), "decode_tok_s": st["decode_tok_s"],
                        "tokens_per_step": round(st["tokens_per_step"], 3),
                        "identical_to_greedy": got == ref}
    for k in (2, 3, 4):
        st = {}
        got, t = timed(lambda: speculative(model, prompt, n_tokens, calibrated_drafter(model, head, full,
                                                                                       REFERENCE_DRAFT_P), k, st),
                       lambda: speculative(model, prompt, 16, calibrated_drafter(model, head, full, REFERENCE_DRAFT_P), k))
        res[f"mtp_at_reference_acceptance_k{k}"] = {
            "tok_s": round(n_tokens / t, 1), "decode_tok_s": st["decode_tok_s"],
            "tokens_per_step": round(st["tokens_per_step"], 3), "identical_to_greedy": got == ref,
            "speedup_vs_greedy": round(t_g / t, 3), "draft_p": REFERENCE_DRAFT_P}
    _progress("speculative decoding at the reference's acceptance done")
    for name, drafter in (("mtp_k3", lambda: MTPDrafter(model, head)), ("replay_k3", lambda: ReplayDrafter(full))):
        st = {}
        got, t = timed(lambda: speculative(model, prompt, n_tokens, drafter(), 3, st, device_loop=False),
                       lambda: speculative(model, prompt, 16, drafter(), 3, device_loop=False))
        res[f"{name}_host_loop"] = {"tok_s": round(n_tokens / t, 1), "tokens_per_step": round(st["tokens_per_step"], 3),
                                    "identical_to_greedy": got == ref}
    from skinny_mlx.sampling import sample, speculative_sample

    _, t = timed(lambda: sample(model, prompt, n_tokens, 1.0, seed=0), lambda: sample(model, prompt, 16, 1.0, seed=0))
    res["sample_T1_tok_s"] = round(n_tokens / t, 1)
    st = {}
    _, t = timed(lambda: speculative_sample(model, prompt, n_tokens, MTPDrafter(model, head), 3, 1.0, seed=0,
                                            stats=st),
                 lambda: speculative_sample(model, prompt, 16, MTPDrafter(model, head), 3, 1.0, seed=0))
    res["mtp_k3_T1"] = {"tok_s": round(n_tokens / t, 1), "tokens_per_step": round(st["tokens_per_step"], 3)}
    _progress("chain speculative decoding done")
    tree = tree_decode(model, head, prompt, ref, full, n_tokens, timed)
    del model, head
    torch.cuda.empty_cache()
    return res, tree


def tree_decode(model, head, prompt, ref, full, n_tokens, timed, reps: int = 30):
    """Draft-tree speculative decoding on the hybrid model: a 16-node tree (branching 4, 2, 1,
    depth 3 below the root) verified by one tree-masked M=16 forward per step."""
    import torch

    from skinny_mlx.cache import KVCache, make_prompt_cache
    from skinny_mlx.graphs import CapturedStep
    from skinny_mlx.rollback import HybridRollback
    from skinny_mlx.spec import forward
    from skinny_mlx.tree import DraftTree, MTPTreeDrafter, tree_speculative

    class ReplayTreeDrafter(MTPTreeDrafter):
        """The model's greedy continuation on the path through nodes 2, 7, 15 (a second-ranked
        branch at the first level), other tokens wrong: three drafts accepted per step. The
        tree is built on the host (draft_tree) or, in tree_speculative's on-device loop, from the
        device token count (tree_into) with the same tokens."""

        def __init__(self):
            super().__init__(model, head)
            self.on_path = {2, 7, 15}
            M, V = self.tree.size, model.args.vocab_size
            depth = torch.tensor(self.tree.depth, device=model.device)
            self.full_dev = torch.tensor(full, dtype=torch.int64, device=model.device)
            self.offset = (depth - 1).clamp(min=0)
            self.root = depth == 0
            self.on = torch.tensor([v in self.on_path for v in range(M)], device=model.device)
            self.wrong = torch.tensor([1 + v for v in range(M)], device=model.device)

        def device_caches(self):
            return []

        def device_start(self):
            pass

        def device_finish(self):
            pass

        def tree_into(self, tokens, emitted):
            true = self.full_dev.index_select(0, (emitted.long() + self.offset).clamp_(max=len(full) - 1))
            true = torch.where(self.root, torch.zeros_like(true), true)
            V = model.args.vocab_size
            tokens[1:].copy_(torch.where(self.on, true, (true + self.wrong) % V)[1:])

        def path_commit(self, pred, h, res):
            pass

        def begin(self, prompt, h, first):
            self.pos = 1

        def draft_tree(self):
            V = model.args.vocab_size
            toks = []
            for v in range(self.tree.size):
                d = self.tree.depth[v]
                true = full[self.pos + d - 1] if d > 0 else 0
                toks.append(true if v in self.on_path else (true + 1 + v) % V)
            return torch.tensor(toks, dtype=torch.int32, device=model.device)

        def update(self, h_kept, new_tokens):
            self.pos += len(new_tokens)

    res = {"workload": f"hybrid decoder of spec_decode, {n_tokens} generated tokens; 16-node draft tree "
                       "(branching 4, 2, 1) from MTP top-k, one tree-masked M=16 verify forward per step"}
    st = {}
    got, t = timed(lambda: tree_speculative(model, prompt, n_tokens, MTPTreeDrafter(model, head), st),
                   lambda: tree_speculative(model, prompt, 16, MTPTreeDrafter(model, head)))
    res["mtp_tree"] = {"tok_s": round(n_tokens / t, 1), "decode_tok_s": st["decode_tok_s"],
                       "tokens_per_step": round(st["tokens_per_step"], 3),
                       "identical_to_greedy": got == ref}
    st = {}
    got, t = timed(lambda: tree_speculative(model, prompt, n_tokens, ReplayTreeDrafter(), st),
                   lambda: tree_speculative(model, prompt, 16, ReplayTreeDrafter()))
    res["replay_tree"] = {"tok_s": round(n_tokens / t, 1), "decode_tok_s": st["decode_tok_s"],
                          "tokens_per_step": round(st["tokens_per_step"], 3),
                          "identical_to_greedy": got == ref}
    st = {}
    tree_speculative(model, prompt, 128, MTPTreeDrafter(model, head), st, profile=True)
    res["mtp_tree_phase_ms_per_step"] = st["ms_per_step"]

    # one captured tree verify forward (M = 16, recording) against one captured M = 1 forward
    cache = make_prompt_cache(model)
    forward(model, prompt, cache)
    rb = HybridRollback.for_model(model)
    tr = DraftTree.from_branching((4, 2, 1), 16, model.device)
    ids16 = torch.tensor(full[:16], dtype=torch.int32, device=model.device)
    ids1 = ids16[:1].clone()
    rb.record()
    s16 = CapturedStep(lambda: forward(model, ids16, cache, tr), cache, 16, recorded=16)
    model.recorder.recording = False
    s1 = CapturedStep(lambda: forward(model, ids1, cache), cache, 1)
    ms = {}
    for m, step in ((1, s1), (16, s16)):
        def once(step=step, m=m):
            step()
            for c in cache:
                if isinstance(c, KVCache):
                    c.trim(m)
        ms[m] = round(min(time_replays(once, reps, 5)[0] for _ in range(3)), 4)
    res["verify_ms"] = {"m1": ms[1], "tree_m16": ms[16], "tree_m16_over_m1": round(ms[16] / ms[1], 3)}
    del s1, s16, cache
    return res


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _host_threads() -> int:
    """Threads for the CPU leg: the cores this process may run on, capped by OMP_NUM_THREADS when it
    is set (a shared host's share for one GPU's job)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(n, 1)


def cpu_baseline(seconds: float):
    """The config-0 matmul (M=8, K=2560, N=9728, the same seeded CPU tensors the GPU gets) on the
    host cores with torch in fp32, standing in for MLX's CPU quantized_matmul (mlx is absent):
    (i) dequantise q*s + b to fp32 and matmul, per call, as a quantized matmul does on the fly;
    (ii) the matmul alone on weights dequantised ahead of time. ~`seconds` of calls per variant.
    `value` is (i), in the algorithmic GB/s of the GPU numbers."""
    import torch

    from skinny_mlx.qmm import random_w4g64

    m, k, n = CONFIG0
    threads = _host_threads()
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    w, s, b = random_w4g64(n, k, generator=g)
    x = torch.randn((m, k), generator=g).to(torch.bfloat16)
    shifts = torch.arange(0, 32, 4, dtype=torch.int32)

    def dequant():
        q = ((w.unsqueeze(-1) >> shifts) & 0xF).reshape(n, k // 64, 64).float()
        return (q * s.float().unsqueeze(-1) + b.float().unsqueeze(-1)).reshape(n, k)

    xf = x.float()
    wd = dequant()

    def timed(fn):
        fn()  # warm-up
        reps, t0 = 0, time.perf_counter()
        while True:
            fn()
            reps += 1
            if time.perf_counter() - t0 >= seconds:
                break
        return (time.perf_counter() - t0) / reps, reps

    t_i, r_i = timed(lambda: (xf @ dequant().t()).to(torch.bfloat16))
    t_ii, r_ii = timed(lambda: (xf @ wd.t()).to(torch.bfloat16))
    nbytes = qmm_bytes(m, k, n)
    return {"value": round(nbytes / t_i / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "ms_per_call": round(t_i * 1e3, 3),
            "matmul_only": {"GB/s": round(nbytes / t_ii / 1e9, 3), "ms_per_call": round(t_ii * 1e3, 3)},
            "sample": f"torch fp32 on the host, config-0 matmul M={m} K={k} N={n} W4 g64: dequantise + matmul per "
                      f"call ({r_i} calls in {seconds:.0f} s; value) and matmul only on pre-dequantised weights "
                      f"({r_ii} calls); {threads} threads",
            "cpu_model": _cpu_model(), "os_cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads()}


def _progress(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def main(argv=None) -> int:
    global FOLD_NORMS
    args = parse_args(argv)
    FOLD_NORMS = False if args.separate_norms else None
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported; this path runs on exactly one GPU "
              "(no multi-GPU sharding is built).", file=sys.stderr)
        return 2
    import torch

    dev = torch.device("cuda:0")
    if args.traffic_probe:
        traffic_probe(args, dev)
        return 0
    if args.spec_only:
        print(json.dumps({"spec_decode": spec_profile(dev, args.spec_only, args.spec_tokens)}), flush=True)
        return 0
    if args.verify_only:
        print(json.dumps({"verify_step": verify_curve(dev, args.steps, (args.verify_only,), args.verify_preset,
                                                      args.verify_tree, synthetic=True)}), flush=True)
        return 0
    gbs, ms, wall_ms, roofline, per_shape, chain, sweep = qmm_stack(args, dev)
    _progress(f"qmm stack: {gbs:.1f} GB/s over {args.streams} stream(s), {chain['GB/s']} GB/s as one chain")
    if args.stack_only:
        print(json.dumps({"value": round(gbs, 1), "unit": "GB/s", "m": args.m, "ms_per_step": round(ms, 4),
                          "streams": args.streams, "stack_chain": chain, "roofline": roofline,
                          "per_shape": per_shape}), flush=True)
        return 0
    config0 = qmm_config0(args, dev)
    _progress(f"config 0: {config0['us']} us, {config0['GB/s']} GB/s")
    library = library_gemm_shapes(dev, args.m, per_shape)
    _progress("bf16 library GEMM per shape: " + ", ".join(f"{s} {r['us']} us" for s, r in library["per_shape"].items()))
    roofline["ceiling"] = {"stream_read": stream_ceiling(dev)}
    _progress("streaming-read ceiling: " + ", ".join(
        f"{r['bytes'] / 1e6:.0f} MB {r['single']['GB/s']:.0f} / {r['graph']['GB/s']:.0f} GB/s"
        for r in roofline["ceiling"]["stream_read"]))
    roofline["decoder"] = decoder_roofline(args, dev)
    _progress("decoder gate|up: " + ", ".join(f"{f} {r['us_per_launch']} us {r['achieved']:.0f} GB/s"
                                             for f, r in roofline["decoder"]["forms"].items()))
    kv_ceiling = next(r for r in roofline["ceiling"]["stream_read"] if r["bytes"] == 8_388_608)
    roofline["attention"] = attention_roofline(dev, kv_ceiling)
    _progress("attention: " + ", ".join(f"M={m} {r['us_per_layer']} us/layer {r['GB/s']:.0f} GB/s"
                                        for m, r in roofline["attention"]["per_m"].items()))
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
        "config": {"workload": f"W4A16 g64 projection stack of a 36-layer hidden-2560 decoder at M={args.m} "
                               "(per layer fused QKV 2560x6144, o 4096x2560, fused gate+up 2560x19456, "
                               "down 9728x2560; plus lm_head 2560x151936), one HIP graph of 145 independent skinny "
                               f"qmm launches spread over {args.streams} stream(s)",
                   "tokens_per_step": args.m, "streams": args.streams},
        "roofline": roofline,
        "stack_frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
        "stack_chain": chain,
        "per_shape": per_shape,
        "config0": config0,
        "library_gemm_bf16": library,
        "stack_sweep": sweep,
    }
    if not args.no_model:
        vs = verify_curve(dev)
        _progress(f"verify step: M8/M1 = {vs['m8_over_m1']}")
        for mode in ("fuse", "stock"):
            c = verify_curve(dev, reps=10, mode=mode, synthetic=True)
            vs[mode] = {"ms": c["ms"], "cost_vs_m1": c["cost_vs_m1"],
                        "path": ("the unpatched linears: every W4 weight dequantised to fp32 and multiplied by a torch "
                                 "GEMM on each call (no quantized matmul kernel; not MLX's qmv/qmm, whose dead zone the "
                                 "reference measured, so it is no comparison for the skinny kernels)"
                                 + ("; projections fused as patch_model fuses them" if mode == "fuse" else ""))}
        c = verify_curve(dev, reps=30, mode="bf16", synthetic=True)
        vs["bf16"] = {"ms": c["ms"], "cost_vs_m1": c["cost_vs_m1"],
                      "skinny_speedup": {m: round(c["ms"][m] / vs["ms"][m], 3) for m in c["ms"]},
                      "path": ("the model run unquantised: every linear's weights dequantised once to bf16 (four "
                               "times the W4 bytes) and multiplied by torch's bf16 GEMM on each call; the same "
                               "captured step and kernels otherwise")}
        vs["protocol"] = ("best of 3 x reps replays of one captured forward per M; skinny: 30 replays over a real "
                          "2048-token prefill; fuse and stock: 10 replays over a synthetic 2048-token cache (the step "
                          "cost does not depend on the cached values)")
        out["verify_step"] = vs
        _progress(f"stock verify curve: M8/M1 = {vs['stock']['cost_vs_m1'][8]}")
        q35 = verify_curve(dev, 20, QWEN35_MS, "qwen35-4b", synthetic=True, context=512)
        q35["reference_m4_max"] = REFERENCE_QWEN35_STEP
        out["verify_step_qwen35_shape"] = q35
        _progress(f"Qwen3.5-4B-shaped verify step: {q35['ms']}")
        out["spec_decode"], out["tree_decode"] = spec_decode(dev, args.spec_tokens)
        _progress("spec and tree decode done")
    if not args.no_cpu:
        cb = cpu_baseline(args.cpu_seconds)
        cb["gpu_speedup_config0"] = round(config0["GB/s"] / cb["value"], 1)
        out["cpu_baseline"] = cb
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
