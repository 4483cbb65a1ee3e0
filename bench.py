"""Benchmark of the flat-cost speculative-verify path on one MI355X.

Default run (`python bench.py`): prints ONE JSON line.

  value     the W4 g64 projection stack of a 36-layer hidden-2560 decoder at M=8 tokens: per
            layer fused QKV (2560->6144), o_proj (4096->2560), fused gate+up (2560->19456),
            down (9728->2560), plus the lm_head (2560->151936) — 145 skinny qmm launches over
            2.29 GB of weights, replayed as one HIP graph with everything resident in HBM (far
            beyond the 256 MB Infinity Cache). value = algorithmic bytes of the step (packs +
            scales + biases + activations in + out) / measured step time, in GB/s.
  roofline  the dominant kernel (the fused gate+up shape, 36 launches per step), timed with HIP
            events on the launch stream over back-to-back launches of its 36 weight sets.
  verify_step  a random-init 36-layer dense decoder (hidden 2560, GQA 32q/8kv x 128, SwiGLU 9728,
            W4 g64 linears, vocab 151936) with 2048 cached tokens: one captured forward of M
            tokens for M in {1, 2, 4, 6, 8, 16}, its ms and the cost relative to M = 1.
  spec_decode  the hybrid model (3 Gated-DeltaNet layers per attention layer), 256-token uniform
            random prompt, 512 generated tokens: greedy tok/s, and speculative tok/s with the
            random-init MTP head (K = 2, 3, 4; random weights draft almost nothing acceptable),
            and with a replay drafter that proposes the model's own greedy continuation (the
            acceptance upper bound; K = 3). Every greedy run is checked token for token against
            greedy decoding. At temperature 1: plain sampled decoding, and speculative decoding with
            rejection sampling (MTP K = 3).
  tree_decode  the same model and prompt with a 16-node draft tree (branching 4, 2, 1) verified
            in one tree-masked M=16 forward per step: tok/s and tokens/step with the MTP head's
            top-k tree and with a replay tree (greedy continuation along a second-ranked branch),
            the per-phase ms of a step, and the captured tree verify forward vs an M=1 forward.
  cpu_baseline  the oracle's numpy dequant+matmul (fp64) of the M=8, K=2560, N=9728 matmul, a
            bounded sample on the host cores.

Options: --gpus N (only 1: this path runs on one GPU), --steps K, --warmup W, --m M,
--no-model (qmm stack only), --no-cpu, --cpu-seconds S, --spec-tokens N, --verify-only M (just the
captured M-token verify forward, K replays over a synthetic 2048-token cache: a clean trace for
profiling; --verify-preset hybrid-36 and --verify-tree select the model and a draft tree).
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
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16


def qmm_bytes(m: int, k: int, n: int) -> int:
    """Algorithmic bytes of one call: packs + scales + biases + x in + y out."""
    return n * k // 2 + 4 * n * (k // 64) + 2 * m * k + 2 * m * n


FOLD_NORMS = False  # --fold-norms: RMSNorms inside the stack folded into the matmuls (Model.fold_norms)


def parse_args(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--m", type=int, default=8)
    ap.add_argument("--no-model", action="store_true", help="only the qmm stack")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--spec-tokens", type=int, default=512)
    ap.add_argument("--verify-only", type=int, default=0, metavar="M",
                    help="only the captured M-token verify forward, over a synthetic 2048-token cache (for profiling)")
    ap.add_argument("--verify-preset", default="dense-36", help="model of --verify-only (dense-36 or hybrid-36)")
    ap.add_argument("--verify-tree", action="store_true", help="--verify-only as a draft tree (branching 4, 2, 1)")
    ap.add_argument("--fold-norms", action="store_true",
                    help="fold the RMSNorms inside the stack into the matmuls around them (Model.fold_norms)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="for rocprofv3 --pmc: one launch of the dominant qmm on each of its 36 weight sets, "
                         "then a 64 MiB device copy and a 64 MiB streaming read as calibration kernels")
    return ap.parse_args(argv)


def traffic_probe(args, dev) -> None:
    """Kernels whose hardware counters (FETCH_SIZE, WRITE_SIZE) give the dominant kernel's HBM
    traffic: 36 launches of the M x 2560 x 19456 qmm on distinct weight sets (2 passes), then the
    calibration kernels of known traffic."""
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
    src = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    red = torch.empty(1024, dtype=torch.float32, device=dev)
    _lib.check(_lib.lib().skinny_stream_read(src.data_ptr(), src.numel(), red.data_ptr(), 1024, _lib.stream_of(src)),
               "stream_read")
    torch.cuda.synchronize()
    print(json.dumps({"traffic_probe": {"qmm": [args.m, k, n], "launches": 2 * LAYERS,
                                        "algorithmic_bytes_per_launch": qmm_bytes(args.m, k, n),
                                        "calibration_bytes": 64 << 20}}), flush=True)


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
        for _ in range(LAYERS):
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


def qmm_stack(args, dev):
    from skinny_mlx import qmm as Q

    m = args.m
    stack = Stack(m, dev)
    graph = capture(stack.run)
    ms, wall_ms = time_replays(graph.replay, args.steps, args.warmup)
    gbs = stack.bytes / (ms * 1e-3) / 1e9
    per_shape = {}
    dom = None
    for k, n in LAYER_SHAPES + [HEAD_SHAPE]:
        gr = capture(lambda k=k, n=n: stack.run(select=(k, n)))
        count = LAYERS if (k, n) != HEAD_SHAPE else 1
        reps = max(args.steps, 20) if count > 1 else max(args.steps, 200)
        sms, _ = time_replays(gr.replay, reps, args.warmup)
        us = sms * 1e3 / count
        per_shape[f"{k}x{n}"] = {"us": round(us, 3), "GB/s": round(qmm_bytes(m, k, n) / (us * 1e-6) / 1e9, 1),
                                 "tile": list(Q.config_for(m, k, n))}
        if (k, n) == LAYER_SHAPES[2]:
            dom = (k, n, us)
        del gr
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
    del stack, graph
    return gbs, ms, wall_ms, roofline, per_shape


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


def verify_curve(dev, reps: int = 30, m_list=(1, 2, 4, 6, 8, 16), preset: str = "dense-36", tree: bool = False,
                 synthetic: bool = False):
    """Captured forward of M tokens with 2048 cached tokens (a draft tree of M nodes, branching
    4, 2, 1, with `tree`). `synthetic` fills the cache directly instead of running the prompt."""
    import torch

    from skinny_mlx.cache import KVCache, make_prompt_cache
    from skinny_mlx.graphs import CapturedStep
    from skinny_mlx.model import build_model
    from skinny_mlx.patch import patch_model
    from skinny_mlx.rollback import HybridRollback
    from skinny_mlx.spec import forward
    from skinny_mlx.tree import DraftTree

    model = build_model(preset)
    patch_model(model)
    model.fold_norms = FOLD_NORMS
    g = torch.Generator().manual_seed(0)
    cache = make_prompt_cache(model)
    if synthetic:
        _synthetic_context(model, cache, 2048, g)
    else:
        model(torch.randint(0, model.args.vocab_size, (2048,), generator=g).tolist(), cache)
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
            step = CapturedStep(lambda ids=ids: forward(model, ids, cache), cache, m)

        def once(step=step, m=m):
            step()
            for c in cache:
                if isinstance(c, KVCache):
                    c.trim(m)  # stay at 2048 cached tokens

        best = min(time_replays(once, reps, 5)[0] for _ in range(3))
        ms[m] = round(best, 4)
        del step
    del model, cache
    torch.cuda.empty_cache()
    return {"workload": f"{preset} decoder (hidden 2560, GQA 32q/8kv x 128, SwiGLU 9728, vocab 151936, W4 g64 "
                        f"linears), 2048 cached tokens; one captured forward of M tokens"
                        + (" as a draft tree (branching 4, 2, 1)" if tree else ""),
            "ms": ms, "cost_vs_m1": {m: round(v / ms[1], 3) for m, v in ms.items()} if 1 in ms else None,
            "m8_over_m1": round(ms[8] / ms[1], 3) if 1 in ms and 8 in ms else None}


def spec_decode(dev, n_tokens: int):
    import torch

    from skinny_mlx.model import build_model
    from skinny_mlx.mtp import load_mtp_head
    from skinny_mlx.patch import patch_model
    from skinny_mlx.spec import MTPDrafter, greedy, speculative

    class ReplayDrafter:
        """Proposes the model's own greedy continuation (every draft accepted)."""

        def __init__(self, ref):
            self.ref = ref

        def begin(self, prompt, h, first):
            self.pos = 1

        def draft(self, k):
            return self.ref[self.pos:self.pos + k]

        def update(self, h_kept, new_tokens):
            self.pos += len(new_tokens)

    model = build_model("hybrid-36")
    patch_model(model)
    model.fold_norms = FOLD_NORMS
    head = load_mtp_head(model)
    g = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, model.args.vocab_size, (256,), generator=g).tolist()

    def timed(fn):
        torch.cuda.synchronize()
        t = time.perf_counter()
        out = fn()
        torch.cuda.synchronize()
        return out, time.perf_counter() - t

    greedy(model, prompt, 8)  # warm-up
    ref, t_g = timed(lambda: greedy(model, prompt, n_tokens))
    _progress(f"greedy: {n_tokens / t_g:.1f} tok/s")
    res = {"workload": f"36-layer hybrid decoder (27 Gated-DeltaNet + 9 attention layers), 256-token random "
                       f"prompt, {n_tokens} generated tokens, greedy",
           "greedy_tok_s": round(n_tokens / t_g, 1)}
    for k in (2, 3, 4):
        st = {}
        got, t = timed(lambda: speculative(model, prompt, n_tokens, MTPDrafter(model, head), k, st))
        res[f"mtp_k{k}"] = {"tok_s": round(n_tokens / t, 1), "tokens_per_step": round(st["tokens_per_step"], 3),
                            "identical_to_greedy": got == ref}
    full = greedy(model, prompt, n_tokens + 8)
    st = {}
    got, t = timed(lambda: speculative(model, prompt, n_tokens, ReplayDrafter(full), 3, st))
    res["replay_k3"] = {"tok_s": round(n_tokens / t, 1), "tokens_per_step": round(st["tokens_per_step"], 3),
                        "identical_to_greedy": got == ref}
    from skinny_mlx.sampling import sample, speculative_sample

    _, t = timed(lambda: sample(model, prompt, n_tokens, 1.0, seed=0))
    res["sample_T1_tok_s"] = round(n_tokens / t, 1)
    st = {}
    _, t = timed(lambda: speculative_sample(model, prompt, n_tokens, MTPDrafter(model, head), 3, 1.0, seed=0,
                                            stats=st))
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
        branch at the first level), other tokens wrong: three drafts accepted per step."""

        def __init__(self):
            super().__init__(model, head, graphs=False)
            self.on_path = {2, 7, 15}

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
    got, t = timed(lambda: tree_speculative(model, prompt, n_tokens, MTPTreeDrafter(model, head), st))
    res["mtp_tree"] = {"tok_s": round(n_tokens / t, 1), "tokens_per_step": round(st["tokens_per_step"], 3),
                       "identical_to_greedy": got == ref}
    st = {}
    got, t = timed(lambda: tree_speculative(model, prompt, n_tokens, ReplayTreeDrafter(), st))
    res["replay_tree"] = {"tok_s": round(n_tokens / t, 1), "tokens_per_step": round(st["tokens_per_step"], 3),
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


def _progress(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def main(argv=None) -> int:
    global FOLD_NORMS
    args = parse_args(argv)
    FOLD_NORMS = args.fold_norms
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported; this path runs on exactly one GPU "
              "(no multi-GPU sharding is built).", file=sys.stderr)
        return 2
    import torch

    dev = torch.device("cuda:0")
    if args.traffic_probe:
        traffic_probe(args, dev)
        return 0
    if args.verify_only:
        print(json.dumps({"verify_step": verify_curve(dev, args.steps, (args.verify_only,), args.verify_preset,
                                                      args.verify_tree, synthetic=True)}), flush=True)
        return 0
    gbs, ms, wall_ms, roofline, per_shape = qmm_stack(args, dev)
    _progress(f"qmm stack: {gbs:.1f} GB/s")
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
                               "down 9728x2560; plus lm_head 2560x151936), one HIP graph of 145 skinny qmm launches",
                   "tokens_per_step": args.m},
        "roofline": roofline,
        "stack_frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
        "per_shape": per_shape,
    }
    if not args.no_model:
        out["verify_step"] = verify_curve(dev)
        _progress(f"verify step: M8/M1 = {out['verify_step']['m8_over_m1']}")
        out["spec_decode"], out["tree_decode"] = spec_decode(dev, args.spec_tokens)
        _progress("spec and tree decode done")
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
