"""Greedy-exact speculative decoding on one GPU, with pluggable drafters.

Call surface kept from the reference (skinny_mlx/spec.py:24-156): `forward`,
`PromptLookupDrafter`, `MTPDrafter` (begin / draft / update), `greedy`, and
`speculative(model, prompt, max_tokens, drafter, k, stats=None, profile=False)`.

One step: the verify forward scores [last emitted token] + K drafts (M = K + 1) in one pass;
the device takes the first-index argmax of every row and the longest prefix where the drafts
match it (the acceptance kernel); the host reads the fed tokens, the predictions and
(n accepted, bonus, keep) back in ONE copy into pinned memory — the step's only
synchronisation, like the reference's single mx.eval (spec.py:138); the cache is rolled back
to the accepted prefix (skinny_mlx.rollback) and the drafter is told what was kept.

Exactness: every kernel on the path computes a token's row without regard to how many rows
share the pass (the skinny qmm's tile depends on (K, N) only; norms, attention and the
recurrence are per row), so the emitted tokens equal plain greedy decoding token for token.
(The reference gets this only up to near-ties between its M=1 and M>1 kernels, spec.py:5-6.)

Steps run as captured HIP graphs by default (`graphs=True`; skinny_mlx.graphs): the decode
step, each verify size, the MTP draft chain and each MTP update size are captured once per
generation and replayed, so the host issues a handful of calls per step instead of hundreds of
launches. `graphs=False` runs the same kernels eagerly.

With a drafter that drafts on the device (MTPDrafter; `device_draft`) the loop itself moves to
the device: one captured graph holds the whole step — drafts, verify, acceptance, the rollback
of the GDN state and of every cache length (skinny_spec_commit, skinny_spec_select_row), the
append of the emitted tokens to a device buffer and the drafter's update — and is replayed back
to back; the host reads the token count once per batch of the fewest steps that can finish.
The tokens, steps and acceptances are the host loop's (`device_loop=False`), which stays the
path for host drafters (prompt lookup) and for `profile`.

Tensors are 2-D ([T, ...]); the reference's leading batch dimension of 1 is dropped.
"""

from __future__ import annotations

import sys
import time

import torch

from . import kernels as K
from .cache import make_prompt_cache
from .graphs import CapturedStep, capture_graph
from .rollback import HybridRollback


class PinnedIds:
    """Host token lists to device int32 without a blocking copy: the list goes into a pinned
    staging buffer, then an asynchronous copy (a copy from pageable memory would hold the host
    until the device had drained). The buffer is refilled only after the copy that last read it
    has completed."""

    def __init__(self, capacity: int):
        self.host = torch.empty((max(capacity, 1),), dtype=torch.int32, pin_memory=True)
        self.event = None

    def upload(self, tokens, out: torch.Tensor) -> torch.Tensor:
        k = len(tokens)
        if k > self.host.numel():
            self.host = torch.empty((2 * k,), dtype=torch.int32, pin_memory=True)
            self.event = None
        if self.event is not None:
            self.event.synchronize()
        self.host[:k] = torch.tensor([int(t) for t in tokens], dtype=torch.int32)
        out[:k].copy_(self.host[:k], non_blocking=True)
        self.event = torch.cuda.Event()
        self.event.record()
        return out


def forward(model, ids, cache, tree=None):
    """(final normed hidden [T, H], logits [T, V]) for tokens `ids`: a list of ints, or an int32
    GPU tensor (drafted tokens then flow into the verify pass without a host round trip).
    `tree` (skinny_mlx.tree.DraftTree) verifies the tokens as a draft tree."""
    h = model.hidden(ids, cache, tree)
    return h, model.logits(h)


class PromptLookupDrafter:
    """Model-free drafting from the context itself: find the latest earlier occurrence of the
    trailing n-gram (n = ngram, ngram-1, ..., 1) and propose the tokens that followed it — the
    reference's search order (spec.py:41-48). Instead of re-scanning the context per draft,
    an index per n maps each n-gram to its latest start among the starts eligible so far
    (start <= len(ctx) - n - 1); it is extended incrementally as tokens are accepted."""

    def __init__(self, ngram: int = 3):
        if ngram < 1:
            raise ValueError("ngram must be >= 1")
        self.ngram = ngram

    def begin(self, prompt, h, first):
        self.ctx = [int(t) for t in prompt] + [int(first)]
        self._latest = {n: {} for n in range(1, self.ngram + 1)}
        self._next_start = {n: 0 for n in range(1, self.ngram + 1)}

    def _extend_index(self) -> None:
        ctx = self.ctx
        for n, table in self._latest.items():
            stop = len(ctx) - n  # starts 0 .. len - n - 1 may match
            for s in range(self._next_start[n], stop):
                table[tuple(ctx[s:s + n])] = s
            self._next_start[n] = max(self._next_start[n], stop)

    def draft(self, k: int) -> list[int]:
        self._extend_index()
        ctx = self.ctx
        for n in range(self.ngram, 0, -1):
            s = self._latest[n].get(tuple(ctx[len(ctx) - n:]))
            if s is not None:
                return ctx[s + n:s + n + k]
        return []

    def update(self, h_kept, new_tokens):
        self.ctx.extend(int(t) for t in new_tokens)


class MTPDrafter:
    """Drafts with the model's MTP head (skinny_mlx.mtp), chained K times on the device.

    The head keeps its own KV cache: `begin` runs it over the prompt (token i+1 paired with the
    target's hidden state of token i), `draft` chains it on its own outputs, and `update` drops
    the chain's K-1 speculative entries and re-runs it on the accepted tokens paired with the
    target's hidden states (reference protocol: spec.py:74-95). Drafts are scored over token
    ids [0, vocab) only — the first `vocab` rows of the model's W4 head, a prefix of its packed
    buffer — while verify scores the full head, so the output is unchanged and only acceptance
    can drop (the reference's pruning, spec.py:57-66). With `graphs`, the chain of each K and the
    update of each length are captured per generation and replayed."""

    def __init__(self, model, head, vocab: int | None = 32768, graphs: bool = True):
        self.model, self.head, self.graphs = model, head, graphs
        V = model.args.vocab_size
        self.vocab = V if vocab is None else min(vocab, V)
        lm = model.lm_head
        packed = getattr(lm, "rweight", None)
        if packed is not None and self.vocab % 16 == 0:
            self._score = self._packed_scorer(packed[:self.vocab])
        else:
            w, s, b = lm.weight[:self.vocab], lm.scales[:self.vocab], lm.biases[:self.vocab]
            self._score = lambda h: K.quantized_matmul(h, w, s, b)
        self.cache = None
        self.n_spec = 0
        self._stage = PinnedIds(64)

    @staticmethod
    def _packed_scorer(rows: torch.Tensor):
        from .qmm import skinny_qmm

        return lambda h: skinny_qmm(h, rows)

    def _run_head(self, tokens: torch.Tensor, hidden: torch.Tensor) -> torch.Tensor:
        return self.head.forward_tokens(tokens, self.model.embed_tokens, hidden, self.cache)

    def _ids(self, tokens) -> torch.Tensor:
        return torch.tensor([int(t) for t in tokens], dtype=torch.int32, device=self.model.device)

    def begin(self, prompt, h, first):
        from .mtp import make_mtp_cache

        self.cache = make_mtp_cache(self.head)
        self._chains, self._updates = {}, {}
        ids = self._ids(list(prompt[1:]) + [int(first)])
        step = self.model.args.max_step_tokens
        last = None
        for i in range(0, ids.shape[0], step):
            last = self._run_head(ids[i:i + step], h[i:i + step])
        self.h_last = last[-1:]
        self.n_spec = 0

    def _chain(self, h0: torch.Tensor, toks: torch.Tensor) -> torch.Tensor:
        h = h0
        k = toks.shape[0]
        for i in range(k):
            K.argmax_rows(self._score(h), out=toks[i:i + 1])
            if i + 1 < k:
                h = self._run_head(toks[i:i + 1], h)
        return toks

    def draft(self, k: int) -> torch.Tensor:
        self.n_spec = max(k - 1, 0)
        dev = self.model.device
        if not self.graphs:
            return self._chain(self.h_last, torch.empty((k,), dtype=torch.int32, device=dev))
        g = self._chains.get(k)
        if g is None:
            h0 = torch.empty_like(self.h_last)
            toks = torch.empty((k,), dtype=torch.int32, device=dev)
            g = (h0, CapturedStep(lambda: self._chain(h0, toks), self.cache, max(k - 1, 0)))
            self._chains[k] = g
        h0, step = g
        h0.copy_(self.h_last)
        return step()

    def _chain_sampled(self, h0, toks, rows, temperature, seed, counter):
        h = h0
        k = toks.shape[0]
        for i in range(k):
            rows[i:i + 1].copy_(self._score(h))
            K.sample_rows(rows[i:i + 1], temperature, seed, counter, offset=i, rng_stream=1, out=toks[i:i + 1])
            if i + 1 < k:
                h = self._run_head(toks[i:i + 1], h)
        return toks, rows

    def draft_sampled(self, k: int, temperature: float, seed: int, counter: torch.Tensor):
        """Sampled drafts for rejection sampling at temperature T: draft i is drawn from
        softmax(scores_i / T) over the pruned vocabulary (counter *counter + i, stream 1), and its
        score row is kept as the draft distribution. Returns (tokens int32 [k], scores bf16 [k, V'])."""
        self.n_spec = max(k - 1, 0)
        dev = self.model.device
        H = self.h_last.shape[-1]
        if not self.graphs:
            return self._chain_sampled(self.h_last, torch.empty((k,), dtype=torch.int32, device=dev),
                                       torch.empty((k, self.vocab), dtype=torch.bfloat16, device=dev),
                                       temperature, seed, counter)
        key = ("sampled", k, temperature, seed, counter.data_ptr())
        g = self._chains.get(key)
        if g is None:
            h0 = torch.empty((1, H), dtype=self.h_last.dtype, device=dev)
            toks = torch.empty((k,), dtype=torch.int32, device=dev)
            rows = torch.empty((k, self.vocab), dtype=torch.bfloat16, device=dev)
            g = (h0, CapturedStep(lambda: self._chain_sampled(h0, toks, rows, temperature, seed, counter), self.cache,
                                  max(k - 1, 0)))
            self._chains[key] = g
        h0, step = g
        h0.copy_(self.h_last)
        return step()

    # The same protocol for the on-device loop of `speculative` (device_draft): the chain and the
    # update run inside the loop's captured step, and the head's hidden state and cache length
    # stay on the device between steps. A drafter built with graphs=False keeps the host loop.
    @property
    def device_draft(self) -> bool:
        return self.graphs

    def device_caches(self) -> list:
        return [self.cache]

    def device_start(self) -> None:
        """Before the step is captured: the last accepted hidden state into a static buffer."""
        self._h_dev = self.h_last.contiguous().clone()

    def draft_into(self, toks: torch.Tensor, emitted: torch.Tensor) -> None:
        """Captured: the chain of len(toks) drafts from the buffered hidden state into toks, then
        the head cache back to its length before the chain (what `update` trims first)."""
        k = toks.shape[0]
        self._chain(self._h_dev, toks)
        if k > 1:
            sh = self.cache.shared
            sh.pos.add_(-(k - 1))
            for c in self.cache:
                c.trim(k - 1)
            sh.dev_pos -= k - 1

    def commit(self, pred: torch.Tensor, h: torch.Tensor, result: torch.Tensor) -> None:
        """Captured: `update` on the device. The head runs over all fed rows, pred[j] paired with
        h[j]; the first keep = result[2] are the emitted tokens (accepted drafts equal their
        predictions, then the bonus) with their verify hidden states, exactly update's input.
        The cache then keeps those rows and the last kept output starts the next chain."""
        out = self._run_head(pred, h)
        K.spec_select_row(result, self.cache.shared.pos, out, self._h_dev)

    def device_finish(self) -> None:
        self.h_last = self._h_dev
        self.n_spec = 0

    def update(self, h_kept, new_tokens):
        for c in self.cache:
            c.trim(self.n_spec)
        self.n_spec = 0
        n = len(new_tokens)
        if not self.graphs:
            ids = self._stage.upload(new_tokens, torch.empty((n,), dtype=torch.int32, device=self.model.device))
            self.h_last = self._run_head(ids, h_kept.contiguous())[-1:]
            return
        g = self._updates.get(n)
        if g is None:
            ids_buf = torch.empty((n,), dtype=torch.int32, device=self.model.device)
            h_buf = torch.empty((n, h_kept.shape[-1]), dtype=h_kept.dtype, device=self.model.device)
            g = (ids_buf, h_buf, CapturedStep(lambda: self._run_head(ids_buf, h_buf)[-1:], self.cache, n))
            self._updates[n] = g
        ids_buf, h_buf, step = g
        self._stage.upload(new_tokens, ids_buf)
        h_buf.copy_(h_kept)
        self.h_last = step()


def _last_argmax(logits: torch.Tensor) -> torch.Tensor:
    return K.argmax_rows(logits[-1:])


def greedy(model, prompt: list[int], max_tokens: int, graphs: bool = True, stats: dict | None = None) -> list[int]:
    """Plain greedy decoding, one token per forward (reference spec.py:98-107). Each step's
    argmax feeds the next step on the device — with `graphs`, the captured step writes it
    straight into its own input — and the tokens are read back once at the end. `stats`, when
    given, receives the decode loop's own time (after the prompt and the step's capture)."""
    cache = make_prompt_cache(model)
    toks = torch.empty((max(max_tokens, 1),), dtype=torch.int32, device=model.device)
    toks[:1].copy_(_last_argmax(model(prompt, cache)))
    clock = _LoopClock(stats)
    if graphs and max_tokens > 1:
        cur = toks[:1].clone()
        step = CapturedStep(lambda: K.argmax_rows(model(cur, cache)[-1:], out=cur), cache, 1)
        clock.start()
        for i in range(1, max_tokens):
            step()
            toks[i:i + 1].copy_(cur)
    else:
        clock.start()
        for i in range(1, max_tokens):
            toks[i:i + 1].copy_(_last_argmax(model(toks[i - 1:i], cache)))
    out = toks[:max_tokens].tolist()
    clock.stop(max(max_tokens - 1, 0))
    return out


class _LoopClock:
    """Wall time of a decode loop alone (the prompt pass and graph captures before it excluded):
    stats["decode_ms"] and stats["decode_tok_s"] over the tokens the loop produced, the loop also a
    roctx range ("skinny:decode_loop") for rocprofv3's marker trace. Synchronises once at the start,
    and only when stats are asked for."""

    def __init__(self, stats: dict | None):
        self.stats, self.t = stats, 0.0

    def start(self):
        if self.stats is not None:
            torch.cuda.synchronize()
            self.t = time.perf_counter()
            torch.cuda.nvtx.range_push("skinny:decode_loop")

    def stop(self, tokens: int):
        if self.stats is not None:
            torch.cuda.synchronize()
            torch.cuda.nvtx.range_pop()
            dt = time.perf_counter() - self.t
            self.stats["decode_ms"] = round(dt * 1e3, 3)
            self.stats["decode_tok_s"] = round(tokens / dt, 1) if dt > 0 else 0.0


class _PhaseClock:
    """Per-phase wall time; synchronises at phase boundaries only when enabled. Each phase is
    also a roctx range ("skinny:<phase>", through torch.cuda.nvtx) for rocprofv3's marker trace.
    The phases run in PHASES order (reference spec.py:112-121, 133-149)."""

    PHASES = ("draft", "verify", "rollback", "drafter update")

    def __init__(self, enabled: bool):
        self.enabled = enabled
        self.total = dict.fromkeys(self.PHASES, 0.0)
        self.t = 0.0
        self.open = False

    def _enter(self, phase: str):
        torch.cuda.nvtx.range_push(f"skinny:{phase}")
        self.open = True

    def _leave(self):
        if self.open:
            torch.cuda.nvtx.range_pop()
            self.open = False

    def start(self):
        if self.enabled:
            torch.cuda.synchronize()
            self._leave()
            self.t = time.perf_counter()
            self._enter(self.PHASES[0])

    def lap(self, phase: str):
        if self.enabled:
            torch.cuda.synchronize()
            now = time.perf_counter()
            self.total[phase] += now - self.t
            self.t = now
            self._leave()
            nxt = self.PHASES.index(phase) + 1
            if nxt < len(self.PHASES):
                self._enter(self.PHASES[nxt])


def speculative(model, prompt: list[int], max_tokens: int, drafter, k: int,
                stats: dict | None = None, profile: bool = False, graphs: bool = True,
                device_loop: bool | None = None) -> list[int]:
    """Greedy-exact speculative decoding. profile=True synchronises at phase boundaries and adds
    per-phase ms/step to `stats`. A drafter that drafts on the device (`device_draft`, e.g.
    MTPDrafter) runs the on-device loop by default (`device_loop`; needs graphs and no profile):
    the same tokens, steps and acceptances, without a host round trip per step."""
    if device_loop is None:
        device_loop = graphs and not profile and getattr(drafter, "device_draft", False)
    if device_loop:
        if not (graphs and not profile and getattr(drafter, "device_draft", False)):
            raise ValueError("the on-device loop needs graphs=True, profile=False and a device drafter")
        return _speculative_on_device(model, prompt, max_tokens, drafter, k, stats)
    dev = model.device
    clock = _PhaseClock(profile)
    cache = make_prompt_cache(model)
    rollback = HybridRollback.for_model(model)
    h, logits = forward(model, prompt, cache)
    out = [int(_last_argmax(logits).item())]
    drafter.begin(prompt, h, out[0])

    result = torch.empty((3,), dtype=torch.int32, device=dev)       # n, bonus, keep
    host = torch.empty((2 * (k + 1) + 3,), dtype=torch.int32, pin_memory=True)
    stage = PinnedIds(k)
    done = torch.cuda.Event()
    verify = {}  # fed -> (token buffer, captured step or None)

    def verify_pass(x: torch.Tensor):
        h, logits = forward(model, x, cache)
        pred = K.argmax_rows(logits)
        K.accept(pred, x[1:] if x.shape[0] > 1 else None, result)
        return h, pred

    steps = accepted = 0
    try:
        while len(out) < max_tokens:
            clock.start()
            d = drafter.draft(k)
            nd = int(d.numel()) if isinstance(d, torch.Tensor) else len(d)
            fed = nd + 1
            if fed not in verify:
                buf = torch.empty((fed,), dtype=torch.int32, device=dev)
                verify[fed] = [buf, None]
            x, captured = verify[fed]
            x[:1].fill_(out[-1])
            if nd:
                if isinstance(d, torch.Tensor):
                    x[1:].copy_(d)
                else:
                    stage.upload(d, x[1:])
            clock.lap("draft")
            rollback.record()
            if graphs:
                if captured is None:
                    captured = verify[fed][1] = CapturedStep(lambda x=x: verify_pass(x), cache, fed, recorded=fed)
                h, pred = captured()
            else:
                h, pred = verify_pass(x)
            host[:fed].copy_(x, non_blocking=True)
            host[fed:2 * fed].copy_(pred, non_blocking=True)
            host[2 * fed:2 * fed + 3].copy_(result, non_blocking=True)
            done.record()
            done.synchronize()  # the step's one host synchronisation
            vals = host[:2 * fed + 3].tolist()
            xs, (n, bonus, keep) = vals[:fed], vals[2 * fed:]
            clock.lap("verify")
            rollback.rollback(cache, fed=fed, keep=keep, keep_device=result[2:3])
            clock.lap("rollback")
            new = xs[1:n + 1] + [bonus]
            drafter.update(h[:n + 1], new)
            clock.lap("drafter update")
            out.extend(new)
            steps += 1
            accepted += n
    finally:
        model.recorder.recording = False  # also when a step raised (e.g. a full cache)
    if stats is not None:
        stats.update(steps=steps, tokens_per_step=len(out) / max(steps, 1), accepted_drafts=accepted)
        if profile:
            stats["ms_per_step"] = {p: round(v / max(steps, 1) * 1e3, 3) for p, v in clock.total.items()}
    return out[:max_tokens]


def _speculative_on_device(model, prompt: list[int], max_tokens: int, drafter, k: int,
                           stats: dict | None) -> list[int]:
    """`speculative` with the whole step in one captured graph: the drafter's K drafts, the verify
    pass over [last token] + drafts, the acceptance, the rollback of the Gated-DeltaNet state
    and of every cache length to the accepted prefix, the append of the emitted tokens to a
    device buffer, and the drafter's update. Nothing of a step goes through the host, so replays
    are queued back to back; the host reads the token count after each batch of ceil(tokens
    still missing / (K + 1)) steps (the fewest that can finish), so it never runs a step the host
    loop would not. Cache capacity is checked per batch against the worst case of K + 1 new
    positions per step."""
    dev = model.device
    cache = make_prompt_cache(model)
    rollback = HybridRollback.for_model(model)
    h, logits = forward(model, prompt, cache)
    first = _last_argmax(logits)
    if max_tokens <= 1:
        return [int(first.item())][:max(max_tokens, 0)]
    fed = k + 1
    drafter.begin(prompt, h, int(first.item()))
    tokens = torch.empty((max_tokens + fed,), dtype=torch.int32, device=dev)
    tokens[:1].copy_(first)
    count = torch.ones((1,), dtype=torch.int32, device=dev)
    x = torch.empty((fed,), dtype=torch.int32, device=dev)
    x[:1].copy_(first)
    result = torch.empty((3,), dtype=torch.int32, device=dev)
    gb = cache.shared.gdn
    drafter.device_start()
    caches = [cache] + list(drafter.device_caches())

    def step():
        drafter.draft_into(x[1:], count)
        rollback.record()
        hh, lg = forward(model, x, cache)
        model.recorder.recording = False
        pred = K.argmax_rows(lg)
        K.accept(pred, x[1:], result)
        if gb is not None:
            K.gdn_select(result[2:3], fed, gb.state, gb.states, gb.conv, gb.window)
        K.spec_commit(result, cache.shared.pos, pred, tokens, count, x[:1])
        drafter.commit(pred, hh, result)

    lengths = []
    for c in caches:
        c.begin_step(0)  # device lengths current, so the capture records no write of them
        lengths.append(c.attention_offset())
    saved = [c.host_state() for c in caches]
    try:
        graph, _ = capture_graph(step)
    finally:
        model.recorder.recording = False
        for c, s in zip(caches, saved):
            c.restore_host_state(s)
    host = torch.empty((1 + len(caches),), dtype=torch.int32, pin_memory=True)
    done = torch.cuda.Event()
    produced, steps = 1, 0
    clock = _LoopClock(stats)
    clock.start()
    try:
        while produced < max_tokens:
            room = min((c.shared.maxlen - n) // fed for c, n in zip(caches, lengths))
            if room < 1:
                c, n = min(zip(caches, lengths), key=lambda cn: cn[0].shared.maxlen - cn[1])
                raise ValueError(f"KV cache full: {n} + {fed} > {c.shared.maxlen}")
            batch = min(-(-(max_tokens - produced) // fed), room)
            for _ in range(batch):
                graph.replay()
            steps += batch
            host[:1].copy_(count, non_blocking=True)
            for i, c in enumerate(caches):
                host[1 + i:2 + i].copy_(c.shared.pos, non_blocking=True)
            done.record()
            done.synchronize()
            vals = host.tolist()
            produced, lengths = vals[0], vals[1:]
    finally:
        del graph
        for c, n in zip(caches, lengths):
            c.resync(n)
        drafter.device_finish()
    clock.stop(min(produced, max_tokens) - 1)
    if stats is not None:
        stats.update(steps=steps, tokens_per_step=produced / max(steps, 1), accepted_drafts=produced - 1 - steps)
    return tokens[:max_tokens].tolist()


def main() -> None:
    """Speculative == greedy on a random-init model: tokens/step, tok/s and the length of the
    identical prefix, for prompt lookup and the MTP head (the reference's main, spec.py:170-204,
    needs a real checkpoint and tokenizer)."""
    from .model import build_model
    from .mtp import load_mtp_head
    from .patch import patch_model

    preset = sys.argv[1] if len(sys.argv) > 1 else "tiny-hybrid"
    model = build_model(preset)
    print("patch:", patch_model(model))
    g = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, model.args.vocab_size, (64,), generator=g).tolist()
    n_tok = 64
    t = time.perf_counter()
    ref = greedy(model, prompt, n_tok)
    t_greedy = time.perf_counter() - t
    for name, drafter, k in [("prompt-lookup", PromptLookupDrafter(), 4),
                             ("mtp", MTPDrafter(model, load_mtp_head(model)), 3)]:
        st = {}
        t = time.perf_counter()
        got = speculative(model, prompt, n_tok, drafter, k, st)
        dt = time.perf_counter() - t
        same = next((i for i, (a, b) in enumerate(zip(ref, got)) if a != b), n_tok)
        print(f"{name:14s} K={k}: {n_tok / dt:7.1f} tok/s (greedy {n_tok / t_greedy:7.1f}) | "
              f"{st['tokens_per_step']:.2f} tok/step | identical first {same}/{n_tok}")


if __name__ == "__main__":
    main()
