"""Decoding at temperature T > 0: plain sampling and speculative decoding with rejection sampling.

The reference decodes greedily (spec.py:98-156) and names rejection sampling for T > 0 as its
next step (docs/flatspec-design.md:19, item F6; README.md:84). This is the standard speculative
sampling: draft i is accepted with probability min(1, p_i(x)/q_i(x)); at the first rejection a
sample of norm(max(0, p_i - q_i)) is emitted; if every draft is accepted, a sample of p_K. The
emitted tokens are distributed exactly as plain sampling from the target (`sample`). The step
loop is the reference's (spec.py:110-156): verify K + 1 tokens in one forward, keep n + 1 of
them (rollback), re-sync the drafter on the kept tokens.

Randomness: one device int64 counter per generation, advanced inside the captured steps, keys a
Philox4x32-10 stream with the given seed (skinny_random_uniform). Plain sampling uses counter
values 0, 1, 2, ...; a speculative step with base c uses c + 2i for the acceptance of draft i and
c + 2n + 1 for the emitted sample (stream 0), and c + i for drafting draft i (stream 1), then
advances the counter by 2(K + 1). A generation is reproducible from its seed.

Drafters: `MTPDrafter.draft_sampled` draws the drafts from the head's pruned-vocabulary
distribution and hands back its score rows (q); a drafter without `draft_sampled` (prompt lookup,
replay) proposes deterministic drafts, which enter as point masses q = delta(x).
"""

from __future__ import annotations

import torch

from . import kernels as K
from .cache import make_prompt_cache
from .graphs import CapturedStep
from .rollback import HybridRollback
from .spec import PinnedIds, forward, greedy, speculative


def _counter(dev) -> torch.Tensor:
    return torch.zeros((1,), dtype=torch.int64, device=dev)


def sample(model, prompt: list[int], max_tokens: int, temperature: float, seed: int = 0,
           graphs: bool = True) -> list[int]:
    """Plain sampled decoding at temperature T (T <= 0: greedy). Token i is drawn with counter i."""
    if temperature <= 0:
        return greedy(model, prompt, max_tokens, graphs)
    cache = make_prompt_cache(model)
    counter = _counter(model.device)
    toks = torch.empty((max(max_tokens, 1),), dtype=torch.int32, device=model.device)
    K.sample_rows(model(prompt, cache)[-1:], temperature, seed, counter, out=toks[:1])
    counter.add_(1)
    cur = toks[:1].clone()

    def step():
        K.sample_rows(model(cur, cache)[-1:], temperature, seed, counter, out=cur)
        counter.add_(1)

    captured = CapturedStep(step, cache, 1) if graphs and max_tokens > 1 else None
    for i in range(1, max_tokens):
        captured() if captured is not None else step()
        toks[i:i + 1].copy_(cur)
    return toks[:max_tokens].tolist()


def speculative_sample(model, prompt: list[int], max_tokens: int, drafter, k: int, temperature: float,
                       seed: int = 0, stats: dict | None = None, graphs: bool = True) -> list[int]:
    """Speculative decoding with rejection sampling at temperature T (T <= 0: the greedy-exact
    `spec.speculative`)."""
    if temperature <= 0:
        return speculative(model, prompt, max_tokens, drafter, k, stats, graphs=graphs)
    dev = model.device
    cache = make_prompt_cache(model)
    rollback = HybridRollback.for_model(model)
    counter = _counter(dev)
    h, logits = forward(model, prompt, cache)
    first = K.sample_rows(logits[-1:], temperature, seed, counter)
    counter.add_(1)
    out = [int(first.item())]
    drafter.begin(prompt, h, out[0])
    sampled_drafts = hasattr(drafter, "draft_sampled")

    result = torch.empty((3,), dtype=torch.int32, device=dev)  # n, emitted token, keep
    host = torch.empty((k + 1 + 3,), dtype=torch.int32, pin_memory=True)
    stage = PinnedIds(k)
    done = torch.cuda.Event()
    verify = {}  # (fed, sampled) -> [token buffer, draft rows buffer, captured step]

    def verify_pass(x: torch.Tensor, rows: torch.Tensor | None):
        hh, lg = forward(model, x, cache)
        nd = x.shape[0] - 1
        st = K.row_stats(lg, temperature)
        sd = K.row_stats(rows, temperature) if rows is not None else None
        K.spec_accept_sampled(lg, st, x[1:], temperature, seed, counter, result, rows, sd)
        counter.add_(2 * (nd + 1))
        return hh

    steps = accepted = 0
    while len(out) < max_tokens:
        if sampled_drafts:
            d, rows = drafter.draft_sampled(k, temperature, seed, counter)
        else:
            d, rows = drafter.draft(k), None
        nd = int(d.numel()) if isinstance(d, torch.Tensor) else len(d)
        fed = nd + 1
        key = (fed, rows is not None)
        if key not in verify:
            verify[key] = [torch.empty((fed,), dtype=torch.int32, device=dev),
                           torch.empty((nd, rows.shape[1]), dtype=torch.bfloat16, device=dev) if rows is not None
                           else None, None]
        x, rbuf, captured = verify[key]
        x[:1].fill_(out[-1])
        if nd:
            if isinstance(d, torch.Tensor):
                x[1:].copy_(d)
            else:
                stage.upload(d, x[1:])
        if rbuf is not None:
            rbuf.copy_(rows[:nd])
        rollback.record()
        if graphs:
            if captured is None:
                captured = verify[key][2] = CapturedStep(lambda x=x, r=rbuf: verify_pass(x, r), cache, fed,
                                                         recorded=fed)
            hv = captured()
        else:
            hv = verify_pass(x, rbuf)
        host[:fed].copy_(x, non_blocking=True)
        host[fed:fed + 3].copy_(result, non_blocking=True)
        done.record()
        done.synchronize()  # the step's one host synchronisation
        vals = host[:fed + 3].tolist()
        xs, (n, tok, keep) = vals[:fed], vals[fed:]
        rollback.rollback(cache, fed=fed, keep=keep, keep_device=result[2:3])
        new = xs[1:n + 1] + [tok]
        drafter.update(hv[:n + 1], new)
        out.extend(new)
        steps += 1
        accepted += n
    if stats is not None:
        stats.update(steps=steps, tokens_per_step=len(out) / max(steps, 1), accepted_drafts=accepted)
    return out[:max_tokens]
