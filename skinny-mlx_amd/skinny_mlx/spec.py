"""Greedy-exact speculative decoding with pluggable drafters.

Same call surface as the reference (skinny_mlx/spec.py:24-156): `forward`,
`PromptLookupDrafter`, `MTPDrafter` (begin / draft / update), `greedy`, `speculative`.

Each step feeds [last emitted token] + K draft tokens (M = K+1) in one forward, takes the
argmax of every row and the longest matching draft prefix on the device (the acceptance
kernel), emits one bonus token, and rolls the hybrid cache back to the accepted prefix
(skinny_mlx.rollback). The step's single host synchronisation copies the drafts, the
predictions and (n, bonus, keep) back together (the reference's one mx.eval, spec.py:138).

Every kernel on the path computes a token's row independently of how many tokens share the
pass, so the output equals plain greedy decoding token for token (the reference's equality
holds up to bf16 near-ties between its batched and single-token kernels, spec.py:5-6).

Tensors are 2-D here ([T, ...]): the reference's leading batch dim of 1 is dropped.
"""

from __future__ import annotations

import sys
import time

import torch

from . import kernels as K
from .cache import make_prompt_cache
from .rollback import HybridRollback


def forward(model, ids, cache):
    """(final normed hidden [T, H], logits [T, V]) for the tokens `ids` (a list, or an int32
    tensor on the GPU so draft tokens flow into verify without a host sync)."""
    h = model.hidden(ids, cache)
    return h, model.logits(h)


def _argmax_last(logits: torch.Tensor) -> torch.Tensor:
    return K.argmax_rows(logits[-1:])


class PromptLookupDrafter:
    """Model-free: propose what followed the latest earlier occurrence of the trailing n-gram
    (reference spec.py:32-51)."""

    def __init__(self, ngram: int = 3):
        self.ngram = ngram

    def begin(self, prompt, h, first):
        self.ctx = list(prompt) + [first]

    def draft(self, k: int) -> list[int]:
        ctx = self.ctx
        for n in range(self.ngram, 0, -1):
            tail = ctx[-n:]
            for start in range(len(ctx) - n - 1, -1, -1):
                if ctx[start:start + n] == tail:
                    return ctx[start + n:start + n + k]
        return []

    def update(self, h_kept, new_tokens):
        self.ctx += list(new_tokens)


class MTPDrafter:
    """Chains the MTP head K times; keeps its own KV cache in sync with accepted tokens
    (reference spec.py:54-95). Drafts score token ids [0, vocab) only — the first `vocab` rows
    of the model's W4 head, a prefix of its packed buffer — while verify uses the full head,
    so output is unchanged and only acceptance can drop."""

    def __init__(self, model, head, vocab: int | None = 32768):
        self.model, self.head = model, head
        lm = model.lm_head
        V = model.args.vocab_size
        self.vocab = V if vocab is None else min(vocab, V)
        rw = getattr(lm, "rweight", None)
        if rw is not None and self.vocab % 16 == 0:
            self._head = ("packed", rw[:self.vocab])
        else:
            self._head = ("linear", (lm.weight[:self.vocab], lm.scales[:self.vocab], lm.biases[:self.vocab]))
        self.cache = None

    def _logits(self, h: torch.Tensor) -> torch.Tensor:
        kind, w = self._head
        if kind == "packed":
            from .qmm import skinny_qmm

            return skinny_qmm(h, w)
        from .patch import _fallback

        return _fallback(h, *w)

    def _step(self, tokens: torch.Tensor, hidden: torch.Tensor) -> torch.Tensor:
        return self.head(K.embed(tokens, self.model.embed_tokens), hidden, self.cache)

    def begin(self, prompt, h, first):
        from .mtp import make_mtp_cache

        self.cache = make_mtp_cache(self.head)
        ids = torch.tensor(list(prompt[1:]) + [int(first)], dtype=torch.int32, device=self.model.device)
        hs = [self._step(ids[i:i + 16], h[i:i + 16]) for i in range(0, ids.shape[0], 16)]
        self.h_last = hs[-1][-1:]
        self.n_spec = 0

    def draft(self, k: int) -> torch.Tensor:
        toks = torch.empty((k,), dtype=torch.int32, device=self.model.device)
        h = self.h_last
        for i in range(k):  # device-resident chain: no host sync between drafts
            K.argmax_rows(self._logits(h), out=toks[i:i + 1])
            if i < k - 1:
                h = self._step(toks[i:i + 1], h)
        self.n_spec = max(k - 1, 0)
        return toks

    def update(self, h_kept, new_tokens):
        for c in self.cache:
            c.trim(self.n_spec)  # drop the speculative chain entries
        ids = torch.tensor(list(new_tokens), dtype=torch.int32, device=self.model.device)
        self.h_last = self._step(ids, h_kept.contiguous())[-1:]
        self.n_spec = 0


def greedy(model, prompt: list[int], max_tokens: int) -> list[int]:
    """Plain greedy decoding, one token per forward (reference spec.py:98-107). The loop never
    waits for the GPU: each step's argmax feeds the next step on the device and the tokens are
    read back once at the end."""
    cache = make_prompt_cache(model)
    y = _argmax_last(model(prompt, cache))
    toks = torch.empty((max_tokens,), dtype=torch.int32, device=model.device)
    for i in range(max_tokens):
        toks[i:i + 1].copy_(y)
        if i < max_tokens - 1:
            y = _argmax_last(model(toks[i:i + 1], cache))
    return toks.tolist()


def speculative(model, prompt: list[int], max_tokens: int, drafter, k: int,
                stats: dict | None = None, profile: bool = False) -> list[int]:
    """profile=True synchronises at phase boundaries and adds per-phase ms/step to stats."""
    phase = {"draft": 0.0, "verify": 0.0, "rollback": 0.0, "drafter update": 0.0}
    clock = [time.perf_counter()]

    def mark(name):
        if profile:
            torch.cuda.synchronize()
            now = time.perf_counter()
            phase[name] += now - clock[0]
            clock[0] = now

    dev = model.device
    cache = make_prompt_cache(model)
    rb = HybridRollback.for_model(model)
    h, logits = forward(model, prompt, cache)
    out = [int(_argmax_last(logits).item())]
    drafter.begin(prompt, h, out[0])
    res = torch.empty((3,), dtype=torch.int32, device=dev)
    steps = accepted = 0
    while len(out) < max_tokens:
        if profile:
            torch.cuda.synchronize()
            clock[0] = time.perf_counter()
        d = drafter.draft(k)
        if not isinstance(d, torch.Tensor):
            d = torch.tensor(list(d), dtype=torch.int32, device=dev)
        mark("draft")
        x = torch.empty((d.numel() + 1,), dtype=torch.int32, device=dev)
        x[0] = out[-1]
        x[1:].copy_(d)
        fed = x.numel()
        rb.record()
        h, logits = forward(model, x, cache)
        pred = K.argmax_rows(logits)
        K.accept(pred, x[1:] if fed > 1 else None, res)
        host = torch.cat([x, pred, res]).tolist()  # the step's one host sync
        xs, pr, (n, bonus, keep) = host[:fed], host[fed:2 * fed], host[2 * fed:]
        mark("verify")
        rb.rollback(cache, fed=fed, keep=keep, keep_device=res[2:3])
        mark("rollback")
        new = xs[1:n + 1] + [bonus]
        drafter.update(h[:n + 1], new)
        mark("drafter update")
        out += new
        steps += 1
        accepted += n
    if stats is not None:
        stats.update(steps=steps, tokens_per_step=len(out) / max(steps, 1), accepted_drafts=accepted)
        if profile:
            stats["ms_per_step"] = {p: round(v / max(steps, 1) * 1e3, 3) for p, v in phase.items()}
    return out[:max_tokens]


def main() -> None:
    """Spec == greedy on a random-init model (the reference's main, spec.py:170-204, needs a
    real checkpoint and tokenizer): prints tokens/step, tok/s and the identical prefix."""
    from .model import build_model
    from .mtp import load_mtp_head
    from .patch import patch_model

    preset = sys.argv[1] if len(sys.argv) > 1 else "tiny-hybrid"
    model = build_model(preset)
    print("patch:", patch_model(model))
    g = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, model.args.vocab_size, (64,), generator=g).tolist()
    N = 64
    t = time.perf_counter()
    ref = greedy(model, prompt, N)
    t_g = time.perf_counter() - t
    for name, drafter, k in [("prompt-lookup", PromptLookupDrafter(), 4),
                             ("mtp", MTPDrafter(model, load_mtp_head(model)), 3)]:
        st = {}
        t = time.perf_counter()
        got = speculative(model, prompt, N, drafter, k, st)
        dt = time.perf_counter() - t
        same = next((i for i, (a, b) in enumerate(zip(ref, got)) if a != b), N)
        print(f"{name:14s} K={k}: {N / dt:7.1f} tok/s (greedy {N / t_g:7.1f}) | "
              f"{st['tokens_per_step']:.2f} tok/step | identical first {same}/{N}")


if __name__ == "__main__":
    main()
