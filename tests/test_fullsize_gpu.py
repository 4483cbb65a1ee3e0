"""The end-to-end workloads at their full size on the GPU, checked by properties that do not depend
on size (the oracle cannot run a 36-layer, 151936-vocabulary decoder over thousands of tokens):

  * dense-36 verify step over a 2048-token prefill: the captured forward of M = 1, 2, 4, 6, 8, 12,
    16 tokens is bitwise the M single-token steps (what makes speculative decoding reproduce greedy
    decoding), and within the path's bf16 bar of the unpatched linears (fp32 dequantise + GEMM,
    SKINNY_RANGE switched off) on the same cache;
  * hybrid-36 (27 Gated-DeltaNet + 9 attention layers), 256-token prompt, 512 tokens: speculative
    decoding with the MTP head (K = 2, 3, 4) and with a replay drafter equals plain greedy token
    for token (reference spec.py:170-204, "identical first N/N");
  * the same model with the (4, 2, 1) 16-node draft tree, MTP top-k and replay trees: tree
    speculative decoding equals greedy.
"""

import numpy as np
import pytest
import torch

from oracle import w4
from skinny_mlx import patch as P
from skinny_mlx.cache import KVCache, make_prompt_cache
from skinny_mlx.graphs import CapturedStep
from skinny_mlx.model import build_model
from skinny_mlx.mtp import load_mtp_head
from skinny_mlx.spec import MTPDrafter, forward, greedy, speculative
from tests.helpers import bits16, near_tie_ok

pytestmark = pytest.mark.gpu


def _trim(cache, n):
    for c in cache:
        if isinstance(c, KVCache):
            c.trim(n)


def _f(t):
    return w4.bf16_to_f32(bits16(t)).astype(np.float64)


@pytest.fixture(scope="module")
def dense36():
    model = build_model("dense-36")
    P.patch_model(model)
    g = torch.Generator().manual_seed(0)
    cache = make_prompt_cache(model)
    forward(model, torch.randint(0, model.args.vocab_size, (2048,), generator=g).tolist(), cache)
    torch.cuda.synchronize()
    assert cache.attention_offset() == 2048
    yield model, cache
    del model, cache
    torch.cuda.empty_cache()


def test_dense36_verify_step_bitwise_equals_single_token_steps(dense36):
    model, cache = dense36
    dev = model.device
    g = torch.Generator().manual_seed(1)
    one = torch.zeros((1,), dtype=torch.int32, device=dev)
    single = CapturedStep(lambda: forward(model, one, cache), cache, 1)
    for M in (1, 2, 4, 6, 8, 12, 16):
        ids = torch.randint(0, model.args.vocab_size, (M,), generator=g).to(torch.int32).to(dev)
        step = CapturedStep(lambda ids=ids: forward(model, ids, cache), cache, M)
        h, logits = (t.clone() for t in step())
        _trim(cache, M)
        hs, ls = [], []
        for t in range(M):
            one.copy_(ids[t:t + 1])
            h1, l1 = single()
            hs.append(h1.clone())
            ls.append(l1.clone())
        _trim(cache, M)
        assert cache.attention_offset() == 2048
        assert torch.equal(logits, torch.cat(ls)), M
        assert torch.equal(h, torch.cat(hs)), M
        del step


def test_dense36_folded_norm_steps_bitwise_equal_separate(dense36):
    """Model.fold_norms at full size: single-token steps with each RMSNorm formed inside the
    q|k|v / gate|up projection after it are bitwise the separate-norm steps."""
    model, cache = dense36
    ids = torch.randint(0, model.args.vocab_size, (4,), generator=torch.Generator().manual_seed(3)).tolist()
    got = []
    for fold in (True, False):
        model.fold_norms = fold
        got.append([forward(model, [t], cache) for t in ids])
        _trim(cache, len(ids))
    model.fold_norms = True
    for (ha, la), (hb, lb) in zip(*got):
        assert torch.equal(ha, hb) and torch.equal(la, lb)


def test_dense36_fused_qkv_attention_bitwise_equals_two_launches(dense36, monkeypatch):
    """Every attention layer's q|k|v projection in one launch with the attention (Attention.fuse_qkv,
    opt-in) against the projection then the attention, on the same 2048-token cache: bitwise the
    same hidden states and logits for a one-token step and an 8-token verify step, and the fused
    form runs once per layer when switched on."""
    from skinny_mlx import kernels as K
    from skinny_mlx.model import Attention

    model, cache = dense36
    layers = [m for m in model.modules() if isinstance(m, Attention)]
    calls = []
    real = K.qkv_attention_fused
    monkeypatch.setattr(K, "qkv_attention_fused", lambda *a, **k: (calls.append(1), real(*a, **k))[1])
    g = torch.Generator().manual_seed(4)
    for m in (1, 8):
        ids = torch.randint(0, model.args.vocab_size, (m,), generator=g).tolist()
        got = []
        for fuse in (True, False):
            for layer in layers:
                layer.fuse_qkv = fuse
            calls.clear()
            got.append(forward(model, ids, cache))
            _trim(cache, m)
            assert len(calls) == (len(layers) if fuse else 0), (m, fuse, len(calls))
        for layer in layers:
            layer.fuse_qkv = False
        (ha, la), (hb, lb) = got
        assert torch.equal(ha, hb) and torch.equal(la, lb), m


def test_dense36_verify_step_matches_unpatched_linears(dense36, monkeypatch):
    """The same M = 8 verify forward with every linear on the unpatched path (fp32 dequantise +
    fp32 GEMM, the mx.quantized_matmul semantics) on the same 2048-token cache: logits within
    rel-err 2e-2 and argmax agreement except near-ties of <= 2 bf16 ulps."""
    model, cache = dense36
    ids = torch.randint(0, model.args.vocab_size, (8,), generator=torch.Generator().manual_seed(2)).tolist()
    _, skinny = forward(model, ids, cache)
    _trim(cache, 8)
    monkeypatch.setattr(P, "SKINNY_RANGE", (99, 99))
    _, stock = forward(model, ids, cache)
    _trim(cache, 8)
    a, b = _f(stock), _f(skinny)
    assert w4.rel_err(b, a) <= 2e-2
    assert near_tie_ok(a, b)


@pytest.fixture(scope="module")
def hybrid36():
    model = build_model("hybrid-36")
    P.patch_model(model)
    head = load_mtp_head(model)
    prompt = torch.randint(0, model.args.vocab_size, (256,), generator=torch.Generator().manual_seed(0)).tolist()
    ref = greedy(model, prompt, 512 + 8)
    yield model, head, prompt, ref
    del model, head
    torch.cuda.empty_cache()


class _Replay:
    """Proposes the target's own greedy continuation with one wrong draft per step at a rotating
    position, so every acceptance length occurs."""

    def __init__(self, ref):
        self.ref, self.step = ref, 0

    def begin(self, prompt, h, first):
        self.pos = 1

    def draft(self, k):
        d = list(self.ref[self.pos:self.pos + k])
        self.step += 1
        j = self.step % (k + 1)
        if j < len(d):
            d[j] = (d[j] + 1) % 151936
        return d

    def update(self, h_kept, new_tokens):
        self.pos += len(new_tokens)


def test_hybrid36_speculative_equals_greedy_512_tokens(hybrid36):
    model, head, prompt, ref = hybrid36
    N = 512
    for k in (2, 3, 4):
        st = {}
        got = speculative(model, prompt, N, MTPDrafter(model, head), k, st)
        assert got == ref[:N], f"MTP K={k}: first difference at {next(i for i, (a, b) in enumerate(zip(got, ref)) if a != b)}"
        assert st["steps"] >= 1
    st = {}
    got = speculative(model, prompt, N, _Replay(ref), 3, st)
    assert got == ref[:N]
    assert st["tokens_per_step"] > 2.0  # drafts were accepted at every length below K


def test_hybrid36_separate_norm_greedy_equals_greedy(hybrid36):
    """Greedy decoding with every RMSNorm as its own launch gives the tokens of the default greedy
    decoding, whose one-token steps form the q|k|v and gate|up norms inside those projections."""
    model, head, prompt, ref = hybrid36
    assert model.fold_norms
    model.fold_norms = False
    try:
        got = greedy(model, prompt, 64)
    finally:
        model.fold_norms = True
    assert got == ref[:64]


def test_hybrid36_tree_speculative_equals_greedy(hybrid36):
    from skinny_mlx.tree import MTPTreeDrafter, tree_speculative

    model, head, prompt, ref = hybrid36
    N = 512
    st = {}
    got = tree_speculative(model, prompt, N, MTPTreeDrafter(model, head), st)
    assert got == ref[:N]

    class ReplayTree(MTPTreeDrafter):
        """The greedy continuation on the path through nodes 2, 7, 15 (a second-ranked branch at the
        first level), every other node wrong: three drafts accepted per step."""

        def __init__(self):
            super().__init__(model, head, graphs=False)

        def begin(self, prompt_, h, first):
            self.pos = 1

        def draft_tree(self):
            V = model.args.vocab_size
            toks = []
            for v in range(self.tree.size):
                d = self.tree.depth[v]
                true = ref[self.pos + d - 1] if d > 0 else 0
                toks.append(true if v in (2, 7, 15) else (true + 1 + v) % V)
            return torch.tensor(toks, dtype=torch.int32, device=model.device)

        def update(self, h_kept, new_tokens):
            self.pos += len(new_tokens)

    st = {}
    got = tree_speculative(model, prompt, N, ReplayTree(), st)
    assert got == ref[:N]
    assert st["tokens_per_step"] > 3.5
