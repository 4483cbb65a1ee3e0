"""Draft-tree verification on the GPU (skinny_mlx.tree): top-k, chain trees equal linear
verification bit for bit, branching trees match forwards along each node's path, the commit
leaves the cache a linear decode of the accepted path would, and tree speculative decoding
emits greedy decoding's tokens."""

import numpy as np
import pytest
import torch

from oracle import accept as A
from skinny_mlx import kernels as K
from skinny_mlx import patch as P
from skinny_mlx.cache import KVCache, make_prompt_cache
from skinny_mlx.model import build_model
from skinny_mlx.mtp import load_mtp_head
from skinny_mlx.rollback import HybridRollback
from skinny_mlx.spec import MTPDrafter, forward, greedy
from skinny_mlx.tree import DraftTree, MTPTreeDrafter, branching_tree, commit_path, tree_speculative
from tests.helpers import near_tie_ok

pytestmark = pytest.mark.gpu


def _steps(st: dict) -> dict:
    """The step statistics both loops report (the device loop adds its own timing)."""
    return {k: st[k] for k in ("steps", "tokens_per_step", "accepted_drafts")}


@pytest.fixture(scope="module", params=["tiny-dense", "tiny-hybrid", "tiny-qwen35"])
def model(request):
    m = build_model(request.param)
    P.patch_model(m)
    return m


def _prompt(n=40, seed=0, vocab=1024):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, vocab, (n,), generator=g).tolist()


def test_topk_rows_matches_sorted_order(dev):
    g = torch.Generator().manual_seed(0)
    rows = (torch.randint(0, 40, (6, 3000), generator=g).float() / 8).to(torch.bfloat16)  # many ties
    for k in (1, 2, 4, 8):
        got = K.topk_rows(rows.to(dev), k).cpu().numpy()
        for r in range(rows.shape[0]):
            v = rows[r].float().numpy()
            order = sorted(range(v.size), key=lambda i: (-v[i], i))[:k]
            assert got[r].tolist() == order
    # masked rows: fewer finite values than k, and every value -inf (ties among -inf by index)
    masked = torch.full((2, 40000), float("-inf")).to(torch.bfloat16)
    masked[0, 39000] = 1.0
    masked[0, 7] = 2.0
    got = K.topk_rows(masked.to(dev), 4).cpu().numpy()
    assert got[0].tolist() == [7, 39000, 0, 1] and got[1].tolist() == [0, 1, 2, 3]


def _linear_and_tree(model, prompt, toks, tree):
    """(h, logits, cache) of a recording forward of `toks` as a chain and as `tree`."""
    rb = HybridRollback.for_model(model)
    out = []
    for t in (None, tree):
        c = make_prompt_cache(model)
        forward(model, prompt, c)
        rb.record()
        h, lg = forward(model, toks, c) if t is None else (lambda hh: (hh, model.logits(hh)))(model.hidden(toks, c, t))
        out.append((h, lg, c))
        rb.model.recorder.recording = False
    return out


def test_chain_tree_is_linear_verify_bitwise(model):
    toks = [5, 17, 300, 2, 999, 64]
    (h1, l1, c1), (h2, l2, c2) = _linear_and_tree(model, _prompt(seed=1), toks, DraftTree.chain(len(toks), model.device))
    assert torch.equal(l1, l2) and torch.equal(h1, h2)
    if c1.shared.gdn is not None:
        g1, g2 = c1.shared.gdn, c2.shared.gdn
        assert torch.equal(g1.window[:, :len(toks) + 3], g2.window[:, :len(toks) + 3])
        # committing the chain's first `keep` nodes by replay gives the linear pass's state after them
        before, conv0 = g2.state.clone(), g2.conv.clone()
        for keep in range(1, len(toks) + 1):
            g2.state.copy_(before)
            g2.conv.copy_(conv0)
            path = torch.tensor([keep] + list(range(keep)), dtype=torch.int32, device=model.device)
            K.gdn_commit_replay(path, g2.state.shape[1], g2.state, g2.record, g2.conv, g2.window)
            assert torch.equal(g2.state, g1.states[:, keep - 1] if keep < len(toks) else g1.state), keep
    assert torch.equal(c1.shared.k_all, c2.shared.k_all) and torch.equal(c1.shared.vt_all, c2.shared.vt_all)


def test_branching_tree_nodes_match_their_paths(model):
    parents, _, _ = branching_tree((4, 2, 1), 16)
    tree = DraftTree(parents, model.device)
    g = torch.Generator().manual_seed(3)
    toks = torch.randint(0, model.args.vocab_size, (tree.size,), generator=g).tolist()
    prompt = _prompt(seed=2)
    rb = HybridRollback.for_model(model)
    c = make_prompt_cache(model)
    forward(model, prompt, c)
    rb.record()
    lt = model.logits(model.hidden(toks, c, tree)).float().cpu().numpy()
    rb.model.recorder.recording = False
    for v in range(tree.size):
        path = [v]
        while parents[path[-1]] >= 0:
            path.append(parents[path[-1]])
        path = path[::-1]
        c2 = make_prompt_cache(model)
        forward(model, prompt, c2)
        _, lp = forward(model, [toks[p] for p in path], c2)
        ref = lp[-1:].float().cpu().numpy()
        err = np.abs(lt[v:v + 1] - ref).max() / np.abs(ref).max()
        assert err <= 2e-2, (v, err)
        assert near_tie_ok(ref, lt[v:v + 1])


@pytest.mark.parametrize("path", [[0, 1, 5, 13], [0, 2, 7, 15], [0, 4], [0]])
def test_commit_leaves_the_cache_of_the_path(model, path):
    parents, _, _ = branching_tree((4, 2, 1), 16)
    tree = DraftTree(parents, model.device)
    assert all(parents[b] == a for a, b in zip(path, path[1:]))
    g = torch.Generator().manual_seed(4)
    toks = torch.randint(0, model.args.vocab_size, (tree.size,), generator=g).tolist()
    prompt = _prompt(seed=5)
    rb = HybridRollback.for_model(model)
    c = make_prompt_cache(model)
    forward(model, prompt, c)
    rb.record()
    model.hidden(toks, c, tree)
    dev_path = torch.tensor([len(path)] + path, dtype=torch.int32, device=model.device)
    commit_path(rb, c, tree.size, dev_path, len(path))
    c2 = make_prompt_cache(model)
    forward(model, prompt, c2)
    forward(model, [toks[p] for p in path], c2)
    assert [x.offset for x in c if isinstance(x, KVCache)] == [x.offset for x in c2 if isinstance(x, KVCache)]
    _, la = forward(model, [11, 12], c)
    _, lb = forward(model, [11, 12], c2)
    a, b = la.float().cpu().numpy(), lb.float().cpu().numpy()
    assert np.abs(a - b).max() / np.abs(b).max() <= 2e-2 and near_tie_ok(b, a)
    if path == [0]:  # the root alone is computed exactly as a one-token forward
        assert torch.equal(la, lb)


def test_chain_tree_drafter_equals_linear_drafter(model):
    head = load_mtp_head(model)
    prompt = _prompt(seed=6)
    c = make_prompt_cache(model)
    h, lg = forward(model, prompt, c)
    first = int(K.argmax_rows(lg[-1:]).item())
    lin = MTPDrafter(model, head, vocab=512)
    lin.begin(prompt, h, first)
    tr = MTPTreeDrafter(model, head, vocab=512, branching=(1, 1, 1), budget=4)
    tr.begin(prompt, h, first)
    d_lin = lin.draft(3).tolist()
    d_tree = tr.draft_tree()[1:].tolist()
    assert d_lin == d_tree


class ReplayTreeDrafter(MTPTreeDrafter):
    """Puts the model's own greedy continuation on the path [0, 2, 7, 15] of the (4, 2, 1) x 16
    tree (through a second child) and wrong tokens elsewhere, so every step accepts three drafts
    along a non-first branch."""

    def __init__(self, model, head, ref):
        super().__init__(model, head, graphs=False)
        self.ref = ref
        self.target = {2: 0, 7: 1, 15: 2}  # node -> depth - 1

    def begin(self, prompt, h, first):
        self.pos = 1

    def draft_tree(self):
        V = self.model.args.vocab_size
        toks = []
        for v in range(self.tree.size):
            d = self.tree.depth[v]
            true = self.ref[self.pos + d - 1] if d > 0 else 0
            toks.append(true if v in self.target else (true + 1 + self.rank[v] + 7 * v) % V)
        return torch.tensor(toks, dtype=torch.int32, device=self.model.device)

    def update(self, h_kept, new_tokens):
        self.pos += len(new_tokens)


class DeviceReplayTreeDrafter(ReplayTreeDrafter):
    """ReplayTreeDrafter's trees, built on the device from the emitted count for the on-device
    loop (the host loop still calls draft_tree): the same tokens at every node, so both loops
    accept three drafts per step along the second branch."""

    def __init__(self, model, head, ref):
        super().__init__(model, head, ref)
        self.graphs = True
        dev = model.device
        M = self.tree.size
        self.ref_dev = torch.tensor(ref, dtype=torch.int64, device=dev)
        depth = torch.tensor(self.tree.depth, device=dev)
        self.offset = (depth - 1).clamp(min=0)
        self.root = depth == 0
        self.on = torch.tensor([v in self.target for v in range(M)], device=dev)
        self.wrong = torch.tensor([1 + self.rank[v] + 7 * v for v in range(M)], device=dev)

    def device_caches(self):
        return []

    def device_start(self):
        pass

    def device_finish(self):
        pass

    def tree_into(self, tokens, emitted):
        V = self.model.args.vocab_size
        true = self.ref_dev.index_select(0, (emitted.long() + self.offset).clamp_(max=len(self.ref) - 1))
        true = torch.where(self.root, torch.zeros_like(true), true)
        tokens[1:].copy_(torch.where(self.on, true, (true + self.wrong) % V)[1:])

    def path_commit(self, pred, h, res):
        pass


def test_tree_device_loop_equals_host_loop(model):
    """The on-device tree loop (tree, tree-masked verify, path commits of the KV and GDN
    state, cache lengths and emitted tokens in one captured step) emits the host loop's tokens
    with its steps and acceptances: drafts accepted along a second-ranked branch, and the MTP
    tree drafter, both equal to greedy."""
    prompt = _prompt(seed=9)
    N = 40
    ref = greedy(model, prompt, N + 8)
    head = load_mtp_head(model)
    st_h, st_d = {}, {}
    host = tree_speculative(model, prompt, N, DeviceReplayTreeDrafter(model, head, ref), st_h, device_loop=False)
    dev = tree_speculative(model, prompt, N, DeviceReplayTreeDrafter(model, head, ref), st_d)
    assert host == dev == ref[:N]
    assert _steps(st_h) == _steps(st_d) and st_d["tokens_per_step"] > 3.0
    st_h, st_d = {}, {}
    host = tree_speculative(model, prompt, N, MTPTreeDrafter(model, head, vocab=512), st_h, device_loop=False)
    dev = tree_speculative(model, prompt, N, MTPTreeDrafter(model, head, vocab=512), st_d)
    assert host == dev == ref[:N] and _steps(st_h) == _steps(st_d)


def test_tree_speculative_equals_greedy(model):
    prompt = _prompt(seed=7)
    N = 40
    ref = greedy(model, prompt, N + 8)
    st = {}
    got = tree_speculative(model, prompt, N, ReplayTreeDrafter(model, load_mtp_head(model), ref), st)
    assert got == ref[:N]
    assert st["tokens_per_step"] > 3.0
    st2 = {}
    head = load_mtp_head(model)
    got2 = tree_speculative(model, prompt, N, MTPTreeDrafter(model, head, vocab=512), st2)
    assert got2 == ref[:N]
    st3 = {}
    got3 = tree_speculative(model, prompt, N, MTPTreeDrafter(model, head, vocab=512, graphs=False), st3, graphs=False)
    assert got3 == got2 and st3["accepted_drafts"] == st2["accepted_drafts"]


def test_tree_accept_kernel_matches_oracle(dev):
    rng = np.random.default_rng(0)
    parents, _, _ = branching_tree((4, 2, 1), 16)
    for _ in range(50):
        toks = rng.integers(0, 5, 16).tolist()
        pred = rng.integers(0, 5, 16).tolist()
        out = torch.empty(19, dtype=torch.int32, device=dev)
        K.tree_accept(torch.tensor(pred, dtype=torch.int32, device=dev), torch.tensor(toks, dtype=torch.int32, device=dev),
                      torch.tensor(parents, dtype=torch.int32, device=dev), out)
        o = out.cpu().tolist()
        n, bonus, path = A.tree_accept(toks, parents, pred)
        assert o[:3] == [n, bonus, n + 1] and o[3:3 + n + 1] == path
