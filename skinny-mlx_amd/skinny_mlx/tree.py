"""Draft-tree speculative decoding: verify a whole tree of drafts in one forward pass.

The reference verifies a chain of K drafts (skinny_mlx/spec.py:110-156) and names tree
verification as its next step (README.md:84; docs/flatspec-design.md:65-69). Here a tree of M
nodes — node 0 the last emitted token, every other node a drafted continuation of its parent —
runs as ONE forward of M tokens:

* attention: each node sees the cache before the tree plus its ancestors (a bit mask per node
  over the tree's cache slots) and is rotated to its depth, not its slot (the `tree`
  descriptor of skinny_attention_fused_bf16, and of skinny_qk_rope_store / skinny_attention_bf16);
* Gated-DeltaNet layers: each node continues from its parent's recurrent state and conv inputs
  (parent pointers into the per-token states the verify pass keeps in HBM anyway), so sibling
  branches fork the state without copies;
* acceptance walks down from the root along children whose token equals the prediction at the
  current node (skinny_tree_accept) — the longest greedy-accepted path;
* the commit moves the path's KV entries into consecutive slots and sets every GDN layer's state
  and conv window to the path's leaf (skinny_kv_commit; skinny_gdn_commit_replay advances the state
  through the path's nodes with the operands the pass recorded); the rest is dropped.

A chain-shaped tree is exactly linear speculative decoding (same masks, positions and states).
For branching trees the emitted tokens are plain greedy decoding's up to near-ties in attention
rounding: a node's ancestors sit in other cache slots than a chain would put them in, so the
attention sums group differently (within bf16 tolerance; the GDN recurrence along a path is
bitwise the chain's).

The drafter chains the model's MTP head (skinny_mlx.mtp) level by level: the children of a node
are the top-k tokens of the head's pruned-vocabulary scores at that node, and the head itself
runs each level's expanding nodes as one call with its own tree mask.
"""

from __future__ import annotations

import time

import torch

from . import kernels as K
from .cache import KVCache, PromptCache, make_prompt_cache
from .graphs import CapturedStep, capture_graph
from .rollback import HybridRollback
from .spec import MTPDrafter, _last_argmax, _LoopClock, _PhaseClock, forward

MAX_TREE = 16  # nodes per tree: one forward of at most 16 tokens (the GDN tree kernels' bound too)


def branching_tree(branching=(4, 2, 1), budget: int = 16):
    """Breadth-first tree: the root gets branching[0] children, each of those branching[1], ...,
    cut at `budget` nodes (root included). Returns (parents, rank, level): rank is a node's
    place among its siblings (which top-k candidate it is)."""
    if budget < 1 or budget > MAX_TREE:
        raise ValueError(f"budget={budget} must be in [1, {MAX_TREE}]")
    parents, rank, level = [-1], [0], [0]
    frontier = [0]
    for depth, b in enumerate(branching, start=1):
        nxt = []
        for p in frontier:
            for r in range(b):
                if len(parents) >= budget:
                    break
                parents.append(p)
                rank.append(r)
                level.append(depth)
                nxt.append(len(parents) - 1)
        frontier = nxt
    return parents, rank, level


def _descriptor(masks, rpos, base: int, device) -> torch.Tensor:
    """The int32 tree descriptor of the attention kernels: [base, masks..., positions...]."""
    signed = [m - (1 << 32) if m >= 1 << 31 else m for m in masks]
    return torch.tensor([base] + signed + list(rpos), dtype=torch.int32, device=device)


class DraftTree:
    """A draft tree verified in one pass: node i occupies cache slot pos0 + i; its mask holds the
    slots of its ancestors and itself; its RoPE position is pos0 + depth."""

    def __init__(self, parents: list[int], device):
        M = len(parents)
        if M < 1 or M > MAX_TREE or parents[0] != -1 or any(not 0 <= parents[i] < i for i in range(1, M)):
            raise ValueError(f"parents must start with -1 and satisfy 0 <= parents[i] < i, at most {MAX_TREE} nodes")
        self.size = M
        self.parents = list(parents)
        self.depth = [0] * M
        masks = [1] + [0] * (M - 1)
        for i in range(1, M):
            self.depth[i] = self.depth[parents[i]] + 1
            masks[i] = masks[parents[i]] | (1 << i)
        self.masks = masks
        self.desc = _descriptor(masks, self.depth, 0, device)
        self.parent = torch.tensor(parents, dtype=torch.int32, device=device)

    @classmethod
    def chain(cls, M: int, device) -> "DraftTree":
        return cls([-1] + list(range(M - 1)), device)

    @classmethod
    def from_branching(cls, branching, budget: int, device) -> "DraftTree":
        return cls(branching_tree(branching, budget)[0], device)


class _HeadCall:
    """One batched MTP-head call of a drafting level: its nodes, their parents' rows and their
    tree descriptor (the head's layer is full attention, so no parent pointers are needed)."""

    def __init__(self, nodes, parent_rows, desc, size):
        self.nodes, self.parent_rows, self.desc, self.size = nodes, parent_rows, desc, size
        self.parent = None


class MTPTreeDrafter(MTPDrafter):
    """Builds a draft tree with the model's MTP head: the children of node v are the top-k
    tokens of the pruned-vocabulary scores of the head's hidden state at v (the root's is the
    head state after the last accepted token, as for chain drafting); each level's expanding
    nodes run through the head as one call in which each node sees the head's cache before the
    tree plus its own ancestors. After verification the head's cache drops the tree and is
    updated with the accepted path exactly as for a chain (MTPDrafter.update)."""

    def __init__(self, model, head, vocab: int | None = 32768, branching=(4, 2, 1), budget: int = 16,
                 graphs: bool = True):
        super().__init__(model, head, vocab, graphs)
        dev = model.device
        self.parents, self.rank, self.level = branching_tree(branching, budget)
        self.tree = DraftTree(self.parents, dev)
        M = self.tree.size
        children = [[] for _ in range(M)]
        for v in range(1, M):
            children[self.parents[v]].append(v)
        self.children = children
        self.depth_max = max(self.level)
        # per level d >= 1: the parents (level d - 1) whose children are scored together
        self._score_plan = []
        for d in range(1, self.depth_max + 1):
            par = [p for p in range(M) if self.level[p] == d - 1 and children[p]]
            kids = [c for p in par for c in children[p]]
            rows = [par.index(self.parents[c]) for c in kids]
            k = max(len(children[p]) for p in par)
            self._score_plan.append((torch.tensor(par, dtype=torch.long, device=dev),
                                     torch.tensor(kids, dtype=torch.long, device=dev),
                                     torch.tensor([r * k + self.rank[c] for r, c in zip(rows, kids)], dtype=torch.long,
                                                  device=dev), k))
        # head calls: per level d >= 1, the level's nodes that have children, in node order
        self._head_calls = []
        slot = {}
        used = 0
        for d in range(1, self.depth_max + 1):
            nodes = [v for v in range(M) if self.level[v] == d and children[v]]
            if not nodes:
                continue
            masks, rpos = [], []
            for j, v in enumerate(nodes):
                slot[v] = used + j
                m, a = 1 << slot[v], self.parents[v]
                while a > 0:
                    m |= 1 << slot[a]
                    a = self.parents[a]
                masks.append(m)
                rpos.append((d - 1) - used)  # head position of level d: tree start + d - 1
            call = _HeadCall(torch.tensor(nodes, dtype=torch.long, device=dev),
                             torch.tensor([self.parents[v] for v in nodes], dtype=torch.long, device=dev),
                             _descriptor(masks, rpos, used, dev), len(nodes))
            self._head_calls.append((d, call))
            used += len(nodes)
        self.head_slots = used
        self._tree_graph = None

    def begin(self, prompt, h, first):
        super().begin(prompt, h, first)
        self._tree_graph = None

    def _expand(self, h_root: torch.Tensor, tokens: torch.Tensor, hs: torch.Tensor) -> torch.Tensor:
        """Fill tokens[1:] level by level (device only)."""
        hs[:1].copy_(h_root)
        calls = dict(self._head_calls)
        for d, (par, kids, pick, k) in enumerate(self._score_plan, start=1):
            top = K.topk_rows(self._score(hs.index_select(0, par)), k)
            tokens.index_copy_(0, kids, top.reshape(-1).index_select(0, pick))
            call = calls.get(d)
            if call is not None:
                ids = tokens.index_select(0, call.nodes)
                out = self.head.forward_tokens(ids, self.model.embed_tokens, hs.index_select(0, call.parent_rows),
                                               self.cache, call)
                hs.index_copy_(0, call.nodes, out)
        return tokens

    # The on-device loop of tree_speculative: the tree's expansion and the update along the
    # accepted path run inside the loop's captured step.

    def tree_into(self, tokens: torch.Tensor, emitted: torch.Tensor) -> None:
        """Captured: the tree's tokens 1..M-1 into `tokens` from the buffered root state
        (device_start), then the head cache back to its length before the tree. `emitted`
        (the device count of tokens produced so far) is not needed here."""
        hs = torch.empty((self.tree.size, self._h_dev.shape[-1]), dtype=self._h_dev.dtype, device=self.model.device)
        self._expand(self._h_dev, tokens, hs)
        sh = self.cache.shared
        sh.pos.add_(-self.head_slots)
        for c in self.cache:
            c.trim(self.head_slots)
        sh.dev_pos -= self.head_slots

    def path_commit(self, pred: torch.Tensor, h: torch.Tensor, res: torch.Tensor) -> None:
        """Captured: `update` along the accepted path, on the device. res = tree_accept's output
        [n, bonus, count, path...]; the head runs over depth + 1 rows, row j = (pred, h) at the
        path's node j (node 0 past the path's end: those rows are never kept), of which the
        first count are update's input (the accepted nodes' tokens equal the predictions at
        their parents, then the bonus). The cache keeps those rows and the last one starts the
        next tree."""
        rows = max(self.level) + 1
        j = torch.arange(rows, device=self.model.device)
        nodes = torch.where(j < res[2:3].long(), res[3:3 + rows].long(), torch.zeros_like(j))
        out = self._run_head(pred.index_select(0, nodes), h.index_select(0, nodes))
        K.spec_select_row(res, self.cache.shared.pos, out, self._h_dev)

    def draft_tree(self) -> torch.Tensor:
        """Device int32 [M]: tokens of nodes 1..M-1 (entry 0 is left for the root token)."""
        M = self.tree.size
        dev = self.model.device
        self.n_spec = self.head_slots
        if not self.graphs:
            tokens = torch.zeros((M,), dtype=torch.int32, device=dev)
            hs = torch.empty((M, self.h_last.shape[-1]), dtype=self.h_last.dtype, device=dev)
            return self._expand(self.h_last, tokens, hs)
        if self._tree_graph is None:
            h0 = torch.empty_like(self.h_last)
            tokens = torch.zeros((M,), dtype=torch.int32, device=dev)
            hs = torch.empty((M, self.h_last.shape[-1]), dtype=self.h_last.dtype, device=dev)
            self._tree_graph = (h0, CapturedStep(lambda: self._expand(h0, tokens, hs), self.cache, self.head_slots))
        h0, step = self._tree_graph
        h0.copy_(self.h_last)
        return step()


def commit_path(rollback: HybridRollback, cache: PromptCache, fed: int, path: torch.Tensor, count: int) -> None:
    """Keep the accepted path of a draft-tree verify pass of `fed` tokens: `path` (device int32)
    = [count, root, ..., leaf]. Every GDN layer takes the leaf's state and conv window, every
    attention layer the path's KV entries in consecutive slots; the host lengths shrink to
    `count` tokens past the tree's start."""
    rollback.model.recorder.recording = False
    sh = cache.shared
    if sh.gdn is not None:
        if sh.gdn.recorded != fed:
            raise RuntimeError(f"commit: the last recording forward fed {sh.gdn.recorded} tokens, not {fed}")
        K.gdn_commit_replay(path, sh.gdn.state.shape[1], sh.gdn.state, sh.gdn.record, sh.gdn.conv, sh.gdn.window)
    if sh.k_all is not None and sh.k_all.shape[0] > 0:
        K.kv_commit(path, sh.pos, fed, sh.k_all, sh.vt_all)
    for c in cache:
        if isinstance(c, KVCache):
            c.trim(fed - count)


def _tree_speculative_on_device(model, prompt: list[int], max_tokens: int, drafter: MTPTreeDrafter,
                                stats: dict | None) -> list[int]:
    """tree_speculative with the whole step in one captured graph (the tree's expansion, the
    tree-masked verify pass, the acceptance, the path commits of the KV caches and GDN states,
    the cache lengths, the emitted tokens and the head's update along the path), batched as in
    spec._speculative_on_device: the host reads the count after ceil(missing / (depth + 1))
    steps."""
    dev = model.device
    cache = make_prompt_cache(model)
    rollback = HybridRollback.for_model(model)
    h, logits = forward(model, prompt, cache)
    first = _last_argmax(logits)
    if max_tokens <= 1:
        return [int(first.item())][:max(max_tokens, 0)]
    drafter.begin(prompt, h, int(first.item()))
    tree = drafter.tree
    M = tree.size
    most = max(drafter.level) + 1  # tokens one step can emit
    tokens = torch.empty((max_tokens + most,), dtype=torch.int32, device=dev)
    tokens[:1].copy_(first)
    count = torch.ones((1,), dtype=torch.int32, device=dev)
    x = torch.zeros((M,), dtype=torch.int32, device=dev)
    x[:1].copy_(first)
    res = torch.zeros((3 + M,), dtype=torch.int32, device=dev)  # n, bonus, count, path
    sh = cache.shared
    drafter.device_start()
    caches = [cache] + list(drafter.device_caches())

    def step():
        drafter.tree_into(x, count)
        rollback.record()
        hh, lg = forward(model, x, cache, tree)
        model.recorder.recording = False
        pred = K.argmax_rows(lg)
        K.tree_accept(pred, x, tree.parent, res)
        path = res[2:]
        if sh.gdn is not None:
            K.gdn_commit_replay(path, sh.gdn.state.shape[1], sh.gdn.state, sh.gdn.record, sh.gdn.conv,
                                sh.gdn.window)
        if sh.k_all is not None and sh.k_all.shape[0] > 0:
            K.kv_commit(path, sh.pos, M, sh.k_all, sh.vt_all)
        K.spec_commit(res, sh.pos, pred, tokens, count, x[:1], path=True)
        drafter.path_commit(pred, hh, res)

    lengths = []
    for c in caches:
        c.begin_step(0)
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
            room = min((c.shared.maxlen - n) // M for c, n in zip(caches, lengths))
            if room < 1:
                c, n = min(zip(caches, lengths), key=lambda cn: cn[0].shared.maxlen - cn[1])
                raise ValueError(f"KV cache full: {n} + {M} > {c.shared.maxlen}")
            batch = min(-(-(max_tokens - produced) // most), room)
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


def tree_speculative(model, prompt: list[int], max_tokens: int, drafter: MTPTreeDrafter, stats: dict | None = None,
                     profile: bool = False, graphs: bool = True, device_loop: bool | None = None) -> list[int]:
    """Greedy speculative decoding with one draft tree verified per step. With graphs and no
    profile the step runs on the device by default (`device_loop`): the same tokens, steps and
    acceptances without a host round trip per step."""
    if device_loop is None:
        device_loop = graphs and not profile and drafter.graphs
    if device_loop:
        if not (graphs and not profile and drafter.graphs):
            raise ValueError("the on-device loop needs graphs=True and profile=False")
        return _tree_speculative_on_device(model, prompt, max_tokens, drafter, stats)
    dev = model.device
    clock = _PhaseClock(profile)
    cache = make_prompt_cache(model)
    rollback = HybridRollback.for_model(model)
    h, logits = forward(model, prompt, cache)
    out = [int(_last_argmax(logits).item())]
    drafter.begin(prompt, h, out[0])
    tree = drafter.tree
    M = tree.size
    x = torch.empty((M,), dtype=torch.int32, device=dev)
    res = torch.empty((3 + M,), dtype=torch.int32, device=dev)  # n, bonus, count, path
    host = torch.empty((3 + 2 * M,), dtype=torch.int32, pin_memory=True)
    done = torch.cuda.Event()

    def verify_pass():
        hh, lg = forward(model, x, cache, tree)
        pred = K.argmax_rows(lg)
        K.tree_accept(pred, x, tree.parent, res)
        return hh

    captured = None
    steps = accepted = 0
    while len(out) < max_tokens:
        clock.start()
        toks = drafter.draft_tree()
        x.copy_(toks)
        x[:1].fill_(out[-1])
        clock.lap("draft")
        rollback.record()
        if graphs:
            if captured is None:
                captured = CapturedStep(verify_pass, cache, M, recorded=M)
            hv = captured()
        else:
            hv = verify_pass()
        host[:3 + M].copy_(res, non_blocking=True)
        host[3 + M:].copy_(x, non_blocking=True)
        done.record()
        done.synchronize()  # the step's one host synchronisation
        vals = host.tolist()
        n, bonus, count = vals[0], vals[1], vals[2]
        path, xs = vals[3:3 + count], vals[3 + M:]
        clock.lap("verify")
        commit_path(rollback, cache, M, res[2:], count)
        clock.lap("rollback")
        new = [xs[p] for p in path[1:]] + [bonus]
        drafter.update(hv.index_select(0, res[3:3 + count]), new)
        clock.lap("drafter update")
        out.extend(new)
        steps += 1
        accepted += n
    if stats is not None:
        stats.update(steps=steps, tokens_per_step=len(out) / max(steps, 1), accepted_drafts=accepted)
        if profile:
            stats["ms_per_step"] = {p: round(v / max(steps, 1) * 1e3, 3) for p, v in clock.total.items()}
    return out[:max_tokens]


def main() -> None:
    """Tree speculative decoding vs greedy on a random-init hybrid model."""
    import sys

    from .model import build_model
    from .mtp import load_mtp_head
    from .patch import patch_model
    from .spec import greedy

    preset = sys.argv[1] if len(sys.argv) > 1 else "tiny-hybrid"
    model = build_model(preset)
    patch_model(model)
    g = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, model.args.vocab_size, (64,), generator=g).tolist()
    n_tok = 64
    ref = greedy(model, prompt, n_tok)
    st = {}
    t = time.perf_counter()
    got = tree_speculative(model, prompt, n_tok, MTPTreeDrafter(model, load_mtp_head(model)), st)
    dt = time.perf_counter() - t
    same = next((i for i, (a, b) in enumerate(zip(ref, got)) if a != b), n_tok)
    print(f"tree (4,2,1)x16: {n_tok / dt:.1f} tok/s | {st['tokens_per_step']:.2f} tok/step | identical first {same}/{n_tok}")


if __name__ == "__main__":
    main()
