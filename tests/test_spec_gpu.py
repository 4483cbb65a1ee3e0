"""Speculative decoding on the GPU: output == plain greedy token for token, acceptance
lengths equal the oracle's, and the replay-free rollback is bitwise a forward over the
accepted prefix."""

import numpy as np
import pytest
import torch

from oracle import accept as A
from skinny_mlx import patch as P
from skinny_mlx.cache import KVCache, make_prompt_cache
from skinny_mlx.model import build_model
from skinny_mlx.mtp import load_mtp_head
from skinny_mlx.rollback import HybridRollback
from skinny_mlx.spec import MTPDrafter, PromptLookupDrafter, forward, greedy, speculative

pytestmark = pytest.mark.gpu


def _steps(st: dict) -> dict:
    """The step statistics both loops report (the device loop adds its own timing)."""
    return {k: st[k] for k in ("steps", "tokens_per_step", "accepted_drafts")}


@pytest.fixture(scope="module", params=["tiny-dense", "tiny-hybrid", "tiny-qwen35"])
def model(request):
    m = build_model(request.param)
    P.patch_model(m)
    return m


def _prompt(n=48, period=7, seed=0):
    g = torch.Generator().manual_seed(seed)
    base = torch.randint(0, 1000, (period,), generator=g).tolist()
    return (base * (n // period + 1))[:n]


class ReplayDrafter:
    """Test drafter: proposes the target's own greedy continuation with every `corrupt`-th
    draft position wrong, so acceptance runs through all lengths deterministically."""

    def __init__(self, ref, corrupt=3):
        self.ref, self.corrupt, self.step = ref, corrupt, 0

    def begin(self, prompt, h, first):
        self.pos = 1  # ref[0] == first

    def draft(self, k):
        d = list(self.ref[self.pos:self.pos + k])
        self.step += 1
        j = self.step % (k + 1)
        if j < len(d):
            d[j] = (d[j] + 1) % 1000
        return d

    def update(self, h_kept, new_tokens):
        self.pos += len(new_tokens)


class DeviceReplayDrafter:
    """The greedy continuation `ref` as drafts, with the draft at position (emitted % (k + 1))
    made wrong, where emitted = tokens produced so far: acceptance runs through every length,
    and the drafts depend only on the emitted count, so the host loop (draft / update) and the
    on-device loop (draft_into, reading the device count) see the same drafts."""

    device_draft = True

    def __init__(self, ref, dev):
        self.ref, self.dev = list(ref), dev
        self.ref_dev = torch.tensor(self.ref, dtype=torch.int64, device=dev)

    def begin(self, prompt, h, first):
        self.pos = 1  # ref[0] == first

    def draft(self, k):
        d = list(self.ref[self.pos:self.pos + k])
        j = self.pos % (k + 1)
        if j < len(d):
            d[j] = (d[j] + 1) % 1000
        return d

    def update(self, h_kept, new_tokens):
        self.pos += len(new_tokens)

    def device_caches(self):
        return []

    def device_start(self):
        pass

    def draft_into(self, toks, emitted):
        k = toks.shape[0]
        ar = torch.arange(k, device=self.dev)
        at = emitted.long()
        vals = self.ref_dev.index_select(0, (at + ar).clamp_(max=len(self.ref) - 1))
        vals = torch.where(ar == at % (k + 1), (vals + 1) % 1000, vals)
        toks.copy_(vals)

    def commit(self, pred, h, result):
        pass

    def device_finish(self):
        pass


@pytest.mark.parametrize("k", [1, 3, 4])
def test_device_loop_equals_host_loop_at_every_acceptance(model, k):
    """The on-device loop (the whole step in one graph, the host reading the count once per
    batch) emits the tokens, and takes the steps and acceptances, of the host loop, which
    equal greedy decoding; drafts accepted up to every position in turn."""
    prompt = _prompt(seed=31)
    N = 45
    full = greedy(model, prompt, N + k + 2)
    st_h, st_d = {}, {}
    host = speculative(model, prompt, N, DeviceReplayDrafter(full, model.device), k, st_h, device_loop=False)
    dev = speculative(model, prompt, N, DeviceReplayDrafter(full, model.device), k, st_d)
    assert host == dev == full[:N]
    assert _steps(st_h) == _steps(st_d) and st_d["accepted_drafts"] > 0


def test_device_loop_mtp_equals_host_loop(model):
    head = load_mtp_head(model)
    prompt = _prompt(seed=33)
    ref = greedy(model, prompt, 30)
    for k in (2, 4):
        st_h, st_d = {}, {}
        host = speculative(model, prompt, 30, MTPDrafter(model, head), k, st_h, device_loop=False)
        dev = speculative(model, prompt, 30, MTPDrafter(model, head), k, st_d, device_loop=True)
        assert host == dev == ref and _steps(st_h) == _steps(st_d)


def test_device_loop_leaves_caches_consistent_and_checks_capacity(model):
    """After the on-device loop the drafter's head cache length is back on the host; a
    generation past the KV cache's capacity raises as the host loop does, with no step run
    beyond it."""
    head = load_mtp_head(model)
    prompt = _prompt(seed=35)
    dr = MTPDrafter(model, head)
    speculative(model, prompt, 20, dr, 3, {})
    assert dr.cache[0].offset == int(dr.cache.shared.pos.item()) and dr.n_spec == 0
    too_many = model.args.max_position - len(prompt) + 8
    for loop in (False, True):
        with pytest.raises(ValueError, match="KV cache full"):
            speculative(model, prompt, too_many, MTPDrafter(model, head), 3, {}, device_loop=loop)


def test_spec_commit_and_select_row_kernels(dev):
    """skinny_spec_commit / skinny_spec_select_row against the host arithmetic: the length
    back by fed - keep, pred[:keep] appended at the count (slots past the buffer dropped), the
    bonus as the next first token, and the row keep - 1 selected."""
    from skinny_mlx import kernels as K

    fed, H = 5, 40
    pred = torch.tensor([11, 12, 13, 14, 15], dtype=torch.int32, device=dev)
    rows = torch.randn((fed, H), generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(dev)
    tokens = torch.full((9,), -1, dtype=torch.int32, device=dev)
    count = torch.tensor([2], dtype=torch.int32, device=dev)
    pos = torch.tensor([100], dtype=torch.int32, device=dev)
    nxt = torch.zeros((1,), dtype=torch.int32, device=dev)
    expect_tokens, c, p = [-1] * 9, 2, 100
    for n in (2, 4, 0, 3):  # keep = n + 1: 3, 5 (= fed), 1, then past the buffer's end
        result = torch.tensor([n, pred[n].item(), n + 1], dtype=torch.int32, device=dev)
        K.spec_commit(result, pos, pred, tokens, count, nxt)
        for j in range(n + 1):
            if c + j < 9:
                expect_tokens[c + j] = 11 + j
        c, p = c + n + 1, p + (n + 1) - fed
        assert tokens.tolist() == expect_tokens and count.item() == c and pos.item() == p
        assert nxt.item() == 11 + n
        out = torch.empty((1, H), dtype=torch.bfloat16, device=dev)
        head_pos = torch.tensor([50], dtype=torch.int32, device=dev)
        K.spec_select_row(result, head_pos, rows, out)
        assert torch.equal(out[0], rows[n]) and head_pos.item() == 50 + (n + 1) - fed


@pytest.mark.parametrize("k", [1, 3, 4])
def test_spec_equals_greedy_prompt_lookup(model, k):
    prompt = _prompt()
    ref = greedy(model, prompt, 40)
    st = {}
    got = speculative(model, prompt, 40, PromptLookupDrafter(), k, st)
    assert got == ref
    assert st["steps"] >= 1


def test_spec_equals_greedy_replay_drafter_and_acceptance(model):
    prompt = _prompt(seed=3)
    N, k = 48, 4
    ref = greedy(model, prompt, N + k + 1)
    dr = ReplayDrafter(ref)
    st = {}
    got = speculative(model, prompt, N, dr, k, st)
    assert got == ref[:N]
    # acceptance lengths: every step accepts exactly up to the corrupted position
    assert st["accepted_drafts"] > 0 and st["tokens_per_step"] > 1.5


def test_spec_equals_greedy_mtp(model):
    head = load_mtp_head(model)
    prompt = _prompt(seed=5)
    gst = {}
    ref = greedy(model, prompt, 32, stats=gst)
    assert gst["decode_ms"] > 0 and gst["decode_tok_s"] > 0
    for k in (2, 3):
        st = {}
        assert speculative(model, prompt, 32, MTPDrafter(model, head), k, st) == ref
        # the device loop's own time, beside the end-to-end one the caller measures
        assert st["decode_ms"] > 0 and st["decode_tok_s"] > 0


def test_rollback_is_bitwise_prefix_forward(model):
    prompt = _prompt(seed=9)
    x = [11, 22, 33, 44, 55, 66]
    fed = len(x)
    rb = HybridRollback.for_model(model)
    for keep in range(1, fed + 1):
        c1 = make_prompt_cache(model)
        forward(model, prompt, c1)
        rb.record()
        forward(model, x, c1)
        rb.rollback(c1, fed, keep)
        c2 = make_prompt_cache(model)
        forward(model, prompt, c2)
        forward(model, x[:keep], c2)
        if c1.shared.gdn is not None:
            assert torch.equal(c1.shared.gdn.state, c2.shared.gdn.state)
            assert torch.equal(c1.shared.gdn.conv, c2.shared.gdn.conv)
        assert [c.offset for c in c1 if isinstance(c, KVCache)] == [c.offset for c in c2 if isinstance(c, KVCache)]
        # and the next step agrees bitwise
        _, l1 = forward(model, [7, 8], c1)
        _, l2 = forward(model, [7, 8], c2)
        assert torch.equal(l1, l2)


def test_rollback_rejects_bad_keep(model):
    rb = HybridRollback.for_model(model)
    c = make_prompt_cache(model)
    forward(model, [1, 2, 3], c)
    rb.record()
    forward(model, [4, 5, 6], c)
    with pytest.raises(ValueError):
        rb.rollback(c, 3, 0)
    with pytest.raises(ValueError):
        rb.rollback(c, 3, 4)
    rb.rollback(c, 3, 3)  # keep == fed: no-op


def test_accept_matches_oracle_on_model_rows(model):
    c = make_prompt_cache(model)
    forward(model, _prompt(seed=11), c)
    _, logits = forward(model, [1, 2, 3, 4, 5], c)
    lg = logits.float().cpu().numpy()
    from skinny_mlx import kernels as K

    pred = K.argmax_rows(logits).cpu().numpy()
    assert pred.tolist() == [A.argmax_first(r) for r in lg]


def test_graph_replay_equals_eager(model):
    """Captured steps (decode, verify, MTP chain and updates) replay exactly what the eager path
    computes: same tokens, same acceptance."""
    prompt = _prompt(seed=13)
    N = 40
    ref = greedy(model, prompt, N, graphs=False)
    assert greedy(model, prompt, N, graphs=True) == ref
    head = load_mtp_head(model)
    st_e, st_g = {}, {}
    e = speculative(model, prompt, N, MTPDrafter(model, head, graphs=False), 3, st_e, graphs=False)
    g = speculative(model, prompt, N, MTPDrafter(model, head, graphs=True), 3, st_g, graphs=True)
    assert e == g == ref
    assert st_e["accepted_drafts"] == st_g["accepted_drafts"]
    full = greedy(model, prompt, N + 6, graphs=False)
    st_r = {}
    r = speculative(model, prompt, N, ReplayDrafter(full), 4, st_r, graphs=True)
    assert r == ref and st_r["tokens_per_step"] > 1.5



def test_capture_runs_without_cyclic_collection(model):
    """A prompt of four or more 16-token pieces keeps a captured piece step on its cache (a
    reference cycle cache -> step -> cache), so dropped caches hold graphs that only the cyclic
    collector frees. A graph freed during another capture is a HIP error that aborts the
    process: CapturedStep captures with the collector off and turns it back on afterwards."""
    import gc

    from skinny_mlx.graphs import CapturedStep

    prompt = _prompt(n=70, seed=21)
    ref = greedy(model, prompt, 6, graphs=False)
    assert greedy(model, prompt, 6, graphs=True) == ref  # leaves a cache cycle behind
    cache = make_prompt_cache(model)
    forward(model, prompt, cache)
    ids = torch.tensor(ref[:1], dtype=torch.int32, device=model.device)
    seen = []

    def fn():
        seen.append(gc.isenabled())
        return forward(model, ids, cache)

    CapturedStep(fn, cache, 1)()
    assert seen == [False] and gc.isenabled()


def test_dropped_cache_frees_its_piece_graph_without_the_collector(model):
    """The captured piece step a long prompt leaves on its cache refers back to the cache only
    weakly, so no reference cycle forms: dropping the cache frees the step and its graph by
    reference counting alone (cyclic collection off), never later inside another capture."""
    import gc
    import weakref

    prompt = _prompt(n=70, seed=22)
    cache = make_prompt_cache(model)
    h, _ = forward(model, prompt, cache)
    step = cache._piece_step[1]
    assert step.cache is cache
    ref = weakref.ref(step)
    del step
    torch.cuda.synchronize()
    was_on = gc.isenabled()
    gc.disable()
    try:
        del cache
        assert ref() is None
    finally:
        if was_on:
            gc.enable()
    # and a fresh cache gets its own piece graph that computes the same states
    c2 = make_prompt_cache(model)
    h2, _ = forward(model, prompt, c2)
    assert torch.equal(h, h2)


def test_profile_mode_reports_phases_and_equals_greedy(model):
    """speculative(profile=True) (reference spec.py:110-156, the phase timers of :112-121) takes
    the host loop, synchronising at each phase boundary inside a roctx range per phase, and still
    gives greedy's tokens; stats carry ms per step for every phase."""
    prompt = _prompt()
    ref = greedy(model, prompt, 24)
    st = {}
    got = speculative(model, prompt, 24, ReplayDrafter(ref), 3, st, profile=True)
    assert got == ref
    ms = st["ms_per_step"]
    assert set(ms) == {"draft", "verify", "rollback", "drafter update"} and all(v >= 0 for v in ms.values())
    assert ms["verify"] > 0 and st["steps"] >= 1
