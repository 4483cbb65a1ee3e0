"""Sampling at T > 0 and speculative rejection sampling on the GPU (csrc/sample.hip,
skinny_mlx.sampling): the Philox stream bit-exact against the oracle; row statistics; samples equal
the oracle's inverse CDF (except when the threshold lies within 1e-4 of a CDF boundary, where fp32
and fp64 sums may order differently); the emitted-token distribution of the acceptance kernel
equals the target's; end to end, generations are reproducible from their seed, graphed and eager
alike, and equal greedy decoding at a vanishing temperature."""

import numpy as np
import pytest
import torch

from oracle import sampling as S
from skinny_mlx import kernels as K
from skinny_mlx import patch as P
from skinny_mlx.model import build_model
from skinny_mlx.mtp import load_mtp_head
from skinny_mlx.sampling import sample, speculative_sample
from skinny_mlx.spec import MTPDrafter, PromptLookupDrafter, greedy

pytestmark = pytest.mark.gpu
MARGIN = 1e-4


def _bf16_logits(rows, v, seed, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn((rows, v), generator=g) * scale).to(torch.bfloat16)


def _counter(dev, value):
    return torch.tensor([value], dtype=torch.int64, device=dev)


@pytest.mark.parametrize("seed", [0, 12345, 2 ** 40 + 7])
@pytest.mark.parametrize("stream", [0, 1])
def test_random_uniform_is_the_oracle_philox(dev, seed, stream):
    base = 2 ** 32 - 100  # crosses into the counter's high word
    got = K.random_uniform(seed, _counter(dev, base), 300, offset=3, rng_stream=stream).cpu().numpy()
    ref = np.array([S.uniform(seed, base + 3 + i, stream) for i in range(300)], dtype=np.float32)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("T", [0.5, 1.0, 2.0])
def test_row_stats(dev, T):
    l = _bf16_logits(5, 3000, 1)
    st = K.row_stats(l.to(dev), T).cpu().double().numpy()
    lf = l.float().double().numpy()
    m = lf.max(1)
    z = np.exp((lf - m[:, None]) / T).sum(1)
    assert np.array_equal(st[:, 0], m)
    assert np.allclose(st[:, 1], z, rtol=1e-5)


def _check_inverse_cdf(tok, w, u):
    """tok is the inverse-CDF sample of weights w at u, or the threshold is within MARGIN of the
    CDF boundary between tok and the exact answer."""
    ref = S.sample_inverse_cdf(w, u)
    if tok == ref:
        return True
    c = np.cumsum(w)
    thr = u * c[-1]
    boundary = c[min(tok, ref)]
    return abs(boundary - thr) <= MARGIN * c[-1]


@pytest.mark.parametrize("T", [0.6, 1.3])
def test_sample_rows_is_the_inverse_cdf(dev, T):
    rows, v, seed, base = 64, 2000, 99, 1000
    l = _bf16_logits(rows, v, 2)
    got = K.sample_rows(l.to(dev), T, seed, _counter(dev, base), offset=5).cpu().numpy()
    lf = l.float().double().numpy()
    for r in range(rows):
        w = np.exp((lf[r] - lf[r].max()) / T)
        assert _check_inverse_cdf(int(got[r]), w, S.uniform(seed, base + 5 + r)), r


def test_sample_rows_distribution(dev):
    v, T, n = 40, 0.8, 50000
    l = _bf16_logits(1, v, 3)
    rows = l.expand(n, v).contiguous().to(dev)
    got = K.sample_rows(rows, T, 7, _counter(dev, 0)).cpu().numpy()
    emp = np.bincount(got, minlength=v) / n
    p = S.probs(l.float().numpy()[0], T)
    assert 0.5 * np.abs(emp - p).sum() < 0.015


def _oracle_step(tl, dl, drafts, T, seed, c, vd):
    """The oracle step: (n accepted, the weights the emitted token is sampled from, its uniform),
    or None when an acceptance decision lies within MARGIN of flipping under fp32 rounding."""
    K_ = len(drafts)
    for i in range(K_):
        p = S.probs(tl[i], T)
        q = np.zeros_like(p)
        if dl is None:
            q[drafts[i]] = 1.0
        else:
            q[:vd] = S.probs(dl[i], T)
        x = drafts[i]
        u = S.uniform(seed, c + 2 * i)
        if abs(u * q[x] - p[x]) <= MARGIN * max(p[x], q[x], 1e-30):
            return None
        if u * q[x] < p[x]:
            continue
        return i, S.residual(p, q), S.uniform(seed, c + 2 * i + 1)
    return K_, S.probs(tl[K_], T), S.uniform(seed, c + 2 * K_ + 1)


@pytest.mark.parametrize("T", [0.7, 1.3])
@pytest.mark.parametrize("point_mass", [False, True])
def test_spec_accept_matches_oracle(dev, T, point_mass):
    rng = np.random.default_rng(0)
    k, v, vd, seed = 3, 700, 500, 4242
    out = torch.empty((3,), dtype=torch.int32, device=dev)
    checked = 0
    for case in range(60):
        tl = _bf16_logits(k + 1, v, 100 + case)
        dl = None if point_mass else _bf16_logits(k, vd, 200 + case)
        tlf = tl.float().double().numpy()
        dlf = None if dl is None else dl.float().double().numpy()
        drafts = []
        for i in range(k):  # draft from q, or the target's argmax so acceptances happen
            if case % 3 == 0:
                drafts.append(int(tlf[i][:vd].argmax()))
            elif dlf is not None:
                drafts.append(int(rng.choice(vd, p=S.probs(dlf[i], T))))
            else:
                drafts.append(int(rng.integers(vd)))
        c = 17 * case
        tld = tl.to(dev)
        st = K.row_stats(tld, T)
        dld = None if dl is None else dl.to(dev)
        sd = None if dld is None else K.row_stats(dld, T)
        K.spec_accept_sampled(tld, st, torch.tensor(drafts, dtype=torch.int32, device=dev), T, seed,
                              _counter(dev, c), out, dld, sd)
        n, tok, keep = out.cpu().tolist()
        ref = _oracle_step(tlf, dlf, drafts, T, seed, c, vd)
        if ref is None:
            continue
        rn, w, u = ref
        assert (n, keep) == (rn, rn + 1), case
        assert _check_inverse_cdf(tok, w, u), case
        checked += 1
    assert checked >= 55


@pytest.mark.parametrize("point_mass", [False, True])
def test_spec_accept_emits_the_target_distribution(dev, point_mass):
    rng = np.random.default_rng(5)
    v, k, T, trials = 10, 2, 0.8, 4000
    tl = _bf16_logits(k + 1, v, 7)
    dl = _bf16_logits(k, v, 8)
    tlf, dlf = tl.float().double().numpy(), dl.float().double().numpy()
    tld = tl.to(dev)
    st = K.row_stats(tld, T)
    dld = None if point_mass else dl.to(dev)
    sd = None if point_mass else K.row_stats(dld, T)
    res = torch.empty((trials, 3), dtype=torch.int32, device=dev)
    counter = _counter(dev, 0)
    firsts = []
    for t in range(trials):
        if point_mass:
            drafts = [int(rng.integers(v)) for _ in range(k)]
        else:
            drafts = [int(rng.choice(v, p=S.probs(dlf[i], T))) for i in range(k)]
        firsts.append(drafts[0])
        counter.fill_(10 * t)
        K.spec_accept_sampled(tld, st, torch.tensor(drafts, dtype=torch.int32, device=dev), T, 3, counter, res[t],
                              dld, sd)
    r = res.cpu().numpy()
    first = np.where(r[:, 0] >= 1, np.array(firsts), r[:, 1])
    emp = np.bincount(first, minlength=v) / trials
    p0 = S.probs(tlf[0], T)
    assert 0.5 * np.abs(emp - p0).sum() < 0.035
    assert (r[:, 2] == r[:, 0] + 1).all() and r[:, 0].max() <= k


@pytest.fixture(scope="module", params=["tiny-dense", "tiny-hybrid", "tiny-qwen35"])
def model(request):
    m = build_model(request.param)
    P.patch_model(m)
    return m


def _prompt(n=40, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 1024, (n,), generator=g).tolist()


def test_sampling_is_reproducible(model):
    prompt = _prompt(seed=1)
    a = sample(model, prompt, 24, 0.8, seed=3)
    assert a == sample(model, prompt, 24, 0.8, seed=3) == sample(model, prompt, 24, 0.8, seed=3, graphs=False)
    assert a != sample(model, prompt, 24, 0.8, seed=4)
    assert all(0 <= t < model.args.vocab_size for t in a)
    head = load_mtp_head(model)
    st = {}
    b = speculative_sample(model, prompt, 24, MTPDrafter(model, head, vocab=512), 3, 0.8, seed=3, stats=st)
    assert b == speculative_sample(model, prompt, 24, MTPDrafter(model, head, vocab=512), 3, 0.8, seed=3)
    assert b == speculative_sample(model, prompt, 24, MTPDrafter(model, head, vocab=512, graphs=False), 3, 0.8,
                                   seed=3, graphs=False)
    assert st["tokens_per_step"] >= 1.0 and all(0 <= t < model.args.vocab_size for t in b)
    c = speculative_sample(model, prompt, 24, PromptLookupDrafter(2), 3, 0.8, seed=3)
    assert len(c) == 24


def _greedy_up_to_exact_ties(model, prompt, ref, got):
    """got == ref, or they first differ where the model's logits hold an exact top tie between
    the two tokens (at T -> 0 a tie is a coin flip for the sampler, first-index for greedy)."""
    from skinny_mlx.cache import make_prompt_cache

    for i, (a, b) in enumerate(zip(ref, got)):
        if a != b:
            logits = model(prompt + ref[:i], make_prompt_cache(model))[-1].float()
            return bool(logits[a] == logits.max() and logits[b] == logits.max())
    return len(ref) == len(got)


def test_vanishing_temperature_is_greedy(model):
    prompt = _prompt(seed=2)
    ref = greedy(model, prompt, 24)
    assert _greedy_up_to_exact_ties(model, prompt, ref, sample(model, prompt, 24, 1e-4, seed=1))
    head = load_mtp_head(model)
    got = speculative_sample(model, prompt, 24, MTPDrafter(model, head, vocab=512), 3, 1e-4, seed=1)
    assert _greedy_up_to_exact_ties(model, prompt, ref, got)
    got = speculative_sample(model, prompt, 24, PromptLookupDrafter(2), 3, 1e-4, seed=1)
    assert _greedy_up_to_exact_ties(model, prompt, ref, got)
