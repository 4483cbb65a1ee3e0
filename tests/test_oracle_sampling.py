"""Pins of oracle/sampling.py: Philox4x32-10 against the published Random123 known-answer
vectors; inverse-CDF sampling on hand cases; the rejection rule through the exact distribution of
the first emitted token (it must equal the target's p0 for every draft distribution q0), with a
planted mistake that the same check catches; and a Monte-Carlo run of the whole step."""

import numpy as np
import pytest

from oracle import sampling as S


@pytest.mark.parametrize("ctr,key,expect", [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
])
def test_philox_known_answers(ctr, key, expect):
    assert S.philox4x32_10(ctr, key) == expect


def test_uniforms():
    u = [S.uniform(7, n) for n in range(2000)]
    assert all(0.0 <= v < 1.0 for v in u)
    assert all((v * 2 ** 24) == int(v * 2 ** 24) for v in u)  # 24-bit grid
    assert abs(np.mean(u) - 0.5) < 0.02
    assert S.uniform(7, 5, stream=0) != S.uniform(7, 5, stream=1)
    assert S.uniform(7, 5) != S.uniform(8, 5)
    assert S.random_u32(3, 2 ** 32 + 1) != S.random_u32(3, 1)  # the counter's high word counts


def test_inverse_cdf_hand_cases():
    w = [1.0, 1.0, 2.0]
    assert S.sample_inverse_cdf(w, 0.0) == 0
    assert S.sample_inverse_cdf(w, 0.49) == 1  # 0.49 * 4 = 1.96 < cumsum 2
    assert S.sample_inverse_cdf(w, 0.5) == 2   # 2.0 is not > 2: the next index
    assert S.sample_inverse_cdf(w, 0.999) == 2
    assert S.sample_inverse_cdf([0.0, 3.0, 0.0], 0.0) == 1  # zero weights are never drawn
    assert S.sample_inverse_cdf([0.0, 3.0, 0.0], 0.99) == 1


def test_probs_and_temperature():
    l = np.array([1.0, 2.0, 4.0])
    p = S.probs(l, 1.0)
    assert np.allclose(p, np.exp(l) / np.exp(l).sum())
    assert np.allclose(S.probs(l, 0.5), np.exp(2 * l) / np.exp(2 * l).sum())
    assert S.probs(l, 1.0, vocab=2)[2] == 0.0


def _rand_dist(rng, v, zeros=0):
    p = rng.random(v) ** 3
    if zeros:
        p[rng.choice(v, zeros, replace=False)] = 0.0
    return p / p.sum()


@pytest.mark.parametrize("seed", range(20))
def test_emitted_distribution_is_the_target(seed):
    rng = np.random.default_rng(seed)
    v = int(rng.integers(2, 12))
    p0 = _rand_dist(rng, v)
    q0 = _rand_dist(rng, v, zeros=int(rng.integers(0, v - 1)))  # a pruned draft vocabulary
    assert np.allclose(S.emitted_first_token_distribution(p0, q0), p0, atol=1e-12)
    point = np.zeros(v)
    point[int(rng.integers(v))] = 1.0  # deterministic drafts
    assert np.allclose(S.emitted_first_token_distribution(p0, point), p0, atol=1e-12)


def test_a_wrong_residual_is_caught():
    rng = np.random.default_rng(0)
    p0, q0 = _rand_dist(rng, 6), _rand_dist(rng, 6)

    def wrong(p, q):  # resampling from p itself instead of max(0, p - q)
        out = np.zeros_like(p)
        for x in range(p.size):
            a = min(1.0, p[x] / q[x])
            out[x] += q[x] * a
            out += q[x] * (1 - a) * p
        return out

    assert not np.allclose(wrong(p0, q0), p0, atol=1e-3)
    assert np.allclose(S.emitted_first_token_distribution(p0, q0), p0, atol=1e-12)


@pytest.mark.parametrize("point_mass", [False, True])
def test_monte_carlo_step(point_mass):
    """The full step function: first emitted token ~ p0 (drafts drawn from q by numpy)."""
    rng = np.random.default_rng(1)
    v, k, T = 6, 2, 0.8
    tl = rng.normal(size=(k + 1, v)) * 2
    dl = rng.normal(size=(k, v)) * 2
    p0 = S.probs(tl[0], T)
    q0 = S.probs(dl[0], T)
    trials = 6000
    counts = np.zeros(v)
    for t in range(trials):
        if point_mass:
            drafts = [int(rng.integers(v)) for _ in range(k)]
            n, tok, keep = S.spec_accept_sampled(tl, drafts, T, seed=5, counter=10 * t)
        else:
            drafts = [int(rng.choice(v, p=S.probs(dl[i], T))) for i in range(k)]
            n, tok, keep = S.spec_accept_sampled(tl, drafts, T, seed=5, counter=10 * t, draft_logits=dl)
        assert keep == n + 1 and 0 <= n <= k
        counts[drafts[0] if n >= 1 else tok] += 1
    emp = counts / trials
    assert 0.5 * np.abs(emp - p0).sum() < 0.03
    if not point_mass:
        assert 0.5 * np.abs(q0 - p0).sum() > 0.1  # the check is not vacuous: q differs from p
