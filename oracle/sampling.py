"""Sampling at temperature T > 0 and speculative rejection sampling, restated (oracle; tests only).

The reference decodes greedily and names rejection sampling for T > 0 as its next step
(docs/flatspec-design.md:19, item F6; README.md:84). The algorithm is the standard speculative
sampling of Leviathan et al. (2023) and Chen et al. (2023):

  for draft i = 0 .. K-1 (x_i drawn from the draft distribution q_i):
      accept x_i with probability min(1, p_i(x_i) / q_i(x_i));
      on the first rejection, emit a sample of norm(max(0, p_i - q_i)) and stop;
  if all K are accepted, emit a sample of p_K (the bonus token).

p_i = softmax(target_logits_i / T), q_i = softmax(draft_logits_i / T) over the draft's
vocabulary [0, Vd) (zero beyond it); a deterministic drafter (prompt lookup, replay) is the
point mass q_i = delta(x_i). The emitted tokens are distributed exactly as sampling from the
target alone.

Random numbers: Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as
1, 2, 3", SC 2011), key = (seed low, seed high), counter = (n low, n high, stream, 0); a uniform
is the first output word's top 24 bits times 2^-24. Draw n of a step with base counter c:
acceptance of draft i uses n = c + 2i, the residual or bonus sample n = c + 2i + 1 (stream 0);
draft sampling uses stream 1.

Sampling by inverse CDF: the smallest index j with cumsum(w)[j] > u * sum(w).

Pins (tests/test_oracle_sampling.py): Philox against the published known-answer vectors of
Random123; inverse-CDF sampling against hand cases; the whole acceptance rule by exact
enumeration of the emitted-token distribution on small vocabularies (it must equal p_0 for every
q), which a wrong acceptance ratio or residual fails.
"""

from __future__ import annotations

import numpy as np

_M0, _M1 = 0xD2511F53, 0xCD9E8D57
_W0, _W1 = 0x9E3779B9, 0xBB67AE85
_MASK = 0xFFFFFFFF


def philox4x32_10(ctr, key):
    """Philox4x32 with 10 rounds: 4 counter words, 2 key words -> 4 output words (Python ints)."""
    c0, c1, c2, c3 = (int(v) & _MASK for v in ctr)
    k0, k1 = (int(v) & _MASK for v in key)
    for r in range(10):
        if r:
            k0 = (k0 + _W0) & _MASK
            k1 = (k1 + _W1) & _MASK
        p0 = _M0 * c0
        p1 = _M1 * c2
        hi0, lo0 = p0 >> 32, p0 & _MASK
        hi1, lo1 = p1 >> 32, p1 & _MASK
        c0, c1, c2, c3 = (hi1 ^ c1 ^ k0) & _MASK, lo1, (hi0 ^ c3 ^ k1) & _MASK, lo0
    return c0, c1, c2, c3


def random_u32(seed: int, n: int, stream: int = 0) -> int:
    return philox4x32_10((n & _MASK, (n >> 32) & _MASK, stream, 0), (seed & _MASK, (seed >> 32) & _MASK))[0]


def uniform(seed: int, n: int, stream: int = 0) -> float:
    """A uniform in [0, 1) with 24 random bits."""
    return (random_u32(seed, n, stream) >> 8) * 2.0 ** -24


def probs(logits, temperature: float, vocab: int | None = None):
    """softmax(logits / T) in float64; entries at or beyond `vocab` are zero."""
    l = np.asarray(logits, dtype=np.float64).copy()
    if vocab is not None:
        l[vocab:] = -np.inf
    z = (l - l.max()) / temperature
    e = np.exp(z)
    return e / e.sum()


def sample_inverse_cdf(w, u: float) -> int:
    w = np.asarray(w, dtype=np.float64)
    c = np.cumsum(w)
    return int(np.searchsorted(c, u * c[-1], side="right"))


def residual(p, q):
    r = np.maximum(p - q, 0.0)
    return r


def spec_accept_sampled(target_logits, drafts, temperature: float, seed: int, counter: int,
                        draft_logits=None, draft_vocab: int | None = None):
    """(n accepted, emitted token, keep = n + 1) for one speculative step; draft_logits None =
    point-mass drafts."""
    K = len(drafts)
    for i in range(K):
        p = probs(target_logits[i], temperature)
        if draft_logits is None:
            q = np.zeros_like(p)
            q[drafts[i]] = 1.0
        else:
            q = np.zeros_like(p)
            qd = probs(draft_logits[i], temperature)
            q[:qd.size] = qd
            if draft_vocab is not None:
                q[draft_vocab:] = 0.0
        x = drafts[i]
        u = uniform(seed, counter + 2 * i)
        if u * q[x] < p[x]:
            continue
        return i, sample_inverse_cdf(residual(p, q), uniform(seed, counter + 2 * i + 1)), i + 1
    p = probs(target_logits[K], temperature)
    return K, sample_inverse_cdf(p, uniform(seed, counter + 2 * K + 1)), K + 1


def emitted_first_token_distribution(p0, q0):
    """Exact distribution of the first emitted token of a step whose first draft is drawn from q0:
    sum over x of q0(x) [min(1, p0(x)/q0(x)) delta_x + (1 - min(1, p0(x)/q0(x))) norm(max(0, p0 - q0))].
    Equals p0 for a correct rule."""
    p0 = np.asarray(p0, dtype=np.float64)
    q0 = np.asarray(q0, dtype=np.float64)
    r = residual(p0, q0)
    rn = r / r.sum() if r.sum() > 0 else r
    out = np.zeros_like(p0)
    for x in range(p0.size):
        if q0[x] == 0:
            continue
        a = min(1.0, p0[x] / q0[x])
        out[x] += q0[x] * a
        out += q0[x] * (1 - a) * rn
    return out
