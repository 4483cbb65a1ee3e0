"""Gated-DeltaNet arithmetic restated in numpy fp64 (oracle; tests only).

Reference:
  * recurrence S <- g S (I - beta k k^T) + beta v k^T, y = S q, state [H, Dv, Dk]
    (bench/reversal_check.py:5, 21-25 `_apply`), with decay g = exp(compute_g(A_log, a,
    dt_bias)) and beta = sigmoid(b) (reversal_check.py:43-46); compute_g lives in the
    third-party mlx_lm (gated_delta.compute_g, version >= 0.31, not vendored) — restated from
    its published form g = -exp(A_log) * softplus(a + dt_bias), which transformers' qwen3_5
    text also gives (transformers/models/qwen3_5/modeling_qwen3_5.py: `g = -self.A_log.float()
    .exp() * F.softplus(a.float() + self.dt_bias)`);
  * q and k l2-normalised (eps 1e-6 inside the square root), q scaled by Dk^-1/2 (the
    transformers restatement `l2norm` + `scale = 1 / query.shape[-1] ** 0.5`);
  * the output norm y / rms(y) * w * silu(z) per head (the gated RMSNorm that follows the
    recurrence in mlx_lm's qwen3_5 layer; transformers' Qwen3_5RMSNormGated restates it);
  * causal depthwise conv of width 4 over [conv_state; x] then SiLU; rollback keeps the state
    after `keep` tokens and conv rows keep .. keep+2 of [conv_state; x]
    (skinny_mlx/rollback.py:58-73).

Pins (tests/test_oracle_gdn.py): closed-form special cases (beta = 0 gives pure decay;
g = 1, beta = 1, |k| = 1 writes v exactly: S'k = v; zero q gives y = 0), the prefix
property, the output norm against torch's rms_norm and silu and its closed forms (z = 0 gives
0; a constant head gives w * silu(z) up to eps; scale invariance), and golden vectors from transformers' torch_recurrent_gated_delta_rule
(tests/golden/gdn_transformers.npz, written by tests/golden/make_gdn_golden.py).
"""

from __future__ import annotations

import numpy as np


def softplus(x):
    x = np.asarray(x, np.float64)
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


def gates(a, b, A_log, dt_bias):
    """(decay g in (0, 1], beta) per (token, head)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    g = np.exp(-np.exp(np.asarray(A_log, np.float64)) * softplus(a + np.asarray(dt_bias, np.float64)))
    beta = 1.0 / (1.0 + np.exp(-b))
    return g, beta


def l2norm(x, eps=1e-6):
    x = np.asarray(x, np.float64)
    return x / np.sqrt((x * x).sum(-1, keepdims=True) + eps)


def step(S, q, k, v, g, beta):
    """One token for all heads. S [H, Dv, Dk]; q, k [H, Dk] (already normalised/scaled);
    v [H, Dv]; g, beta [H]. Returns (S', y [H, Dv])."""
    S = g[:, None, None] * S
    kv = np.einsum("hvk,hk->hv", S, k)
    S = S + np.einsum("hv,hk->hvk", beta[:, None] * (v - kv), k)
    return S, np.einsum("hvk,hk->hv", S, q)


def recurrence(q, k, v, a, b, A_log, dt_bias, S0):
    """Tokens t = 0..T-1: q, k [T, H, Dk] raw (normalised here), v [T, H, Dv], a, b [T, H].
    Returns (y [T, H, Dv], states [T, H, Dv, Dk]) in fp64."""
    q = l2norm(q) / np.sqrt(np.asarray(q).shape[-1])
    k = l2norm(k)
    v = np.asarray(v, np.float64)
    g, beta = gates(a, b, A_log, dt_bias)
    S = np.asarray(S0, np.float64).copy()
    ys, states = [], []
    for t in range(q.shape[0]):
        S, y = step(S, q[t], k[t], v[t], g[t], beta[t])
        ys.append(y)
        states.append(S)
    return np.stack(ys), np.stack(states)


def conv_silu(x, conv_state, w):
    """x [T, C], conv_state [KW-1, C], w [C, KW] -> (silu(conv) [T, C], new conv_state, window
    [T+KW-1, C] = [conv_state; x])."""
    x = np.asarray(x, np.float64)
    window = np.concatenate([np.asarray(conv_state, np.float64), x], axis=0)
    kw = w.shape[1]
    T = x.shape[0]
    out = np.zeros_like(x)
    for t in range(T):
        out[t] = (window[t:t + kw] * np.asarray(w, np.float64).T).sum(0)
    out = out / (1.0 + np.exp(-out))
    return out, window[T:T + kw - 1], window


def gated_rmsnorm(y, z, w, eps):
    """The mixer's output norm per head (qwen3_5's gated RMSNorm, the layer after
    gated_delta_update): y [..., D] fp64, z [..., D], w [D] -> y / sqrt(mean(y^2) + eps) * w *
    silu(z)."""
    y = np.asarray(y, np.float64)
    z = np.asarray(z, np.float64)
    inv = 1.0 / np.sqrt((y * y).mean(-1, keepdims=True) + eps)
    return y * inv * np.asarray(w, np.float64) * (z / (1.0 + np.exp(-z)))


def select(states, window, keep: int, fed: int, state_now, conv_now, kw: int = 4):
    """Rollback selection (rollback.py:61-70): keep == fed leaves the state as the forward left
    it; 1 <= keep < fed takes states[keep-1] and window rows keep .. keep+kw-2."""
    if keep == fed:
        return state_now, conv_now
    if not 1 <= keep < fed:
        raise ValueError("keep out of range")
    return states[keep - 1], window[keep:keep + kw - 1]
