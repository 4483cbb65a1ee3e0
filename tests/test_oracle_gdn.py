"""Pins the Gated-DeltaNet oracle (oracle/gdn.py): closed forms, the prefix property, and
golden vectors from an independent implementation (transformers' recurrent gated delta rule,
tests/golden/gdn_transformers.npz; its state is [H, Dk, Dv], the transpose of ours)."""

import os

import numpy as np
import torch

from oracle import gdn as G

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "gdn_transformers.npz")


def test_matches_transformers_golden():
    # transformers casts its inputs to fp32 inside the recurrence, so agreement is to fp32
    # rounding (~1e-6 relative); a dropped term or a wrong index would be off by O(1).
    z = np.load(GOLDEN)
    S0 = np.swapaxes(z["S0_kv"], -1, -2)  # [H, Dv, Dk]
    y, states = G.recurrence(z["q"], z["k"], z["v"], z["a"], z["b"], z["A_log"], z["dt_bias"], S0)
    np.testing.assert_allclose(y, z["y"], rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(states, np.swapaxes(z["states_kv"], -1, -2), rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(states[-1], np.swapaxes(z["S_final_kv"], -1, -2), rtol=2e-5, atol=2e-6)


def test_beta_zero_is_pure_decay():
    rng = np.random.default_rng(0)
    H, Dk, Dv = 2, 8, 4
    S = rng.standard_normal((H, Dv, Dk))
    q, k, v = rng.standard_normal((H, Dk)), rng.standard_normal((H, Dk)), rng.standard_normal((H, Dv))
    g = np.array([0.5, 0.9])
    S1, y = G.step(S, q, k, v, g, np.zeros(H))
    np.testing.assert_allclose(S1, g[:, None, None] * S)
    np.testing.assert_allclose(y, np.einsum("hvk,hk->hv", S1, q))


def test_unit_key_full_write_stores_v():
    # g = 1, beta = 1, |k| = 1: S' = S (I - k k^T) + v k^T, so S' k = v exactly (delta-rule write)
    rng = np.random.default_rng(1)
    H, Dk, Dv = 3, 16, 8
    S = rng.standard_normal((H, Dv, Dk))
    k = rng.standard_normal((H, Dk))
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((H, Dv))
    S1, _ = G.step(S, np.zeros((H, Dk)), k, v, np.ones(H), np.ones(H))
    np.testing.assert_allclose(np.einsum("hvk,hk->hv", S1, k), v, rtol=1e-12, atol=1e-12)


def test_zero_query_gives_zero_output_and_gates_range():
    rng = np.random.default_rng(2)
    T, H, D = 4, 2, 8
    y, _ = G.recurrence(np.zeros((T, H, D)), rng.standard_normal((T, H, D)), rng.standard_normal((T, H, D)),
                        rng.standard_normal((T, H)), rng.standard_normal((T, H)), np.zeros(H), np.zeros(H),
                        np.zeros((H, D, D)))
    assert np.all(y == 0)
    g, beta = G.gates(np.array([-50.0, 0.0, 50.0]), np.array([-50.0, 0.0, 50.0]), 0.0, 0.0)
    assert np.all((g > 0) & (g <= 1)) and np.isclose(g[1], np.exp(-np.log(2.0)))
    assert np.isclose(beta[1], 0.5) and beta[0] < 1e-20 and np.isclose(beta[2], 1.0)


def test_prefix_property_and_select():
    rng = np.random.default_rng(3)
    T, H, Dk, Dv = 6, 2, 8, 8
    args = [rng.standard_normal((T, H, Dk)), rng.standard_normal((T, H, Dk)), rng.standard_normal((T, H, Dv)),
            rng.standard_normal((T, H)), rng.standard_normal((T, H)), rng.standard_normal(H), rng.standard_normal(H)]
    S0 = rng.standard_normal((H, Dv, Dk))
    y, states = G.recurrence(*args, S0)
    for keep in range(1, T + 1):
        yk, sk = G.recurrence(*[a[:keep] for a in args[:5]], *args[5:], S0)
        np.testing.assert_array_equal(sk[-1], states[keep - 1])
        np.testing.assert_array_equal(yk, y[:keep])


def test_conv_window_selection_exhaustive():
    rng = np.random.default_rng(4)
    C, kw = 5, 4
    w = rng.standard_normal((C, kw))
    st0 = rng.standard_normal((kw - 1, C))
    for fed in range(1, 7):
        x = rng.standard_normal((fed, C))
        out, st_full, window = G.conv_silu(x, st0, w)
        for keep in range(1, fed + 1):
            out_k, st_k, _ = G.conv_silu(x[:keep], st0, w)
            _, conv_sel = G.select(None if keep == fed else np.zeros((fed, 1)), window, keep, fed, None, st_full)
            np.testing.assert_array_equal(conv_sel, st_k)
            np.testing.assert_array_equal(out_k, out[:keep])


def test_gated_rmsnorm_closed_forms_and_torch():
    rng = np.random.default_rng(11)
    D, eps = 128, 1e-6
    y = rng.standard_normal((3, 4, D))
    z = rng.standard_normal((3, 4, D)) * 2
    w = rng.uniform(0.5, 1.5, D)
    got = G.gated_rmsnorm(y, z, w, eps)
    yt, zt, wt = (torch.tensor(a, dtype=torch.float64) for a in (y, z, w))
    ref = torch.nn.functional.rms_norm(yt, (D,), weight=wt, eps=eps) * torch.nn.functional.silu(zt)
    np.testing.assert_allclose(got, ref.numpy(), rtol=1e-12, atol=1e-12)
    assert np.array_equal(G.gated_rmsnorm(y, np.zeros_like(z), w, eps), np.zeros_like(y))  # silu(0) = 0
    c = np.full((D,), -2.5)  # a constant head normalises to -1 (up to eps)
    np.testing.assert_allclose(G.gated_rmsnorm(c, z[0, 0], w, eps),
                               -w * z[0, 0] / (1 + np.exp(-z[0, 0])) / np.sqrt(1 + eps / 6.25), rtol=1e-12)
    np.testing.assert_allclose(G.gated_rmsnorm(7.0 * y, z, w, 0.0), G.gated_rmsnorm(y, z, w, 0.0), rtol=1e-12)


def test_conv_impulse_response_fixes_the_tap_order():
    """Zero state and a unit impulse at token 0 of channel c: out[t, c] = silu(w[c, KW-1-t]) for
    t < KW and 0 after, every other channel 0. The newest token meets the last tap (Conv1d over
    [state; x] with the window ending at the current token), so a reversed tap order fails."""
    rng = np.random.default_rng(12)
    C, kw, T = 6, 4, 7
    w = rng.standard_normal((C, kw))
    w[:, 0] += 3.0  # taps made distinct in size so no order coincides with another
    silu = lambda v: v / (1 + np.exp(-v))
    for c in range(C):
        x = np.zeros((T, C))
        x[0, c] = 1.0
        out, state, window = G.conv_silu(x, np.zeros((kw - 1, C)), w)
        expect = np.zeros((T, C))
        for t in range(kw):
            expect[t, c] = silu(w[c, kw - 1 - t])
        np.testing.assert_array_equal(out, expect)
        np.testing.assert_array_equal(state, x[T - kw + 1:])
        np.testing.assert_array_equal(window[kw - 1:], x)


def test_conv_matches_torch_depthwise_conv1d():
    """The conv of transformers' and mlx_lm's Qwen3.5 mixer is a depthwise Conv1d (groups = C,
    weight [C, 1, KW], no bias) over [conv_state; x] along time, then SiLU; torch's conv1d in fp64
    with asymmetric taps and a nonzero state must agree to rounding."""
    rng = np.random.default_rng(13)
    C, kw, T = 10, 4, 9
    w = rng.standard_normal((C, kw)) * np.array([0.2, -0.7, 1.3, 2.1])
    st = rng.standard_normal((kw - 1, C))
    x = rng.standard_normal((T, C))
    got, new_state, _ = G.conv_silu(x, st, w)
    seq = torch.tensor(np.concatenate([st, x]).T[None], dtype=torch.float64)  # [1, C, KW-1+T]
    ref = torch.nn.functional.conv1d(seq, torch.tensor(w[:, None, :], dtype=torch.float64), groups=C)
    ref = torch.nn.functional.silu(ref)[0].T.numpy()  # [T, C]
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)
    np.testing.assert_array_equal(new_state, np.concatenate([st, x])[-(kw - 1):])
