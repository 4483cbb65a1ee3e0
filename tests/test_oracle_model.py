"""Pins the decoder oracle's building blocks (oracle/model.py) by closed forms, so that a wrong
sign, index or dropped term in the restatement fails here rather than agreeing with the device."""

import numpy as np

from oracle import model as OM
from oracle import w4


def _ones_bits(n):
    return w4.f32_to_bf16(np.ones(n, np.float32))


def test_rmsnorm_closed_forms():
    # a constant row normalises to +-1 (up to eps), for any magnitude
    for c in (0.25, -3.0, 40.0):
        y = OM.rmsnorm(np.full(64, c), _ones_bits(64), 0.0)
        assert np.allclose(y, np.sign(c), atol=2 ** -8)
    # scale invariance, and the weight multiplies element-wise
    rng = np.random.default_rng(0)
    x = rng.standard_normal(128)
    w = w4.f32_to_bf16(rng.uniform(0.5, 2.0, 128).astype(np.float32))
    assert np.allclose(OM.rmsnorm(7.0 * x, w, 0.0), OM.rmsnorm(x, w, 0.0), rtol=2 ** -7, atol=1e-6)
    ref = x / np.sqrt((x * x).mean()) * w4.bf16_to_f32(w)
    assert np.allclose(OM.rmsnorm(x, w, 0.0), ref, rtol=2 ** -7, atol=1e-6)


def test_rope_closed_forms():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(128)
    assert np.allclose(OM.rope(x, 0, 1e6), x)  # position 0 is the identity
    y = OM.rope(x, 37, 1e6)
    half = 64
    # each (i, i + D/2) pair is rotated: its norm is preserved
    assert np.allclose(x[:half] ** 2 + x[half:] ** 2, y[:half] ** 2 + y[half:] ** 2)
    # rotations compose: rope(rope(x, p), q) == rope(x, p + q)
    assert np.allclose(OM.rope(OM.rope(x, 11, 1e4), 26, 1e4), OM.rope(x, 37, 1e4))
    # D = 2: inverse frequency 1, the pair (a, b) turns by `pos` radians counter-clockwise
    a, b, p = 0.3, -1.2, 2
    assert np.allclose(OM.rope(np.array([a, b]), p, 1e6),
                       [a * np.cos(p) - b * np.sin(p), b * np.cos(p) + a * np.sin(p)])
    # frequency of pair i is theta^(-2i/D): pair 1 of D = 4 at theta 100 turns by pos / 10
    z = OM.rope(np.array([0.0, 1.0, 0.0, 0.0]), 5, 100.0)
    assert np.allclose(z, [0.0, np.cos(0.5), 0.0, np.sin(0.5)])


def test_attention_row_closed_forms():
    rng = np.random.default_rng(2)
    q = rng.standard_normal(16)
    keys = rng.standard_normal((1, 16))
    vals = rng.standard_normal((1, 16))
    assert np.allclose(OM.attention_row(q, keys, vals, 0.25), vals[0])  # one key: its value
    keys = np.zeros((5, 16))
    vals = rng.standard_normal((5, 16))
    assert np.allclose(OM.attention_row(q, keys, vals, 0.25), vals.mean(0))  # equal scores: the mean
    keys = np.zeros((3, 16))
    keys[1] = q * 100.0  # one dominant score selects its value
    assert np.allclose(OM.attention_row(q, keys, vals[:3], 1.0), vals[1])
