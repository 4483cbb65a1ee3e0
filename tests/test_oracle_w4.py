"""Pins the W4 g64 oracle (oracle/w4.py) before the device path is checked against it.

Each check is chosen so a plausible slip (wrong nibble order, group broadcast along the
wrong axis, scale/bias swapped, bf16 rounding toward zero) fails at least one of them.
"""

import numpy as np
import pytest
import torch

from oracle import w4


def test_pack_known_answer():
    # element i of a word sits at bits 4i (reference qmm.py:104)
    q = np.array([[1, 2, 3, 4, 5, 6, 7, 8, 15, 0, 0, 0, 0, 0, 0, 9]], dtype=np.uint8)
    w = w4.pack_mlx(q)
    assert w.dtype == np.uint32
    assert w.tolist() == [[0x87654321, 0x9000000F]]
    assert np.array_equal(w4.unpack_mlx(w), q)


def test_pack_roundtrip_random():
    rng = np.random.default_rng(0)
    q = rng.integers(0, 16, size=(48, 256), dtype=np.uint8)
    assert np.array_equal(w4.unpack_mlx(w4.pack_mlx(q)), q)
    words = rng.integers(0, 2 ** 32, size=(16, 32), dtype=np.uint64).astype(np.uint32)
    assert np.array_equal(w4.pack_mlx(w4.unpack_mlx(words)), words)


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10 ** rng.uniform(-30, 30, 20000),
                        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 3.4e38, -1e-40], np.float32)]).astype(np.float32)
    ours = w4.f32_to_bf16(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    # ties go to even: 1 + 2^-8 is halfway between 1 and 1 + 2^-7
    assert w4.f32_to_bf16(np.array([1.00390625], np.float32))[0] == 0x3F80
    assert w4.f32_to_bf16(np.array([1.01171875], np.float32))[0] == 0x3F82
    assert np.array_equal(w4.bf16_to_f32(theirs), torch.from_numpy(x).to(torch.bfloat16).float().numpy())


def _rand_case(m, n, k, seed):
    g = torch.Generator().manual_seed(seed)
    from skinny_mlx.qmm import random_w4g64

    w, s, b = random_w4g64(n, k, generator=g)
    x = torch.randn((m, k), generator=g).to(torch.bfloat16)
    bits = lambda t: t.view(torch.int16).numpy().view(np.uint16)
    return bits(x), w4.as_u32(w), bits(s), bits(b)


def test_dequant_closed_forms():
    n, k = 16, 128
    rng = np.random.default_rng(2)
    s = w4.f32_to_bf16(np.abs(rng.standard_normal((n, k // 64))).astype(np.float32) * 0.02)
    # q = 8 everywhere with b = -8 s  ->  every weight is exactly 0
    q8 = np.full((n, k), 8, np.uint8)
    b = w4.f32_to_bf16(-8.0 * w4.bf16_to_f32(s))
    assert np.all(w4.dequant(w4.pack_mlx(q8), s, b) == 0.0)
    # q = 0 with b = 0 -> 0 ; q = 1 with b = 0 -> the group's scale, broadcast over 64 columns
    zero = np.zeros_like(s)
    assert np.all(w4.dequant(w4.pack_mlx(np.zeros((n, k), np.uint8)), s, zero) == 0.0)
    d1 = w4.dequant(w4.pack_mlx(np.ones((n, k), np.uint8)), s, zero)
    assert np.array_equal(d1, np.repeat(w4.bf16_to_f32(s).astype(np.float64), 64, axis=1))
    # bias only: q = 0 gives b broadcast over the group (catches s/b swaps)
    d2 = w4.dequant(w4.pack_mlx(np.zeros((n, k), np.uint8)), s, b)
    assert np.array_equal(d2, np.repeat(w4.bf16_to_f32(b).astype(np.float64), 64, axis=1))


def test_qmm_one_hot_selects_a_column():
    xb, w, s, b = _rand_case(1, 32, 256, 3)
    ref_w = w4.dequant(w, s, b)
    for col in (0, 63, 64, 200, 255):
        x = np.zeros((1, 256), np.float32)
        x[0, col] = 1.0
        y = w4.qmm(w4.f32_to_bf16(x), w, s, b)
        assert np.array_equal(y[0], ref_w[:, col])


def test_qmm_ones_gives_row_sums_and_affine_identity():
    xb, w, s, b = _rand_case(4, 48, 192, 4)
    deq = w4.dequant(w, s, b)
    ones = w4.f32_to_bf16(np.ones((1, 192), np.float32))
    assert np.allclose(w4.qmm(ones, w, s, b)[0], deq.sum(1), rtol=0, atol=1e-12)
    # the affine identity of reference qmm.py:8-9 gives the same product
    assert np.allclose(w4.qmm(xb, w, s, b), w4.qmm_affine(xb, w, s, b), rtol=1e-12, atol=1e-12)


def test_rel_err_metric():
    ref = np.array([[1.0, -4.0], [2.0, 0.5]])
    assert w4.rel_err(ref, ref) == 0.0
    assert w4.rel_err(ref + np.array([[0.0, 0.4], [0.0, 0.0]]), ref) == pytest.approx(0.1)


def _rand_pack(n, k, seed):
    rng = np.random.default_rng(seed)
    w = rng.integers(0, 2 ** 32, size=(n, k // 8), dtype=np.uint64).astype(np.uint32)
    s = w4.f32_to_bf16(np.abs(rng.standard_normal((n, k // 64))).astype(np.float32) * 0.02)
    b = w4.f32_to_bf16(rng.standard_normal((n, k // 64)).astype(np.float32) * 0.1)
    return w, s, b


def test_pack_roundtrip_and_multiset():
    for n, k in ((16, 128), (32, 256), (48, 640)):
        w, s, b = _rand_pack(n, k, 5)
        wf = w4.pack_frag(w, s, b)
        assert wf.shape == (n, k // 8 + k // 64) and wf.dtype == np.uint32
        w2, s2, b2 = w4.unpack_frag(wf)
        assert np.array_equal(w2, w) and np.array_equal(s2, s) and np.array_equal(b2, b)
        # same nibbles, different order: the code histogram of each 16-row tile is preserved
        qa = w4.unpack_mlx(w).reshape(n // 16, -1)
        T, P = n // 16, k // 128
        nib = wf.reshape(T, P, w4.BLOCK_WORDS)[:, :, :256].reshape(T, -1)
        qb = w4.unpack_mlx(nib)
        for t in range(T):
            assert np.array_equal(np.bincount(qa[t], minlength=16), np.bincount(qb[t], minlength=16))


def test_pack_lane_readout_reproduces_codes_scales_biases():
    """Emulating the kernel's read of each lane must give 128 + q of the documented element and
    the scale/bias of the lane's row and group."""
    rng = np.random.default_rng(6)
    n, k = 32, 256
    q = rng.integers(0, 16, size=(n, k), dtype=np.uint8)
    _, s, b = _rand_pack(n, k, 7)
    wf = w4.pack_frag(w4.pack_mlx(q), s, b)
    sf, bf = w4.bf16_to_f32(s), w4.bf16_to_f32(b)
    for t in range(n // 16):
        for g in range(k // 64):
            ops = w4.lane_operands(wf, t, g)
            for h in range(2):
                for lane in range(64):
                    row = 16 * t + lane % 16
                    c0 = 64 * g + 32 * h + 8 * (lane // 16)
                    assert np.array_equal(ops[h, lane], 128.0 + q[row, c0:c0 + 8].astype(np.float32))
            sb = w4.lane_scale_bias(wf, t, g)
            assert np.array_equal(sb[:, 0], sf[16 * t:16 * t + 16, g])
            assert np.array_equal(sb[:, 1], bf[16 * t:16 * t + 16, g])


def test_relayout_is_the_nibble_part_of_the_packed_blocks():
    """The one-argument relayout (repack_for_skinny(w)) keeps MLX's [N, K/8] shape, holds the
    same nibbles as each 16-row tile of w (per-tile code histogram), and is word for word the
    first 256 words of every packed block, so completing it with the scales and biases gives
    pack_frag exactly."""
    for n, k in ((16, 128), (48, 640)):
        w, s, b = _rand_pack(n, k, 8)
        rl = w4.relayout_frag(w)
        assert rl.shape == w.shape and rl.dtype == np.uint32
        T, P = n // 16, k // 128
        full = w4.pack_frag(w, s, b).reshape(T, P, w4.BLOCK_WORDS)
        assert np.array_equal(rl.reshape(T, P, 256), full[:, :, :256])
        qa, qb = w4.unpack_mlx(w).reshape(T, -1), w4.unpack_mlx(rl).reshape(T, -1)
        for t in range(T):
            assert np.array_equal(np.bincount(qa[t], minlength=16), np.bincount(qb[t], minlength=16))
        assert not np.array_equal(rl, w)  # a different order, not the identity
