"""GPU parity of the W4 g64 relayout and skinny qmm (HIP, through the C ABI) against the
oracle, on seeded inputs of the benchmark distributions.

Bars (from the path's contract):
  * relayout: bit-exact vs the oracle's fragment order; unrelayout(relayout(w)) == w.
  * qmm: max|y - ref| / max|ref| <= 2e-2 against fp64 dequant+matmul (reference
    qmm.py:185-186). The kernel rounds once to bf16 at the end, so the test also holds it to
    a tighter 4e-3 to catch a dropped term that the loose bar would hide.
  * bitwise M-invariance: a token's output row is identical for every M = 1..16.
"""

import numpy as np
import pytest
import torch

from oracle import w4
from skinny_mlx import qmm as Q
from tests.helpers import bits16, qmm_case, u32

pytestmark = pytest.mark.gpu

CONFIG1 = [(2560, 6144), (4096, 2560), (2560, 19456), (9728, 2560), (2560, 151936)]
# Qwen3.5-4B's own projection shapes: fused q|gate|k|v, the Gated-DeltaNet input projection, the
# MLP's gate|up and down, the 248k-row head
QWEN35 = [(2560, 10240), (2560, 12352), (2560, 18432), (9216, 2560), (2560, 248320)]


def _to(dev, *ts):
    return [t.to(dev) for t in ts]


@pytest.mark.parametrize("n,k", [(16, 128), (48, 384), (9728, 2560)])
def test_pack_bit_exact(dev, n, k):
    _, w, s, b = qmm_case(1, n, k, seed=11)
    wf = Q.repack_for_skinny(w.to(dev), s.to(dev), b.to(dev))
    assert np.array_equal(u32(wf), w4.pack_frag(u32(w), bits16(s), bits16(b)))
    w2, s2, b2 = Q.unrepack(wf)
    assert np.array_equal(u32(w2), u32(w))
    assert np.array_equal(bits16(s2), bits16(s)) and np.array_equal(bits16(b2), bits16(b))


@pytest.mark.parametrize("k,n", [(2560, 9728), (9728, 2560)])
def test_reference_two_call_sequence(dev, k, n):
    """The reference's drop-in sequence, unchanged (bench/model_matmuls.py:20, 37; qmm.py:96, 132):
    rw = repack_for_skinny(w), then skinny_qmm(x, rw, scales, biases), against the oracle. The
    relayout keeps MLX's shape and is bit-exact; its completion with the scales and biases equals the
    one-step packing, is kept for later calls and is redone when the scales change in place."""
    x, w, s, b = qmm_case(8, n, k, seed=12)
    xd, wd, sd, bd = _to(dev, x, w, s, b)
    rw = Q.repack_for_skinny(wd)
    assert rw.shape == wd.shape and rw.dtype == torch.int32
    assert np.array_equal(u32(rw), w4.relayout_frag(u32(w)))
    assert np.array_equal(u32(Q.unrepack(rw)), u32(w))
    y = Q.skinny_qmm(xd, rw, sd, bd)
    ref = w4.qmm(bits16(x), u32(w), bits16(s), bits16(b))
    err = w4.rel_err(w4.bf16_to_f32(bits16(y)), ref)
    assert err <= 2e-2 and err <= 4e-3
    full = Q.repack_for_skinny(wd, sd, bd)
    assert np.array_equal(u32(rw._skinny_full[1]), u32(full))
    assert np.array_equal(bits16(Q.skinny_qmm(xd, full)), bits16(y))
    kept = rw._skinny_full[1]
    assert np.array_equal(bits16(Q.skinny_qmm(xd, rw, sd, bd)), bits16(y)) and rw._skinny_full[1] is kept
    sd.mul_(2.0)  # exact in bf16: the product becomes x . (2 q s + b)
    y2 = Q.skinny_qmm(xd, rw, sd, bd)
    assert rw._skinny_full[1] is not kept
    ref2 = w4.qmm(bits16(x), u32(w), bits16(sd), bits16(b))
    assert w4.rel_err(w4.bf16_to_f32(bits16(y2)), ref2) <= 4e-3
    with pytest.raises(ValueError):
        Q.skinny_qmm(xd, full, sd, bd)  # packed before the scales changed
    with pytest.raises(ValueError):
        Q.skinny_qmm(xd, wd, sd, bd)    # MLX packs that were never relaid
    with pytest.raises(ValueError):
        Q.skinny_qmm(xd, rw)            # a relayout needs its scales and biases


@pytest.mark.parametrize("m", list(range(1, 17)))
def test_qmm_config0_all_m(dev, m):
    x, w, s, b = qmm_case(m, 9728, 2560, seed=0)
    ref = w4.qmm(bits16(x), u32(w), bits16(s), bits16(b))
    xd, wd, sd, bd = _to(dev, x, w, s, b)
    y = Q.skinny_qmm(xd, Q.repack_for_skinny(wd, sd, bd), sd, bd)
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == (m, 9728)
    err = w4.rel_err(w4.bf16_to_f32(bits16(y)), ref)
    assert err <= 2e-2
    assert err <= 4e-3


@pytest.mark.parametrize("k,n", CONFIG1 + QWEN35)
@pytest.mark.parametrize("m", [1, 2, 4, 6, 8, 12, 16])
def test_qmm_config1_shapes(dev, k, n, m):
    x, w, s, b = qmm_case(m, n, k, seed=1)
    xd, wd, sd, bd = _to(dev, x, w, s, b)
    y = bits16(Q.skinny_qmm(xd, Q.repack_for_skinny(wd, sd, bd), sd, bd))
    # the oracle on a bounded row sample (head, a middle slice, tail) keeps the CPU time small
    rows = np.unique(np.concatenate([np.arange(0, min(n, 2048)), np.arange(n // 2, n // 2 + 512), np.arange(n - 1024, n)]))
    ref = w4.qmm(bits16(x), u32(w)[rows], bits16(s)[rows], bits16(b)[rows])
    err = w4.rel_err(w4.bf16_to_f32(y[:, rows]), ref)
    assert err <= 2e-2
    assert err <= 4e-3


def test_reference_sweep_loop_runs_unchanged(dev):
    """The reference's tile sweep (qmm.py:201-213) as its code runs it: CONFIG_OVERRIDE = (rf, sk)
    for rf in {1, 2, 4} and sk in {1, 2, 4, 8}, then skinny_qmm(x, rw, scales, biases) on a
    repack_for_skinny(w) relayout, at M = 8 and 16. Every tile is within the qmm bars of the
    oracle at (K, N) = (2560, 9728); config_for(m, k) returns the pair; the split-K shape (9728,
    2560) takes the forced unsplit tile."""
    k, n = 2560, 9728
    x, w, s, b = qmm_case(16, n, k, seed=31)
    xd, wd, sd, bd = _to(dev, x, w, s, b)
    rw = Q.repack_for_skinny(wd)  # the reference's Rs entry: (repack_for_skinny(q), s, b)
    x2, w2, s2, b2 = qmm_case(8, 2560, 9728, seed=32)
    rw2 = Q.repack_for_skinny(w2.to(dev))
    rows2 = np.arange(0, 2560, 3)
    ref2 = w4.qmm(bits16(x2), u32(w2)[rows2], bits16(s2)[rows2], bits16(b2)[rows2])
    assert Q.CONFIG_OVERRIDE is None
    try:
        for m in (8, 16):
            ref = w4.qmm(bits16(x[:m]), u32(w), bits16(s), bits16(b))
            for rf in (1, 2, 4):
                for sk in (1, 2, 4, 8):
                    Q.CONFIG_OVERRIDE = (rf, sk)
                    assert Q.config_for(m, k) == (rf, sk)
                    assert Q.config_for(m, k, n) == (1, rf, sk, 2)
                    y = Q.skinny_qmm(xd[:m], rw, sd, bd)
                    err = w4.rel_err(w4.bf16_to_f32(bits16(y)), ref)
                    assert err <= 2e-2 and err <= 4e-3, (m, rf, sk, err)
                    if m == 8:
                        y2 = Q.skinny_qmm(x2.to(dev), rw2, s2.to(dev), b2.to(dev))
                        err2 = w4.rel_err(w4.bf16_to_f32(bits16(y2)[:, rows2]), ref2)
                        assert err2 <= 4e-3, (rf, sk, err2)
    finally:
        Q.CONFIG_OVERRIDE = None
    assert len(Q.config_for(8, k)) == 2


def _down_case(dev, sets: int, m: int, seed: int):
    """`sets` packed 9728 x 2560 weights (the split-K shape) and their inputs."""
    g = torch.Generator(device=dev).manual_seed(seed)
    ws = [Q.repack_for_skinny(*Q.random_w4g64(2560, 9728, generator=g, device=dev)) for _ in range(sets)]
    xs = [torch.randn((m, 9728), generator=g, device=dev).to(torch.bfloat16) for _ in range(sets)]
    return ws, xs


def test_splitk_calls_on_two_streams_overlap_safely(dev):
    """skinny_qmm is re-entrant across streams: two streams each issue a chain of split-K calls
    (9728 x 2560, M = 8) with nothing ordering one stream's calls against the other's, eagerly and
    as two branches of one captured graph, and every output is bitwise the same call's output when
    all the calls run one after another on one stream. Each stream has its own workspace."""
    assert Q._plain_config(9728, 2560)[0] > 1
    sets, reps = 4, 6
    ws, xs = _down_case(dev, sets, 8, seed=41)
    ref = [Q.skinny_qmm(x, w) for x, w in zip(xs, ws)]  # serialized, one stream
    torch.cuda.synchronize()
    a, b = torch.cuda.Stream(), torch.cuda.Stream()
    ya = [[torch.empty((8, 2560), dtype=torch.bfloat16, device=dev) for _ in range(sets)] for _ in range(reps)]
    yb = [[torch.empty((8, 2560), dtype=torch.bfloat16, device=dev) for _ in range(sets)] for _ in range(reps)]

    def both():
        main = torch.cuda.current_stream()
        a.wait_stream(main)
        b.wait_stream(main)
        for r in range(reps):
            with torch.cuda.stream(a):
                for i in range(sets):
                    Q.skinny_qmm(xs[i], ws[i], out=ya[r][i])
            with torch.cuda.stream(b):
                for i in reversed(range(sets)):
                    Q.skinny_qmm(xs[i], ws[i], out=yb[r][i])
        main.wait_stream(a)
        main.wait_stream(b)

    def check():
        for r in range(reps):
            for i in range(sets):
                assert torch.equal(ya[r][i], ref[i]) and torch.equal(yb[r][i], ref[i]), (r, i)

    both()
    torch.cuda.synchronize()
    check()
    keys = {key for key in Q._SPLITK_WS if key[1] in (a.cuda_stream, b.cuda_stream)}
    assert len(keys) == 2
    assert Q._SPLITK_WS[(dev, a.cuda_stream)].data_ptr() != Q._SPLITK_WS[(dev, b.cuda_stream)].data_ptr()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        both()
    for _ in range(3):
        for y in [t for row in ya + yb for t in row]:
            y.zero_()
        graph.replay()
        torch.cuda.synchronize()
        check()
    assert not Q.splitk_workspace_failed(dev)


def test_splitk_workspace_error_word_is_sticky(dev):
    """A split-K workspace whose header says a last split gave up makes every later call on it
    write NaN rows (no silent use of words a late slice may still overwrite); a fresh workspace
    computes the product again. The mark is set from the host here: no wait is made to fail."""
    ws, xs = _down_case(dev, 1, 4, seed=42)
    good = Q.skinny_qmm(xs[0], ws[0])
    work = Q.splitk_workspace(dev, 2560, Q._plain_config(9728, 2560)[0])
    torch.cuda.synchronize()
    assert not Q.splitk_workspace_failed(dev)
    work.view(torch.int32)[0] = 1
    torch.cuda.synchronize()
    try:
        assert Q.splitk_workspace_failed(dev)
        assert bool(torch.isnan(Q.skinny_qmm(xs[0], ws[0]).float()).all())
    finally:
        Q.reset_splitk_workspaces()
    assert torch.equal(Q.skinny_qmm(xs[0], ws[0]), good)
    assert not Q.splitk_workspace_failed(dev)


def test_qmm_bitwise_m_invariant(dev):
    x, w, s, b = qmm_case(16, 2560, 4096, seed=2)
    xd, wd, sd, bd = _to(dev, x, w, s, b)
    wf = Q.repack_for_skinny(wd, sd, bd)
    full = bits16(Q.skinny_qmm(xd, wf, sd, bd))
    for m in range(1, 16):
        part = bits16(Q.skinny_qmm(xd[:m].contiguous(), wf, sd, bd))
        assert np.array_equal(part, full[:m]), m
    # and a token's row does not depend on which other rows share the call
    perm = torch.randperm(16, generator=torch.Generator().manual_seed(3))
    shuffled = bits16(Q.skinny_qmm(xd[perm.to(dev)].contiguous(), wf, sd, bd))
    assert np.array_equal(shuffled, full[perm.numpy()])


def test_qmm_deterministic(dev):
    x, w, s, b = qmm_case(8, 2560, 9728, seed=4)
    xd, wd, sd, bd = _to(dev, x, w, s, b)
    wf = Q.repack_for_skinny(wd, sd, bd)
    a = bits16(Q.skinny_qmm(xd, wf, sd, bd))
    for _ in range(3):
        assert np.array_equal(bits16(Q.skinny_qmm(xd, wf, sd, bd)), a)


def test_qmm_known_answers(dev):
    n, k = 64, 256
    g = torch.Generator().manual_seed(5)
    s = (torch.randn((n, k // 64), generator=g) * 0.02).abs().to(torch.bfloat16)
    # q = 8 everywhere with b = -8 s: every weight is exactly zero. The kernel feeds 128+q to
    # the MFMA and removes 128*sum(x) per group in fp32, so the exact zero comes back as a
    # cancellation residue of a few fp32 ulps of 136*sum(x)*s (~1e-6 here), not as 0.
    q8 = np.full((n, k), 8, np.uint8)
    w8 = torch.from_numpy(w4.pack_mlx(q8).view(np.int32))
    b8 = (s.float() * -8).to(torch.bfloat16)
    x = torch.randn((16, k), generator=g).to(torch.bfloat16)
    y = Q.skinny_qmm(x.to(dev), Q.repack_for_skinny(w8.to(dev), s.to(dev), b8.to(dev)))
    assert y.float().abs().max().item() < 1e-4
    # one-hot x selects a dequantized column (to within one bf16 rounding)
    q = np.random.default_rng(6).integers(0, 16, size=(n, k), dtype=np.uint8)
    wq = torch.from_numpy(w4.pack_mlx(q).view(np.int32))
    bq = (torch.randn((n, k // 64), generator=g) * 0.1).to(torch.bfloat16)
    cols = [0, 5, 63, 64, 130, 255]
    xo = torch.zeros((len(cols), k))
    for i, c in enumerate(cols):
        xo[i, c] = 1.0
    y = Q.skinny_qmm(xo.to(torch.bfloat16).to(dev), Q.repack_for_skinny(wq.to(dev), s.to(dev), bq.to(dev)))
    deq = w4.dequant(u32(wq), bits16(s), bits16(bq))
    got = w4.bf16_to_f32(bits16(y)).astype(np.float64)
    for i, c in enumerate(cols):
        ref = deq[:, c]
        assert np.all(np.abs(got[i] - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-30), c


def test_qmm_m_over_16_chunks(dev):
    x, w, s, b = qmm_case(40, 256, 512, seed=7)
    xd, wd, sd, bd = _to(dev, x, w, s, b)
    wf = Q.repack_for_skinny(wd, sd, bd)
    y = bits16(Q.skinny_qmm(xd, wf, sd, bd))
    for m0 in (0, 16, 32):
        part = bits16(Q.skinny_qmm(xd[m0:m0 + 8].contiguous(), wf, sd, bd))
        assert np.array_equal(part, y[m0:m0 + 8])
    assert w4.rel_err(w4.bf16_to_f32(y), w4.qmm(bits16(x), u32(w), bits16(s), bits16(b))) <= 4e-3


def test_qmm_strided_input_and_leading_dims(dev):
    x, w, s, b = qmm_case(6, 128, 256, seed=8)
    xd, wd, sd, bd = _to(dev, x, w, s, b)
    wf = Q.repack_for_skinny(wd, sd, bd)
    base = bits16(Q.skinny_qmm(xd, wf, sd, bd))
    wide = torch.zeros((6, 512), dtype=torch.bfloat16, device=dev)
    wide[:, 128:384] = xd
    y = bits16(Q.skinny_qmm(wide[:, 128:384], wf, sd, bd))  # row stride 512
    assert np.array_equal(y, base)
    y3 = Q.skinny_qmm(xd.reshape(2, 3, 256), wf, sd, bd)
    assert tuple(y3.shape) == (2, 3, 128)
    assert np.array_equal(bits16(y3.reshape(6, 128)), base)


def test_qmm_rejects_bad_arguments(dev):
    x, w, s, b = qmm_case(4, 64, 128, seed=9)
    xd, wd, sd, bd = _to(dev, x, w, s, b)
    wf = Q.repack_for_skinny(wd, sd, bd)
    with pytest.raises(ValueError):
        Q.skinny_qmm(xd[:, :64], wf, sd, bd)
    with pytest.raises(ValueError):
        Q.skinny_qmm(xd, wf, sd[:32], bd)
    with pytest.raises(ValueError):
        Q.skinny_qmm(xd, wd, sd, bd)  # raw MLX packs are not a packed buffer
    with pytest.raises(ValueError):
        Q.skinny_qmm(xd, wf, sd.clone(), bd)  # scales other than the packed ones
    with pytest.raises(ValueError):
        Q.repack_for_skinny(wd[:40].contiguous(), sd[:40].contiguous(), bd[:40].contiguous())
    with pytest.raises(ValueError):
        Q.repack_for_skinny(wd, sd.float(), bd)


@pytest.mark.parametrize("k,f", [(256, 512), (2560, 9728), (2560, 9216)])
@pytest.mark.parametrize("m", [1, 8, 16])
def test_gate_up_layout_and_swiglu(dev, k, f, m):
    """The gate|up layout returns [gate | up] in the unfused column order (within the qmm bar of
    the oracle), and its SwiGLU epilogue is bitwise the activation kernel applied to that."""
    from skinny_mlx import kernels as KK

    x, wg, sg, bg = qmm_case(m, f, k, seed=21)
    _, wu, su, bu = qmm_case(1, f, k, seed=22)
    w, s, b = torch.cat([wg, wu]), torch.cat([sg, su]), torch.cat([bg, bu])
    xd, wd, sd, bd = _to(dev, x, w, s, b)
    packed = Q.repack_gate_up(wd, sd, bd)
    split = Q.skinny_glu(xd, packed, swiglu=False)
    act = Q.skinny_glu(xd, packed, swiglu=True)
    assert tuple(split.shape) == (m, 2 * f) and tuple(act.shape) == (m, f)
    assert np.array_equal(bits16(act), bits16(KK.silu_mul(split)))
    rows = np.unique(np.concatenate([np.arange(0, 256), np.arange(f - 128, f + 128), np.arange(2 * f - 256, 2 * f)]))
    ref = w4.qmm(bits16(x), u32(w)[rows], bits16(s)[rows], bits16(b)[rows])
    assert w4.rel_err(w4.bf16_to_f32(bits16(split)[:, rows]), ref) <= 4e-3
    # a token's activation row does not depend on M
    one = Q.skinny_glu(xd[-1:].contiguous(), packed, swiglu=True)
    assert np.array_equal(bits16(one), bits16(act)[-1:])


@pytest.mark.parametrize("k,f", [(2560, 9728), (2560, 9216), (2560, 256)])
def test_one_wave_form_of_the_gate_up_tile_is_bitwise_its_four_waves(dev, k, f):
    """From two tokens on the 4-wave gate|up + SwiGLU tile over K = 2560 runs as one wave holding
    the four K groups of five pairs in separate accumulators (added in group order): every row of
    2..16-token calls equals the one-token call (four waves) on that row alone, and the SwiGLU
    output equals the activation kernel applied to the split output (four waves at every M)."""
    from skinny_mlx import _lib
    from skinny_mlx import kernels as KK

    x, wg, sg, bg = qmm_case(16, f, k, seed=40 + k)
    _, wu, su, bu = qmm_case(1, f, k, seed=41 + k)
    w, s, b = torch.cat([wg, wu]), torch.cat([sg, su]), torch.cat([bg, bu])
    xd, wd, sd, bd = _to(dev, x, w, s, b)
    packed = Q.repack_gate_up(wd, sd, bd)
    saved = Q._GLU_TILES.pop((k, f), None)
    try:
        Q._GLU_TILES[(k, f)] = _lib.QmmTile(1, 2, 4, 2)
        ones = [bits16(Q.skinny_glu(xd[t:t + 1].contiguous(), packed, swiglu=True)) for t in range(16)]
        for m in (2, 3, 8, 16):
            act = bits16(Q.skinny_glu(xd[:m].contiguous(), packed, swiglu=True))
            for t in range(m):
                assert np.array_equal(act[t:t + 1], ones[t]), (m, t)
            split = Q.skinny_glu(xd[:m].contiguous(), packed, swiglu=False)
            assert np.array_equal(act, bits16(KK.silu_mul(split))), m
    finally:
        Q._GLU_TILES.pop((k, f), None)
        if saved is not None:
            Q._GLU_TILES[(k, f)] = saved


@pytest.mark.parametrize("m", [1, 5, 16])
def test_slab_tile_equals_single_wave_tile_bitwise(dev, m):
    """The slab kernel (X staged once per workgroup in LDS by DMA) and a one-wave wave-X tile
    both sum K in pair order per wave, so they agree bit for bit; both meet the oracle."""
    x, w, s, b = qmm_case(m, 1024, 2560, seed=31)
    xd, wd, sd, bd = _to(dev, x, w, s, b)
    wf = Q.repack_for_skinny(wd, sd, bd)
    try:
        Q.CONFIG_OVERRIDE = (2, 1, 8, 4)
        slab = bits16(Q.skinny_qmm(xd, wf))
        Q.CONFIG_OVERRIDE = (2, 2, 4, 3)
        slab2 = bits16(Q.skinny_qmm(xd, wf))
        Q.CONFIG_OVERRIDE = (1, 1, 1, 2)
        one = bits16(Q.skinny_qmm(xd, wf))
    finally:
        Q.CONFIG_OVERRIDE = None
    assert np.array_equal(slab, one) and np.array_equal(slab2, one)
    ref = w4.qmm(bits16(x), u32(w), bits16(s), bits16(b))
    assert w4.rel_err(w4.bf16_to_f32(slab), ref) <= 4e-3


@pytest.mark.parametrize("k,n", [(9728, 2560), (4096, 2560), (2048, 2560), (9216, 2560), (2560, 1024)])
@pytest.mark.parametrize("m", [1, 8, 16])
def test_split_k_partial_sums(dev, k, n, m):
    """The split-K slices, summed in order and rounded to bf16, match the fp64 oracle to the qmm
    bar (and 4e-3)."""
    from skinny_mlx.kernels import PartialSum

    x, w, s, b = qmm_case(m, n, k, seed=4)
    xd, wd, sd, bd = _to(dev, x, w, s, b)
    ps = Q.skinny_qmm_partial(xd, Q.repack_for_skinny(wd, sd, bd))
    assert isinstance(ps, PartialSum) and ps.parts.shape[1:] == (m, n)
    splits, _ = Q.partial_config(k, n)
    assert ps.parts.shape[0] == splits and (splits > 1 or (k, n) == (2560, 1024))
    ref = w4.qmm(bits16(x), u32(w), bits16(s), bits16(b))
    err = w4.rel_err(w4.bf16_to_f32(bits16(ps.value())), ref)
    assert err <= 2e-2 and err <= 4e-3


def test_one_split_is_the_plain_kernel(dev):
    """With one split the slice is the plain kernel's fp32 result before its bf16 rounding."""
    from skinny_mlx import _lib

    m, k, n = 8, 2560, 2048
    x, w, s, b = qmm_case(m, n, k, seed=5)
    xd, wd, sd, bd = _to(dev, x, w, s, b)
    wf = Q.repack_for_skinny(wd, sd, bd)
    for tile in ((1, 2, 8, 2), (1, 1, 4, 3), (1, 4, 2, 2)):
        t = _lib.QmmTile(*tile)
        y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        _lib.check(_lib.lib().skinny_qmm_w4g64_bf16(xd.data_ptr(), m, k, k, wf.data_ptr(), n, y.data_ptr(), n, t,
                                                    _lib.stream_of(xd)), "qmm")
        part = torch.empty((1, m, n), dtype=torch.float32, device=dev)
        _lib.check(_lib.lib().skinny_qmm_w4g64_partial_f32(xd.data_ptr(), m, k, k, wf.data_ptr(), n, part.data_ptr(),
                                                           n, 1, t, _lib.stream_of(xd)), "partial")
        assert torch.equal(part[0].to(torch.bfloat16), y), tile


@pytest.mark.parametrize("k,n", [(9728, 2560), (4096, 2560), (9216, 2560)])
def test_split_k_bitwise_m_invariant(dev, k, n):
    x, w, s, b = qmm_case(16, n, k, seed=6)
    xd, wd, sd, bd = _to(dev, x, w, s, b)
    wf = Q.repack_for_skinny(wd, sd, bd)
    full = Q.skinny_qmm_partial(xd, wf).parts
    for m in (1, 3, 8):
        part = Q.skinny_qmm_partial(xd[:m].contiguous(), wf).parts
        assert torch.equal(part, full[:, :m]), m


@pytest.mark.parametrize("splits", [1, 2, 3, 4])
def test_rmsnorm_with_partial_residual(dev, splits):
    """rmsnorm(h + residual slices) is bitwise rmsnorm(h + bf16(sum of the slices))."""
    from skinny_mlx import kernels as K

    g = torch.Generator().manual_seed(splits)
    rows, H = 8, 2560
    h = torch.randn((rows, H), generator=g).to(torch.bfloat16).to(dev)
    parts = (torch.randn((splits, rows, H), generator=g) * 0.5).to(dev)
    wn = (torch.randn(H, generator=g) * 0.1 + 1).to(torch.bfloat16).to(dev)
    ps = K.PartialSum(parts)
    h1, h2 = h.clone(), h.clone()
    a = K.rmsnorm(h1, wn, 1e-6, residual=ps, sum_out=h1)
    b = K.rmsnorm(h2, wn, 1e-6, residual=ps.value(), sum_out=h2)
    assert torch.equal(a, b) and torch.equal(h1, h2)


@pytest.mark.parametrize("splits,tile", [(2, (1, 1, 8, 2)), (3, (1, 2, 4, 3)), (4, (1, 1, 4, 4))])
def test_splitk_matches_oracle_and_is_m_invariant(dev, splits, tile):
    """The split-K plain kernel (skinny_qmm_w4g64_splitk_bf16): within the qmm bars of the oracle at
    the down projection's shape, bitwise the same row for every M = 1..16 and every repeat, and its
    workspace back at the "not yet written" mark after each call."""
    k, n = 9728, 2560
    x, w, s, b = qmm_case(16, n, k, seed=13)
    xd, wd, sd, bd = _to(dev, x, w, s, b)
    wf = Q.repack_for_skinny(wd, sd, bd)
    Q.SPLITK_OVERRIDE = (splits,) + tile
    try:
        full = bits16(Q.skinny_qmm(xd, wf))
        rows = np.arange(0, n, 7)
        ref = w4.qmm(bits16(x), u32(w)[rows], bits16(s)[rows], bits16(b)[rows])
        err = w4.rel_err(w4.bf16_to_f32(full[:, rows]), ref)
        assert err <= 2e-2 and err <= 4e-3
        for m in (1, 3, 8, 15):
            assert np.array_equal(bits16(Q.skinny_qmm(xd[:m].contiguous(), wf)), full[:m]), m
        assert np.array_equal(bits16(Q.skinny_qmm(xd, wf)), full)
        ws = Q.splitk_workspace(dev, n, splits)
        torch.cuda.synchronize()
        assert bool((ws.view(torch.int32) == -1).all())
    finally:
        Q.SPLITK_OVERRIDE = None


def test_splitk_table_shape_takes_the_split_kernel(dev):
    """(9728, 2560) is in the split-K table: skinny_qmm takes it, and stays within the oracle's bars."""
    splits, _ = Q._plain_config(9728, 2560)
    assert splits >= 2
    x, w, s, b = qmm_case(8, 2560, 9728, seed=14)
    xd, wd, sd, bd = _to(dev, x, w, s, b)
    y = bits16(Q.skinny_qmm(xd, Q.repack_for_skinny(wd, sd, bd)))
    rows = np.arange(0, 2560, 5)
    ref = w4.qmm(bits16(x), u32(w)[rows], bits16(s)[rows], bits16(b)[rows])
    assert w4.rel_err(w4.bf16_to_f32(y[:, rows]), ref) <= 4e-3


def test_launches_spread_over_streams_equal_one_chain(dev):
    """Independent skinny_qmm calls spread over four streams in one captured graph (the split-K
    shape's calls on three different streams, each with its own workspace) give bitwise the
    outputs of the same calls as one chain on one stream, over several replays: the batch form of
    the projection stack (the reference evaluates its matmuls as one list, qmm.py:195-197)."""
    g = torch.Generator(device=dev).manual_seed(21)
    shapes = [(2560, 6144), (4096, 2560), (2560, 19456), (9728, 2560)] * 3
    assert Q._plain_config(9728, 2560)[0] > 1 and all(Q._plain_config(*t)[0] == 1 for t in shapes[:3])
    ws = []
    for k, n in shapes:
        w, s, b = Q.random_w4g64(n, k, generator=g, device=dev)
        ws.append((Q.repack_for_skinny(w, s, b), s, b))
    xs = {k: torch.randn((8, k), generator=g, device=dev).to(torch.bfloat16) for k in {2560, 4096, 9728}}
    ys = [torch.empty((8, n), dtype=torch.bfloat16, device=dev) for _, n in shapes]
    streams = [torch.cuda.Stream() for _ in range(4)]

    def chain():
        for (k, _), (wf, s, b), y in zip(shapes, ws, ys):
            Q.skinny_qmm(xs[k], wf, s, b, out=y)

    def batch():
        main = torch.cuda.current_stream()
        for st in streams:
            st.wait_stream(main)
        for i, ((k, _), (wf, s, b), y) in enumerate(zip(shapes, ws, ys)):
            with torch.cuda.stream(streams[(i + i // 4) % 4]):  # the split-K shape on streams 3, 0, 1
                Q.skinny_qmm(xs[k], wf, s, b, out=y)
        for st in streams:
            main.wait_stream(st)

    chain()
    torch.cuda.synchronize()
    ref = [y.clone() for y in ys]
    batch()  # first calls outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        batch()
    for _ in range(3):
        for y in ys:
            y.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(ref, ys))
