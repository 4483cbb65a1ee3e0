"""The Gated-DeltaNet mixer's launches around its recurrence.

* The fused input projection with the conv + SiLU in its epilogue (skinny_qmm_w4g64_conv_bf16)
  against skinny_qmm_w4g64_bf16 then skinny_gdn_conv_silu, bit for bit: outputs, conv state and
  rollback window, for a chain with and without recording and for draft trees.
* A hybrid decoder whose GDN projections fuse, with the fusion on and off, bit for bit through a
  prompt, a recorded verify step and a draft-tree step.
* The output norm (skinny_gated_rmsnorm) against the oracle.
* The out_proj with that norm formed inside its launch (skinny_qmm_w4g64_gated_partial_f32)
  against skinny_gated_rmsnorm then skinny_qmm_w4g64_partial_f32, bit for bit, and a hybrid
  decoder with the fusion on and off.
* The one-token recurrence with the output norm in its launch (skinny_gdn_recurrence_gated_bf16)
  against skinny_gdn_recurrence then skinny_gated_rmsnorm, bit for bit (output and state), and a
  hybrid decoder's one-token steps with the fusion on and off."""

import numpy as np
import pytest
import torch

from skinny_mlx import kernels as K
from skinny_mlx import patch as P
from skinny_mlx import qmm as Q
from skinny_mlx.cache import make_prompt_cache
from skinny_mlx.model import build_model
from skinny_mlx.rollback import HybridRollback
from skinny_mlx.spec import forward
from skinny_mlx.tree import DraftTree
from oracle import gdn as G
from oracle import w4
from tests.helpers import qmm_case

pytestmark = pytest.mark.gpu


def _tree_parents(m):
    return [-1] + [(i - 1) // 2 for i in range(1, m)]  # a binary tree: several branches per level


@pytest.mark.parametrize("m", [1, 3, 8, 16])
@pytest.mark.parametrize("mode", ["chain", "record", "tree"])
@pytest.mark.parametrize("n,c", [(8224, 6144), (12352, 8192)])
def test_conv_epilogue_is_bitwise_the_two_launch_path(dev, m, mode, n, c):
    # the fused q|k|v|z|b|a projections of the hybrid decoder (16 heads) and of Qwen3.5-4B's
    # Gated-DeltaNet (16 key heads, 32 value heads)
    k = 2560
    x, w, s, b = qmm_case(m, n, k, seed=80 + m)
    xd = x.to(dev)
    wf = Q.repack_for_skinny(w.to(dev), s.to(dev), b.to(dev))
    g = torch.Generator().manual_seed(m)
    conv_w = ((torch.rand((c, 4), generator=g) - 0.5)).to(torch.bfloat16).to(dev)
    state0 = torch.randn((3, c), generator=g).to(torch.bfloat16).to(dev)
    recording = mode != "chain"
    parent = torch.tensor(_tree_parents(m), dtype=torch.int32, device=dev) if mode == "tree" else None
    win_ref = torch.zeros((3 + 16, c), dtype=torch.bfloat16, device=dev) if recording else None
    win = torch.zeros_like(win_ref) if recording else None

    y_ref = Q.skinny_qmm(xd, wf)
    st_ref = state0.clone()
    xc_ref = K.gdn_conv_silu(y_ref[:, :c], st_ref, conv_w, win_ref, parent)
    st = state0.clone()
    y = Q.skinny_qmm_conv(xd, wf, c, st, conv_w, win, parent)
    torch.cuda.synchronize()
    assert torch.equal(y[:, :c], xc_ref), mode
    assert torch.equal(y[:, c:], y_ref[:, c:])
    assert torch.equal(st, st_ref)  # advanced for a chain, untouched for a tree (the commit does it)
    if recording:
        assert torch.equal(win[:3 + m], win_ref[:3 + m])


def test_conv_epilogue_rejects_bad_arguments(dev):
    x, w, s, b = qmm_case(4, 256, 256, seed=90)
    xd = x.to(dev)
    wf = Q.repack_for_skinny(w.to(dev), s.to(dev), b.to(dev))
    st = torch.zeros((3, 128), dtype=torch.bfloat16, device=dev)
    cw = torch.zeros((128, 4), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="draft tree needs the window"):
        Q.skinny_qmm_conv(xd, wf, 128, st, cw, None, torch.tensor([-1, 0, 0, 1], dtype=torch.int32, device=dev))
    with pytest.raises(ValueError, match="conv_state"):
        Q.skinny_qmm_conv(xd, wf, 128, st[:, :64].contiguous(), cw)
    st3 = torch.zeros((4, 128), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="kernel width 5 unsupported"):
        Q.skinny_qmm_conv(xd, wf, 128, st3, torch.zeros((128, 5), dtype=torch.bfloat16, device=dev))


@pytest.mark.parametrize("m,h", [(1, 16), (8, 16), (5, 3)])
def test_gated_rmsnorm_matches_oracle(dev, m, h):
    """The mixer's output norm (skinny_gated_rmsnorm) against the oracle: fp32 y, bf16 z rows of
    a strided view, within bf16 rounding of the output."""
    g = torch.Generator().manual_seed(200 + m)
    y = torch.randn((m, h, 128), generator=g).to(dev)
    z = (torch.randn((m, h * 128 + 24), generator=g) * 2).to(torch.bfloat16).to(dev)[:, 24:]
    w = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16).to(dev)
    out = K.gated_rmsnorm(y, z, w, 1e-6)
    want = G.gated_rmsnorm(y.double().cpu().numpy(), z.double().cpu().numpy().reshape(m, h, 128),
                           w.double().cpu().numpy(), 1e-6).reshape(m, h * 128)
    assert w4.rel_err(out.double().cpu().numpy(), want) <= 4e-3


def test_hybrid_with_fused_conv_is_bitwise_the_two_launch_path():
    # 16 linear heads: the b and a projections are 16 wide, so the four GDN input projections fuse
    model = build_model("tiny-hybrid", linear_num_heads=16)
    P.patch_model(model)
    gdn = [layer.linear_attn for layer in model.layers if layer.is_linear]
    assert gdn and all(getattr(m.in_proj_qkv, "projection", None) is not None for m in gdn)
    prompt = torch.randint(0, model.args.vocab_size, (37,), generator=torch.Generator().manual_seed(4)).tolist()
    step = [5, 99, 7, 12, 500, 3, 8, 1000]
    tree = DraftTree(_tree_parents(8), model.device)

    def run():
        cache = make_prompt_cache(model)
        rb = HybridRollback.for_model(model)
        h1, l1 = forward(model, prompt, cache)
        rb.record()
        h2, l2 = forward(model, step, cache)           # a recorded verify step (chain)
        rb.rollback(cache, fed=8, keep=3)
        rb.record()
        h3, l3 = forward(model, step, cache, tree)     # a draft-tree step
        rb.rollback(cache, fed=8, keep=8)              # ends the recording
        return [h1, l1, h2, l2, h3, l3, cache.shared.gdn.state.clone(), cache.shared.gdn.conv.clone()]

    fused = run()
    for m in gdn:
        m.fuse_conv = False
    separate = run()
    for a, b in zip(fused, separate):
        assert torch.equal(a, b)


@pytest.mark.parametrize("k,n", [(2048, 2560), (256, 256)])  # the 36-layer and the test hybrid's out_proj
@pytest.mark.parametrize("m", [1, 2, 5, 8, 16])
def test_gated_norm_in_out_proj_is_bitwise_the_two_launches(dev, k, n, m):
    """X = rmsnorm(y) * w * silu(z) per head formed by each lane of the split-K projection: the
    slices equal skinny_gated_rmsnorm followed by skinny_qmm_partial exactly. z is a column slice of
    a wider projection output (row stride > K); heads of all-zero y, of large y and of large |z|
    cover the sum's edge cases."""
    h = k // 128
    _, w, s, b = qmm_case(1, n, k, seed=300 + m)
    wf = Q.repack_for_skinny(w.to(dev), s.to(dev), b.to(dev))
    g = torch.Generator().manual_seed(400 + m)
    y = torch.randn((m, h, 128), generator=g)
    y[0, 0] = 0.0
    if h > 1:
        y[m - 1, 1] *= 1e4
    y = y.to(dev)
    zw = (torch.randn((m, k + 136), generator=g) * 3).to(torch.bfloat16)
    zw[:, 136] = 40.0
    zw[:, 137] = -40.0
    z = zw.to(dev)[:, 136:]
    nw = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16).to(dev)
    eps = 1e-6
    assert Q.gated_partial_supported(k, n)
    ref = Q.skinny_qmm_partial(K.gated_rmsnorm(y, z, nw, eps), wf).parts
    got = Q.skinny_qmm_partial_gated(y, z, nw, eps, wf).parts
    torch.cuda.synchronize()
    assert got.shape == ref.shape
    assert torch.equal(got, ref), (k, n, m)


def test_gated_norm_in_out_proj_rejects_bad_arguments(dev):
    _, w, s, b = qmm_case(1, 256, 256, seed=310)
    wf = Q.repack_for_skinny(w.to(dev), s.to(dev), b.to(dev))
    y = torch.zeros((4, 2, 128), device=dev)
    z = torch.zeros((4, 256), dtype=torch.bfloat16, device=dev)
    nw = torch.ones(128, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="y must be fp32"):
        Q.skinny_qmm_partial_gated(y.to(torch.bfloat16), z, nw, 1e-6, wf)
    with pytest.raises(ValueError, match="z must be bf16"):
        Q.skinny_qmm_partial_gated(y, z[:, :128], nw, 1e-6, wf)
    with pytest.raises(ValueError, match="1..16 tokens"):
        Q.skinny_qmm_partial_gated(torch.zeros((17, 2, 128), device=dev), z, nw, 1e-6, wf)


def test_hybrid_with_gated_norm_in_out_proj_is_bitwise_the_two_launch_path(monkeypatch):
    """The test hybrid (2 linear heads: out_proj K = N = 256) through a 37-token prompt (passes of
    16, 16 and 5 tokens), a one-token step, a recorded verify step and a draft-tree step with the
    output norm inside the out_proj (GatedDeltaNet.fuse_norm, opt-in), then with it switched off:
    the same hidden states, logits and states; the fused form runs in every GDN layer of each of
    the six passes."""
    model = build_model("tiny-hybrid")
    P.patch_model(model)
    gdn = [layer.linear_attn for layer in model.layers if layer.is_linear]
    calls = []
    real = Q.skinny_qmm_partial_gated
    monkeypatch.setattr(P, "skinny_qmm_partial_gated", lambda *a, **kw: (calls.append(1), real(*a, **kw))[1])
    prompt = torch.randint(0, model.args.vocab_size, (37,), generator=torch.Generator().manual_seed(5)).tolist()
    step = [5, 99, 7, 12, 500, 3, 8, 1000]
    tree = DraftTree(_tree_parents(8), model.device)

    def run():
        cache = make_prompt_cache(model)
        rb = HybridRollback.for_model(model)
        out = list(forward(model, prompt, cache))
        out += forward(model, [17], cache)
        rb.record()
        out += forward(model, step, cache)
        rb.rollback(cache, fed=8, keep=3)
        rb.record()
        out += forward(model, step, cache, tree)
        rb.rollback(cache, fed=8, keep=8)
        return out + [cache.shared.gdn.state.clone(), cache.shared.gdn.conv.clone()]

    for m in gdn:
        m.fuse_norm = True
        m.fuse_head_norm = False  # the one-token step's norm in the out_proj too, not in the recurrence
    fused = run()
    assert len(calls) == 6 * len(gdn)
    for m in gdn:
        m.fuse_norm = False
    calls.clear()
    separate = run()
    assert not calls
    for a, b in zip(fused, separate):
        assert torch.equal(a, b)


@pytest.mark.parametrize("h", [16, 3])
def test_head_gated_recurrence_is_bitwise_the_two_launches(dev, h):
    """Three one-token steps in a row from one state: the fused launch's output and state equal
    skinny_gdn_recurrence followed by skinny_gated_rmsnorm exactly. z is a column slice of a wider
    projection row, as the mixer passes it."""
    rng = np.random.default_rng(40 + h)
    g = torch.Generator(device=dev).manual_seed(h)
    A_log = torch.tensor(np.log(rng.uniform(1, 16, h)), dtype=torch.float32, device=dev)
    dt = torch.tensor(rng.uniform(-1, 1, h), dtype=torch.float32, device=dev)
    nw = (1.0 + 0.1 * torch.randn((128,), generator=g, device=dev)).to(torch.bfloat16)
    s_fused = (0.1 * torch.randn((h, 128, 128), generator=g, device=dev)).contiguous()
    s_two = s_fused.clone()
    for step in range(3):
        qkv = torch.randn((1, 3 * h * 128), generator=g, device=dev).to(torch.bfloat16)
        ab = torch.randn((1, 2 * h), generator=g, device=dev).to(torch.bfloat16)
        row = torch.randn((1, h * 128 + 40), generator=g, device=dev).to(torch.bfloat16)
        z = row[:, 24:24 + h * 128]
        out = K.gdn_recurrence_gated(qkv, ab[:, :h], ab[:, h:], A_log, dt, s_fused, z, nw, 1e-6, h, 128, 128)
        y = K.gdn_recurrence(qkv, ab[:, :h], ab[:, h:], A_log, dt, s_two, None, h, 128, 128)
        want = K.gated_rmsnorm(y, z, nw, 1e-6)
        assert torch.equal(out, want), step
        assert torch.equal(s_fused, s_two), step


def test_head_gated_recurrence_rejects_bad_arguments(dev):
    h = 2
    qkv = torch.zeros((2, 3 * h * 128), dtype=torch.bfloat16, device=dev)
    ab = torch.zeros((2, 2 * h), dtype=torch.bfloat16, device=dev)
    st = torch.zeros((h, 128, 128), device=dev)
    f = torch.zeros((h,), device=dev)
    nw = torch.ones((128,), dtype=torch.bfloat16, device=dev)
    z = torch.zeros((1, h * 128), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="one token"):
        K.gdn_recurrence_gated(qkv, ab[:, :h], ab[:, h:], f, f, st, z, nw, 1e-6, h, 128, 128)
    with pytest.raises(ValueError, match="z must be bf16"):
        K.gdn_recurrence_gated(qkv[:1], ab[:1, :h], ab[:1, h:], f, f, st, z[:, :128], nw, 1e-6, h, 128, 128)
    with pytest.raises(ValueError, match="head dims"):
        K.gdn_recurrence_gated(qkv[:1], ab[:1, :h], ab[:1, h:], f, f, st, z, nw, 1e-6, h, 64, 128)


def test_hybrid_one_token_steps_with_the_head_norm_are_bitwise_the_two_launches(monkeypatch):
    """The test hybrid through a 37-token prompt, four one-token steps, a recorded verify step
    and two more one-token steps with the output norm inside the one-token recurrence's launch
    (GatedDeltaNet.fuse_head_norm, the default), then with it switched off: the same hidden
    states, logits and states; the fused form runs in every GDN layer of each one-token step and
    nowhere else."""
    from skinny_mlx import model as Mo

    model = build_model("tiny-hybrid")
    P.patch_model(model)
    gdn = [layer.linear_attn for layer in model.layers if layer.is_linear]
    assert all(m.fuse_head_norm for m in gdn)
    calls = []
    real = K.gdn_recurrence_gated
    monkeypatch.setattr(Mo.K, "gdn_recurrence_gated", lambda *a, **kw: (calls.append(1), real(*a, **kw))[1])
    prompt = torch.randint(0, model.args.vocab_size, (37,), generator=torch.Generator().manual_seed(6)).tolist()
    step = [5, 99, 7, 12]

    def run():
        cache = make_prompt_cache(model)
        rb = HybridRollback.for_model(model)
        out = list(forward(model, prompt, cache))
        for t in (17, 400, 3, 61):
            out += forward(model, [t], cache)
        rb.record()
        out += forward(model, step, cache)
        rb.rollback(cache, fed=4, keep=2)
        for t in (8, 1000):
            out += forward(model, [t], cache)
        return out + [cache.shared.gdn.state.clone(), cache.shared.gdn.conv.clone()]

    fused = run()
    assert len(calls) == 6 * len(gdn)
    for m in gdn:
        m.fuse_head_norm = False
    calls.clear()
    separate = run()
    assert not calls
    for a, b in zip(fused, separate):
        assert torch.equal(a, b)
