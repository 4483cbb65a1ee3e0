"""The Gated-DeltaNet mixer's launches around its recurrence.

* The fused input projection with the conv + SiLU in its epilogue (skinny_qmm_w4g64_conv_bf16)
  against skinny_qmm_w4g64_bf16 then skinny_gdn_conv_silu, bit for bit: outputs, conv state and
  rollback window, for a chain with and without recording and for draft trees.
* A hybrid decoder whose GDN projections fuse, with the fusion on and off, bit for bit through a
  prompt, a recorded verify step and a draft-tree step.
* The output norm (skinny_gated_rmsnorm) against the oracle."""

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
def test_conv_epilogue_is_bitwise_the_two_launch_path(dev, m, mode):
    k, n, c = 2560, 8224, 6144  # the hybrid decoder's fused q|k|v|z|b|a projection
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
