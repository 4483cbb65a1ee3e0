"""The allocation-free attention entry point (skinny_attention_fused_noalloc_bf16, through the C
ABI) against the entry it varies, skinny_attention_fused_bf16 with a caller workspace: the same
kernels, so outputs and cache writes must be bit-identical, over two calls in a row (the second
smaller, on the scratch the first one left), and in a replayed HIP graph."""

import numpy as np
import pytest
import torch

from oracle import w4
from skinny_mlx import kernels as K

pytestmark = pytest.mark.gpu

HQ, HKV, D = 32, 8, 128


def _bf(x, dev):
    return torch.as_tensor(x, dtype=torch.float32).to(torch.bfloat16).to(dev)


def _case(seed, M, L, maxlen, dev):
    rng = np.random.default_rng(seed)
    return dict(
        qkv=_bf(w4.round_bf16(rng.standard_normal((M, (HQ + 2 * HKV) * D))), dev),
        qn=_bf(w4.round_bf16(1 + 0.1 * rng.standard_normal(D)), dev),
        kn=_bf(w4.round_bf16(1 + 0.1 * rng.standard_normal(D)), dev),
        k=_bf(w4.round_bf16(rng.standard_normal((HKV, maxlen, D))), dev),
        vt=_bf(w4.round_bf16(rng.standard_normal((HKV, D, maxlen))), dev),
        pos=torch.tensor([L], dtype=torch.int32, device=dev),
        table=K.rope_table(1e6, maxlen, dev))


def _with_workspace(c, tree):
    k, vt = c["k"].clone(), c["vt"].clone()
    ws = K.attn_workspace(HKV, k.shape[1], k.device)
    out = K.attention_fused(c["qkv"], HQ, HKV, D, c["qn"], c["kn"], 1e-6, c["table"], c["pos"], k, vt, D ** -0.5, ws,
                            tree)
    return out, k, vt


def _no_alloc(c, tree, out=None):
    k, vt = c["k"].clone(), c["vt"].clone()
    out = K.attention_fused_noalloc(c["qkv"], HQ, HKV, D, c["qn"], c["kn"], 1e-6, c["table"], c["pos"], k, vt,
                                    D ** -0.5, tree, out=out)
    return out, k, vt


def test_no_alloc_attention_equals_workspace_entry_on_two_calls(dev):
    from skinny_mlx.tree import DraftTree, branching_tree

    # the first call at the scratch's maximum (8 kv heads x 4096 positions), the second smaller and
    # a draft tree, reading the scratch the first call left behind
    for seed, M, L, maxlen, tree in ((1, 16, 2040, 4096, False), (2, 5, 300, 1024, True)):
        print(f"no-alloc attention: M={M} L={L} maxlen={maxlen} tree={tree}", flush=True)
        c = _case(seed, M, L, maxlen, dev)
        desc = DraftTree(branching_tree((4, 2, 1), M)[0], dev).desc if tree else None
        ref, k1, v1 = _with_workspace(c, desc)
        got, k2, v2 = _no_alloc(c, desc)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (M, L)
        assert torch.equal(k1, k2) and torch.equal(v1, v2), (M, L)


def test_no_alloc_attention_rejects_shapes_beyond_its_scratch(dev):
    c = _case(3, 2, 100, 8192, dev)  # 8 kv heads x 8192 positions = 512 chunk pairs > 256
    with pytest.raises(ValueError, match="scratch maximum"):
        _no_alloc(c, None)


def test_no_alloc_attention_replays_in_a_graph(dev):
    """Captured once (after a first eager call on the device), replayed with eager work and a
    synchronisation between replays; every replay equals the workspace entry's result."""
    c = _case(4, 8, 1500, 2048, dev)
    ref, k_ref, v_ref = _with_workspace(c, None)
    out = torch.empty_like(ref)
    _no_alloc(c, None, out=out)  # first call on the device outside the capture
    k, vt = c["k"].clone(), c["vt"].clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            K.attention_fused_noalloc(c["qkv"], HQ, HKV, D, c["qn"], c["kn"], 1e-6, c["table"], c["pos"], k, vt,
                                      D ** -0.5, None, out=out)
    torch.cuda.current_stream().wait_stream(stream)
    for i in range(3):
        out.zero_()
        k.copy_(c["k"])
        vt.copy_(c["vt"])
        _with_workspace(c, None)  # other work on the device between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), i
        assert torch.equal(k, k_ref) and torch.equal(vt, v_ref), i
