"""The MLP sublayer in one launch (skinny_mlp_fused_partial_f32): gate|up + SwiGLU and the down
projection's split-K slices, bitwise the two launches it replaces (skinny_qmm_w4g64_glu_bf16 with
the SwiGLU epilogue, then skinny_qmm_w4g64_partial_f32), at the 36-layer decoders' shape for every
token count it takes; its hand-off counters are left at zero by every call, eagerly and in replayed
graphs; and the dense decoder's verify forward with the launch switched on (MLP.fuse_mlp, off by
default) is bitwise the forward without it."""

import pytest
import torch

from skinny_mlx import qmm as Q

pytestmark = pytest.mark.gpu

K, F, N = 2560, 9728, 2560


@pytest.fixture(scope="module")
def weights(dev):
    g = torch.Generator(device=dev).manual_seed(40)
    wgu = Q.repack_gate_up(*Q.random_w4g64(2 * F, K, generator=g, device=dev))
    wdn = Q.repack_for_skinny(*Q.random_w4g64(N, F, generator=g, device=dev))
    act, sync = Q.mlp_fused_buffers(F, dev)
    return wgu, wdn, act, sync, g


def _two_launches(x, wgu, wdn):
    h = Q.skinny_glu(x, wgu, swiglu=True)
    return h, Q.skinny_qmm_partial(h, wdn).parts


@pytest.mark.parametrize("m", [2, 3, 5, 8, 12, 16])
def test_fused_mlp_is_bitwise_the_two_launches(dev, weights, m):
    wgu, wdn, act, sync, g = weights
    assert Q.mlp_fused_supported(m, K, F, N)
    x = torch.randn((m, K), generator=g, device=dev).to(torch.bfloat16)
    h, ref = _two_launches(x, wgu, wdn)
    got = Q.skinny_mlp_fused_partial(x, wgu, wdn, act, sync).parts
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    assert torch.equal(act[:m], h)
    assert int(sync.abs().sum()) == 0  # every counter back at zero


def test_fused_mlp_calls_in_a_row_and_in_a_graph(dev, weights):
    """Calls of different token counts back to back, then the same calls captured in one graph and
    replayed three times (outputs cleared between replays): every output bitwise its reference."""
    wgu, wdn, act, sync, g = weights
    xs = [torch.randn((m, K), generator=g, device=dev).to(torch.bfloat16) for m in (8, 2, 16, 3)]
    refs = [_two_launches(x, wgu, wdn)[1] for x in xs]
    outs = [Q.skinny_mlp_fused_partial(x, wgu, wdn, act, sync).parts for x in xs]
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(outs, refs))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = [Q.skinny_mlp_fused_partial(x, wgu, wdn, act, sync).parts for x in xs]
    for _ in range(3):
        for o in outs:
            o.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(outs, refs))
        assert int(sync.abs().sum()) == 0


def test_fused_mlp_in_the_dense_decoder_is_bitwise_the_unfused_mlp(dev):
    """The dense-36 decoder's verify forward at M = 2, 8 and 16 over a short prompt with
    MLP.fuse_mlp on (one launch per MLP) and off (two): the same hidden states and logits."""
    from skinny_mlx import patch as P
    from skinny_mlx.cache import KVCache, make_prompt_cache
    from skinny_mlx.model import build_model
    from skinny_mlx.spec import forward

    model = build_model("dense-36", num_hidden_layers=4, max_position=1024)
    P.patch_model(model)
    prompt = list(range(100, 160))
    for m in (2, 8, 16):
        ids = list(range(500, 500 + m))
        got = []
        for fuse in (True, False):
            for layer in model.layers:
                layer.mlp.fuse_mlp = fuse
            cache = make_prompt_cache(model)
            forward(model, prompt, cache)
            got.append(forward(model, ids, cache))
        assert torch.equal(got[0][0], got[1][0]) and torch.equal(got[0][1], got[1][1]), m
    assert all(isinstance(c, KVCache) for c in cache)
