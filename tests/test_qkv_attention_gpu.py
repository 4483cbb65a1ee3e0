"""GPU parity of the q|k|v projection fused with the attention (skinny_qkv_attention_fused_bf16),
through the C ABI.

Bar, bitwise: at the 36-layer decoders' shape (K = 2560, Hq = 32, Hkv = 8, D = 128, so N = 6144),
the output and both caches equal skinny_qmm_w4g64_bf16 followed by skinny_attention_fused_bf16 on
copies of the same caches, for chains and a draft tree, over cache lengths from empty to past
2000 keys and at chunk boundaries; the hand-off buffer is back to all 0xFFFF after every call, so
calls in a row and replays of a captured graph keep agreeing. The two-launch path itself is pinned
against the oracle by the attention tests of test_kernels_gpu.py and the qmm tests.
"""

import pytest
import torch

from skinny_mlx import kernels as K
from skinny_mlx import qmm as Q
from skinny_mlx.tree import DraftTree, branching_tree
from tests.helpers import qmm_case

pytestmark = pytest.mark.gpu

Hq, Hkv, D, HIDDEN, MAXLEN, THETA, EPS = 32, 8, 128, 2560, 4096, 1e6, 1e-6
N = (Hq + 2 * Hkv) * D


@pytest.fixture(scope="module")
def setup(dev):
    _, w, s, b = qmm_case(1, N, HIDDEN, seed=41)
    packed = Q.repack_for_skinny(w.to(dev), s.to(dev), b.to(dev))
    g = torch.Generator().manual_seed(42)
    qn = (torch.randn(D, generator=g) * 0.1 + 1).to(torch.bfloat16).to(dev)
    kn = (torch.randn(D, generator=g) * 0.1 + 1).to(torch.bfloat16).to(dev)
    kc = torch.randn((Hkv, MAXLEN, D), generator=g).to(torch.bfloat16).to(dev)
    vt = torch.randn((Hkv, D, MAXLEN), generator=g).to(torch.bfloat16).to(dev)
    table = K.rope_table(THETA, MAXLEN, dev)
    handoff = torch.full((16, N), -1, dtype=torch.int16, device=dev)
    return dict(packed=packed, qn=qn, kn=kn, kc=kc, vt=vt, table=table, handoff=handoff,
                ws1=K.attn_workspace(Hkv, MAXLEN, dev), ws2=K.attn_workspace(Hkv, MAXLEN, dev))


def _x(dev, m, seed):
    return torch.randn((m, HIDDEN), generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16).to(dev)


def _two_launches(st, x, pos, kc, vt, desc):
    y = Q.skinny_qmm(x, st["packed"])
    return K.attention_fused(y, Hq, Hkv, D, st["qn"], st["kn"], EPS, st["table"], pos, kc, vt, D ** -0.5, st["ws1"],
                             desc)


def _fused(st, x, pos, kc, vt, desc):
    return K.qkv_attention_fused(x, st["packed"], Hq, Hkv, D, st["qn"], st["kn"], EPS, st["table"], pos, kc, vt,
                                 D ** -0.5, st["ws2"], st["handoff"], desc)


def test_supported_at_the_decoder_shape():
    assert K.qkv_attention_supported(HIDDEN, N, Hkv, MAXLEN)
    assert not K.qkv_attention_supported(256, 768, 2, 512)  # the test decoders' two-wave tile


@pytest.mark.parametrize("m,length", [(1, 0), (1, 2048), (2, 127), (4, 128), (8, 2040), (16, 300), (12, 1000),
                                      (3, 4093 - 3)])
def test_fused_equals_projection_then_attention(dev, setup, m, length):
    st = setup
    x = _x(dev, m, 100 + m)
    pos = torch.tensor([length], dtype=torch.int32, device=dev)
    k1, v1, k2, v2 = st["kc"].clone(), st["vt"].clone(), st["kc"].clone(), st["vt"].clone()
    ref = _two_launches(st, x, pos, k1, v1, None)
    got = _fused(st, x, pos, k2, v2, None)
    torch.cuda.synchronize()
    assert torch.equal(got, ref), (m, length)
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    assert bool((st["handoff"] == -1).all())


@pytest.mark.parametrize("m,length", [(16, 700), (7, 0), (16, 2040)])
def test_fused_draft_tree(dev, setup, m, length):
    st = setup
    desc = DraftTree(branching_tree((4, 2, 1), m)[0], dev).desc
    x = _x(dev, m, 200 + m)
    pos = torch.tensor([length], dtype=torch.int32, device=dev)
    k1, v1, k2, v2 = st["kc"].clone(), st["vt"].clone(), st["kc"].clone(), st["vt"].clone()
    ref = _two_launches(st, x, pos, k1, v1, desc)
    got = _fused(st, x, pos, k2, v2, desc)
    assert torch.equal(got, ref) and torch.equal(k1, k2) and torch.equal(v1, v2)
    assert bool((st["handoff"] == -1).all())


def test_calls_in_a_row_and_graph_replays(dev, setup):
    """Consecutive calls at growing lengths, then a captured call replayed three times with eager
    work between the replays: every result equals the two-launch path's."""
    st = setup
    k1, v1, k2, v2 = st["kc"].clone(), st["vt"].clone(), st["kc"].clone(), st["vt"].clone()
    pos1 = torch.tensor([500], dtype=torch.int32, device=dev)
    pos2 = pos1.clone()
    for i, m in enumerate((4, 1, 16, 2)):
        x = _x(dev, m, 300 + i)
        ref = _two_launches(st, x, pos1, k1, v1, None)
        got = _fused(st, x, pos2, k2, v2, None)
        assert torch.equal(got, ref), i
        pos1 += m
        pos2 += m
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    from skinny_mlx.graphs import capture_graph

    xs = _x(dev, 8, 400)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _fused(st, xs, pos2, k2, v2, None)  # first-use work outside the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    pos1 += 8
    _two_launches(st, xs, pos1 - 8, k1, v1, None)
    graph, out = capture_graph(lambda: _fused(st, xs, pos2, k2, v2, None))
    for r in range(3):
        xs.copy_(_x(dev, 8, 500 + r))
        pos2.fill_(600 + 10 * r)
        pos1.fill_(600 + 10 * r)
        graph.replay()
        ref = _two_launches(st, xs, pos1, k1, v1, None)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), r
        assert bool((st["handoff"] == -1).all())
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    del graph
