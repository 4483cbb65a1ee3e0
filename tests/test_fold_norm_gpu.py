"""GPU parity of the norm-in projections (the RMSNorm before a fused projection formed inside its
launch), through the C ABI.

Bars, all bitwise: for the plain (q|k|v), SwiGLU (gate|up) and conv (Gated-DeltaNet input)
forms, the product equals the separate norm kernel (skinny_rmsnorm_partials_bf16, or
skinny_rmsnorm_bf16 without slices) followed by the plain projection of its output with the same
tile, and h_out equals that norm's sum_out, at the decoders' shapes, M = 1..4 within the LDS
budget, with 0 to 4 residual slices; the conv form also leaves the conv state and the rollback
window as the separate path does. The norm itself is pinned against the oracle by the RMSNorm
tests of test_kernels_gpu.py (the same kernel computes the reference here).
"""

import pytest
import torch

from skinny_mlx import kernels as K
from skinny_mlx import qmm as Q
from tests.helpers import qmm_case

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _rows(dev, m, k, splits, seed):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn((m, k), generator=g).to(torch.bfloat16).to(dev)
    parts = (torch.randn((splits, m, k), generator=g) * 0.3).to(dev) if splits else None
    w = (torch.randn(k, generator=g) * 0.1 + 1.0).to(torch.bfloat16).to(dev)
    return h, parts, w


def _inputs(h, parts, w):
    """(NormIn, the separate path's normed rows, its residual stream) for the same rows."""
    res = None if parts is None else K.PartialSum(parts)
    h_out = None if parts is None else torch.full_like(h, float("nan"))
    nx = K.NormIn(h, res, w, EPS, h_out)
    if parts is None:
        return nx, K.rmsnorm(h, w, EPS), h
    h_ref = torch.empty_like(h)
    return nx, K.rmsnorm(h, w, EPS, residual=res, sum_out=h_ref), h_ref


def _weights(dev, n, k, seed, gate_up=False):
    _, w, s, b = qmm_case(1, n, k, seed=seed)
    w, s, b = w.to(dev), s.to(dev), b.to(dev)
    return (Q.repack_gate_up if gate_up else Q.repack_for_skinny)(w, s, b)


@pytest.mark.parametrize("k,n", [(2560, 6144), (256, 768)])
@pytest.mark.parametrize("m,splits", [(1, 0), (1, 1), (1, 2), (1, 3), (1, 4), (2, 3), (4, 0)])
def test_normin_plain_is_bitwise_the_separate_path(dev, k, n, m, splits):
    if not Q.normin_supported(Q.NORMIN_PLAIN, m, k, n, splits):
        pytest.skip("rows past the norm-in LDS budget")
    wf = _weights(dev, n, k, 10 + m)
    h, parts, w = _rows(dev, m, k, splits, 20 + 7 * m + splits)
    nx, x_ref, h_ref = _inputs(h, parts, w)
    y = Q.skinny_qmm_normin(nx, wf)
    torch.cuda.synchronize()
    assert torch.equal(y, Q.skinny_qmm(x_ref, wf)), (m, splits)
    if parts is not None:
        assert torch.equal(nx.h_out, h_ref)


@pytest.mark.parametrize("k,f", [(2560, 9728), (256, 512)])
@pytest.mark.parametrize("m,splits", [(1, 3), (1, 0), (1, 1), (1, 2), (2, 3)])
def test_normin_swiglu_is_bitwise_the_separate_path(dev, k, f, m, splits):
    if not Q.normin_supported(Q.NORMIN_SWIGLU, m, k, 2 * f, splits):
        pytest.skip("rows past the norm-in LDS budget")
    gu = _weights(dev, 2 * f, k, 30 + m, gate_up=True)
    h, parts, w = _rows(dev, m, k, splits, 40 + m)
    nx, x_ref, h_ref = _inputs(h, parts, w)
    a = Q.skinny_glu_normin(nx, gu)
    assert torch.equal(a, Q.skinny_glu(x_ref, gu, swiglu=True)), (m, splits)
    if parts is not None:
        assert torch.equal(nx.h_out, h_ref)


@pytest.mark.parametrize("m,tree", [(1, False), (2, False), (2, True)])
def test_normin_conv_is_bitwise_the_separate_path(dev, m, tree):
    k, n, c, kw = 2560, 8224, 6144, 4
    if not Q.normin_supported(Q.NORMIN_CONV, m, k, n, 3):
        pytest.skip("rows past the norm-in LDS budget")
    wf = _weights(dev, n, k, 50 + m)
    h, parts, w = _rows(dev, m, k, 3, 60 + m)
    g = torch.Generator().manual_seed(70 + m)
    conv_w = (torch.randn((c, kw), generator=g) * 0.5).to(torch.bfloat16).to(dev)
    state0 = torch.randn((kw - 1, c), generator=g).to(torch.bfloat16).to(dev)
    parent = torch.tensor([-1, 0][:m], dtype=torch.int32, device=dev) if tree else None
    nx, x_ref, h_ref = _inputs(h, parts, w)
    s1, s2 = state0.clone(), state0.clone()
    w1 = torch.zeros((kw - 1 + m, c), dtype=torch.bfloat16, device=dev)
    w2 = torch.zeros_like(w1)
    y = Q.skinny_qmm_conv_normin(nx, wf, c, s1, conv_w, w1, parent)
    y_ref = Q.skinny_qmm_conv(x_ref, wf, c, s2, conv_w, w2, parent)
    assert torch.equal(y, y_ref) and torch.equal(s1, s2) and torch.equal(w1, w2)
    assert torch.equal(nx.h_out, h_ref)


def test_normin_value_and_kernel_agree_in_the_model_order(dev):
    """The order the decoder uses: a NormIn consumed by the norm-in kernel, then value() (the
    separate kernel, writing h_out again with the same bits) — both views agree."""
    k, n = 2560, 6144
    wf = _weights(dev, n, k, 80)
    h, parts, w = _rows(dev, 1, k, 3, 81)
    nx, x_ref, h_ref = _inputs(h, parts, w)
    y = Q.skinny_qmm_normin(nx, wf)
    first = nx.h_out.clone()
    assert torch.equal(nx.value(), x_ref) and torch.equal(nx.h_out, first) and torch.equal(first, h_ref)
    assert torch.equal(y, Q.skinny_qmm(nx.value(), wf))
