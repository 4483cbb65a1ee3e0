"""GPU parity of the RMSNorm folded into the matmuls around it, through the C ABI.

Producer (skinny_qmm_w4g64_resnorm_bf16): the split-K projection whose output is a residual
finishes the residual add and the norm's input side in its epilogue. Bars: the new residual
stream is bitwise what the split-K slices + partial-residual RMSNorm store as sum_out; xw is
exactly bf16(v * w); the per-tile sums of v^2 match fp32 sums; the tile-group counters are zero
after every call, so a second call (fewer tokens) is right too.

Consumer (skinny_qmm_w4g64_scaled_bf16 and the glu form): y = inv[t] * (xw @ W^T) against the
fp64 oracle (dequant + matmul of the same xw, times 1/rms from the rows themselves) to the qmm
bar and 4e-3; bitwise M-invariant rows.
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle import w4
from skinny_mlx import _lib
from skinny_mlx import kernels as K
from skinny_mlx import qmm as Q
from tests.helpers import bits16, qmm_case, u32

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _to(dev, *ts):
    return [t.to(dev) for t in ts]


def _norm_weight(n, seed, dev):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(n, generator=g) * 0.1 + 1.0).to(torch.bfloat16).to(dev)


def _resnorm_raw(xd, wf, res, nw, splits, tile, counters):
    m, k = xd.shape
    n = wf.shape[0]
    xw = torch.empty((m, n), dtype=torch.bfloat16, device=xd.device)
    ss = torch.full((n // 16, 16), float("nan"), dtype=torch.float32, device=xd.device)
    part = torch.empty((splits, m, n), dtype=torch.float32, device=xd.device)
    _lib.check(_lib.lib().skinny_qmm_w4g64_resnorm_bf16(
        xd.data_ptr(), m, k, k, wf.data_ptr(), n, res.data_ptr(), n, nw.data_ptr(), res.data_ptr(), n,
        xw.data_ptr(), n, ss.data_ptr(), part.data_ptr(), n, counters.data_ptr(), splits, ctypes.byref(tile),
        _lib.stream_of(xd)), "resnorm")
    return xw, ss


@pytest.mark.parametrize("k,n", [(9728, 2560), (4096, 2560), (2048, 2560)])
@pytest.mark.parametrize("splits", [1, 2, 4])
def test_resnorm_residual_is_bitwise_the_partial_path(dev, k, n, splits):
    _, tile = Q.partial_config(k, n)
    counters = torch.zeros((n // 16,), dtype=torch.int32, device=dev)
    nw = _norm_weight(n, 3, dev)
    for m in (8, 3):  # the second call also checks that the counters were left at zero
        x, w, s, b = qmm_case(m, n, k, seed=20 + m)
        xd, wd, sd, bd = _to(dev, x, w, s, b)
        wf = Q.repack_for_skinny(wd, sd, bd)
        h = torch.randn((m, n), generator=torch.Generator().manual_seed(m)).to(torch.bfloat16).to(dev)
        part = torch.empty((splits, m, n), dtype=torch.float32, device=dev)
        _lib.check(_lib.lib().skinny_qmm_w4g64_partial_f32(xd.data_ptr(), m, k, k, wf.data_ptr(), n, part.data_ptr(),
                                                           n, splits, ctypes.byref(tile), _lib.stream_of(xd)),
                   "partial")
        h_ref = h.clone()
        K.rmsnorm(h_ref, nw, EPS, residual=K.PartialSum(part), sum_out=h_ref)
        h_new = h.clone()
        xw, ss = _resnorm_raw(xd, wf, h_new, nw, splits, tile, counters)
        torch.cuda.synchronize()
        assert torch.equal(h_new, h_ref), (m, splits)
        assert torch.equal(xw, (h_ref.float() * nw.float()).to(torch.bfloat16))
        ref_ss = (h_ref.double() ** 2).view(m, n // 16, 16).sum(-1).t()
        torch.testing.assert_close(ss[:, :m].double(), ref_ss, rtol=2e-6, atol=1e-6)
        assert int(counters.abs().sum()) == 0


def test_resnorm_module_path_and_defaults(dev):
    """qmm.skinny_qmm_resnorm (its default split and tile, shared counters) = the raw call; the
    NormedInput it returns materialises to rmsnorm(v) * w within bf16 rounding."""
    k, n, m = 9728, 2560, 8
    x, w, s, b = qmm_case(m, n, k, seed=30)
    xd, wd, sd, bd = _to(dev, x, w, s, b)
    wf = Q.repack_for_skinny(wd, sd, bd)
    nw = _norm_weight(n, 4, dev)
    h = torch.randn((m, n), generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).to(dev)
    splits, tile = Q.resnorm_config(k, n)
    h1 = h.clone()
    xw1, ss1 = _resnorm_raw(xd, wf, h1, nw, splits, tile, torch.zeros((n // 16,), dtype=torch.int32, device=dev))
    h2 = h.clone()
    nx = Q.skinny_qmm_resnorm(xd, wf, h2, nw, EPS)
    assert torch.equal(h1, h2) and torch.equal(nx.xw, xw1) and torch.equal(nx.ss[:, :m], ss1[:, :m])
    ref = K.rmsnorm(h1, nw, EPS)
    torch.testing.assert_close(nx.value().float(), ref.float(), rtol=1.6e-2, atol=1e-2)


def _scaled_reference(v, nw, x_w, wd, sd, bd):
    """fp64 oracle: inv[t] * (xw @ dequant(W)^T), inv from the rows of v."""
    v64 = v.double().cpu().numpy()
    inv = 1.0 / np.sqrt((v64 ** 2).mean(axis=1) + EPS)
    y = w4.qmm(bits16(x_w.cpu()), u32(wd.cpu()), bits16(sd.cpu()), bits16(bd.cpu()))
    return y * inv[:, None]


@pytest.mark.parametrize("k,n", [(2560, 6144), (2560, 8224), (4096, 1024)])
@pytest.mark.parametrize("m", [1, 8, 16])
def test_scaled_projection_matches_oracle(dev, k, n, m):
    x, w, s, b = qmm_case(m, n, k, seed=40 + m)
    xd, wd, sd, bd = _to(dev, x, w, s, b)
    nw = _norm_weight(k, 6, dev)
    nx = K.rms_prep(xd, nw, EPS)
    assert torch.equal(nx.xw, (xd.float() * nw.float()).to(torch.bfloat16))
    ref_ss = (xd.double() ** 2).view(m, k // 16, 16).sum(-1).t()
    torch.testing.assert_close(nx.ss[:, :m].double(), ref_ss, rtol=2e-6, atol=1e-6)
    y = Q.skinny_qmm_scaled(nx, Q.repack_for_skinny(wd, sd, bd))
    ref = _scaled_reference(xd, nw, nx.xw, wd, sd, bd)
    err = w4.rel_err(w4.bf16_to_f32(bits16(y.cpu())), ref)
    assert err <= 2e-2 and err <= 4e-3


@pytest.mark.parametrize("m", [1, 8, 16])
def test_scaled_glu_matches_oracle_and_swiglu_bitwise(dev, m):
    k, f = 2560, 1024
    x, w, s, b = qmm_case(m, 2 * f, k, seed=50 + m)
    xd, wd, sd, bd = _to(dev, x, w, s, b)
    nw = _norm_weight(k, 7, dev)
    nx = K.rms_prep(xd, nw, EPS)
    wf = Q.repack_gate_up(wd, sd, bd)
    split = Q.skinny_glu_scaled(nx, wf, swiglu=False)  # [gate | up], the unfused column order
    ref = _scaled_reference(xd, nw, nx.xw, wd, sd, bd)
    err = w4.rel_err(w4.bf16_to_f32(bits16(split.cpu())), ref)
    assert err <= 2e-2 and err <= 4e-3
    act = Q.skinny_glu_scaled(nx, wf, swiglu=True)
    assert torch.equal(act, K.silu_mul(split))


def test_scaled_rows_bitwise_m_invariant(dev):
    k, n = 2560, 6144
    x, w, s, b = qmm_case(16, n, k, seed=60)
    xd, wd, sd, bd = _to(dev, x, w, s, b)
    wf = Q.repack_for_skinny(wd, sd, bd)
    gu = Q.repack_gate_up(wd, sd, bd)
    nw = _norm_weight(k, 8, dev)
    full = K.rms_prep(xd, nw, EPS)
    y16, a16 = Q.skinny_qmm_scaled(full, wf), Q.skinny_glu_scaled(full, gu, swiglu=True)
    for m in (1, 5, 8):
        part = K.rms_prep(xd[:m].contiguous(), nw, EPS)
        assert torch.equal(Q.skinny_qmm_scaled(part, wf), y16[:m]), m
        assert torch.equal(Q.skinny_glu_scaled(part, gu, swiglu=True), a16[:m]), m


def test_scaled_rejects_bad_arguments(dev):
    x, w, s, b = qmm_case(4, 256, 8192, seed=70)
    xd, wd, sd, bd = _to(dev, x, w, s, b)
    nx = K.NormedInput(xd, torch.zeros((8192 // 16, 16), dtype=torch.float32, device=dev), EPS)
    with pytest.raises(ValueError, match="exceeds"):
        Q.skinny_qmm_scaled(nx, Q.repack_for_skinny(wd, sd, bd))
    with pytest.raises(ValueError, match="ss must be"):
        Q.skinny_qmm_scaled(K.NormedInput(xd[:, :2560].contiguous(), nx.ss, EPS),
                            Q.repack_for_skinny(wd[:, :320].contiguous(), sd[:, :40].contiguous(),
                                                bd[:, :40].contiguous()))
