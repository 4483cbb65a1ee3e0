"""GPU parity of the decoder kernels (through the C ABI) against the oracle, on seeded inputs."""

import numpy as np
import pytest
import torch

from oracle import accept as A
from oracle import gdn as G
from oracle import model as OM
from oracle import w4
from skinny_mlx import kernels as K
from tests.helpers import bits16

pytestmark = pytest.mark.gpu


def _bf(x, dev):
    return torch.as_tensor(x, dtype=torch.float32).to(torch.bfloat16).to(dev)


def _f(t):
    return w4.bf16_to_f32(bits16(t)).astype(np.float64)


def test_rmsnorm_residual_inplace(dev):
    g = torch.Generator().manual_seed(0)
    x = torch.randn((7, 2560), generator=g).to(torch.bfloat16)
    r = torch.randn((7, 2560), generator=g).to(torch.bfloat16)
    w = (torch.randn(2560, generator=g) * 0.1 + 1).to(torch.bfloat16)
    xd, rd, wd = x.to(dev), r.to(dev), w.to(dev)
    out = K.rmsnorm(xd, wd, 1e-6, residual=rd, sum_out=xd)  # in-place residual add
    h = w4.round_bf16(_f(x) + _f(r))
    assert np.array_equal(_f(xd), h)
    ref = OM.rmsnorm(h, bits16(w), 1e-6)
    assert np.max(np.abs(_f(out) - ref)) <= np.max(np.abs(ref)) * 2 ** -7
    plain = K.rmsnorm(rd, wd, 1e-6)
    assert w4.rel_err(_f(plain), OM.rmsnorm(_f(r), bits16(w), 1e-6)) <= 8e-3


def test_mtp_input_is_bitwise_embed_norms_concat(dev):
    """skinny_mtp_input_bf16: the MTP head's fc input in one launch is bitwise
    cat(rmsnorm(embed(ids)), rmsnorm(hidden)), with out-of-range ids clamped like embed and
    hidden rows read at a row stride; and it matches the oracle's norms."""
    g = torch.Generator().manual_seed(11)
    V, H = 300, 2560
    table = torch.randn((V, H), generator=g).to(torch.bfloat16).to(dev)
    w_e = (torch.randn(H, generator=g) * 0.1 + 1).to(torch.bfloat16).to(dev)
    w_h = (torch.randn(H, generator=g) * 0.1 + 1).to(torch.bfloat16).to(dev)
    wide = (torch.randn((9, H + 64), generator=g) * 3).to(torch.bfloat16).to(dev)
    for t in (1, 3, 9):
        ids = torch.tensor([5, -4, 299, 300, 77, 0, 1000, 12, 150][:t], dtype=torch.int32, device=dev)
        hidden = wide[:t, 64:]  # stride H + 64
        out = K.mtp_input(ids, table, hidden, w_e, w_h, 1e-6)
        want = torch.cat([K.rmsnorm(K.embed(ids, table), w_e, 1e-6), K.rmsnorm(hidden.contiguous(), w_h, 1e-6)], -1)
        torch.cuda.synchronize()
        assert torch.equal(out, want), t
        rows = np.clip(ids.cpu().numpy(), 0, V - 1)
        ref = OM.rmsnorm(_f(table)[rows], bits16(w_e.cpu()), 1e-6)
        assert np.max(np.abs(_f(out[:, :H]) - ref)) <= np.max(np.abs(ref)) * 2 ** -7
    with pytest.raises(ValueError, match="aligned"):
        K.mtp_input(ids[:1], table, wide[:1, 4:4 + H], w_e, w_h, 1e-6)


def test_silu_mul_and_embed(dev):
    g = torch.Generator().manual_seed(1)
    gu = torch.randn((5, 2 * 300), generator=g).to(torch.bfloat16)
    act = K.silu_mul(gu.to(dev))
    gg, uu = _f(gu)[:, :300], _f(gu)[:, 300:]
    ref = w4.round_bf16(gg / (1 + np.exp(-gg)) * uu)
    assert np.max(np.abs(_f(act) - ref)) <= np.max(np.abs(ref)) * 2 ** -7
    table = torch.randn((100, 64), generator=g).to(torch.bfloat16)
    ids = torch.tensor([3, 0, 99, 3, 57], dtype=torch.int32)
    e = K.embed(ids.to(dev), table.to(dev))
    assert np.array_equal(bits16(e), bits16(table)[ids.numpy()])


def test_argmax_first_index_and_accept(dev):
    rng = np.random.default_rng(2)
    # few distinct values -> many exact ties, as with flat random-init logits in bf16
    logits = rng.integers(-3, 4, size=(9, 151936)).astype(np.float32)
    logits[3, 150000] = 10.0
    logits[4, :] = 0.0
    logits[5, :] = -np.inf          # a fully masked row: index 0
    logits[6, :140000] = -np.inf    # masked except the tail
    logits[6, 150001] = 3.0
    lt = _bf(logits, dev)
    pred = K.argmax_rows(lt).cpu().numpy()
    assert pred.tolist() == [A.argmax_first(r) for r in logits]
    # rows not 16-byte aligned (one value at a time), and rows longer than one round trip holds
    odd = _bf(rng.integers(-3, 4, size=(3, 151937)).astype(np.float32), dev)[:, 1:]
    assert K.argmax_rows(odd).cpu().numpy().tolist() == [A.argmax_first(r) for r in odd.float().cpu().numpy()]
    long = rng.integers(-3, 4, size=(2, 200000)).astype(np.float32)
    long[1, 199990] = 9.0
    assert K.argmax_rows(_bf(long, dev)).cpu().numpy().tolist() == [A.argmax_first(r) for r in long]
    out = torch.empty(3, dtype=torch.int32, device=dev)
    for k in range(0, 9):
        for trial in range(4):
            draft = pred[:k].copy()
            if trial and k:
                draft[rng.integers(0, k)] += 1  # a mismatch somewhere
            K.accept(torch.tensor(pred[:k + 1], dtype=torch.int32, device=dev),
                     torch.tensor(draft, dtype=torch.int32, device=dev) if k else None, out)
            assert tuple(out.cpu().tolist()) == A.accept(list(draft), list(pred[:k + 1]))


def test_conv_silu_and_window(dev):
    rng = np.random.default_rng(3)
    T, C = 6, 300
    x = w4.round_bf16(rng.standard_normal((T, C)))
    st = w4.round_bf16(rng.standard_normal((3, C)))
    wc = w4.round_bf16(rng.standard_normal((C, 4)) * 0.5)
    xd, std_, wd = _bf(x, dev), _bf(st, dev), _bf(wc, dev)
    window = torch.zeros((T + 3, C), dtype=torch.bfloat16, device=dev)
    out = K.gdn_conv_silu(xd, std_, wd, window)
    ref, st_ref, win_ref = G.conv_silu(x, st, wc)
    assert np.max(np.abs(_f(out) - ref)) <= np.max(np.abs(ref)) * 2 ** -7
    assert np.array_equal(_f(std_), st_ref) and np.array_equal(_f(window), win_ref)


def _gdn_inputs(rng, T, H, dev):
    qkv = w4.round_bf16(rng.standard_normal((T, 3 * H * 128)))
    ab = w4.round_bf16(rng.standard_normal((T, 2 * H)))
    A_log = np.log(rng.uniform(1, 16, H))
    dt = rng.uniform(-1, 1, H)
    S0 = rng.standard_normal((H, 128, 128)) * 0.1
    return qkv, ab, A_log, dt, S0


def _split_qkv(qkv, T, H):
    return (qkv[:, :H * 128].reshape(T, H, 128), qkv[:, H * 128:2 * H * 128].reshape(T, H, 128),
            qkv[:, 2 * H * 128:].reshape(T, H, 128))


@pytest.mark.parametrize("T,H,record", [(5, 4, True), (5, 16, False), (5, 16, True), (16, 16, False),
                                        (16, 16, True)])
def test_gdn_recurrence_matches_oracle(dev, T, H, record):
    """The recurrence against the oracle, up to the hybrid decoder's shape (16 heads of 128 x 128
    state) and a whole 16-token staging block, with and without the per-token states."""
    rng = np.random.default_rng(4 + 100 * T + H)
    qkv, ab, A_log, dt, S0 = _gdn_inputs(rng, T, H, dev)
    qd, abd = _bf(qkv, dev), _bf(ab, dev)
    state = torch.tensor(S0, dtype=torch.float32, device=dev)
    states = torch.zeros((T, H, 128, 128), dtype=torch.float32, device=dev) if record else None
    y = K.gdn_recurrence(qd, abd[:, :H], abd[:, H:], torch.tensor(A_log, dtype=torch.float32, device=dev),
                         torch.tensor(dt, dtype=torch.float32, device=dev), state, states, H, 128, 128)
    q, k, v = _split_qkv(qkv, T, H)
    S0f = S0.astype(np.float32).astype(np.float64)
    y_ref, st_ref = G.recurrence(q, k, v, ab[:, H:], ab[:, :H], A_log.astype(np.float32), dt.astype(np.float32), S0f)
    assert w4.rel_err(y.cpu().numpy(), y_ref) <= 1e-4
    assert w4.rel_err(state.cpu().numpy(), st_ref[-1]) <= 1e-4
    if record:
        assert w4.rel_err(states.cpu().numpy(), st_ref) <= 1e-4
        assert np.array_equal(state.cpu().numpy(), states[-1].cpu().numpy())


def test_gdn_tree_recurrence_matches_oracle_per_path(dev):
    """A 16-node draft tree (branching 4, 2, 1) over the hybrid decoder's 16 heads: every node's
    output and recorded state equal the oracle's recurrence run along that node's own path from
    the root, and the state before the pass is left as it was."""
    from skinny_mlx.tree import branching_tree

    rng = np.random.default_rng(9)
    M, H = 16, 16
    parents, _, _ = branching_tree((4, 2, 1), M)
    qkv, ab, A_log, dt, S0 = _gdn_inputs(rng, M, H, dev)
    state = torch.tensor(S0, dtype=torch.float32, device=dev)
    before = state.clone()
    states = torch.zeros((M, H, 128, 128), dtype=torch.float32, device=dev)
    par = torch.tensor(parents, dtype=torch.int32, device=dev)
    y = K.gdn_recurrence(_bf(qkv, dev), _bf(ab, dev)[:, :H], _bf(ab, dev)[:, H:],
                         torch.tensor(A_log, dtype=torch.float32, device=dev),
                         torch.tensor(dt, dtype=torch.float32, device=dev), state, states, H, 128, 128, par)
    assert torch.equal(state, before)
    q, k, v = _split_qkv(qkv, M, H)
    S0f = S0.astype(np.float32).astype(np.float64)
    yc, sc = y.cpu().numpy(), states.cpu().numpy()
    for node in range(M):
        path = [node]
        while parents[path[-1]] >= 0:
            path.append(parents[path[-1]])
        path = path[::-1]
        y_ref, st_ref = G.recurrence(q[path], k[path], v[path], ab[path, H:], ab[path, :H], A_log.astype(np.float32),
                                     dt.astype(np.float32), S0f)
        assert w4.rel_err(yc[node], y_ref[-1]) <= 1e-4, node
        assert w4.rel_err(sc[node], st_ref[-1]) <= 1e-4, node


@pytest.mark.parametrize("path", [[0], [0, 1], [0, 1, 5, 13], [0, 2, 7, 15], [0, 4, 12]])
def test_gdn_tree_commit_replay_equals_recorded_states(dev, path):
    """A draft tree's pass over two layers keeping both its node states and its update operands:
    the commit by replay from the operands (skinny_gdn_commit_replay) leaves every layer's state,
    and its conv state, bitwise as the commit from the recorded node states (skinny_gdn_commit),
    the leaf's state of the pass."""
    from skinny_mlx.tree import branching_tree

    rng = np.random.default_rng(8)
    M, H, L, C = 16, 4, 2, 3 * 4 * 128
    parents, _, _ = branching_tree((4, 2, 1), M)
    assert all(parents[b] == a for a, b in zip(path, path[1:]))
    par = torch.tensor(parents, dtype=torch.int32, device=dev)
    state = torch.zeros((L, H, 128, 128), dtype=torch.float32, device=dev)
    states = torch.zeros((L, M, H, 128, 128), dtype=torch.float32, device=dev)
    record = torch.zeros((L, K.gdn_record_words(H)), dtype=torch.float32, device=dev)
    for l in range(L):
        qkv, ab, A_log, dt, S0 = _gdn_inputs(rng, M, H, dev)
        state[l] = torch.tensor(S0, dtype=torch.float32, device=dev)
        K.gdn_recurrence(_bf(qkv, dev), _bf(ab, dev)[:, :H], _bf(ab, dev)[:, H:],
                         torch.tensor(A_log, dtype=torch.float32, device=dev),
                         torch.tensor(dt, dtype=torch.float32, device=dev), state[l], states[l], H, 128, 128, par,
                         record[l])
    before = state.clone()
    conv = _bf(w4.round_bf16(rng.standard_normal((L, 3, C))), dev)
    window = _bf(w4.round_bf16(rng.standard_normal((L, M + 3, C))), dev)
    dev_path = torch.tensor([len(path)] + path, dtype=torch.int32, device=dev)
    s1, s2, c1, c2 = state.clone(), state.clone(), conv.clone(), conv.clone()
    K.gdn_commit(dev_path, M, s1, states, c1, window)
    K.gdn_commit_replay(dev_path, H, s2, record, c2, window)
    assert torch.equal(before, state)  # a tree pass leaves the state as it was
    assert torch.equal(s1, s2) and torch.equal(c1, c2)
    assert torch.equal(s2, states[:, path[-1]])


def test_gdn_prefix_bitwise_and_select(dev):
    """S_keep from a verify over `fed` tokens is bitwise the state of a run over only `keep`."""
    rng = np.random.default_rng(5)
    fed, H = 6, 2
    qkv, ab, A_log, dt, S0 = _gdn_inputs(rng, fed, H, dev)
    qd, abd = _bf(qkv, dev), _bf(ab, dev)
    Al, dtt = torch.tensor(A_log, dtype=torch.float32, device=dev), torch.tensor(dt, dtype=torch.float32, device=dev)
    st_all = torch.tensor(S0, dtype=torch.float32, device=dev)[None].repeat(2, 1, 1, 1).contiguous()
    states = torch.zeros((2, 16, H, 128, 128), dtype=torch.float32, device=dev)
    conv = torch.zeros((2, 3, 8), dtype=torch.bfloat16, device=dev)
    window = torch.zeros((2, 19, 8), dtype=torch.bfloat16, device=dev)
    window[:, :fed + 3] = torch.arange((fed + 3) * 8, dtype=torch.float32, device=dev).reshape(fed + 3, 8).to(torch.bfloat16)
    y_full = K.gdn_recurrence(qd, abd[:, :H], abd[:, H:], Al, dtt, st_all[1], states[1], H, 128, 128)
    for keep in range(1, fed + 1):
        s_k = torch.tensor(S0, dtype=torch.float32, device=dev)
        y_k = K.gdn_recurrence(qd[:keep].contiguous(), abd[:keep, :H], abd[:keep, H:], Al, dtt, s_k, None, H, 128, 128)
        assert torch.equal(y_k, y_full[:keep])
        assert torch.equal(s_k, states[1, keep - 1])
        # device select picks the same state for layer 1 (and the conv rows keep .. keep+2)
        sel = st_all.clone()
        cv = conv.clone()
        K.gdn_select(torch.tensor([keep], dtype=torch.int32, device=dev), fed, sel, states, cv, window)
        if keep < fed:
            assert torch.equal(sel[1], s_k)
            assert torch.equal(cv[1], window[1, keep:keep + 3])
        else:
            assert torch.equal(sel, st_all) and torch.equal(cv, conv)  # keep == fed: no-op


def _attn_case(rng, L, M, Hq, Hkv, maxlen, dev):
    D = 128
    kc = np.zeros((Hkv, maxlen, D))
    vc = np.zeros((Hkv, maxlen, D))
    kc[:, :L + M] = w4.round_bf16(rng.standard_normal((Hkv, L + M, D)))
    vc[:, :L + M] = w4.round_bf16(rng.standard_normal((Hkv, L + M, D)))
    q = w4.round_bf16(rng.standard_normal((M, Hq, D)))
    return q, kc, vc


@pytest.mark.parametrize("L,M", [(0, 1), (5, 8), (300, 16), (1000, 3), (9000, 5)])
def test_attention_matches_oracle(dev, L, M):
    """Up to 9000 cached keys: more than one block of 32 chunk partials, which the merge folds with
    several waves."""
    rng = np.random.default_rng(6 + L)
    Hq, Hkv, maxlen = 32, 8, max(1280, -(-(L + M) // 128) * 128)
    q, kc, vc = _attn_case(rng, L, M, Hq, Hkv, maxlen, dev)
    kd = _bf(kc, dev)
    vtd = _bf(np.swapaxes(vc, 1, 2), dev).contiguous()
    ws = K.attn_workspace(Hkv, maxlen, dev)
    pos = torch.tensor([L], dtype=torch.int32, device=dev)
    out = K.attention(_bf(q, dev), kd, vtd, pos, 128 ** -0.5, ws).cpu()
    got = w4.bf16_to_f32(out.view(torch.int16).numpy().view(np.uint16)).reshape(M, Hq, 128)
    G_ = Hq // Hkv
    ref = np.stack([np.stack([OM.attention_row(q[t, h], kc[h // G_, :L + t + 1], vc[h // G_, :L + t + 1], 128 ** -0.5)
                              for h in range(Hq)]) for t in range(M)])
    assert w4.rel_err(got, ref) <= 2e-2
    assert np.max(np.abs(got - ref)) <= 2e-2


def test_attention_bitwise_m_invariant(dev):
    """Token t's output is identical whether it is verified in a batch of M or alone."""
    rng = np.random.default_rng(7)
    Hq, Hkv, maxlen, L, M = 32, 8, 768, 200, 12
    q, kc, vc = _attn_case(rng, L, M, Hq, Hkv, maxlen, dev)
    kd, vtd = _bf(kc, dev), _bf(np.swapaxes(vc, 1, 2), dev).contiguous()
    ws = K.attn_workspace(Hkv, maxlen, dev)
    qd = _bf(q, dev)
    full = K.attention(qd, kd, vtd, torch.tensor([L], dtype=torch.int32, device=dev), 128 ** -0.5, ws)
    for t in range(M):
        one = K.attention(qd[t:t + 1].contiguous(), kd, vtd, torch.tensor([L + t], dtype=torch.int32, device=dev),
                          128 ** -0.5, ws)
        assert torch.equal(one, full[t:t + 1]), t


def test_qk_rope_store_matches_oracle(dev):
    rng = np.random.default_rng(8)
    M, Hq, Hkv, D, maxlen, p0 = 3, 4, 2, 128, 256, 17
    qkv = w4.round_bf16(rng.standard_normal((M, (Hq + 2 * Hkv) * D)))
    qn = w4.f32_to_bf16(1 + 0.1 * rng.standard_normal(D))
    kn = w4.f32_to_bf16(1 + 0.1 * rng.standard_normal(D))
    kc = torch.zeros((Hkv, maxlen, D), dtype=torch.bfloat16, device=dev)
    vt = torch.zeros((Hkv, D, maxlen), dtype=torch.bfloat16, device=dev)
    qnd = torch.from_numpy(qn.view(np.int16)).view(torch.bfloat16).to(dev)
    knd = torch.from_numpy(kn.view(np.int16)).view(torch.bfloat16).to(dev)
    q = K.qk_rope_store(_bf(qkv, dev), Hq, Hkv, D, qnd, knd, 1e-6, torch.tensor([p0], dtype=torch.int32, device=dev),
                        1e6, kc, vt)
    qg, kg, vg = _f(q), _f(kc), _f(vt)
    for t in range(M):
        for h in range(Hq + 2 * Hkv):
            x = qkv[t, h * D:(h + 1) * D]
            if h < Hq:
                ref = OM.rope(OM.rmsnorm(x, qn, 1e-6), p0 + t, 1e6)
                assert np.max(np.abs(qg[t, h] - ref)) <= 2 ** -6 * np.max(np.abs(ref))
            elif h < Hq + Hkv:
                ref = OM.rope(OM.rmsnorm(x, kn, 1e-6), p0 + t, 1e6)
                assert np.max(np.abs(kg[h - Hq, p0 + t] - ref)) <= 2 ** -6 * np.max(np.abs(ref))
            else:
                assert np.array_equal(vg[h - Hq - Hkv, :, p0 + t], x)


@pytest.mark.parametrize("M,L,tree", [(1, 0, False), (8, 2040, False), (16, 300, False), (5, 126, False),
                                      (16, 700, True), (7, 0, True), (8, 16380, False), (16, 16300, True)])
@pytest.mark.parametrize("norms", [True, False])
def test_fused_attention_equals_rope_store_then_attention(dev, M, L, tree, norms):
    """skinny_attention_fused_bf16 against the two-launch path it replaces (skinny_qk_rope_store +
    skinny_attention_bf16, both HIP): the same cache bits (keys and values of the new tokens) and
    outputs within bf16 rounding (the query RMSNorm sums its squares in another order). The oracle
    check of the fused path is test_fused_attention_matches_oracle_at_config_context."""
    from skinny_mlx.tree import DraftTree, branching_tree

    rng = np.random.default_rng(M * 1000 + L)
    Hq, Hkv, D, theta = 32, 8, 128, 1e6
    maxlen = max(2176, -(-(L + M) // 128) * 128 + 128)  # past 4096 slots the merge runs several waves
    qkv = _bf(w4.round_bf16(rng.standard_normal((M, (Hq + 2 * Hkv) * D))), dev)
    qn = _bf(w4.round_bf16(1 + 0.1 * rng.standard_normal(D)), dev) if norms else None
    kn = _bf(w4.round_bf16(1 + 0.1 * rng.standard_normal(D)), dev) if norms else None
    base_k = _bf(w4.round_bf16(rng.standard_normal((Hkv, maxlen, D))), dev)
    base_v = _bf(w4.round_bf16(rng.standard_normal((Hkv, D, maxlen))), dev)
    pos = torch.tensor([L], dtype=torch.int32, device=dev)
    desc = DraftTree(branching_tree((4, 2, 1), M)[0], dev).desc if tree else None
    ws = K.attn_workspace(Hkv, maxlen, dev)
    k1, v1 = base_k.clone(), base_v.clone()
    q = K.qk_rope_store(qkv, Hq, Hkv, D, qn, kn, 1e-6, pos, theta, k1, v1, desc)
    ref = K.attention(q, k1, v1, pos, D ** -0.5, ws, desc)
    k2, v2 = base_k.clone(), base_v.clone()
    table = K.rope_table(theta, maxlen, dev)
    got = K.attention_fused(qkv, Hq, Hkv, D, qn, kn, 1e-6, table, pos, k2, v2, D ** -0.5, ws, desc)
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    a, b = _f(got), _f(ref)
    assert np.max(np.abs(a - b)) <= 2 ** -6 * np.max(np.abs(b))
    assert np.mean(a == b) > 0.9


@pytest.mark.parametrize("maxlen,L", [(1024, 300), (20480, 20000)])
def test_fused_attention_bitwise_m_invariant(dev, maxlen, L):
    """Token t's output is identical whether it is verified in a batch of 12 or alone, also over 160
    chunks (five blocks of partials, folded by the merge's four waves)."""
    rng = np.random.default_rng(9)
    Hq, Hkv, D, M = 32, 8, 128, 12
    qkv = _bf(w4.round_bf16(rng.standard_normal((M, (Hq + 2 * Hkv) * D))), dev)
    qn = _bf(w4.round_bf16(1 + 0.1 * rng.standard_normal(D)), dev)
    kn = _bf(w4.round_bf16(1 + 0.1 * rng.standard_normal(D)), dev)
    kc = _bf(w4.round_bf16(rng.standard_normal((Hkv, maxlen, D))), dev)
    vt = _bf(w4.round_bf16(rng.standard_normal((Hkv, D, maxlen))), dev)
    ws = K.attn_workspace(Hkv, maxlen, dev)
    table = K.rope_table(1e6, maxlen, dev)
    full = K.attention_fused(qkv, Hq, Hkv, D, qn, kn, 1e-6, table, torch.tensor([L], dtype=torch.int32, device=dev),
                             kc.clone(), vt.clone(), D ** -0.5, ws)
    k2, v2 = kc.clone(), vt.clone()
    for t in range(M):
        one = K.attention_fused(qkv[t:t + 1], Hq, Hkv, D, qn, kn, 1e-6, table,
                                torch.tensor([L + t], dtype=torch.int32, device=dev), k2, v2, D ** -0.5, ws)
        assert torch.equal(one, full[t:t + 1]), t


def test_rope_table_matches_oracle(dev):
    """cos/sin of pos * theta^(-2i/128); the fp32 angle carries ~pos * 2^-24 of rounding, as in
    the separate RoPE kernel, so the bound grows with the position."""
    table = K.rope_table(1e6, 4096, dev).cpu().double().numpy()
    i = np.arange(64)
    for p in (0, 1, 17, 299, 4095):
        ang = p * 1e6 ** (-2.0 * i / 128)
        tol = 1e-6 + 2.4e-7 * p
        assert np.max(np.abs(table[p, :, 0] - np.cos(ang))) <= tol, p
        assert np.max(np.abs(table[p, :, 1] - np.sin(ang))) <= tol, p


@pytest.mark.parametrize("tree", [False, True])
@pytest.mark.parametrize("M", [1, 8, 16])
def test_fused_attention_matches_oracle_at_config_context(dev, M, tree):
    """The attention the decoder calls (skinny_attention_fused_bf16) against the oracle at the
    verify step's shape: Hq = 32, Hkv = 8, D = 128, 2040 cached keys plus M new ones (crossing
    the 2048-key chunk boundary), chain and (4, 2, 1) draft tree. The oracle normalises and rotates
    q and the new keys (oracle.model.rmsnorm, rope at the token's position, its depth in a tree),
    then softmax-attends over the cached rows and the new rows each token sees. Bars: logits-style
    rel-err <= 2e-2 and max |diff| <= 2e-2 (the path's bf16 tolerance); new key rows within bf16
    rounding of the oracle's; value rows bit-exact."""
    from skinny_mlx.tree import DraftTree, branching_tree

    rng = np.random.default_rng(100 + 10 * M + int(tree))
    Hq, Hkv, D, maxlen, theta, L, eps = 32, 8, 128, 2176, 1e6, 2040, 1e-6
    G_ = Hq // Hkv
    raw = w4.round_bf16(rng.standard_normal((M, (Hq + 2 * Hkv) * D)))
    qn = w4.f32_to_bf16(1 + 0.1 * rng.standard_normal(D))
    kn = w4.f32_to_bf16(1 + 0.1 * rng.standard_normal(D))
    kc = w4.round_bf16(rng.standard_normal((Hkv, maxlen, D)))
    vc = w4.round_bf16(rng.standard_normal((Hkv, maxlen, D)))
    if tree:
        parents, _, depth = branching_tree((4, 2, 1), M)
    else:
        parents, depth = [-1] + list(range(M - 1)), list(range(M))
    desc = DraftTree(parents, dev).desc if tree else None
    bits = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(dev)
    k_dev = _bf(kc, dev)
    vt_dev = _bf(np.swapaxes(vc, 1, 2), dev).contiguous()
    pos = torch.tensor([L], dtype=torch.int32, device=dev)
    ws = K.attn_workspace(Hkv, maxlen, dev)
    table = K.rope_table(theta, maxlen, dev)
    got = _f(K.attention_fused(_bf(raw, dev), Hq, Hkv, D, bits(qn), bits(kn), eps, table, pos, k_dev, vt_dev,
                               D ** -0.5, ws, desc)).reshape(M, Hq, D)
    q_rows = raw[:, :Hq * D].reshape(M, Hq, D)
    k_rows = raw[:, Hq * D:(Hq + Hkv) * D].reshape(M, Hkv, D)
    v_rows = raw[:, (Hq + Hkv) * D:].reshape(M, Hkv, D)
    k_new = np.stack([[w4.round_bf16(OM.rope(OM.rmsnorm(k_rows[t, h], kn, eps), L + depth[t], theta))
                       for h in range(Hkv)] for t in range(M)])
    ref = np.zeros((M, Hq, D))
    for t in range(M):
        seen, a = [], t
        while a >= 0:
            seen.append(a)
            a = parents[a]
        seen = sorted(seen)
        for h in range(Hq):
            hk = h // G_
            q = w4.round_bf16(OM.rope(OM.rmsnorm(q_rows[t, h], qn, eps), L + depth[t], theta))
            keys = np.concatenate([kc[hk, :L], k_new[seen, hk]])
            vals = np.concatenate([vc[hk, :L], v_rows[seen, hk]])
            ref[t, h] = OM.attention_row(q, keys, vals, D ** -0.5)
    assert w4.rel_err(got, ref) <= 2e-2
    assert np.max(np.abs(got - ref)) <= 2e-2
    kg = _f(k_dev)[:, L:L + M]                  # [Hkv, M, D]
    assert np.max(np.abs(kg - np.swapaxes(k_new, 0, 1))) <= 2 ** -7 * np.max(np.abs(k_new))
    vg = _f(vt_dev)[:, :, L:L + M]              # [Hkv, D, M]
    assert np.array_equal(vg, np.transpose(v_rows, (1, 2, 0)))
