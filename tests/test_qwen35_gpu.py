"""The Qwen3.5 architecture on the GPU (the reference loads Qwen3.5-4B, spec.py:175): the general
attention kernels (head_dim 64/128/256, RoPE over part of each head, query heads at a stride, the
sigmoid output gate) and the Gated-DeltaNet kernels with key heads shared by value heads, each
against the oracle, whose Qwen3.5 composition is pinned to transformers' Qwen3_5ForCausalLM
(tests/test_oracle_model.py). The tiny Qwen3.5-shaped decoder ("tiny-qwen35") runs through the
decoder, speculative, draft-tree and sampling tests with the other tiny presets.

Bars: attention outputs within the path's bf16 tolerance of the fp64 oracle (rel-err and max
|diff| <= 2e-2); new key rows within bf16 rounding; value rows bit-exact; GDN outputs and states
within 1e-4 of the fp64 recurrence; bitwise M-invariance where the device path promises it."""

import numpy as np
import pytest
import torch

from oracle import gdn as G
from oracle import model as OM
from oracle import w4
from skinny_mlx import kernels as K
from tests.helpers import bits16

pytestmark = pytest.mark.gpu


def _bf(x, dev):
    return torch.from_numpy(w4.f32_to_bf16(np.asarray(x, np.float32)).view(np.int16)).view(torch.bfloat16).to(dev)


def _f(t):
    return w4.bf16_to_f32(bits16(t)).astype(np.float64)


def _layout(Hq, Hkv, D, gated):
    """(q_stride, k_offset, v_offset, gate_offset, row width) of Qwen3.5's q|k|v rows."""
    qs = 2 * D if gated else D
    return qs, Hq * qs, Hq * qs + Hkv * D, (D if gated else None), Hq * qs + 2 * Hkv * D


@pytest.mark.parametrize("D,rd,gated", [(256, 64, True), (256, 256, False), (128, 64, True), (64, 64, False),
                                        (128, 128, True)])
@pytest.mark.parametrize("M,L,tree", [(1, 0, False), (8, 300, False), (16, 2040, False), (16, 700, True),
                                      (5, 126, True)])
def test_general_attention_matches_oracle(dev, D, rd, gated, M, L, tree):
    """skinny_attention_general_bf16 against the oracle: q/k RMSNorm, RoPE over the first rd dims
    at the token's position (its depth in a draft tree), softmax attention over the cached rows and
    the new rows each token sees (causal or its ancestors), then bf16(o) * bf16(sigmoid(gate)).
    Hq = 4, Hkv = 2 (two query heads per kv head)."""
    from skinny_mlx.tree import DraftTree, branching_tree

    rng = np.random.default_rng(1000 * D + 100 * M + rd + int(tree) + L)
    Hq, Hkv, maxlen, theta, eps = 4, 2, 2176, 1e7, 1e-6
    G_ = Hq // Hkv
    qs, koff, voff, goff, width = _layout(Hq, Hkv, D, gated)
    raw = w4.round_bf16(rng.standard_normal((M, width)))
    qn = w4.f32_to_bf16(1 + 0.1 * rng.standard_normal(D))
    kn = w4.f32_to_bf16(1 + 0.1 * rng.standard_normal(D))
    kc = w4.round_bf16(rng.standard_normal((Hkv, maxlen, D)))
    vc = w4.round_bf16(rng.standard_normal((Hkv, maxlen, D)))
    kcd, vtd = _bf(kc, dev), _bf(np.swapaxes(vc, 1, 2), dev).contiguous()
    pos = torch.tensor([L], dtype=torch.int32, device=dev)
    parents = branching_tree((4, 2, 1), M)[0] if tree else None
    desc = DraftTree(parents, dev).desc if tree else None
    table = K.rope_table_dim(theta, rd, maxlen, dev)
    ws = K.attn_general_workspace(Hq, Hkv, D, maxlen, dev)
    out = K.attention_general(_bf(raw, dev), Hq, Hkv, D, qs, koff, voff, goff, _bf(w4.bf16_to_f32(qn), dev),
                              _bf(w4.bf16_to_f32(kn), dev), eps, rd, table, pos, kcd, vtd, D ** -0.5, ws, desc)
    got = _f(out).reshape(M, Hq, D)
    depth = list(range(M))  # RoPE position offset: the token's index in a chain, its depth in a tree
    if tree:
        for t in range(1, M):
            depth[t] = depth[parents[t]] + 1
        depth[0] = 0
    ks_new = np.stack([[OM.rope(OM.rmsnorm(raw[t, koff + j * D:koff + (j + 1) * D], kn, eps), L + depth[t], theta, rd)
                        for j in range(Hkv)] for t in range(M)])
    vs_new = np.stack([[raw[t, voff + j * D:voff + (j + 1) * D] for j in range(Hkv)] for t in range(M)])
    kg, vg = _f(kcd), _f(vtd)
    for t in range(M):  # the new rows in the caches
        for j in range(Hkv):
            assert np.max(np.abs(kg[j, L + t] - ks_new[t, j])) <= 2 ** -6 * np.max(np.abs(ks_new[t, j]))
            assert np.array_equal(vg[j, :, L + t], vs_new[t, j])
    ref = np.zeros((M, Hq, D))
    for t in range(M):
        seen = [u for u in range(M) if (u <= t if not tree else u in _ancestors(parents, t))]
        for h in range(Hq):
            j = h // G_
            q = OM.rope(OM.rmsnorm(raw[t, h * qs:h * qs + D], qn, eps), L + depth[t], theta, rd)
            keys = np.concatenate([kc[j, :L], np.stack([w4.round_bf16(ks_new[u, j]) for u in seen])])
            vals = np.concatenate([vc[j, :L], np.stack([vs_new[u, j] for u in seen])])
            o = OM.attention_row(w4.round_bf16(q), keys, vals, D ** -0.5)
            ref[t, h] = OM.sigmoid_gate(o, raw[t, goff + h * qs:goff + h * qs + D]) if gated else o
    assert w4.rel_err(got, ref) <= 2e-2
    assert np.max(np.abs(got - ref)) <= 2e-2


def _ancestors(parents, t):
    out = {t}
    while parents[t] >= 0:
        t = parents[t]
        out.add(t)
    return out


def test_general_attention_bitwise_m_invariant(dev):
    """A token's output (and its cache rows) is the same whether it shares the step or not."""
    rng = np.random.default_rng(11)
    Hq, Hkv, D, rd, maxlen, L, M = 4, 2, 256, 64, 1024, 300, 12
    qs, koff, voff, goff, width = _layout(Hq, Hkv, D, True)
    raw = _bf(w4.round_bf16(rng.standard_normal((M, width))), dev)
    qn = _bf(1 + 0.1 * rng.standard_normal(D), dev)
    kn = _bf(1 + 0.1 * rng.standard_normal(D), dev)
    kc = _bf(w4.round_bf16(rng.standard_normal((Hkv, maxlen, D))), dev)
    vt = _bf(w4.round_bf16(rng.standard_normal((Hkv, D, maxlen))), dev)
    table = K.rope_table_dim(1e7, rd, maxlen, dev)
    ws = K.attn_general_workspace(Hq, Hkv, D, maxlen, dev)
    k1, v1 = kc.clone(), vt.clone()
    full = K.attention_general(raw, Hq, Hkv, D, qs, koff, voff, goff, qn, kn, 1e-6, rd, table,
                               torch.tensor([L], dtype=torch.int32, device=dev), k1, v1, D ** -0.5, ws)
    k2, v2 = kc.clone(), vt.clone()
    for t in range(M):
        one = K.attention_general(raw[t:t + 1], Hq, Hkv, D, qs, koff, voff, goff, qn, kn, 1e-6, rd, table,
                                  torch.tensor([L + t], dtype=torch.int32, device=dev), k2, v2, D ** -0.5, ws)
        assert torch.equal(one, full[t:t + 1]), t
    assert torch.equal(k1, k2) and torch.equal(v1, v2)


def test_rope_table_dim_matches_oracle(dev):
    """cos/sin of pos * theta^(-2i/R) for a RoPE over R = 64 dims (and R = 128 equals the 128-dim
    kernels' table bit for bit)."""
    table = K.rope_table_dim(1e7, 64, 4096, dev).cpu().double().numpy()
    i = np.arange(32)
    for p in (0, 1, 17, 299, 4095):
        ang = p * 1e7 ** (-2.0 * i / 64)
        tol = 1e-6 + 2.4e-7 * p
        assert np.max(np.abs(table[p, :, 0] - np.cos(ang))) <= tol, p
        assert np.max(np.abs(table[p, :, 1] - np.sin(ang))) <= tol, p
    assert torch.equal(K.rope_table_dim(1e6, 128, 512, dev).reshape(512, -1),
                       K.rope_table(1e6, 512, dev).reshape(512, -1))


@pytest.mark.parametrize("T,record", [(1, False), (5, True), (16, True)])
def test_gdn_shared_key_heads_match_oracle(dev, T, record):
    """The recurrence with 2 key heads over 4 value heads (value head h reads key head h // 2, as
    transformers' qwen3_5 repeat_interleave does) against the oracle."""
    rng = np.random.default_rng(20 + T)
    Hk, H = 2, 4
    qk = w4.round_bf16(rng.standard_normal((T, 2 * Hk * 128)))
    v = w4.round_bf16(rng.standard_normal((T, H * 128)))
    qkv = np.concatenate([qk, v], axis=1)
    ab = w4.round_bf16(rng.standard_normal((T, 2 * H)))
    A_log = np.log(rng.uniform(1, 16, H))
    dt = rng.uniform(-1, 1, H)
    S0 = rng.standard_normal((H, 128, 128)) * 0.1
    state = torch.tensor(S0, dtype=torch.float32, device=dev)
    states = torch.zeros((T, H, 128, 128), dtype=torch.float32, device=dev) if record else None
    abd = _bf(ab, dev)
    y = K.gdn_recurrence(_bf(qkv, dev), abd[:, :H], abd[:, H:], torch.tensor(A_log, dtype=torch.float32, device=dev),
                         torch.tensor(dt, dtype=torch.float32, device=dev), state, states, H, 128, 128,
                         n_key_heads=Hk)
    q = np.repeat(qk[:, :Hk * 128].reshape(T, Hk, 128), H // Hk, axis=1)
    k = np.repeat(qk[:, Hk * 128:].reshape(T, Hk, 128), H // Hk, axis=1)
    y_ref, st_ref = G.recurrence(q, k, v.reshape(T, H, 128), ab[:, H:], ab[:, :H], A_log.astype(np.float32),
                                 dt.astype(np.float32), S0.astype(np.float32).astype(np.float64))
    assert w4.rel_err(y.cpu().numpy(), y_ref) <= 1e-4
    assert w4.rel_err(state.cpu().numpy(), st_ref[-1]) <= 1e-4
    if record:
        assert w4.rel_err(states.cpu().numpy(), st_ref) <= 1e-4


def test_gdn_shared_key_heads_one_token_gated_form_is_bitwise(dev):
    """The one-token recurrence with the output norm in its launch equals the recurrence followed
    by the gated norm, bit for bit, with 2 key heads over 4 value heads."""
    rng = np.random.default_rng(30)
    Hk, H = 2, 4
    qkv = _bf(w4.round_bf16(rng.standard_normal((1, 2 * Hk * 128 + H * 128))), dev)
    ab = _bf(w4.round_bf16(rng.standard_normal((1, 2 * H))), dev)
    z = _bf(w4.round_bf16(rng.standard_normal((1, H * 128))), dev)
    nw = _bf(1 + 0.1 * rng.standard_normal(128), dev)
    A_log = torch.tensor(np.log(rng.uniform(1, 16, H)), dtype=torch.float32, device=dev)
    dt = torch.tensor(rng.uniform(-1, 1, H), dtype=torch.float32, device=dev)
    S0 = torch.tensor(rng.standard_normal((H, 128, 128)) * 0.1, dtype=torch.float32, device=dev)
    s1, s2 = S0.clone(), S0.clone()
    y = K.gdn_recurrence(qkv, ab[:, :H], ab[:, H:], A_log, dt, s1, None, H, 128, 128, n_key_heads=Hk)
    ref = K.gated_rmsnorm(y, z, nw, 1e-6)
    got = K.gdn_recurrence_gated(qkv, ab[:, :H], ab[:, H:], A_log, dt, s2, z, nw, 1e-6, H, 128, 128, n_key_heads=Hk)
    assert torch.equal(got, ref) and torch.equal(s1, s2)


def test_qwen35_widths_speculative_equals_greedy():
    """Four layers at Qwen3.5-4B's widths (three Gated-DeltaNet layers of 16 key / 32 value heads,
    one gated attention layer of 16 query / 4 kv heads of dim 256, hidden 2560, MLP 9216, a
    248320-row head), so every projection runs its own full-size tile: speculative decoding with a
    drafter that proposes the greedy continuation with one wrong token at a rotating position
    (5-token verify steps, every acceptance length, every rollback) gives plain greedy's tokens."""
    from skinny_mlx import patch as P
    from skinny_mlx.model import ModelArgs, build_model
    from skinny_mlx.spec import greedy, speculative

    args = ModelArgs(hidden_size=2560, num_hidden_layers=4, num_attention_heads=16, num_key_value_heads=4,
                     head_dim=256, intermediate_size=9216, vocab_size=248320, rope_theta=1e7,
                     full_attention_interval=4, linear_num_heads=32, linear_num_key_heads=16,
                     partial_rotary_factor=0.25, attn_output_gate=True, max_position=512)
    model = build_model(args)
    P.patch_model(model)
    prompt = torch.randint(0, args.vocab_size, (64,), generator=torch.Generator().manual_seed(5)).tolist()
    N, K = 48, 4
    ref = greedy(model, prompt, N + K + 1)

    class Replay:
        def begin(self, prompt_, h, first):
            self.pos, self.step = 1, 0

        def draft(self, k):
            d = list(ref[self.pos:self.pos + k])
            self.step += 1
            j = self.step % (k + 1)
            if j < len(d):
                d[j] = (d[j] + 1) % args.vocab_size
            return d

        def update(self, h_kept, new_tokens):
            self.pos += len(new_tokens)

    st = {}
    got = speculative(model, prompt, N, Replay(), K, st)
    assert got == ref[:N]
    assert st["tokens_per_step"] > 2.0
    del model
    torch.cuda.empty_cache()
