"""Pins the decoder oracle's building blocks (oracle/model.py) by closed forms, so that a wrong
sign, index or dropped term in the restatement fails here rather than agreeing with the device."""

import numpy as np

from oracle import model as OM
from oracle import w4


def _ones_bits(n):
    return w4.f32_to_bf16(np.ones(n, np.float32))


def test_rmsnorm_closed_forms():
    # a constant row normalises to +-1 (up to eps), for any magnitude
    for c in (0.25, -3.0, 40.0):
        y = OM.rmsnorm(np.full(64, c), _ones_bits(64), 0.0)
        assert np.allclose(y, np.sign(c), atol=2 ** -8)
    # scale invariance, and the weight multiplies element-wise
    rng = np.random.default_rng(0)
    x = rng.standard_normal(128)
    w = w4.f32_to_bf16(rng.uniform(0.5, 2.0, 128).astype(np.float32))
    assert np.allclose(OM.rmsnorm(7.0 * x, w, 0.0), OM.rmsnorm(x, w, 0.0), rtol=2 ** -7, atol=1e-6)
    ref = x / np.sqrt((x * x).mean()) * w4.bf16_to_f32(w)
    assert np.allclose(OM.rmsnorm(x, w, 0.0), ref, rtol=2 ** -7, atol=1e-6)


def test_rope_closed_forms():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(128)
    assert np.allclose(OM.rope(x, 0, 1e6), x)  # position 0 is the identity
    y = OM.rope(x, 37, 1e6)
    half = 64
    # each (i, i + D/2) pair is rotated: its norm is preserved
    assert np.allclose(x[:half] ** 2 + x[half:] ** 2, y[:half] ** 2 + y[half:] ** 2)
    # rotations compose: rope(rope(x, p), q) == rope(x, p + q)
    assert np.allclose(OM.rope(OM.rope(x, 11, 1e4), 26, 1e4), OM.rope(x, 37, 1e4))
    # D = 2: inverse frequency 1, the pair (a, b) turns by `pos` radians counter-clockwise
    a, b, p = 0.3, -1.2, 2
    assert np.allclose(OM.rope(np.array([a, b]), p, 1e6),
                       [a * np.cos(p) - b * np.sin(p), b * np.cos(p) + a * np.sin(p)])
    # frequency of pair i is theta^(-2i/D): pair 1 of D = 4 at theta 100 turns by pos / 10
    z = OM.rope(np.array([0.0, 1.0, 0.0, 0.0]), 5, 100.0)
    assert np.allclose(z, [0.0, np.cos(0.5), 0.0, np.sin(0.5)])


def test_attention_row_closed_forms():
    rng = np.random.default_rng(2)
    q = rng.standard_normal(16)
    keys = rng.standard_normal((1, 16))
    vals = rng.standard_normal((1, 16))
    assert np.allclose(OM.attention_row(q, keys, vals, 0.25), vals[0])  # one key: its value
    keys = np.zeros((5, 16))
    vals = rng.standard_normal((5, 16))
    assert np.allclose(OM.attention_row(q, keys, vals, 0.25), vals.mean(0))  # equal scores: the mean
    keys = np.zeros((3, 16))
    keys[1] = q * 100.0  # one dominant score selects its value
    assert np.allclose(OM.attention_row(q, keys, vals[:3], 1.0), vals[1])


# --- the composition, against an independent implementation and identity constructions ---------

import os  # noqa: E402

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _golden(name):
    z = np.load(os.path.join(GOLDEN, name))
    params = {k[2:]: z[k] for k in z.files if k.startswith("p:")}
    cfg = {k[2:]: z[k].item() for k in z.files if k.startswith("c:")}
    return z, params, cfg


def test_dense_decoder_matches_transformers_qwen3():
    """The whole dense decoder (block order, residuals, q/k-norm before RoPE, GQA head mapping,
    SwiGLU, final norm, head) against transformers' Qwen3ForCausalLM on the same W4 weights
    (tests/golden/qwen3_dense_transformers.npz). transformers runs its norms and RoPE tables in
    fp32, so agreement is to ~1e-6 relative; a wrong composition is off by O(1)."""
    z, p, c = _golden("qwen3_dense_transformers.npz")
    cfg = dict(c, full_attention_interval=0, num_hidden_layers=int(c["num_hidden_layers"]),
               num_attention_heads=int(c["num_attention_heads"]), num_key_value_heads=int(c["num_key_value_heads"]),
               head_dim=int(c["head_dim"]))
    hid, logits = OM.Decoder(p, cfg, exact=True).forward(z["tokens"])
    assert w4.rel_err(logits, z["logits"]) < 1e-5
    assert w4.rel_err(hid, z["hidden"]) < 1e-5
    # the bf16 form (what the device is held to) stays within the path's bar of the same reference
    _, lb = OM.Decoder(p, cfg).forward(z["tokens"])
    assert w4.rel_err(lb, z["logits"]) < 2e-2


def _qwen3_5_cfg(c):
    ints = ("num_hidden_layers", "num_attention_heads", "num_key_value_heads", "head_dim", "full_attention_interval",
            "linear_num_heads", "linear_num_key_heads", "linear_key_head_dim", "linear_value_head_dim",
            "linear_conv_kernel_dim")
    return dict(c, **{k: int(c[k]) for k in ints}, attn_output_gate=bool(c["attn_output_gate"]))


def test_qwen3_5_decoder_matches_transformers():
    """The Qwen3.5 architecture the reference runs (spec.py:175 loads Qwen3.5-4B): the attention
    output gate from the second half of each head's q_proj rows, RoPE over a quarter of a 256-dim
    head, and Gated-DeltaNet layers whose 2 key heads serve 4 value heads, in a 3:1 hybrid stack,
    against transformers' Qwen3_5ForCausalLM on the same W4 weights
    (tests/golden/qwen3_5_hybrid_transformers.npz), to 1e-5 relative in fp64. The bf16 form is not
    held to this reference: in this small random decoder bf16 rounding alone moves single logits
    by up to ~15% (the device is held to the bf16 oracle, rounded at its own points)."""
    z, p, c = _golden("qwen3_5_hybrid_transformers.npz")
    cfg = _qwen3_5_cfg(c)
    assert OM.rotary_dim(cfg) == 64 and cfg["attn_output_gate"] and cfg["linear_num_key_heads"] == 2
    hid, logits = OM.Decoder(p, cfg, exact=True).forward(z["tokens"])
    assert w4.rel_err(logits, z["logits"]) < 1e-5
    assert w4.rel_err(hid, z["hidden"]) < 1e-5
    # the features are exercised at this size: RoPE over the whole head, or the gate rows read as
    # queries of an ungated layer of the same width, miss the reference by far
    _, lfull = OM.Decoder(p, dict(cfg, partial_rotary_factor=1.0), exact=True).forward(z["tokens"])
    assert w4.rel_err(lfull, z["logits"]) > 1e-3
    ungated = dict(p)
    for k in ("weight", "scales", "biases"):  # query rows only: heads of [query; gate] rows
        w = p[f"layers.3.self_attn.q_proj.{k}"]
        ungated[f"layers.3.self_attn.q_proj.{k}"] = w.reshape(2, 2, -1, w.shape[-1])[:, 0].reshape(-1, w.shape[-1])
    _, lung = OM.Decoder(ungated, dict(cfg, attn_output_gate=False), exact=True).forward(z["tokens"])
    assert w4.rel_err(lung, z["logits"]) > 1e-3


def test_partial_rope_and_gate_closed_forms():
    """Partial RoPE turns the first R dims exactly as a full RoPE of an R-dim head and leaves the
    rest; the gate multiplies by sigmoid: gate 0 halves the output, a large gate keeps it, a very
    negative one zeroes it."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal(256)
    y = OM.rope(x, 19, 1e7, 64)
    assert np.array_equal(y[64:], x[64:])
    assert np.allclose(y[:64], OM.rope(x[:64], 19, 1e7))
    assert np.allclose(OM.rope(x, 19, 1e7, 256), OM.rope(x, 19, 1e7))
    assert np.allclose(OM.rope(x, 0, 1e7, 64), x)
    o = w4.round_bf16(rng.standard_normal(64)).astype(np.float64)
    assert np.array_equal(OM.sigmoid_gate(o, np.zeros(64)), w4.round_bf16(o * 0.5))
    assert np.array_equal(OM.sigmoid_gate(o, np.full(64, 40.0)), o)
    assert np.array_equal(OM.sigmoid_gate(o, np.full(64, -200.0)), np.zeros(64) * o)


def test_gdn_mixer_matches_transformers_qwen3_5():
    """One Gated-DeltaNet mixer (projection split q|k|v, conv taps and state, gates, delta rule,
    gated RMSNorm, out_proj) against transformers' Qwen3_5GatedDeltaNet over 7 tokens from zero
    state (tests/golden/qwen3_5_gdn_layer_transformers.npz; its recurrence runs in fp32)."""
    z, p, c = _golden("qwen3_5_gdn_layer_transformers.npz")
    cfg = dict(c, num_hidden_layers=1, full_attention_interval=2, linear_num_heads=int(c["linear_num_heads"]),
               linear_key_head_dim=int(c["linear_key_head_dim"]), linear_value_head_dim=int(c["linear_value_head_dim"]),
               linear_conv_kernel_dim=int(c["linear_conv_kernel_dim"]))
    dec = OM.Decoder(p, cfg, exact=True)
    assert dec.is_linear(0)
    got = np.stack([dec.gdn_layer(0, row) for row in z["x"]])
    assert w4.rel_err(got, z["y"]) < 1e-5


def test_hybrid_layer_pattern_matches_qwen3_5_layer_types():
    """Which layers are Gated-DeltaNet: transformers' Qwen3.5 config builds layer_types from
    full_attention_interval as 'linear_attention' iff (i + 1) % interval != 0."""
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig

    for layers, interval in ((36, 4), (8, 2), (6, 3)):
        hf = Qwen3_5TextConfig(num_hidden_layers=layers, full_attention_interval=interval).layer_types
        dec = OM.Decoder.__new__(OM.Decoder)
        dec.c = {"full_attention_interval": interval}
        assert [dec.is_linear(i) for i in range(layers)] == [t == "linear_attention" for t in hf]


def _zero_w4(n, k):
    """W4 g64 weight that dequantises to exactly 0 (q = 8, b = -8 s)."""
    s = w4.f32_to_bf16(np.full((n, k // 64), 0.125, np.float32))
    return w4.pack_mlx(np.full((n, k), 8, np.uint8)), s, w4.f32_to_bf16(np.full((n, k // 64), -1.0, np.float32))


def _identity_w4(n, k, col0=0):
    """W4 g64 weight [n, k] that dequantises to exactly [0 | I | 0] with I at columns col0..col0+n
    (s = 1, b = -8, q = 9 on that diagonal and 8 elsewhere)."""
    q = np.full((n, k), 8, np.uint8)
    q[np.arange(n), col0 + np.arange(n)] = 9
    return (w4.pack_mlx(q), w4.f32_to_bf16(np.ones((n, k // 64), np.float32)),
            w4.f32_to_bf16(np.full((n, k // 64), -8.0, np.float32)))


def test_hybrid_stack_with_identity_mixers_reduces_to_its_attention_layers():
    """Zeroed out_proj and down_proj make every Gated-DeltaNet layer the identity on the residual
    stream, so a 3:1 hybrid's logits must equal the dense decoder made of its attention layers alone
    (layers 3 and 7 as 0 and 1), whose composition the Qwen3 golden pins. A GDN layer that touched
    the stream, or attention layers that read the wrong cache or layer index, would fail."""
    z, p, c = _golden("qwen3_dense_transformers.npz")
    H, L = int(c["hidden_size"]), int(c["num_hidden_layers"])
    nh, dk, dv, kw = 2, 32, 32, 4
    conv_dim = 2 * nh * dk + nh * dv
    rng = np.random.default_rng(3)
    hyb = {k: v for k, v in p.items() if not k.startswith("layers.")}
    for j in range(2 * 4):
        src = f"layers.{j // 4}." if (j + 1) % 4 == 0 else None
        pre = f"layers.{j}."
        if src is not None:
            hyb.update({pre + k[len(src):]: v for k, v in p.items() if k.startswith(src)})
            continue
        hyb[pre + "input_layernorm"] = p["layers.0.input_layernorm"]
        hyb[pre + "post_attention_layernorm"] = p["layers.1.post_attention_layernorm"]
        la = pre + "linear_attn."
        for name, n in (("in_proj_qkv", conv_dim), ("in_proj_z", nh * dv), ("in_proj_b", nh), ("in_proj_a", nh)):
            q = rng.integers(0, 16, size=(n, H), dtype=np.uint8)
            s = w4.f32_to_bf16(np.abs(rng.standard_normal((n, H // 64))).astype(np.float32) * 0.02)
            hyb[la + name + ".weight"], hyb[la + name + ".scales"], hyb[la + name + ".biases"] = (
                w4.pack_mlx(q), s, w4.f32_to_bf16(-8 * w4.bf16_to_f32(s)))
        hyb[la + "out_proj.weight"], hyb[la + "out_proj.scales"], hyb[la + "out_proj.biases"] = _zero_w4(H, nh * dv)
        hyb[la + "conv1d_weight"] = w4.f32_to_bf16(rng.standard_normal((conv_dim, kw)).astype(np.float32))
        hyb[la + "A_log"] = rng.random(nh)
        hyb[la + "dt_bias"] = rng.random(nh)
        hyb[la + "norm_weight"] = p["layers.0.self_attn.q_norm"]
        F = p["layers.0.mlp.gate_proj.scales"].shape[0]
        for name, n, k in (("gate_proj", F, H), ("up_proj", F, H)):
            hyb[pre + "mlp." + name + ".weight"] = p["layers.0.mlp." + name + ".weight"]
            hyb[pre + "mlp." + name + ".scales"] = p["layers.0.mlp." + name + ".scales"]
            hyb[pre + "mlp." + name + ".biases"] = p["layers.0.mlp." + name + ".biases"]
        hyb[pre + "mlp.down_proj.weight"], hyb[pre + "mlp.down_proj.scales"], hyb[pre + "mlp.down_proj.biases"] = (
            _zero_w4(H, F))
    base = dict(c, num_hidden_layers=L, num_attention_heads=int(c["num_attention_heads"]),
                num_key_value_heads=int(c["num_key_value_heads"]), head_dim=int(c["head_dim"]),
                linear_num_heads=nh, linear_key_head_dim=dk, linear_value_head_dim=dv, linear_conv_kernel_dim=kw)
    dense = OM.Decoder(p, dict(base, full_attention_interval=0), exact=True)
    hybrid = OM.Decoder(hyb, dict(base, num_hidden_layers=8, full_attention_interval=4), exact=True)
    toks = z["tokens"][:6]
    hd, ld = dense.forward(toks)
    hh, lh = hybrid.forward(toks)
    np.testing.assert_allclose(lh, ld, rtol=0, atol=1e-12 * np.abs(ld).max())
    np.testing.assert_allclose(hh, hd, rtol=0, atol=1e-12 * np.abs(hd).max())
    assert any(np.abs(s["S"]).max() > 0 for s in hybrid.gdn.values())  # the mixers did run


def test_mtp_head_composition_by_identity_fc():
    """The MTP head (reference mtp.py:51-67) with fc = [I | 0] is norm(layer(rmsnorm_e(emb))):
    exactly a one-layer decoder whose embedding row is rmsnorm_e(emb); with fc = [0 | I] it is the
    same with rmsnorm_h(hidden). This fixes the concat order [embedding; hidden], the per-half
    norms and the layer/final-norm placement against the Qwen3-pinned decoder."""
    z, p, c = _golden("qwen3_dense_transformers.npz")
    H = int(c["hidden_size"])
    cfg = dict(c, num_hidden_layers=1, full_attention_interval=0, num_attention_heads=int(c["num_attention_heads"]),
               num_key_value_heads=int(c["num_key_value_heads"]), head_dim=int(c["head_dim"]))
    layer = {("layer." + k[len("layers.0."):]): v for k, v in p.items() if k.startswith("layers.0.")}
    rng = np.random.default_rng(4)
    e_norm = w4.f32_to_bf16((1 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    h_norm = w4.f32_to_bf16((1 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    embs = w4.round_bf16(rng.standard_normal((5, H))).astype(np.float64)
    hids = w4.round_bf16(2 * rng.standard_normal((5, H))).astype(np.float64)
    for half, src, nw in ((0, embs, e_norm), (1, hids, h_norm)):
        head_p = dict(layer, pre_fc_norm_embedding=e_norm, pre_fc_norm_hidden=h_norm, norm=p["norm"])
        head_p["fc.weight"], head_p["fc.scales"], head_p["fc.biases"] = _identity_w4(H, 2 * H, col0=half * H)
        head = OM.MTPHead(head_p, cfg)
        got = np.stack([head.step(e, h) for e, h in zip(embs, hids)])
        rows = np.stack([w4.f32_to_bf16(OM.rmsnorm(r, nw, cfg["rms_norm_eps"]).astype(np.float32)) for r in src])
        dec_p = {k: v for k, v in p.items() if k.startswith("layers.0.")}
        dec_p.update(embed_tokens=rows, norm=p["norm"], **{f"lm_head.{k}": v for k, v in
                                                           zip(("weight", "scales", "biases"), _zero_w4(16, H))})
        dec = OM.Decoder(dec_p, cfg)
        ref = np.stack([dec.step(t)[0] for t in range(5)])
        np.testing.assert_array_equal(got, ref)
