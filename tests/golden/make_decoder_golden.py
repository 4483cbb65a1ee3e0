"""Writes golden vectors for the oracle decoder's composition from an independent implementation,
transformers 5.x (third-party text installed in this container; not the reference, which is never
imported):

  qwen3_dense_transformers.npz      a 2-layer dense decoder in the Qwen3 layout (pre-norm blocks,
                                    per-head q/k RMSNorm, rotate-half RoPE, GQA, SwiGLU, final
                                    norm, untied head): transformers' Qwen3ForCausalLM in float64
  qwen3_5_gdn_layer_transformers.npz one Gated-DeltaNet mixer (in_proj_qkv/z/b/a, causal conv 4 +
                                    SiLU, gated delta rule, gated RMSNorm, out_proj):
                                    transformers' Qwen3_5GatedDeltaNet in float64
  qwen3_5_hybrid_transformers.npz   a 4-layer Qwen3.5-architecture decoder: attention output gate,
                                    partial RoPE over a 256-dim head, GDN key heads shared by two
                                    value heads: transformers' Qwen3_5ForCausalLM in float64

The weights are seeded W4 g64 packs in MLX's format (packs, bf16 scales and biases), bf16 norms
and embeddings, fp32 gates; transformers gets their exact dequantised values. Each file holds
those inputs, the token ids or input rows, and transformers' outputs (data only, no code).

Run from the repo root: python tests/golden/make_decoder_golden.py [dense] [gdn] [qwen3_5]
"""

import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import w4  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def _bf16_bits(x: np.ndarray) -> np.ndarray:
    return w4.f32_to_bf16(np.asarray(x, np.float32))


def _w4(rng, n: int, k: int):
    """Packs [N, K/8] uint32, scales and biases [N, K/64] bf16 bits: codes uniform, scales
    |N(0, s)| with s giving weights of std ~1/sqrt(K), biases -8 s plus a small offset."""
    q = rng.integers(0, 16, size=(n, k), dtype=np.uint8)
    std = 1.0 / (3.7 * np.sqrt(k))
    s = np.abs(rng.standard_normal((n, k // 64))) * std
    b = -8.0 * s + rng.standard_normal((n, k // 64)) * std * 0.5
    return w4.pack_mlx(q), _bf16_bits(s), _bf16_bits(b)


def _add_linear(params, name, rng, n, k):
    params[name + ".weight"], params[name + ".scales"], params[name + ".biases"] = _w4(rng, n, k)


def _deq(params, name) -> torch.Tensor:
    return torch.from_numpy(w4.dequant(params[name + ".weight"], params[name + ".scales"], params[name + ".biases"]))


def _f(bits) -> torch.Tensor:
    return torch.from_numpy(w4.bf16_to_f32(bits).astype(np.float64))


def dense_golden():
    from transformers import Qwen3Config, Qwen3ForCausalLM

    rng = np.random.default_rng(0)
    cfg = dict(hidden_size=128, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2, head_dim=32,
               intermediate_size=256, vocab_size=96, rms_norm_eps=1e-6, rope_theta=1e6)
    H, L, Hq, Hkv, D, F, V = (cfg[k] for k in ("hidden_size", "num_hidden_layers", "num_attention_heads",
                                               "num_key_value_heads", "head_dim", "intermediate_size", "vocab_size"))
    p = {"embed_tokens": _bf16_bits(rng.standard_normal((V, H)))}
    for i in range(L):
        pre = f"layers.{i}."
        p[pre + "input_layernorm"] = _bf16_bits(1 + 0.1 * rng.standard_normal(H))
        p[pre + "post_attention_layernorm"] = _bf16_bits(1 + 0.1 * rng.standard_normal(H))
        p[pre + "self_attn.q_norm"] = _bf16_bits(1 + 0.1 * rng.standard_normal(D))
        p[pre + "self_attn.k_norm"] = _bf16_bits(1 + 0.1 * rng.standard_normal(D))
        for name, n, k in (("q_proj", Hq * D, H), ("k_proj", Hkv * D, H), ("v_proj", Hkv * D, H),
                           ("o_proj", H, Hq * D)):
            _add_linear(p, pre + "self_attn." + name, rng, n, k)
        for name, n, k in (("gate_proj", F, H), ("up_proj", F, H), ("down_proj", H, F)):
            _add_linear(p, pre + "mlp." + name, rng, n, k)
    p["norm"] = _bf16_bits(1 + 0.1 * rng.standard_normal(H))
    _add_linear(p, "lm_head", rng, V, H)

    hf_cfg = Qwen3Config(hidden_size=H, num_hidden_layers=L, num_attention_heads=Hq, num_key_value_heads=Hkv,
                         head_dim=D, intermediate_size=F, vocab_size=V, rms_norm_eps=cfg["rms_norm_eps"],
                         rope_parameters={"rope_type": "default", "rope_theta": cfg["rope_theta"]},
                         max_position_embeddings=64, tie_word_embeddings=False, attention_bias=False,
                         attn_implementation="eager")
    model = Qwen3ForCausalLM(hf_cfg).to(torch.float64).eval()
    sd = {"model.embed_tokens.weight": _f(p["embed_tokens"]), "model.norm.weight": _f(p["norm"]),
          "lm_head.weight": _deq(p, "lm_head")}
    for i in range(L):
        pre, hp = f"layers.{i}.", f"model.layers.{i}."
        sd[hp + "input_layernorm.weight"] = _f(p[pre + "input_layernorm"])
        sd[hp + "post_attention_layernorm.weight"] = _f(p[pre + "post_attention_layernorm"])
        sd[hp + "self_attn.q_norm.weight"] = _f(p[pre + "self_attn.q_norm"])
        sd[hp + "self_attn.k_norm.weight"] = _f(p[pre + "self_attn.k_norm"])
        for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
            sd[hp + f"self_attn.{name}.weight"] = _deq(p, pre + "self_attn." + name)
        for name in ("gate_proj", "up_proj", "down_proj"):
            sd[hp + f"mlp.{name}.weight"] = _deq(p, pre + "mlp." + name)
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected and all("rotary" in m for m in missing), (missing, unexpected)
    tokens = rng.integers(0, V, size=12)
    with torch.no_grad():
        ids = torch.tensor(tokens[None], dtype=torch.long)
        hidden = model.model(ids).last_hidden_state[0].numpy()
        logits = model(ids).logits[0].numpy()
    out = {f"p:{k}": v for k, v in p.items()}
    out.update({f"c:{k}": np.float64(v) for k, v in cfg.items()}, tokens=tokens, hidden=hidden, logits=logits)
    path = os.path.join(HERE, "qwen3_dense_transformers.npz")
    np.savez_compressed(path, **out)
    print("wrote", path)


def gdn_layer_golden():
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5GatedDeltaNet

    rng = np.random.default_rng(1)
    H, nh, dk, dv, kw, T, eps = 128, 2, 32, 32, 4, 7, 1e-6
    conv_dim = 2 * nh * dk + nh * dv
    pre = "layers.0.linear_attn."
    p = {}
    for name, n in (("in_proj_qkv", conv_dim), ("in_proj_z", nh * dv), ("in_proj_b", nh), ("in_proj_a", nh)):
        _add_linear(p, pre + name, rng, n, H)
    _add_linear(p, pre + "out_proj", rng, H, nh * dv)
    p[pre + "conv1d_weight"] = _bf16_bits((rng.random((conv_dim, kw)) - 0.5) * (2.0 / np.sqrt(kw)))
    p[pre + "A_log"] = np.log(rng.random(nh) * 15.0 + 1.0).astype(np.float32).astype(np.float64)
    p[pre + "dt_bias"] = (rng.random(nh) * 2.0 - 1.0).astype(np.float32).astype(np.float64)
    p[pre + "norm_weight"] = _bf16_bits(1 + 0.1 * rng.standard_normal(dv))
    x = w4.round_bf16(rng.standard_normal((T, H))).astype(np.float64)

    hf_cfg = Qwen3_5TextConfig(hidden_size=H, num_hidden_layers=1, layer_types=["linear_attention"],
                               linear_num_key_heads=nh, linear_num_value_heads=nh, linear_key_head_dim=dk,
                               linear_value_head_dim=dv, linear_conv_kernel_dim=kw, rms_norm_eps=eps,
                               hidden_act="silu")
    layer = Qwen3_5GatedDeltaNet(hf_cfg, layer_idx=0).to(torch.float64).eval()
    sd = {f"{n}.weight": _deq(p, pre + n) for n in ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a",
                                                       "out_proj")}
    sd["conv1d.weight"] = _f(p[pre + "conv1d_weight"])[:, None, :]
    sd["A_log"] = torch.from_numpy(p[pre + "A_log"])
    sd["dt_bias"] = torch.from_numpy(p[pre + "dt_bias"])
    sd["norm.weight"] = _f(p[pre + "norm_weight"])
    layer.load_state_dict(sd, strict=True)
    with torch.no_grad():
        y = layer(torch.from_numpy(x)[None])[0].numpy()
    cfg = dict(hidden_size=H, linear_num_heads=nh, linear_key_head_dim=dk, linear_value_head_dim=dv,
               linear_conv_kernel_dim=kw, rms_norm_eps=eps)
    out = {f"p:{k}": v for k, v in p.items()}
    out.update({f"c:{k}": np.float64(v) for k, v in cfg.items()}, x=x, y=y)
    path = os.path.join(HERE, "qwen3_5_gdn_layer_transformers.npz")
    np.savez_compressed(path, **out)
    print("wrote", path)


def qwen3_5_golden():
    """A 4-layer Qwen3.5-architecture decoder (three Gated-DeltaNet layers, then full attention)
    with the features the dense and GDN-layer files do not cover: the attention output gate (q_proj
    rows per head: query then gate), partial RoPE (a quarter of a 256-dim head), and GDN layers with
    2 key heads shared by 4 value heads. transformers' Qwen3_5ForCausalLM in float64; its RMSNorms
    multiply by (1 + w), so it gets w - 1 for the oracle's gammas w (the GDN output norm multiplies by
    w itself)."""
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5ForCausalLM

    rng = np.random.default_rng(2)
    cfg = dict(hidden_size=128, num_hidden_layers=4, num_attention_heads=2, num_key_value_heads=1, head_dim=256,
               intermediate_size=256, vocab_size=128, rms_norm_eps=1e-6, rope_theta=1e7, full_attention_interval=4,
               partial_rotary_factor=0.25, attn_output_gate=1, linear_num_heads=4, linear_num_key_heads=2,
               linear_key_head_dim=64, linear_value_head_dim=64, linear_conv_kernel_dim=4)
    H, L, Hq, Hkv, D, F, V = (cfg[k] for k in ("hidden_size", "num_hidden_layers", "num_attention_heads",
                                               "num_key_value_heads", "head_dim", "intermediate_size", "vocab_size"))
    nv, nk, dk, dv, kw = (cfg[k] for k in ("linear_num_heads", "linear_num_key_heads", "linear_key_head_dim",
                                           "linear_value_head_dim", "linear_conv_kernel_dim"))
    conv_dim = 2 * nk * dk + nv * dv
    layer_types = ["linear_attention"] * 3 + ["full_attention"]
    p = {"embed_tokens": _bf16_bits(rng.standard_normal((V, H)))}
    for i in range(L):
        pre = f"layers.{i}."
        p[pre + "input_layernorm"] = _bf16_bits(1 + 0.1 * rng.standard_normal(H))
        p[pre + "post_attention_layernorm"] = _bf16_bits(1 + 0.1 * rng.standard_normal(H))
        if layer_types[i] == "full_attention":
            a = pre + "self_attn."
            p[a + "q_norm"] = _bf16_bits(1 + 0.1 * rng.standard_normal(D))
            p[a + "k_norm"] = _bf16_bits(1 + 0.1 * rng.standard_normal(D))
            for name, n, k in (("q_proj", 2 * Hq * D, H), ("k_proj", Hkv * D, H), ("v_proj", Hkv * D, H),
                               ("o_proj", H, Hq * D)):
                _add_linear(p, a + name, rng, n, k)
        else:
            g = pre + "linear_attn."
            for name, n in (("in_proj_qkv", conv_dim), ("in_proj_z", nv * dv), ("in_proj_b", nv), ("in_proj_a", nv)):
                _add_linear(p, g + name, rng, n, H)
            _add_linear(p, g + "out_proj", rng, H, nv * dv)
            p[g + "conv1d_weight"] = _bf16_bits((rng.random((conv_dim, kw)) - 0.5) * (2.0 / np.sqrt(kw)))
            p[g + "A_log"] = np.log(rng.random(nv) * 15.0 + 1.0).astype(np.float32).astype(np.float64)
            p[g + "dt_bias"] = (rng.random(nv) * 2.0 - 1.0).astype(np.float32).astype(np.float64)
            p[g + "norm_weight"] = _bf16_bits(1 + 0.1 * rng.standard_normal(dv))
        for name, n, k in (("gate_proj", F, H), ("up_proj", F, H), ("down_proj", H, F)):
            _add_linear(p, pre + "mlp." + name, rng, n, k)
    p["norm"] = _bf16_bits(1 + 0.1 * rng.standard_normal(H))
    _add_linear(p, "lm_head", rng, V, H)

    hf_cfg = Qwen3_5TextConfig(hidden_size=H, num_hidden_layers=L, num_attention_heads=Hq, num_key_value_heads=Hkv,
                               head_dim=D, intermediate_size=F, vocab_size=V, rms_norm_eps=cfg["rms_norm_eps"],
                               rope_parameters={"rope_type": "default", "rope_theta": cfg["rope_theta"],
                                                "partial_rotary_factor": cfg["partial_rotary_factor"]},
                               layer_types=layer_types, linear_num_key_heads=nk, linear_num_value_heads=nv,
                               linear_key_head_dim=dk, linear_value_head_dim=dv, linear_conv_kernel_dim=kw,
                               max_position_embeddings=64, tie_word_embeddings=False, attention_bias=False,
                               hidden_act="silu", attn_implementation="eager")
    model = Qwen3_5ForCausalLM(hf_cfg).to(torch.float64).eval()
    one = lambda bits: _f(bits) - 1.0  # noqa: E731  (zero-centred RMSNorm gammas)
    sd = {"model.embed_tokens.weight": _f(p["embed_tokens"]), "model.norm.weight": one(p["norm"]),
          "lm_head.weight": _deq(p, "lm_head")}
    for i in range(L):
        pre, hp = f"layers.{i}.", f"model.layers.{i}."
        sd[hp + "input_layernorm.weight"] = one(p[pre + "input_layernorm"])
        sd[hp + "post_attention_layernorm.weight"] = one(p[pre + "post_attention_layernorm"])
        if layer_types[i] == "full_attention":
            sd[hp + "self_attn.q_norm.weight"] = one(p[pre + "self_attn.q_norm"])
            sd[hp + "self_attn.k_norm.weight"] = one(p[pre + "self_attn.k_norm"])
            for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
                sd[hp + f"self_attn.{name}.weight"] = _deq(p, pre + "self_attn." + name)
        else:
            g, hg = pre + "linear_attn.", hp + "linear_attn."
            for name in ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a", "out_proj"):
                sd[hg + f"{name}.weight"] = _deq(p, g + name)
            sd[hg + "conv1d.weight"] = _f(p[g + "conv1d_weight"])[:, None, :]
            sd[hg + "A_log"] = torch.from_numpy(p[g + "A_log"])
            sd[hg + "dt_bias"] = torch.from_numpy(p[g + "dt_bias"])
            sd[hg + "norm.weight"] = _f(p[g + "norm_weight"])
        for name in ("gate_proj", "up_proj", "down_proj"):
            sd[hp + f"mlp.{name}.weight"] = _deq(p, pre + "mlp." + name)
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected and all("rotary" in m for m in missing), (missing, unexpected)
    tokens = rng.integers(0, V, size=10)
    with torch.no_grad():
        ids = torch.tensor(tokens[None], dtype=torch.long)
        hidden = model.model(ids).last_hidden_state[0].numpy()
        logits = model(ids).logits[0].numpy()
    out = {f"p:{k}": v for k, v in p.items()}
    out.update({f"c:{k}": np.float64(v) for k, v in cfg.items()}, tokens=tokens, hidden=hidden, logits=logits)
    path = os.path.join(HERE, "qwen3_5_hybrid_transformers.npz")
    np.savez_compressed(path, **out)
    print("wrote", path)


if __name__ == "__main__":
    which = sys.argv[1:] or ["dense", "gdn", "qwen3_5"]
    if "dense" in which:
        dense_golden()
    if "gdn" in which:
        gdn_layer_golden()
    if "qwen3_5" in which:
        qwen3_5_golden()
