"""The decoder forward restated in numpy (oracle; tests only).

What it restates: the verify forward of the decoder the reference runs (skinny_mlx/spec.py:
24-29 -> mlx_lm's model), for skinny_mlx's random-init dense and hybrid decoders — RMSNorm
pre-norm blocks, W4 g64 linears (oracle/w4.py), per-head q/k RMSNorm, rotate-half RoPE,
causal GQA attention with a KV cache, SwiGLU MLP, and Gated-DeltaNet mixers (oracle/gdn.py).
Values are rounded to bf16 at the same points as the device path (every op output that the
model keeps in bf16); everything else is fp64. Softmax is exact (the device rounds P to bf16
and merges 32-key blocks), so attention agrees within the bf16 tolerance, not bitwise.

Tokens are processed one at a time: every op is per token and causal, so this equals a
batched forward. `exact=True` drops every bf16 rounding point (fp64 throughout, linears as
x . dequant(w)^T in fp64): the form in which the composition is compared with an independent
implementation. Pins (tests/test_oracle_model.py): the parts (w4, gdn, accept), closed forms
(RoPE rotation, single-key attention, softmax of equal scores), the whole dense decoder against
transformers' Qwen3ForCausalLM and the Gated-DeltaNet mixer against transformers'
Qwen3_5GatedDeltaNet (golden vectors in tests/golden/, written by make_decoder_golden.py), the
hybrid layer pattern against transformers' Qwen3.5 layer_types, the Qwen3.5 architecture
(attention output gate, partial RoPE, head_dim 256, Gated-DeltaNet key heads shared by two value
heads) against transformers' Qwen3_5ForCausalLM, and identity constructions for the hybrid stack
and the MTP head (layers made the identity reduce them to pinned decoders).
"""

from __future__ import annotations

import numpy as np

from . import gdn as G
from . import w4

bf = w4.round_bf16


def _f(bits) -> np.ndarray:
    """bf16 bit patterns -> float64."""
    return w4.bf16_to_f32(np.asarray(bits, np.uint16)).astype(np.float64)


def _exact(x):
    return np.asarray(x, np.float64)


def rmsnorm(x, w_bits, eps, rnd=bf):
    x = np.asarray(x, np.float64)
    inv = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    return rnd(x * inv * _f(w_bits))


def rope(x, pos: int, theta: float, rotary_dim: int | None = None):
    """Rotate-half RoPE of one head vector x [D] at position pos (fp64 angles). With rotary_dim
    R < D only the first R dims turn, as pairs (i, i + R/2) at frequency theta^(-2i/R); the rest
    pass through (Qwen3.5's partial rotary factor, transformers qwen3_5 apply_rotary_pos_emb)."""
    D = x.shape[-1]
    R = D if rotary_dim is None else int(rotary_dim)
    half = R // 2
    inv_freq = theta ** (-2.0 * np.arange(half) / R)
    ang = pos * inv_freq
    c, s = np.cos(ang), np.sin(ang)
    a, b = x[:half], x[half:R]
    return np.concatenate([a * c - b * s, b * c + a * s, x[R:]])


def rotary_dim(cfg) -> int:
    """Dims of each head that RoPE turns: head_dim x partial_rotary_factor (1 when absent)."""
    return int(cfg["head_dim"] * float(cfg.get("partial_rotary_factor", 1.0)))


def sigmoid_gate(o, gate, rnd=bf):
    """Qwen3.5's attention output gate, o * sigmoid(gate), both operands and the product rounded
    at the device's points (transformers qwen3_5 Attention: attn_output * torch.sigmoid(gate))."""
    g = np.asarray(gate, np.float64)
    return rnd(rnd(o) * rnd(1.0 / (1.0 + np.exp(-g))))


def attention_row(q, keys, values, scale):
    """softmax(q . keys^T * scale) . values for one query over all visible keys (fp64)."""
    s = keys @ q * scale
    p = np.exp(s - s.max())
    return (p[:, None] * values).sum(0) / p.sum()


class Decoder:
    """params: name -> numpy array (bf16 as uint16 bits, packs as uint32, fp32 gates), as in
    skinny_mlx.model.Model.state_dict(); cfg: the ModelArgs fields as a dict."""

    def __init__(self, params: dict, cfg: dict, exact: bool = False):
        self.p, self.c = params, cfg
        self.exact = exact
        self.rnd = _exact if exact else bf
        self.reset()

    def norm(self, x, name):
        return rmsnorm(x, self.p[name], self.c["rms_norm_eps"], self.rnd)

    def gdn_heads(self):
        """(key heads, value heads) of the Gated-DeltaNet layers: linear_num_heads value heads, and
        linear_num_key_heads key heads (0 or absent: as many as value heads)."""
        nv = self.c["linear_num_heads"]
        return int(self.c.get("linear_num_key_heads", 0) or nv), nv

    def reset(self):
        c = self.c
        self.pos = 0
        self.kv = {}
        self.gdn = {}
        for i in range(c["num_hidden_layers"]):
            if self.is_linear(i):
                (nk, nh), dk, dv = self.gdn_heads(), c["linear_key_head_dim"], c["linear_value_head_dim"]
                conv_dim = 2 * nk * dk + nh * dv
                self.gdn[i] = {"conv": np.zeros((c["linear_conv_kernel_dim"] - 1, conv_dim)),
                               "S": np.zeros((nh, dv, dk))}
            else:
                self.kv[i] = ([], [])

    def is_linear(self, i):
        fai = self.c["full_attention_interval"]
        return fai > 0 and (i + 1) % fai != 0

    def linear(self, name, x):
        p = self.p
        if self.exact:
            return w4.dequant(p[name + ".weight"], p[name + ".scales"], p[name + ".biases"]) @ _exact(x)
        y = w4.qmm(w4.f32_to_bf16(np.atleast_2d(x).astype(np.float32)), p[name + ".weight"], p[name + ".scales"],
                   p[name + ".biases"])
        return bf(y)[0]

    def attn(self, i, x):
        """Full attention of layer i for one token. With attn_output_gate, q_proj holds per head
        the query rows then the gate rows (transformers qwen3_5 Attention: q_proj to 2 x heads x
        head_dim, viewed [heads, 2 D] and chunked), and the attention output is multiplied by
        sigmoid(gate) before o_proj."""
        c, p, rnd = self.c, self.p, self.rnd
        pre = f"layers.{i}.self_attn."
        Hq, Hkv, D = c["num_attention_heads"], c["num_key_value_heads"], c["head_dim"]
        gated = bool(c.get("attn_output_gate", False))
        qg = self.linear(pre + "q_proj", x).reshape(Hq, 2 * D if gated else D)
        q, gate = qg[:, :D], (qg[:, D:] if gated else None)
        k = self.linear(pre + "k_proj", x).reshape(Hkv, D)
        v = self.linear(pre + "v_proj", x).reshape(Hkv, D)
        th, rd = c["rope_theta"], rotary_dim(c)
        q = np.stack([rnd(rope(self.norm(q[h], pre + "q_norm"), self.pos, th, rd)) for h in range(Hq)])
        k = np.stack([rnd(rope(self.norm(k[h], pre + "k_norm"), self.pos, th, rd)) for h in range(Hkv)])
        ks, vs = self.kv[i]
        ks.append(k)
        vs.append(v)
        K_ = np.stack(ks)  # [L, Hkv, D]
        V_ = np.stack(vs)
        G_ = Hq // Hkv
        o = np.stack([attention_row(q[h], K_[:, h // G_], V_[:, h // G_], D ** -0.5) for h in range(Hq)])
        o = sigmoid_gate(o, gate, rnd) if gated else rnd(o)
        return self.linear(pre + "o_proj", o.reshape(-1))

    def gdn_layer(self, i, x):
        c, p, rnd = self.c, self.p, self.rnd
        pre = f"layers.{i}.linear_attn."
        (nk, nh), dk, dv = self.gdn_heads(), c["linear_key_head_dim"], c["linear_value_head_dim"]
        qkv = self.linear(pre + "in_proj_qkv", x)
        z = self.linear(pre + "in_proj_z", x)
        b = self.linear(pre + "in_proj_b", x)
        a = self.linear(pre + "in_proj_a", x)
        st = self.gdn[i]
        xc, st["conv"], _ = G.conv_silu(qkv[None], st["conv"], _f(p[pre + "conv1d_weight"]))
        xc = rnd(xc[0])
        # value head j reads key head j // (nh / nk) (transformers qwen3_5: q and k
        # repeat_interleave'd to the value heads)
        q = np.repeat(xc[:nk * dk].reshape(nk, dk), nh // nk, axis=0)
        k = np.repeat(xc[nk * dk:2 * nk * dk].reshape(nk, dk), nh // nk, axis=0)
        v = xc[2 * nk * dk:].reshape(nh, dv)
        y, S = G.recurrence(q[None], k[None], v[None], a[None], b[None], p[pre + "A_log"], p[pre + "dt_bias"],
                            st["S"])
        st["S"] = S[0]
        y = y[0]
        o = rnd(G.gated_rmsnorm(y, z.reshape(nh, dv), _f(p[pre + "norm_weight"]), c["rms_norm_eps"]))
        return self.linear(pre + "out_proj", o.reshape(-1))

    def mlp(self, i, x):
        pre = f"layers.{i}.mlp."
        gt = self.linear(pre + "gate_proj", x)
        up = self.linear(pre + "up_proj", x)
        return self.linear(pre + "down_proj", self.rnd(gt / (1.0 + np.exp(-gt)) * up))

    def step(self, token: int):
        """One token through every layer -> (final normed hidden [H], logits [V])."""
        c, p, rnd = self.c, self.p, self.rnd
        h = _f(p["embed_tokens"][token])
        for i in range(c["num_hidden_layers"]):
            x = self.norm(h, f"layers.{i}.input_layernorm")
            r = self.gdn_layer(i, x) if self.is_linear(i) else self.attn(i, x)
            h = rnd(h + r)
            x = self.norm(h, f"layers.{i}.post_attention_layernorm")
            h = rnd(h + self.mlp(i, x))
        hn = self.norm(h, "norm")
        self.pos += 1
        return hn, self.linear("lm_head", hn)

    def forward(self, tokens):
        hs, ls = zip(*[self.step(int(t)) for t in tokens])
        return np.stack(hs), np.stack(ls)


class MTPHead:
    """The MTP draft head restated (reference skinny_mlx/mtp.py:51-67): per token,
    h' = norm(layer(fc([rmsnorm_e(embed(tok)); rmsnorm_h(hidden)]))) with one full-attention
    decoder layer and its own KV cache. params: MTPHead.state_dict() in the numpy form of
    Decoder; the layer's tensors are read through a one-layer Decoder (names "layer." ->
    "layers.0.")."""

    def __init__(self, params: dict, cfg: dict):
        self.p = params
        layer = {"layers.0." + k[len("layer."):]: v for k, v in params.items() if k.startswith("layer.")}
        c = dict(cfg, num_hidden_layers=1, full_attention_interval=0)
        self.dec = Decoder(layer, c)
        self.eps = cfg["rms_norm_eps"]

    def step(self, emb, hidden):
        """emb, hidden: [H] (bf16 values) -> the head's hidden state [H] for this position."""
        p, eps, d = self.p, self.eps, self.dec
        x = np.concatenate([rmsnorm(emb, p["pre_fc_norm_embedding"], eps), rmsnorm(hidden, p["pre_fc_norm_hidden"], eps)])
        y = w4.qmm(w4.f32_to_bf16(x[None].astype(np.float32)), p["fc.weight"], p["fc.scales"], p["fc.biases"])
        h = bf(y)[0]
        r = d.attn(0, rmsnorm(h, d.p["layers.0.input_layernorm"], eps))
        h = bf(h + r)
        h = bf(h + d.mlp(0, rmsnorm(h, d.p["layers.0.post_attention_layernorm"], eps)))
        d.pos += 1
        return rmsnorm(h, p["norm"], eps)
