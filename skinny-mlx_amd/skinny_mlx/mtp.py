"""Multi-token-prediction (MTP) draft head.

Same structure and call surface as the reference (skinny_mlx/mtp.py:51-84): `MTPHead(args)`
computes h' = norm(layer(fc([rmsnorm_e(embed(tok_{t+1})); rmsnorm_h(h_t)]))) with one
full-attention decoder layer and its own KV cache; `load_mtp_head(model, ...)` builds it.

No checkpoint can be fetched here (the reference range-fetches `mtp.*` tensors from the Hub,
mtp.py:25-48), so the head is random-init W4 g64 by default. `load_mtp_head(model,
path=...)` loads a local safetensors file of `mtp.*` tensors with the reference's name map
(mtp.py:76: drop "mtp.", "layers.0." -> "layer."), the +1 shift of the zero-centred 1-D
norm weights (mtp.py:77-78), and W4 g64 affine quantisation of the linears (mtp.py:81-82).
"""

from __future__ import annotations

import torch
from torch import nn

from . import kernels as K
from .cache import KVCache, PromptCache, Shared
from .model import DecoderLayer, ModelArgs, QuantizedLinear, Recorder, _bf16_param


class MTPHead(nn.Module):
    """h_next = norm(layer(fc([norm_e(embed(tok_{t+1})), norm_h(h_t)]))); scored by the model's
    head, it predicts tok_{t+2}."""

    def __init__(self, args: ModelArgs, device="cuda", seed: int = 1):
        super().__init__()
        dev = torch.device(device)
        g = torch.Generator(device=dev).manual_seed(seed)
        H = args.hidden_size
        self.args, self.device = args, dev
        self.register_buffer("pre_fc_norm_embedding", _bf16_param((H,), g, dev))
        self.register_buffer("pre_fc_norm_hidden", _bf16_param((H,), g, dev))
        self.fc = QuantizedLinear(2 * H, H, g, dev)
        fai = args.full_attention_interval or 1
        self.layer = DecoderLayer(args, fai - 1, g, dev, Recorder())  # a full-attention layer
        assert not self.layer.is_linear
        self.register_buffer("norm", _bf16_param((H,), g, dev))

    def forward(self, emb: torch.Tensor, hidden: torch.Tensor, cache: PromptCache, tree=None) -> torch.Tensor:
        """`tree` (a skinny_mlx.tree.DraftTree descriptor) lets the tokens of one call be
        siblings in a draft tree: each attends to the cache before the tree plus its ancestors."""
        eps = self.args.rms_norm_eps
        x = self.fc(torch.cat([K.rmsnorm(emb, self.pre_fc_norm_embedding, eps),
                               K.rmsnorm(hidden.contiguous(), self.pre_fc_norm_hidden, eps)], dim=-1))
        return self._layer(x, cache, tree)

    def forward_tokens(self, tokens: torch.Tensor, table: torch.Tensor, hidden: torch.Tensor, cache: PromptCache,
                       tree=None) -> torch.Tensor:
        """forward(embed(tokens), hidden, ...) with the embedding lookup, the two input norms and
        their concatenation in one launch (kernels.mtp_input); bitwise the same."""
        x = self.fc(K.mtp_input(tokens, table, hidden, self.pre_fc_norm_embedding, self.pre_fc_norm_hidden,
                                self.args.rms_norm_eps))
        return self._layer(x, cache, tree)

    def _layer(self, x: torch.Tensor, cache: PromptCache, tree) -> torch.Tensor:
        eps = self.args.rms_norm_eps
        T = x.shape[0]
        cache.begin_step(T)
        h = x
        y = K.rmsnorm(h, self.layer.input_layernorm, eps)
        r = self.layer.mixer(y, cache[0], tree)
        y = K.rmsnorm(h, self.layer.post_attention_layernorm, eps, residual=r, sum_out=h)
        out = K.rmsnorm(h, self.norm, eps, residual=self.layer.mlp(y), sum_out=h)
        cache.advance(T)
        cache.end_step(T)
        return out


def make_mtp_cache(head: MTPHead) -> PromptCache:
    """A one-layer KV cache for the head (the reference uses a fresh KVCache, spec.py:78)."""
    a = head.args
    shared = Shared(head.device, a.num_key_value_heads, a.max_position,
                    K.attn_workspace_bytes(a.num_key_value_heads, a.max_position))
    shared.allocate_kv(1, a.num_key_value_heads, a.head_dim, a.rope_theta,
                       (a.num_attention_heads, a.rotary_dim) if a.general_attention else None)
    shared.allocate_handoff((a.num_attention_heads + 2 * a.num_key_value_heads) * a.head_dim)
    cache = PromptCache([KVCache(shared, 0)])
    cache.shared = shared
    return cache


def quantize_w4g64(w: torch.Tensor):
    """Affine 4-bit, group-64 quantisation of a float [N, K] weight -> MLX-format
    (packs int32 [N, K/8], scales, biases bf16 [N, K/64]): per group, bias = min and
    scale = (max - min) / 15, codes rounded to nearest and clamped to 0..15."""
    n, k = w.shape
    g = w.float().reshape(n, k // 64, 64)
    lo = g.amin(-1)
    hi = g.amax(-1)
    scale = ((hi - lo) / 15.0).to(torch.bfloat16)
    bias = lo.to(torch.bfloat16)
    sf = scale.float().unsqueeze(-1)
    q = torch.where(sf > 0, torch.round((g - bias.float().unsqueeze(-1)) / torch.where(sf > 0, sf, 1.0)),
                    torch.zeros_like(g)).clamp(0, 15).to(torch.int64).reshape(n, k // 8, 8)
    words = torch.zeros((n, k // 8), dtype=torch.int64, device=w.device)
    for i in range(8):
        words |= q[:, :, i] << (4 * i)
    words = torch.where(words >= 2 ** 31, words - 2 ** 32, words).to(torch.int32)
    return words, scale, bias


def load_mtp_head(model, path: str | None = None, bits: int | None = 4, seed: int = 1, patch: bool = True) -> MTPHead:
    """The MTP head for `model`: random-init W4 g64 (path=None), or the `mtp.*` tensors of a
    local safetensors file, renamed and +1-shifted as in the reference and quantised to W4 g64.
    With `patch` (the default) its linears are patched like the trunk's (patch.patch_model), so
    drafting runs on the skinny kernels."""
    head = MTPHead(model.args, model.device, seed=seed)
    if path is not None:
        _load_mtp_weights(head, path, bits)
    if patch:
        from .patch import patch_model

        patch_model(head)
    return head


@torch.no_grad()
def _load_mtp_weights(head: MTPHead, path: str, bits: int | None) -> None:
    if bits not in (4, None):
        raise ValueError("only 4-bit heads are supported")
    from safetensors.torch import load_file

    raw = load_file(path, device=str(head.device))
    weights = {}
    for k, v in raw.items():
        if not k.startswith("mtp."):
            continue
        k = k.removeprefix("mtp.").replace("layers.0.", "layer.")
        if v.dim() == 1:  # zero-centred RMSNorm gammas
            v = v.float() + 1.0
        weights[k] = v
    for name, mod in head.named_modules():
        if isinstance(mod, QuantizedLinear) and f"{name}.weight" in weights:
            w, s, b = quantize_w4g64(weights.pop(f"{name}.weight"))
            mod.weight.copy_(w)
            mod.scales.copy_(s)
            mod.biases.copy_(b)
    for name, buf in head.named_buffers():
        key = name[:-len(".weight")] if name.endswith(".weight") else name
        for cand in (name, key, name.replace("_layernorm", "_layernorm.weight")):
            if cand in weights and weights[cand].shape == buf.shape:
                buf.copy_(weights.pop(cand).to(buf.dtype))
                break
