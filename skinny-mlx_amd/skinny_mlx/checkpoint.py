"""Local MLX 4-bit checkpoints: load the trunk of an mlx_lm Qwen3.5-style decoder into a
`skinny_mlx.model.Model`, and write one out.

The reference gets its model from `mlx_lm.load(...)` of an MLX 4-bit checkpoint (spec.py:175;
patch.py:122) and its MTP head from the `mtp.*` tensors of the original checkpoint (mtp.py:22-48,
76-78). Nothing is fetched here: a checkpoint is a local `*.safetensors` file or a directory of
shards (with its `config.json`). The format is MLX's, byte for byte:

* every W4 linear is `<name>.weight` (int32 [N, K/8], eight 4-bit codes per word, element i at
  bits 4i), `<name>.scales` and `<name>.biases` ([N, K/64]), group size 64;
* norm gammas are stored as used (mlx_lm's sanitize has already applied the +1 of the
  zero-centred RMSNorms when it converted the checkpoint);
* the GDN conv weight is MLX's Conv1d layout [C, KW, 1];
* a quantised embedding (`embed_tokens.{weight,scales,biases}`) is dequantised to the model's
  bf16 table (q·s + b, exact in fp32, rounded once to bf16; MLX's own dequantisation rounding is
  not pinned here), and it doubles as the LM head when the checkpoint has no `lm_head` (the tied
  head the reference routes through `QuantizedEmbedding.as_linear`, patch.py:85-87).

Key prefixes `language_model.model.`, `model.` and `language_model.` are accepted (the
multimodal Qwen3.5 nests its text model under `language_model`).

What the decoder computes is the dense Qwen3 block and the Qwen3.5 Gated-DeltaNet hybrid,
including Qwen3.5's attention (the output gated by sigmoid of the second half of each head's
q_proj rows, RoPE over a quarter of each 256-dim head) and its GDN layers with 16 key heads over
32 value heads. `args_from_config` reads those settings; configs with features it does not
compute (mixture of experts, other head sizes, RoPE scaling) raise NotImplementedError rather than
load into a model that would compute something else.
"""

from __future__ import annotations

import json
import os
import re

import torch

from .model import GROUP, ModelArgs

_PREFIXES = ("language_model.model.", "model.language_model.", "model.", "language_model.")


def _files(path: str) -> list[str]:
    if os.path.isdir(path):
        files = sorted(os.path.join(path, f) for f in os.listdir(path) if f.endswith(".safetensors"))
        if not files:
            raise FileNotFoundError(f"no .safetensors files in {path}")
        return files
    if not os.path.exists(path):
        raise FileNotFoundError(path)
    return [path]


def _strip(key: str) -> str:
    for p in _PREFIXES:
        if key.startswith(p):
            return key[len(p):]
    return key


def args_from_config(path: str, **overrides) -> ModelArgs:
    """ModelArgs from an mlx_lm / HF `config.json` (a directory or the file itself); the text
    model's settings may sit under `text_config`. Only 4-bit group-64 quantisation is supported.

    The Qwen3.5 features are read as transformers' qwen3_5 configuration states them: the
    attention output gate (always on for the qwen3_5 / qwen3_next families, else the config's
    `attn_output_gate`), `partial_rotary_factor` (in `rope_parameters` or at the top level; 0.25 by
    default for those families), `head_dim`, and GDN layers with `linear_num_key_heads` key heads
    over `linear_num_value_heads` value heads. The interleaved multimodal RoPE sections
    (`mrope_section`) turn text positions exactly as a plain RoPE does (all three position streams
    equal the token position), so they are accepted and ignored. Features this decoder does not
    compute raise NotImplementedError (_reject_unsupported)."""
    cfg_path = os.path.join(path, "config.json") if os.path.isdir(path) else path
    with open(cfg_path) as f:
        cfg = json.load(f)
    q = cfg.get("quantization") or cfg.get("quantization_config")
    text = cfg.get("text_config", cfg)
    if q is not None and (q.get("bits", 4) != 4 or q.get("group_size", GROUP) != GROUP):
        raise ValueError(f"only 4-bit group-{GROUP} checkpoints are supported, got {q}")
    rope = text.get("rope_parameters") or text.get("rope_scaling") or {}
    family = {str(cfg.get("model_type", "")), str(text.get("model_type", ""))}
    gated_family = bool(family & set(_GATED_FAMILIES))
    _reject_unsupported(cfg, text, rope)
    head_dim = text.get("head_dim", text["hidden_size"] // text["num_attention_heads"])
    factor = rope.get("partial_rotary_factor", text.get("partial_rotary_factor", 0.25 if gated_family else 1.0))
    kw = dict(
        hidden_size=text["hidden_size"],
        num_hidden_layers=text["num_hidden_layers"],
        num_attention_heads=text["num_attention_heads"],
        num_key_value_heads=text.get("num_key_value_heads", text["num_attention_heads"]),
        head_dim=head_dim,
        intermediate_size=text["intermediate_size"],
        vocab_size=text["vocab_size"],
        rms_norm_eps=text.get("rms_norm_eps", 1e-6),
        rope_theta=rope.get("rope_theta", text.get("rope_theta", 1e6)),
        full_attention_interval=_attention_interval(text),
        partial_rotary_factor=float(factor),
        attn_output_gate=bool(text.get("attn_output_gate", cfg.get("attn_output_gate", gated_family))),
    )
    if kw["full_attention_interval"]:
        nk = text.get("linear_num_key_heads", 16)
        nv = text.get("linear_num_value_heads", nk)
        kw.update(linear_num_heads=nv, linear_num_key_heads=0 if nk == nv else nk,
                  linear_key_head_dim=text.get("linear_key_head_dim", 128),
                  linear_value_head_dim=text.get("linear_value_head_dim", 128),
                  linear_conv_kernel_dim=text.get("linear_conv_kernel_dim", 4))
    kw.update(overrides)
    return ModelArgs(**kw)


def _attention_interval(text: dict) -> int:
    """full_attention_interval, or derived from `layer_types` (transformers qwen3_5: a layer is
    linear attention iff (i + 1) % interval != 0); 0 for a dense stack."""
    interval = int(text.get("full_attention_interval", 0) or 0)
    types = text.get("layer_types")
    if not types:
        return interval
    full = [i for i, t in enumerate(types) if t == "full_attention"]
    if len(full) == len(types):
        return 0
    step = full[0] + 1 if full else 0
    if not step or any(t != ("full_attention" if (i + 1) % step == 0 else "linear_attention")
                       for i, t in enumerate(types)):
        raise NotImplementedError(f"layer_types {types[:8]}...: only a repeating pattern of linear layers ending in "
                                  "one full-attention layer is implemented")
    return step


# Model families whose attention layers gate their output with sigmoid(gate), the gate being the
# second half of each head's q_proj rows (transformers qwen3_5 / qwen3_next Attention: q_proj of
# 2 x heads x head_dim, `attn_output * sigmoid(gate)`), and whose RoPE covers a fraction of the head
# (partial_rotary_factor, 0.25 by default in those configs).
_GATED_FAMILIES = ("qwen3_5", "qwen3_5_text", "qwen3_next")


def _reject_unsupported(cfg: dict, text: dict, rope: dict) -> None:
    """Raise NotImplementedError for architecture features this decoder does not compute, so that
    a checkpoint whose tensors would still fit the shapes is never run as another model: mixture
    of experts, head sizes the attention kernels do not take, an odd rotary dimension, GDN head
    sizes other than 128, and RoPE scaling other than the plain one."""
    family = {str(cfg.get("model_type", "")), str(text.get("model_type", ""))}
    if any("moe" in f for f in family) or text.get("num_experts") or text.get("num_local_experts"):
        raise NotImplementedError(f"model type {sorted(family - {''})}: mixture-of-experts layers are not implemented")
    hd = text.get("head_dim", text["hidden_size"] // text["num_attention_heads"])
    if hd not in (64, 128, 256):
        raise NotImplementedError(f"head_dim={hd}: the attention kernels take head_dim 64, 128 or 256")
    gated_family = bool(family & set(_GATED_FAMILIES))
    factor = float(rope.get("partial_rotary_factor", text.get("partial_rotary_factor", 0.25 if gated_family else 1.0)))
    rd = int(hd * factor)
    if rd < 2 or rd % 2 or rd > hd:
        raise NotImplementedError(f"partial_rotary_factor={factor}: {rd} rotary dims of a {hd}-dim head")
    kind = rope.get("rope_type", rope.get("type", "default"))
    if kind not in ("default", None):
        raise NotImplementedError(f"rope_type {kind!r}: only the plain RoPE is implemented")
    if text.get("full_attention_interval") or text.get("layer_types"):
        for key in ("linear_key_head_dim", "linear_value_head_dim"):
            if text.get(key, 128) != 128:
                raise NotImplementedError(f"{key}={text[key]}: the Gated-DeltaNet kernels take 128")
        nk = text.get("linear_num_key_heads", 16)
        nv = text.get("linear_num_value_heads", nk)
        if nv % nk:
            raise NotImplementedError(f"{nv} GDN value heads over {nk} key heads: not a whole number per key head")


def _mlx_name(name: str) -> str:
    """Model buffer name -> the checkpoint key (without prefix)."""
    name = re.sub(r"(input_layernorm|post_attention_layernorm|q_norm|k_norm)$", r"\1.weight", name)
    if name == "norm":
        return "norm.weight"
    name = name.replace("linear_attn.conv1d_weight", "linear_attn.conv1d.weight")
    name = name.replace("linear_attn.norm_weight", "linear_attn.norm.weight")
    if name == "embed_tokens":
        return "embed_tokens.weight"
    return name


def _dequant_rows(w: torch.Tensor, s: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """MLX W4 g64 rows -> fp32 (q * s + b), q element i of a word at bits 4i."""
    n = w.shape[0]
    words = w.to(torch.int64) & 0xFFFFFFFF
    q = torch.stack([(words >> (4 * i)) & 0xF for i in range(8)], dim=-1).reshape(n, -1).float()
    sf = s.float().repeat_interleave(GROUP, dim=1)
    bf = b.float().repeat_interleave(GROUP, dim=1)
    return q * sf + bf


@torch.no_grad()
def load_mlx_checkpoint(model, path: str, strict: bool = True) -> dict:
    """Copy the checkpoint at `path` into `model` (built with matching ModelArgs). Returns
    {"loaded", "missing", "unexpected", "tied_head"}; with `strict`, missing or unexpected trunk
    tensors raise. Shapes must match exactly (W4 packs, scales and biases are copied as they are;
    floating tensors are cast to the buffer's dtype). Load before patch_model(model)."""
    from safetensors.torch import load_file

    from .patch import FusedSliceLinear, SkinnyQuantizedLinear

    if any(isinstance(m, (SkinnyQuantizedLinear, FusedSliceLinear)) for m in model.modules()):
        raise RuntimeError("load the checkpoint before patch_model: patched linears hold packed copies")
    raw = {}
    for f in _files(path):
        for k, v in load_file(f).items():
            k = _strip(k)
            if k.startswith("mtp.") or k.startswith("vision") or k.startswith("visual"):
                continue
            raw[k] = v
    targets = {_mlx_name(n): t for n, t in model.state_dict(keep_vars=True).items()}
    loaded, tied = [], False
    emb_q = "embed_tokens.scales" in raw
    if emb_q:  # quantised embedding table -> bf16 rows
        table = _dequant_rows(raw.pop("embed_tokens.weight"), raw.pop("embed_tokens.scales"),
                              raw.pop("embed_tokens.biases"))
        raw["embed_tokens.weight"] = table
        if "lm_head.weight" not in raw:  # tied head: the quantised table is the head's W4 pack
            tied = True
    for key, buf in targets.items():
        if key not in raw:
            continue
        src = raw.pop(key)
        if key.endswith("conv1d.weight") and src.dim() == 3:  # MLX Conv1d [C, KW, 1]
            src = src.reshape(src.shape[0], src.shape[1])
        if tuple(src.shape) != tuple(buf.shape):
            raise ValueError(f"{key}: checkpoint shape {tuple(src.shape)} != model {tuple(buf.shape)}")
        if buf.dtype == torch.int32 and src.dtype not in (torch.int32, torch.uint32):
            raise ValueError(f"{key}: expected packed int32 codes, got {src.dtype}")
        buf.data.copy_(src.view(torch.int32) if src.dtype == torch.uint32 else src.to(buf.dtype))
        loaded.append(key)
    if tied:
        head = model.lm_head
        emb = load_file_tensors(path, "embed_tokens")
        for part in ("weight", "scales", "biases"):
            getattr(head, part).data.copy_(emb[part])
            loaded.append(f"lm_head.{part} (tied)")
    missing = [k for k in targets if k not in loaded and not (tied and k.startswith("lm_head."))]
    unexpected = sorted(raw)
    if strict and (missing or unexpected):
        raise ValueError(f"checkpoint mismatch: missing {missing[:8]}{'...' if len(missing) > 8 else ''}, "
                         f"unexpected {unexpected[:8]}{'...' if len(unexpected) > 8 else ''}")
    return {"loaded": len(loaded), "missing": missing, "unexpected": unexpected, "tied_head": tied}


def load_file_tensors(path: str, module: str) -> dict:
    """The weight / scales / biases of one module of the checkpoint at `path` (prefix-stripped)."""
    from safetensors.torch import load_file

    out = {}
    for f in _files(path):
        for k, v in load_file(f).items():
            k = _strip(k)
            if k.startswith(module + "."):
                out[k[len(module) + 1:]] = v
    return out


@torch.no_grad()
def save_mlx_checkpoint(model, path: str, prefix: str = "model.") -> None:
    """Write `model`'s trunk as an MLX-format safetensors file (keys under `prefix`, the LM head
    as `lm_head.*`, the conv weight as [C, KW, 1])."""
    from safetensors.torch import save_file

    out = {}
    for name, t in model.state_dict().items():
        key = _mlx_name(name)
        t = t.detach().cpu().contiguous()
        if key.endswith("conv1d.weight"):
            t = t.reshape(t.shape[0], t.shape[1], 1)
        out[key if key.startswith("lm_head.") else prefix + key] = t
    save_file(out, path)


__all__ = ["args_from_config", "load_mlx_checkpoint", "save_mlx_checkpoint"]
