"""Local MLX 4-bit checkpoints (skinny_mlx.checkpoint): MLX key names and layouts in, the model's
buffers out, byte for byte; quantised tied embeddings; config.json; error paths. CPU only, except
the last test (a loaded model's forward on the GPU)."""

import json

import numpy as np
import pytest
import torch

from oracle import w4
from skinny_mlx.checkpoint import args_from_config, load_mlx_checkpoint, save_mlx_checkpoint
from skinny_mlx.model import build_model
from skinny_mlx.mtp import quantize_w4g64


def _same_state(a, b):
    sa, sb = a.state_dict(), b.state_dict()
    assert sa.keys() == sb.keys()
    for k in sa:
        assert sa[k].dtype == sb[k].dtype and torch.equal(sa[k].cpu(), sb[k].cpu()), k


@pytest.mark.parametrize("preset", ["tiny-dense", "tiny-hybrid", "tiny-qwen35"])
@pytest.mark.parametrize("prefix", ["model.", "language_model.model.", ""])
def test_round_trip_is_byte_exact(tmp_path, preset, prefix):
    src = build_model(preset, device="cpu")
    path = str(tmp_path / "ckpt.safetensors")
    save_mlx_checkpoint(src, path, prefix=prefix)
    dst = build_model(preset, device="cpu", seed=7)
    stats = load_mlx_checkpoint(dst, path)
    assert stats["missing"] == [] and stats["unexpected"] == [] and not stats["tied_head"]
    assert stats["loaded"] == len(src.state_dict())
    _same_state(src, dst)


def test_mlx_layouts_in_the_file(tmp_path):
    from safetensors.torch import load_file

    m = build_model("tiny-hybrid", device="cpu")
    path = str(tmp_path / "ckpt.safetensors")
    save_mlx_checkpoint(m, path)
    f = load_file(path)
    C = m.layers[0].linear_attn.conv1d_weight.shape[0]
    assert f["model.layers.0.linear_attn.conv1d.weight"].shape == (C, 4, 1)  # MLX Conv1d [C, KW, 1]
    assert f["model.layers.0.linear_attn.norm.weight"].dtype == torch.bfloat16
    assert f["model.layers.3.self_attn.q_norm.weight"].shape == (m.args.head_dim,)
    assert f["model.layers.0.mlp.down_proj.weight"].dtype == torch.int32
    assert f["model.norm.weight"].shape == (m.args.hidden_size,)
    assert "lm_head.scales" in f and "model.embed_tokens.weight" in f


def test_sharded_directory_and_extra_tensors_are_skipped(tmp_path):
    from safetensors.torch import load_file, save_file

    src = build_model("tiny-dense", device="cpu")
    full = str(tmp_path / "one.safetensors")
    save_mlx_checkpoint(src, full, prefix="language_model.model.")
    tensors = load_file(full)
    keys = sorted(tensors)
    d = tmp_path / "shards"
    d.mkdir()
    save_file({k: tensors[k] for k in keys[::2]}, str(d / "model-00001-of-00002.safetensors"))
    rest = {k: tensors[k] for k in keys[1::2]}
    rest["mtp.fc.weight"] = torch.zeros(4, 4)  # the MTP head's tensors belong to load_mtp_head
    save_file(rest, str(d / "model-00002-of-00002.safetensors"))
    dst = build_model("tiny-dense", device="cpu", seed=3)
    load_mlx_checkpoint(dst, str(d))
    _same_state(src, dst)


def test_quantised_tied_embedding(tmp_path):
    from safetensors.torch import save_file

    src = build_model("tiny-dense", device="cpu")
    path = str(tmp_path / "tied.safetensors")
    save_mlx_checkpoint(src, path)
    from safetensors.torch import load_file

    f = load_file(path)
    for part in ("weight", "scales", "biases"):
        del f[f"lm_head.{part}"]
    qw, qs, qb = quantize_w4g64(src.embed_tokens.float())
    f["model.embed_tokens.weight"], f["model.embed_tokens.scales"], f["model.embed_tokens.biases"] = qw, qs, qb
    save_file(f, path)
    dst = build_model("tiny-dense", device="cpu", seed=9)
    stats = load_mlx_checkpoint(dst, path)
    assert stats["tied_head"] and stats["missing"] == []
    # the table is the oracle's dequantisation of the pack, rounded to bf16
    ref = w4.dequant(qw.numpy().view(np.uint32), qs.view(torch.int16).numpy().view(np.uint16),
                     qb.view(torch.int16).numpy().view(np.uint16))
    got = dst.embed_tokens.float().numpy()
    assert np.array_equal(got, torch.from_numpy(np.asarray(ref, dtype=np.float32)).to(torch.bfloat16).float().numpy())
    # and the head holds the same W4 pack
    assert torch.equal(dst.lm_head.weight, qw) and torch.equal(dst.lm_head.scales, qs)
    assert torch.equal(dst.lm_head.biases, qb)


def test_errors(tmp_path):
    from safetensors.torch import load_file, save_file

    src = build_model("tiny-dense", device="cpu")
    path = str(tmp_path / "c.safetensors")
    save_mlx_checkpoint(src, path)
    f = load_file(path)
    del f["model.layers.1.mlp.up_proj.scales"]
    f["model.layers.9.extra.weight"] = torch.zeros(2)
    save_file(f, path)
    with pytest.raises(ValueError, match="missing.*up_proj.scales.*unexpected.*layers.9"):
        load_mlx_checkpoint(build_model("tiny-dense", device="cpu"), path)
    stats = load_mlx_checkpoint(build_model("tiny-dense", device="cpu"), path, strict=False)
    assert stats["missing"] == ["layers.1.mlp.up_proj.scales"] and stats["unexpected"] == ["layers.9.extra.weight"]
    f = load_file(path)
    f["model.norm.weight"] = torch.zeros(7, dtype=torch.bfloat16)
    save_file(f, path)
    with pytest.raises(ValueError, match="norm.weight: checkpoint shape"):
        load_mlx_checkpoint(build_model("tiny-dense", device="cpu"), path, strict=False)
    with pytest.raises(FileNotFoundError):
        load_mlx_checkpoint(build_model("tiny-dense", device="cpu"), str(tmp_path / "absent.safetensors"))


def test_args_from_config(tmp_path):
    cfg = {"model_type": "skinny_hybrid", "quantization": {"group_size": 64, "bits": 4},
           "text_config": {"hidden_size": 2560, "num_hidden_layers": 36, "num_attention_heads": 32,
                           "num_key_value_heads": 8, "head_dim": 128, "intermediate_size": 9728,
                           "vocab_size": 151936, "rms_norm_eps": 1e-6, "rope_parameters": {"rope_theta": 1e7},
                           "full_attention_interval": 4, "linear_num_key_heads": 16,
                           "linear_num_value_heads": 16, "linear_key_head_dim": 128, "linear_value_head_dim": 128,
                           "linear_conv_kernel_dim": 4}}
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    a = args_from_config(str(tmp_path), max_position=8192)
    assert (a.hidden_size, a.num_hidden_layers, a.num_key_value_heads, a.full_attention_interval) == (2560, 36, 8, 4)
    assert a.rope_theta == 1e7 and a.linear_num_heads == 16 and a.max_position == 8192
    cfg["quantization"]["bits"] = 8
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    with pytest.raises(ValueError, match="4-bit"):
        args_from_config(str(tmp_path))
    cfg["quantization"]["bits"] = 4
    cfg["text_config"]["linear_num_value_heads"] = 32
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    a = args_from_config(str(tmp_path))
    assert (a.linear_num_heads, a.linear_num_key_heads, a.gdn_key_heads) == (32, 16, 16)
    cfg["text_config"]["linear_num_value_heads"] = 24
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    with pytest.raises(NotImplementedError, match="24 GDN value heads over 16 key heads"):
        args_from_config(str(tmp_path))


def _qwen35_style_config(**text):
    """A Qwen3.5-4B-style text config (transformers qwen3_5 field names): 256-dim heads with a
    quarter rotated, 16 GDN key heads over 32 value heads, the layer pattern as layer_types."""
    t = {"hidden_size": 2560, "num_hidden_layers": 32, "num_attention_heads": 16, "num_key_value_heads": 4,
         "head_dim": 256, "intermediate_size": 9216, "vocab_size": 248320, "rms_norm_eps": 1e-6,
         "rope_parameters": {"rope_type": "default", "rope_theta": 1e7, "partial_rotary_factor": 0.25,
                             "mrope_section": [11, 11, 10], "mrope_interleaved": True},
         "layer_types": (["linear_attention"] * 3 + ["full_attention"]) * 8,
         "linear_num_key_heads": 16, "linear_num_value_heads": 32, "linear_key_head_dim": 128,
         "linear_value_head_dim": 128, "linear_conv_kernel_dim": 4, "model_type": "qwen3_5_text"}
    t.update(text)
    return {"model_type": "qwen3_5", "quantization": {"group_size": 64, "bits": 4}, "text_config": t}


def test_qwen3_5_config_reads_the_gate_partial_rope_and_gdn_heads(tmp_path):
    """The reference's model family (spec.py:175: Qwen3.5-4B): a qwen3_5 config becomes ModelArgs with
    the attention output gate on, RoPE over 64 of 256 head dims, 16 key heads over 32 value heads,
    and the 3:1 pattern from layer_types (transformers qwen3_5/configuration_qwen3_5.py: linear iff
    (i + 1) % interval != 0). What the decoder does not compute is still refused."""
    path = tmp_path / "config.json"
    path.write_text(json.dumps(_qwen35_style_config()))
    a = args_from_config(str(tmp_path))
    assert a.attn_output_gate and a.general_attention
    assert (a.head_dim, a.rotary_dim, a.rope_theta) == (256, 64, 1e7)
    assert (a.full_attention_interval, a.linear_num_heads, a.gdn_key_heads) == (4, 32, 16)
    assert [a.is_linear(i) for i in range(8)] == [True, True, True, False] * 2
    cfg = _qwen35_style_config(partial_rotary_factor=0.5)  # a top-level factor is read when rope_parameters has none
    del cfg["text_config"]["rope_parameters"]["partial_rotary_factor"]
    path.write_text(json.dumps(cfg))
    assert args_from_config(str(tmp_path)).rotary_dim == 128
    for change, match in ((dict(head_dim=192), "head_dim=192"), (dict(num_experts=64), "mixture-of-experts"),
                          (dict(linear_key_head_dim=64), "linear_key_head_dim=64"),
                          (dict(layer_types=["linear_attention", "full_attention", "full_attention"] * 4),
                           "repeating pattern")):
        path.write_text(json.dumps(_qwen35_style_config(**change)))
        with pytest.raises(NotImplementedError, match=match):
            args_from_config(str(tmp_path))
    cfg = _qwen35_style_config()
    cfg["text_config"]["rope_parameters"]["rope_type"] = "yarn"
    path.write_text(json.dumps(cfg))
    with pytest.raises(NotImplementedError, match="yarn"):
        args_from_config(str(tmp_path))
    cfg = _qwen35_style_config()  # an ungated family reads the flag, and a full RoPE by default
    cfg["model_type"] = cfg["text_config"]["model_type"] = "custom"
    del cfg["text_config"]["rope_parameters"]["partial_rotary_factor"]
    path.write_text(json.dumps(cfg))
    a = args_from_config(str(tmp_path))
    assert not a.attn_output_gate and a.rotary_dim == 256


def test_qwen35_4b_preset_is_what_the_loader_reads(tmp_path):
    """The bench's qwen35-4b decoder (model.PRESETS) is the model a Qwen3.5-4B-style config loads
    as: every field that shapes the step is equal."""
    import dataclasses

    from skinny_mlx.model import PRESETS

    (tmp_path / "config.json").write_text(json.dumps(_qwen35_style_config()))
    loaded, preset = args_from_config(str(tmp_path)), PRESETS["qwen35-4b"]
    skip = {"max_position", "seed"}
    for f in dataclasses.fields(preset):
        if f.name not in skip:
            assert getattr(loaded, f.name) == getattr(preset, f.name), f.name
    assert preset.general_attention and preset.rotary_dim == 64 and preset.gdn_key_heads == 16
    assert [preset.is_linear(i) for i in range(preset.num_hidden_layers)] == [loaded.is_linear(i) for i in range(32)]


def test_qwen3_5_checkpoint_round_trip_keeps_the_gated_q_proj(tmp_path):
    """A Qwen3.5-shaped model's q_proj holds 2 x heads x head_dim rows (query then gate rows per
    head, the checkpoint layout), its GDN in_proj_qkv 2 Hk Dk + Hv Dv rows; both go through a
    save / load byte for byte."""
    src = build_model("tiny-qwen35", device="cpu")
    a = src.args
    attn = src.layers[3].self_attn
    assert attn.q_proj.out_features == 2 * a.num_attention_heads * a.head_dim
    gdn = src.layers[0].linear_attn
    assert gdn.in_proj_qkv.out_features == 2 * 2 * 128 + 4 * 128 and gdn.A_log.shape == (4,)
    path = str(tmp_path / "q.safetensors")
    save_mlx_checkpoint(src, path, prefix="language_model.model.")
    dst = build_model("tiny-qwen35", device="cpu", seed=5)
    stats = load_mlx_checkpoint(dst, path)
    assert stats["missing"] == [] and stats["unexpected"] == []
    _same_state(src, dst)


@pytest.mark.gpu
def test_loaded_model_runs_like_the_original(tmp_path):
    from skinny_mlx.cache import make_prompt_cache
    from skinny_mlx.patch import patch_model

    src = build_model("tiny-hybrid")
    path = str(tmp_path / "ckpt.safetensors")
    save_mlx_checkpoint(src, path)
    dst = build_model("tiny-hybrid", seed=11)
    load_mlx_checkpoint(dst, path)
    patch_model(src)
    with pytest.raises(RuntimeError, match="before patch_model"):
        load_mlx_checkpoint(src, path)
    patch_model(dst)
    ids = list(range(5, 40))
    a = src(ids, make_prompt_cache(src))
    b = dst(ids, make_prompt_cache(dst))
    assert torch.equal(a, b)


@pytest.mark.gpu
def test_loaded_qwen3_5_model_runs_like_the_original(tmp_path):
    from skinny_mlx.cache import make_prompt_cache
    from skinny_mlx.patch import patch_model

    src = build_model("tiny-qwen35")
    path = str(tmp_path / "q.safetensors")
    save_mlx_checkpoint(src, path)
    dst = build_model("tiny-qwen35", seed=11)
    load_mlx_checkpoint(dst, path)
    patch_model(src)
    patch_model(dst)
    ids = list(range(5, 40))
    assert torch.equal(src(ids, make_prompt_cache(src)), dst(ids, make_prompt_cache(dst)))
