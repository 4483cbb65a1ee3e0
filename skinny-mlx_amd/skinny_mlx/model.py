"""Random-init decoders of the verify-step workloads (PyTorch-ROCm + the HIP kernels).

The reference patches an mlx_lm Qwen3.5 model (skinny_mlx/patch.py:90-115) and runs it at
skinny_mlx/spec.py:24-29; no checkpoint is available here, so the build defines its own
decoders with the same structure and the workload dimensions:

  dense   every layer: RMSNorm -> fused-able q/k/v (W4) -> per-head q/k RMSNorm + RoPE ->
          causal GQA attention over the KV cache -> o_proj (W4) -> residual -> RMSNorm ->
          gate/up (W4) -> SwiGLU -> down (W4) -> residual; final RMSNorm; W4 lm_head.
  hybrid  the same, except that in each group of `full_attention_interval` layers the first
          ones are Gated-DeltaNet mixers (qkv/z/b/a projections, causal conv 4, gated delta
          rule, gated RMSNorm, out_proj) and the last one is full attention (Qwen3.5 layout).

Linears are `QuantizedLinear`s holding MLX's W4 g64 format; their unpatched forward is
fp32 dequantise + fp32 GEMM (the mx.quantized_matmul semantics the reference keeps for M outside its
skinny range). `skinny_mlx.patch.patch_model` swaps them for the skinny kernel.
Embeddings and norms are bf16; GDN gates (A_log, dt_bias) are fp32.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field, replace

import torch
from torch import nn

from . import kernels as K
from .cache import ArraysCache, KVCache, PromptCache
from .qmm import GROUP, random_w4g64

MAX_STEP = 16  # tokens per forward pass (longer inputs are processed in pieces)
# Forwards of at most this many tokens form each RMSNorm inside the fused projection after it (its
# norm-in form: every workgroup repeats the norm, which for one token costs less than a launch).
FOLD_TOKENS = 1


@dataclass
class ModelArgs:
    hidden_size: int = 2560
    num_hidden_layers: int = 36
    num_attention_heads: int = 32
    num_key_value_heads: int = 8
    head_dim: int = 128
    intermediate_size: int = 9728
    vocab_size: int = 151936
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    full_attention_interval: int = 0  # 0: dense (all attention); 4: three GDN layers per attention layer
    linear_num_heads: int = 16
    linear_key_head_dim: int = 128
    linear_value_head_dim: int = 128
    linear_conv_kernel_dim: int = 4
    max_position: int = 4096  # KV cache capacity (multiple of 256)
    max_step_tokens: int = MAX_STEP  # tokens whose GDN states a recording forward keeps
    seed: int = 0
    # Qwen3.5 attention (transformers qwen3_5 Attention): RoPE over the first head_dim x factor dims
    # of each head, and q_proj holding per head the query rows then gate rows, the attention output
    # multiplied by sigmoid(gate) before o_proj
    partial_rotary_factor: float = 1.0
    attn_output_gate: bool = False
    # Gated-DeltaNet key heads (0: one per value head); each serves linear_num_heads / this many value
    # heads (Qwen3.5: 16 key heads over 32 value heads)
    linear_num_key_heads: int = 0

    def is_linear(self, i: int) -> bool:
        return self.full_attention_interval > 0 and (i + 1) % self.full_attention_interval != 0

    @property
    def rotary_dim(self) -> int:
        return int(self.head_dim * self.partial_rotary_factor)

    @property
    def general_attention(self) -> bool:
        """Whether the attention layers take the general kernels (kernels.attention_general)
        rather than the 128-dim ones: another head size, a partial RoPE, or an output gate."""
        return self.head_dim != 128 or self.rotary_dim != self.head_dim or self.attn_output_gate

    @property
    def gdn_key_heads(self) -> int:
        return self.linear_num_key_heads or self.linear_num_heads


PRESETS = {
    # the benchmark decoders: 36 layers of hidden 2560, dense, and its 3:1 Gated-DeltaNet hybrid
    "dense-36": ModelArgs(),
    "hybrid-36": ModelArgs(full_attention_interval=4),
    # small shapes for the parity tests
    "tiny-dense": ModelArgs(hidden_size=256, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=1,
                            intermediate_size=512, vocab_size=1024, max_position=512),
    "tiny-hybrid": ModelArgs(hidden_size=256, num_hidden_layers=4, num_attention_heads=4, num_key_value_heads=1,
                             intermediate_size=512, vocab_size=1024, max_position=512, full_attention_interval=4,
                             linear_num_heads=2),
    # the Qwen3.5 architecture at a small size: gated attention over 256-dim heads with a quarter
    # of each head rotated, and GDN layers whose 2 key heads serve 4 value heads
    "tiny-qwen35": ModelArgs(hidden_size=256, num_hidden_layers=4, num_attention_heads=2, num_key_value_heads=1,
                             head_dim=256, intermediate_size=512, vocab_size=1024, max_position=512, rope_theta=1e7,
                             full_attention_interval=4, linear_num_heads=4, linear_num_key_heads=2,
                             partial_rotary_factor=0.25, attn_output_gate=True),
    # the shape of the reference's model, Qwen3.5-4B (spec.py:175), random-init: 24 GDN + 8 gated
    # attention layers (docs/roofline-and-plan.md:12); 16 query / 4 kv heads of 256 dims with a
    # quarter rotated, GDN 16 key / 32 value heads of 128, vocabulary 248320 and RoPE base 1e7 as
    # transformers' qwen3_5 configuration has them; hidden 2560 and FFN 9216 are assumed for the 4B
    # member (the reference holds no config)
    "qwen35-4b": ModelArgs(hidden_size=2560, num_hidden_layers=32, num_attention_heads=16, num_key_value_heads=4,
                           head_dim=256, intermediate_size=9216, vocab_size=248320, rope_theta=1e7,
                           full_attention_interval=4, linear_num_heads=32, linear_num_key_heads=16,
                           partial_rotary_factor=0.25, attn_output_gate=True),
}


def weight_scale_std(k: int) -> float:
    """std of |N(0, std)| scales giving dequantised weights of std ~1/sqrt(K) (codes centred
    by bias = -8 s have std ~4.6, and E|N(0, std)| = 0.8 std)."""
    return 1.0 / (3.7 * math.sqrt(k))


class QuantizedLinear(nn.Module):
    """W4 g64 linear without bias, MLX format (mlx.nn.QuantizedLinear with bits=4, group_size=64):
    weight int32 [N, K/8] (eight codes per word, element i at bits 4i), scales/biases bf16
    [N, K/64]. The unpatched forward dequantises to fp32 and runs an fp32 GEMM."""

    def __init__(self, in_features: int, out_features: int, generator: torch.Generator, device):
        super().__init__()
        self.in_features, self.out_features = in_features, out_features
        self.bits, self.group_size = 4, GROUP
        w, s, b = random_w4g64(out_features, in_features, generator=generator, device=device,
                               scale_std=weight_scale_std(in_features))
        self.register_buffer("weight", w)
        self.register_buffer("scales", s)
        self.register_buffer("biases", b)

    def forward(self, x) -> torch.Tensor:
        if isinstance(x, K.NormIn):
            x = x.value()
        return K.quantized_matmul(x, self.weight, self.scales, self.biases)


def _bf16_param(shape, generator, device, mean=1.0, std=0.02) -> torch.Tensor:
    return (torch.randn(shape, generator=generator, device=device) * std + mean).to(torch.bfloat16)


def residual_out(proj, x: torch.Tensor):
    """A projection whose output is only ever the residual of the next RMSNorm (o_proj, the GDN
    out_proj, down_proj): a patched one returns its split-K slices (kernels.PartialSum), which
    the norm adds, an unpatched one its output."""
    partial = getattr(proj, "partial", None)
    return partial(x) if partial is not None else proj(x)


def norm_input(h: torch.Tensor, residual, weight: torch.Tensor, eps: float, spare: torch.Tensor):
    """The input rmsnorm(h + residual) * weight of the next projections, and the tensor that holds
    the residual stream h + residual once they have run. A split-K residual (kernels.PartialSum)
    or none gives a kernels.NormIn, which a fused projection forms inside its own launch (the new
    stream going to `spare`); any other residual runs the norm kernel now, in place."""
    if residual is None:
        return K.NormIn(h, None, weight, eps), h
    if isinstance(residual, K.PartialSum):
        return K.NormIn(h, residual, weight, eps, spare), spare
    return K.rmsnorm(h, weight, eps, residual=residual, sum_out=h), h


def joined(parts: list[torch.Tensor]) -> torch.Tensor:
    """Concatenate [T, n_i] outputs along the last dim; if they are adjacent slices of one
    buffer (a fused projection), return a view of that buffer instead of copying."""
    first = parts[0]
    t = first.shape[0]
    base = first.untyped_storage().data_ptr()
    ok = all(p.dim() == 2 and p.shape[0] == t and p.stride(1) == 1 and p.stride(0) == first.stride(0)
             and p.untyped_storage().data_ptr() == base for p in parts)
    if ok:
        addr = first.data_ptr()
        for p in parts:
            if p.data_ptr() != addr:
                ok = False
                break
            addr += p.shape[1] * p.element_size()
    width = sum(p.shape[1] for p in parts)
    if ok and first.stride(0) >= width:
        return first.as_strided((t, width), (first.stride(0), 1))
    return torch.cat(parts, dim=-1)


class Attention(nn.Module):
    def __init__(self, a: ModelArgs, g: torch.Generator, dev):
        super().__init__()
        H, D = a.hidden_size, a.head_dim
        self.a = a
        # gated: per head the query rows, then the gate rows (the checkpoint's q_proj layout)
        self.q_proj = QuantizedLinear(H, a.num_attention_heads * D * (2 if a.attn_output_gate else 1), g, dev)
        self.k_proj = QuantizedLinear(H, a.num_key_value_heads * D, g, dev)
        self.v_proj = QuantizedLinear(H, a.num_key_value_heads * D, g, dev)
        self.o_proj = QuantizedLinear(a.num_attention_heads * D, H, g, dev)
        self.register_buffer("q_norm", _bf16_param((D,), g, dev))
        self.register_buffer("k_norm", _bf16_param((D,), g, dev))
        # Opt-in: the fused q|k|v projection in one launch with the attention (bitwise the two
        # launches). Measured on the 36-layer dense step: 1.436 -> 1.442 / 1.524 -> 1.554 /
        # 1.751 -> 1.799 ms at M = 1 / 8 / 16; the hand-off and the reset of its rows cost more
        # than the hidden KV staging saves. Its chunk workgroups wait (bounded) for the projection's
        # rows, counting on the GPU to themselves: not for a model run beside other streams' work.
        self.fuse_qkv = False

    def forward(self, x, cache: KVCache, tree=None):
        a = self.a
        sh = cache.shared
        desc = None if tree is None else tree.desc
        if sh.rope_theta != a.rope_theta:
            raise ValueError(f"cache RoPE table for theta={sh.rope_theta}, layer uses {a.rope_theta}")
        if a.general_attention:
            # Qwen3.5 layouts (another head size, a partial RoPE, the output gate): the general kernels
            if sh.rope_dim != a.rotary_dim:
                raise ValueError(f"cache RoPE table over {sh.rope_dim} dims, layer rotates {a.rotary_dim}")
            Hq, Hkv, D = a.num_attention_heads, a.num_key_value_heads, a.head_dim
            qs = 2 * D if a.attn_output_gate else D
            qkv = joined([self.q_proj(x), self.k_proj(x), self.v_proj(x)])
            o = K.attention_general(qkv, Hq, Hkv, D, qs, Hq * qs, Hq * qs + Hkv * D,
                                    D if a.attn_output_gate else None, self.q_norm, self.k_norm, a.rms_norm_eps,
                                    a.rotary_dim, sh.rope, sh.pos, cache.k, cache.vt, D ** -0.5,
                                    sh.attn_general_workspace, desc)
            return residual_out(self.o_proj, o)
        # With fuse_qkv, a fused q|k|v projection runs in one launch with the attention (the chunk
        # workgroups stage their KV while it streams its weights; bitwise the two launches);
        # otherwise, or where that form does not apply, the projection, then the attention.
        proj = getattr(self.q_proj, "projection", None)
        o = None
        if (self.fuse_qkv and proj is not None and hasattr(proj, "attention_output")
                and all(getattr(m, "projection", None) is proj for m in (self.k_proj, self.v_proj))
                and [m.columns for m in (self.q_proj, self.k_proj, self.v_proj)] == proj.columns):
            o = proj.attention_output(x, dict(
                n_q=a.num_attention_heads, n_kv=a.num_key_value_heads, head_dim=a.head_dim, q_norm=self.q_norm,
                k_norm=self.k_norm, eps=a.rms_norm_eps, table=sh.rope, pos=sh.pos, k_cache=cache.k,
                vt_cache=cache.vt, scale=a.head_dim ** -0.5, workspace=sh.attn_workspace, handoff=sh.handoff,
                tree=desc))
        if o is None:
            qkv = joined([self.q_proj(x), self.k_proj(x), self.v_proj(x)])
            o = K.attention_fused(qkv, a.num_attention_heads, a.num_key_value_heads, a.head_dim, self.q_norm,
                                  self.k_norm, a.rms_norm_eps, sh.rope, sh.pos, cache.k, cache.vt, a.head_dim ** -0.5,
                                  sh.attn_workspace, desc)
        return residual_out(self.o_proj, o)


class GatedDeltaNet(nn.Module):
    def __init__(self, a: ModelArgs, g: torch.Generator, dev, recorder: "Recorder"):
        super().__init__()
        H = a.hidden_size
        nh, dk, dv = a.linear_num_heads, a.linear_key_head_dim, a.linear_value_head_dim
        self.a, self.recorder = a, recorder
        self.conv_dim = 2 * a.gdn_key_heads * dk + nh * dv
        self.in_proj_qkv = QuantizedLinear(H, self.conv_dim, g, dev)
        self.in_proj_z = QuantizedLinear(H, nh * dv, g, dev)
        self.in_proj_b = QuantizedLinear(H, nh, g, dev)
        self.in_proj_a = QuantizedLinear(H, nh, g, dev)
        self.out_proj = QuantizedLinear(nh * dv, H, g, dev)
        kw = a.linear_conv_kernel_dim
        self.register_buffer("conv1d_weight", ((torch.rand((self.conv_dim, kw), generator=g, device=dev) - 0.5)
                                               * (2.0 / math.sqrt(kw))).to(torch.bfloat16))
        self.register_buffer("A_log", torch.log(torch.rand((nh,), generator=g, device=dev) * 15.0 + 1.0))
        self.register_buffer("dt_bias", torch.rand((nh,), generator=g, device=dev) * 2.0 - 1.0)
        self.register_buffer("norm_weight", _bf16_param((dv,), g, dev))
        self.fuse_conv = True  # conv + SiLU in a fused input projection's epilogue when it has one
        # The output norm formed inside a patched out_proj's launch (bitwise the separate norm):
        # opt-in, since every lane then forms 32 gated values per head in front of its first
        # MFMA, measured slower than the separate launch (hybrid-36 one-token step 1.461 against
        # 1.426 ms, recorded 2- / 4- / 8-token verify 1.513 / 1.552 / 1.651 against 1.486 / 1.512 /
        # 1.599 ms, 16-node tree 1.903 against 1.837 ms).
        self.fuse_norm = False
        # A one-token step that keeps no per-token state forms the output norm inside the
        # recurrence's launch (one workgroup per head; bitwise the two launches).
        self.fuse_head_norm = True

    def forward(self, x, cache: ArraysCache, tree=None):
        a = self.a
        T = x.shape[0]
        rec = self.recorder.recording
        if tree is not None and not rec:
            raise ValueError("a draft-tree forward must record (HybridRollback.record()) so it can be committed")
        if rec and T > cache.buffers.max_step:
            raise ValueError(f"recording forward of {T} tokens exceeds {cache.buffers.max_step}")
        parent = None if tree is None else tree.parent
        window = cache.window if rec else None
        # A fused q|k|v|z|b|a projection runs the conv + SiLU in its own epilogue (bitwise the
        # separate conv kernel's output); anything else takes the two launches.
        members = (self.in_proj_qkv, self.in_proj_z, self.in_proj_b, self.in_proj_a)
        proj = getattr(self.in_proj_qkv, "projection", None)
        y = None
        if (self.fuse_conv and proj is not None and hasattr(proj, "conv_output")
                and all(getattr(m, "projection", None) is proj for m in members)
                and self.in_proj_qkv.columns == slice(0, self.conv_dim)):
            y = proj.conv_output(x, self.conv_dim, cache.conv_state, self.conv1d_weight, window, parent)
        if y is not None:
            xc, z, b, ag = (y[:, m.columns] for m in members)
        else:
            qkv, z, b, ag = self.in_proj_qkv(x), self.in_proj_z(x), self.in_proj_b(x), self.in_proj_a(x)
            xc = K.gdn_conv_silu(qkv, cache.conv_state, self.conv1d_weight, window, parent)
        if b.stride(0) != ag.stride(0):
            b, ag = b.contiguous(), ag.contiguous()
        # A recording chain keeps every per-token state for the rollback's selection; a draft tree
        # keeps its nodes' update operands, from which the commit replays the accepted path.
        tree_rec = rec and parent is not None
        if self.fuse_head_norm and T == 1 and not rec and parent is None:
            o = K.gdn_recurrence_gated(xc, b, ag, self.A_log, self.dt_bias, cache.state, z, self.norm_weight,
                                       a.rms_norm_eps, a.linear_num_heads, a.linear_key_head_dim,
                                       a.linear_value_head_dim, a.gdn_key_heads)
            return residual_out(self.out_proj, o)
        y = K.gdn_recurrence(xc, b, ag, self.A_log, self.dt_bias, cache.state,
                             cache.states if rec and not tree_rec else None, a.linear_num_heads,
                             a.linear_key_head_dim, a.linear_value_head_dim, parent,
                             cache.record if tree_rec else None, a.gdn_key_heads)
        # A patched out_proj forms the output norm per head inside its own launch (bitwise the
        # separate norm); otherwise the norm, then the projection.
        gated = getattr(self.out_proj, "partial_gated", None) if self.fuse_norm else None
        r = gated(y, z, self.norm_weight, a.rms_norm_eps) if gated is not None else None
        if r is not None:
            return r
        o = K.gated_rmsnorm(y, z, self.norm_weight, a.rms_norm_eps)
        return residual_out(self.out_proj, o)


def swiglu(gate: nn.Module, up: nn.Module, x: torch.Tensor) -> torch.Tensor:
    """silu(gate(x)) * up(x). When both are slices of one fused gate|up projection (see
    skinny_mlx.patch), its matmul applies the activation in the same launch."""
    proj = getattr(gate, "projection", None)
    if proj is not None and getattr(proj, "gate_up", False) and getattr(up, "projection", None) is proj:
        return proj.swiglu(x)
    return K.silu_mul(joined([gate(x), up(x)]))


class MLP(nn.Module):
    def __init__(self, a: ModelArgs, g: torch.Generator, dev):
        super().__init__()
        self.gate_proj = QuantizedLinear(a.hidden_size, a.intermediate_size, g, dev)
        self.up_proj = QuantizedLinear(a.hidden_size, a.intermediate_size, g, dev)
        self.down_proj = QuantizedLinear(a.intermediate_size, a.hidden_size, g, dev)
        # Opt-in: a patched MLP of the decoders' shape then runs from two tokens on as one launch
        # (gate|up + SwiGLU, then the down projection's split-K slices; bitwise the two launches).
        # Off by default: on the 36-layer dense verify step at M=8 the one launch takes 20.9 us
        # where the two take 10.9 + 4.8 us, so the step is slower (1.80 ms against 1.54 ms). Like
        # fuse_qkv, its down tiles wait (bounded) for the gate|up tiles, counting on the GPU to
        # themselves.
        self.fuse_mlp = False

    def forward(self, x):
        proj = getattr(self.gate_proj, "projection", None)
        if self.fuse_mlp and proj is not None and getattr(self.up_proj, "projection", None) is proj:
            fused = getattr(proj, "mlp_partial", None)
            r = fused(x, self.down_proj) if fused is not None else None
            if r is not None:
                return r
        return residual_out(self.down_proj, swiglu(self.gate_proj, self.up_proj, x))


class DecoderLayer(nn.Module):
    def __init__(self, a: ModelArgs, i: int, g: torch.Generator, dev, recorder: "Recorder"):
        super().__init__()
        self.is_linear = a.is_linear(i)
        self.register_buffer("input_layernorm", _bf16_param((a.hidden_size,), g, dev))
        self.register_buffer("post_attention_layernorm", _bf16_param((a.hidden_size,), g, dev))
        if self.is_linear:
            self.linear_attn = GatedDeltaNet(a, g, dev, recorder)
        else:
            self.self_attn = Attention(a, g, dev)
        self.mlp = MLP(a, g, dev)

    def mixer(self, x, cache, tree=None):
        if self.is_linear:
            return self.linear_attn(x, cache, tree)
        return self.self_attn(x, cache, tree)


@dataclass
class Recorder:
    """Whether GDN layers keep per-token states and conv inputs for rollback (set by
    HybridRollback.record(), cleared by rollback())."""
    recording: bool = False


class Model(nn.Module):
    """The decoder. `model(ids, cache)` -> logits [T, V]; `hidden(ids, cache)` -> the final
    normed hidden states [T, H] (what spec.forward hands to the drafter)."""

    def __init__(self, args: ModelArgs, device="cuda"):
        super().__init__()
        self.args = args
        self.device = torch.device(device)
        g = torch.Generator(device=self.device).manual_seed(args.seed)
        self.recorder = Recorder()
        self.register_buffer("embed_tokens",
                             torch.randn((args.vocab_size, args.hidden_size), generator=g, device=self.device)
                             .to(torch.bfloat16))
        self.layers = nn.ModuleList([DecoderLayer(args, i, g, self.device, self.recorder)
                                     for i in range(args.num_hidden_layers)])
        self.register_buffer("norm", _bf16_param((args.hidden_size,), g, self.device))
        self.lm_head = QuantizedLinear(args.hidden_size, args.vocab_size, g, self.device)
        # True: in forwards of at most FOLD_TOKENS tokens each RMSNorm before a fused projection
        # runs inside that projection's launch (norm_input) where patch.NORMIN_TOKENS allows it
        # (q|k|v and gate|up; the Gated-DeltaNet input keeps its norm launch), with the bits of the
        # separate norm launch. Measured on MI355X (one-token step of the 36-layer decoders over
        # 2048 cached tokens, same box): dense 1.381 against 1.442 ms, hybrid 1.329 against 1.385 ms.
        self.fold_norms = True

    def _ids(self, ids) -> torch.Tensor:
        if isinstance(ids, torch.Tensor):
            t = ids.reshape(-1)
            if t.device != self.device or t.dtype != torch.int32:
                t = t.to(device=self.device, dtype=torch.int32)
            return t.contiguous()
        ids = list(ids)
        if any(i < 0 or i >= self.args.vocab_size for i in ids):
            raise ValueError("token id out of range")
        return torch.tensor(ids, dtype=torch.int32, device=self.device)

    def hidden(self, ids, cache: PromptCache, tree=None) -> torch.Tensor:
        """Final normed hidden states of the tokens `ids`, appended to `cache`. Inputs longer
        than MAX_STEP tokens run as consecutive pieces (each a full pass over the layers).
        `tree` (skinny_mlx.tree.DraftTree) makes the tokens a draft tree instead of a chain."""
        ids = self._ids(ids)
        T = ids.shape[0]
        if tree is not None and tree.size != T:
            raise ValueError(f"draft tree of {tree.size} nodes for {T} tokens")
        if T > MAX_STEP:
            if self.recorder.recording or tree is not None:
                raise ValueError("a recording or draft-tree forward takes at most MAX_STEP tokens")
            return self._pieces(ids, cache)
        a = self.args
        eps = a.rms_norm_eps
        cache.begin_step(T)
        h = K.embed(ids, self.embed_tokens)
        pending = None
        if self.fold_norms and T <= FOLD_TOKENS and h.is_cuda:
            spare = torch.empty_like(h)
            for layer, c in zip(self.layers, cache):
                x, h_next = norm_input(h, pending, layer.input_layernorm, eps, spare)
                r = layer.mixer(x, c, tree)
                if h_next is not h:
                    h, spare = h_next, h
                x, h_next = norm_input(h, r, layer.post_attention_layernorm, eps, spare)
                pending = layer.mlp(x)
                if h_next is not h:
                    h, spare = h_next, h
            out = K.rmsnorm(h, self.norm, eps, residual=pending, sum_out=h)
        else:
            for layer, c in zip(self.layers, cache):
                if pending is None:
                    x = K.rmsnorm(h, layer.input_layernorm, eps)
                else:
                    x = K.rmsnorm(h, layer.input_layernorm, eps, residual=pending, sum_out=h)
                r = layer.mixer(x, c, tree)
                x = K.rmsnorm(h, layer.post_attention_layernorm, eps, residual=r, sum_out=h)
                pending = layer.mlp(x)
            out = K.rmsnorm(h, self.norm, eps, residual=pending, sum_out=h)
        cache.advance(T)
        cache.end_step(T)
        if self.recorder.recording and cache.shared.gdn is not None:
            cache.shared.gdn.recorded = T
        return out

    def _pieces(self, ids: torch.Tensor, cache: PromptCache) -> torch.Tensor:
        """A long input as consecutive MAX_STEP-token passes. With four or more full pieces on the
        GPU, the full pieces replay one captured pass (graphs.CapturedStep, kept on the cache for
        its later prompts): issued kernel by kernel from Python, a pass costs about twice its GPU
        time, and a capture about two passes. The remainder runs eagerly."""
        T = ids.shape[0]
        full = T // MAX_STEP if ids.is_cuda and not torch.cuda.is_current_stream_capturing() else 0
        if full < 4:
            full = 0
        outs = []
        if full:
            piece = getattr(cache, "_piece_step", None)
            if piece is None:
                import weakref

                from .graphs import CapturedStep

                # The step lives on the cache and refers back to it only weakly (the closure too),
                # so a dropped cache frees the graph by reference counting, not by the collector.
                buf = ids[:MAX_STEP].clone()
                wc = weakref.ref(cache)
                piece = cache._piece_step = (buf, CapturedStep(lambda: self.hidden(buf, wc()), cache, MAX_STEP,
                                                               weak_cache=True))
            buf, step = piece
            for i in range(full):
                buf.copy_(ids[i * MAX_STEP:(i + 1) * MAX_STEP])
                outs.append(step().clone())
        for i in range(full * MAX_STEP, T, MAX_STEP):
            outs.append(self.hidden(ids[i:i + MAX_STEP], cache))
        return torch.cat(outs)

    def logits(self, h: torch.Tensor) -> torch.Tensor:
        return self.lm_head(h)

    def forward(self, ids, cache: PromptCache, tree=None) -> torch.Tensor:
        return self.logits(self.hidden(ids, cache, tree))


def build_model(preset: str | ModelArgs = "dense-36", device="cuda", **overrides) -> Model:
    args = PRESETS[preset] if isinstance(preset, str) else preset
    if overrides:
        args = replace(args, **overrides)
    return Model(args, device)
