"""Per-layer caches of the decoders: attention KV caches and Gated-DeltaNet state.

Counterparts of mlx_lm's `KVCache` (offset, `trim`) and `ArraysCache` ([conv_state,
recurrent_state]) and of `make_prompt_cache`, which the reference uses at
skinny_mlx/spec.py:19, 78, 93, 99, 123 and rollback.py:14, 64-73.

Memory is laid out for the device, not per object:
  * every attention layer has K [Hkv, maxlen, D] and V transposed [Hkv, D, maxlen] (bf16,
    zero-initialised so rolled-back or never-written positions hold finite values), as views of
    model-wide [L, ...] tensors so that one launch can move an accepted draft-tree path in all
    layers;
  * all attention layers share one device int32 `pos` (tokens cached before the step) that
    the kernels read, so a captured launch sequence replays at any length; each layer still
    keeps its own host-side `offset`, trimmed per layer like mlx_lm's KVCache;
  * the Gated-DeltaNet layers' conv windows, states, per-token states and recorded conv
    inputs live in four model-wide tensors, so one launch rolls back every layer.
"""

from __future__ import annotations

import torch


class Shared:
    """State common to every layer cache of one generation."""

    def __init__(self, device, n_kv: int, maxlen: int, workspace_bytes: int):
        self.device = device
        self.maxlen = maxlen
        self.pos = torch.zeros(1, dtype=torch.int32, device=device)
        self.dev_pos = 0  # value last written to `pos`
        self.attn_workspace = torch.empty(max(workspace_bytes // 4, 1), dtype=torch.float32, device=device)
        self.gdn = None  # GDNBuffers when the model has Gated-DeltaNet layers
        self.k_all = self.vt_all = None  # [L, Hkv, maxlen, D] / [L, Hkv, D, maxlen] bf16
        self.rope = None  # fp32 [maxlen, R/2, 2] (cos, sin) of every cache position (allocate_kv)
        self.rope_theta = None
        self.rope_dim = None  # R of a general-attention table (None: the 128-dim kernels' table)
        self.attn_general_workspace = None  # kernels.attention_general's workspace, when its layers need it
        self.handoff = None  # int16 [16, q|k|v width], all -1: the fused q|k|v + attention's rows

    def allocate_handoff(self, width: int) -> None:
        """The hand-off rows of kernels.qkv_attention_fused (16 tokens of `width` q|k|v columns),
        made before any step is captured; every call leaves them all -1 again."""
        self.handoff = torch.full((16, width), -1, dtype=torch.int16, device=self.device)

    def allocate_kv(self, layers: int, n_kv: int, head_dim: int, rope_theta: float,
                    general: tuple[int, int] | None = None) -> None:
        """The model-wide K / V^T caches and the RoPE table, made before any step is captured.
        `general` = (query heads, rotary dims) for attention layers that take the general kernels
        (kernels.attention_general): their table covers the rotary dims, and their workspace is
        made here too."""
        from . import kernels as K

        self.k_all = torch.zeros((layers, n_kv, self.maxlen, head_dim), dtype=torch.bfloat16, device=self.device)
        self.vt_all = torch.zeros((layers, n_kv, head_dim, self.maxlen), dtype=torch.bfloat16, device=self.device)
        if general is None:
            self.rope = K.rope_table(rope_theta, self.maxlen, self.device)
        else:
            n_q, rd = general
            self.rope = K.rope_table_dim(rope_theta, rd, self.maxlen, self.device)
            self.rope_dim = rd
            self.attn_general_workspace = K.attn_general_workspace(n_q, n_kv, head_dim, self.maxlen, self.device)
        self.rope_theta = rope_theta


class KVCache:
    """Attention layer cache (mlx_lm KVCache semantics: `offset`, `trim(n)`): K [Hkv, maxlen, D]
    and V^T [Hkv, D, maxlen], views of the model-wide `shared.k_all` / `shared.vt_all`."""

    def __init__(self, shared: Shared, index: int):
        self.shared = shared
        self.index = index
        self.k = shared.k_all[index]
        self.vt = shared.vt_all[index]
        self.offset = 0

    def is_trimmable(self) -> bool:
        return True

    def trim(self, n: int) -> int:
        n = min(self.offset, n)
        self.offset -= n
        return n


class GDNBuffers:
    """Model-wide Gated-DeltaNet buffers; layer j owns index j of each tensor."""

    def __init__(self, device, layers: int, heads: int, dk: int, dv: int, conv_dim: int, conv_kernel: int,
                 max_step: int):
        self.max_step = max_step
        self.conv_rows = conv_kernel - 1
        self.conv = torch.zeros((layers, conv_kernel - 1, conv_dim), dtype=torch.bfloat16, device=device)
        self.state = torch.zeros((layers, heads, dv, dk), dtype=torch.float32, device=device)
        self.states = torch.zeros((layers, max_step, heads, dv, dk), dtype=torch.float32, device=device)
        self.window = torch.zeros((layers, max_step + conv_kernel - 1, conv_dim), dtype=torch.bfloat16, device=device)
        # a draft tree's pass keeps its nodes' update operands here (not their states); the commit replays the path
        from .kernels import gdn_record_words
        self.record = torch.zeros((layers, gdn_record_words(heads)), dtype=torch.float32, device=device)
        self.recorded = 0  # tokens recorded by the last recording forward (0 = none)


class ArraysCache:
    """Gated-DeltaNet layer cache: views of the model-wide buffers (mlx_lm ArraysCache:
    cache[0] is the conv window, cache[1] the recurrent state)."""

    def __init__(self, buffers: GDNBuffers, j: int):
        self.buffers = buffers
        self.index = j

    @property
    def conv_state(self) -> torch.Tensor:
        return self.buffers.conv[self.index]

    @property
    def state(self) -> torch.Tensor:
        return self.buffers.state[self.index]

    @property
    def states(self) -> torch.Tensor:
        return self.buffers.states[self.index]

    @property
    def window(self) -> torch.Tensor:
        return self.buffers.window[self.index]

    @property
    def record(self) -> torch.Tensor:
        return self.buffers.record[self.index]

    def __getitem__(self, i: int) -> torch.Tensor:
        return (self.conv_state, self.state)[i]


class PromptCache(list):
    """The list of per-layer caches (what mlx_lm's make_prompt_cache returns), plus the
    shared device position."""

    shared: Shared

    def attention_offset(self) -> int:
        offs = {c.offset for c in self if isinstance(c, KVCache)}
        if len(offs) > 1:
            raise RuntimeError(f"attention caches disagree on their length: {sorted(offs)}")
        return offs.pop() if offs else 0

    # A forward of T tokens is begin_step(T) (host: capacity check, and a device write of the
    # length only when the device copy is stale, e.g. after a trim), the kernels, advance(T)
    # (device: the length moves past the step — a kernel, so a captured step carries it), and
    # end_step(T) (host bookkeeping, which a replayed capture redoes).

    def begin_step(self, tokens: int) -> None:
        """Check capacity and make the device length current before a forward of `tokens` tokens."""
        off = self.attention_offset()
        if off + tokens > self.shared.maxlen:
            raise ValueError(f"KV cache full: {off} + {tokens} > {self.shared.maxlen}")
        if self.shared.dev_pos != off:
            self.shared.pos.fill_(off)
            self.shared.dev_pos = off

    def advance(self, tokens: int) -> None:
        """Device side of a step's end: the shared length grows by `tokens`."""
        self.shared.pos.add_(tokens)

    def end_step(self, tokens: int) -> None:
        """Host side of a step's end: every attention layer's length, and the tracked device length."""
        for c in self:
            if isinstance(c, KVCache):
                c.offset += tokens
        self.shared.dev_pos += tokens

    def resync(self, length: int) -> None:
        """Host bookkeeping after steps that moved the device length by amounts only the device
        knew (an on-device decode loop): every attention layer and the tracked device length
        become `length`, the value read back from `shared.pos`."""
        for c in self:
            if isinstance(c, KVCache):
                c.offset = length
        self.shared.dev_pos = length

    def host_state(self) -> tuple:
        """The host-side bookkeeping (restored after a capture, during which no kernel ran)."""
        gdn = self.shared.gdn
        return (tuple(c.offset for c in self if isinstance(c, KVCache)), self.shared.dev_pos,
                None if gdn is None else gdn.recorded)

    def restore_host_state(self, state: tuple) -> None:
        offsets, dev_pos, recorded = state
        kv = [c for c in self if isinstance(c, KVCache)]
        for c, off in zip(kv, offsets):
            c.offset = off
        self.shared.dev_pos = dev_pos
        if self.shared.gdn is not None:
            self.shared.gdn.recorded = recorded


def make_prompt_cache(model) -> PromptCache:
    """Fresh caches for `model` (counterpart of mlx_lm.models.cache.make_prompt_cache)."""
    from . import kernels as K

    a = model.args
    dev = model.device
    shared = Shared(dev, a.num_key_value_heads, a.max_position,
                    K.attn_workspace_bytes(a.num_key_value_heads, a.max_position))
    n_gdn = sum(1 for l in model.layers if l.is_linear)
    if n_gdn:
        conv_dim = 2 * a.gdn_key_heads * a.linear_key_head_dim + a.linear_num_heads * a.linear_value_head_dim
        shared.gdn = GDNBuffers(dev, n_gdn, a.linear_num_heads, a.linear_key_head_dim, a.linear_value_head_dim,
                                conv_dim, a.linear_conv_kernel_dim, a.max_step_tokens)
    shared.allocate_kv(len(model.layers) - n_gdn, a.num_key_value_heads, a.head_dim, a.rope_theta,
                       (a.num_attention_heads, a.rotary_dim) if a.general_attention else None)
    shared.allocate_handoff((a.num_attention_heads + 2 * a.num_key_value_heads) * a.head_dim)
    cache = PromptCache()
    cache.shared = shared
    j = i = 0
    for layer in model.layers:
        if layer.is_linear:
            cache.append(ArraysCache(shared.gdn, j))
            j += 1
        else:
            cache.append(KVCache(shared, i))
            i += 1
    return cache
