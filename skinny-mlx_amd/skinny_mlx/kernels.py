"""Thin, validated Python wrappers over the decoder kernels of libskinny_hip.so.

Each function launches on torch's current stream, allocates only its output (when `out` is
not given) and never synchronises. Shapes and dtypes are checked here; the C side checks
them again and reports through skinny_last_error().
"""

from __future__ import annotations

import torch

from . import _lib

BF16 = torch.bfloat16


def _req(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _bf16_2d(t: torch.Tensor, name: str) -> None:
    _req(t.is_cuda and t.dtype == BF16 and t.dim() == 2 and t.stride(-1) == 1, f"{name} must be a bf16 2-D GPU tensor")


class PartialSum:
    """The output of a split-K projection not yet summed: fp32 slices [splits, M, N]; their sum in
    slice order, rounded to bf16, is the projection's output. `rmsnorm` takes it as a residual;
    `value()` gives the bf16 tensor."""

    def __init__(self, parts: torch.Tensor):
        self.parts = parts

    @property
    def shape(self):
        return self.parts.shape[1:]

    def value(self) -> torch.Tensor:
        acc = self.parts[0].clone()
        for s in range(1, self.parts.shape[0]):
            acc += self.parts[s]
        return acc.to(torch.bfloat16)


class NormIn:
    """rmsnorm(h + residual) * weight, not yet formed: the input of a projection that can form it
    inside its own launch (the norm-in matmuls of skinny_mlx.qmm). `residual` is a PartialSum or
    None. Once the consuming projection has run, h_out (which must not be h) holds h + residual in
    bf16, as rmsnorm's sum_out would. Anything else that takes it calls value(): the separate norm
    kernel, with the same bits (cached)."""

    def __init__(self, h: torch.Tensor, residual, weight: torch.Tensor, eps: float,
                 h_out: torch.Tensor | None = None):
        _bf16_2d(h, "h")
        _req(h.is_contiguous(), "h must be contiguous")
        _req(residual is None or isinstance(residual, PartialSum), "residual must be a PartialSum or None")
        _req(h_out is None or (h_out.shape == h.shape and h_out.dtype == BF16 and h_out.is_contiguous()
                               and h_out.data_ptr() != h.data_ptr()), "h_out must be a bf16 buffer like h, not h")
        _req(residual is None or h_out is not None, "a residual needs h_out")
        self.h, self.residual, self.weight, self.eps, self.h_out = h, residual, weight, float(eps), h_out
        self._value = None

    @property
    def shape(self):
        return self.h.shape

    @property
    def device(self):
        return self.h.device

    @property
    def dtype(self):
        return BF16

    def dim(self) -> int:
        return 2

    def numel(self) -> int:
        return self.h.numel()

    @property
    def splits(self) -> int:
        return 0 if self.residual is None else self.residual.parts.shape[0]

    def abi(self) -> "_lib.NormIn":
        p = None if self.residual is None else self.residual.parts
        return _lib.NormIn(self.h.data_ptr(), _lib.ptr(p), self.splits, self.weight.data_ptr(), self.eps,
                           _lib.ptr(self.h_out))

    def value(self) -> torch.Tensor:
        if self._value is None:
            self._value = rmsnorm(self.h, self.weight, self.eps, residual=self.residual, sum_out=self.h_out)
        return self._value


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, residual=None,
            sum_out: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """rmsnorm(x + residual) * weight; with sum_out, x + residual is stored there (may be x).
    `residual` may be a PartialSum (split-K slices, summed in order and rounded to bf16)."""
    if isinstance(residual, PartialSum):
        _bf16_2d(x, "x")
        rows, H = x.shape
        p = residual.parts
        _req(p.dtype == torch.float32 and p.dim() == 3 and tuple(p.shape[1:]) == (rows, H) and p.is_contiguous(),
             "partial residual must be contiguous fp32 [splits, rows, H]")
        y = torch.empty_like(x) if out is None else out
        _lib.check(_lib.lib().skinny_rmsnorm_partials_bf16(x.data_ptr(), p.data_ptr(), p.shape[0], p.stride(0), H,
                                                           weight.data_ptr(), eps, y.data_ptr(), _lib.ptr(sum_out),
                                                           rows, H, _lib.stream_of(x)), "rmsnorm_partials")
        return y
    _bf16_2d(x, "x")
    rows, H = x.shape
    _req(x.is_contiguous(), "x must be contiguous")
    _req(weight.dtype == BF16 and weight.numel() == H, "weight must be bf16 [H]")
    if residual is not None:
        _req(residual.shape == x.shape and residual.dtype == BF16 and residual.is_contiguous(), "residual mismatch")
    if sum_out is not None:
        _req(residual is not None and sum_out.shape == x.shape and sum_out.is_contiguous(), "sum_out mismatch")
    y = torch.empty_like(x) if out is None else out
    _lib.check(_lib.lib().skinny_rmsnorm_bf16(x.data_ptr(), _lib.ptr(residual), weight.data_ptr(), eps, y.data_ptr(),
                                              _lib.ptr(sum_out), rows, H, _lib.stream_of(x)), "rmsnorm")
    return y


def mtp_input(ids: torch.Tensor, table: torch.Tensor, hidden: torch.Tensor, w_e: torch.Tensor, w_h: torch.Tensor,
              eps: float) -> torch.Tensor:
    """[rmsnorm(embed(ids)) * w_e | rmsnorm(hidden) * w_h] -> bf16 [T, 2H] in one launch: the MTP
    head's fc input, bitwise embed + two rmsnorm calls + concatenation."""
    _req(ids.is_cuda and ids.dtype == torch.int32 and ids.dim() == 1 and ids.is_contiguous(), "ids must be int32 [T]")
    _req(table.dtype == BF16 and table.dim() == 2 and table.is_contiguous(), "table must be contiguous bf16 [V, H]")
    _bf16_2d(hidden, "hidden")
    T = ids.shape[0]
    V, H = table.shape
    _req(hidden.shape == (T, H) and hidden.stride(1) == 1, "hidden must be bf16 [T, H] rows")
    out = torch.empty((T, 2 * H), dtype=BF16, device=ids.device)
    _lib.check(_lib.lib().skinny_mtp_input_bf16(ids.data_ptr(), T, table.data_ptr(), V, hidden.data_ptr(),
                                                hidden.stride(0), w_e.data_ptr(), w_h.data_ptr(), eps, out.data_ptr(), H,
                                                _lib.stream_of(ids)), "mtp_input")
    return out


def gated_rmsnorm(y: torch.Tensor, z: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """Per head: rmsnorm(y) * weight * silu(z). y fp32 [T, H, D]; z bf16 [T, >= H*D] rows."""
    _req(y.is_cuda and y.dtype == torch.float32 and y.dim() == 3 and y.is_contiguous(), "y must be fp32 [T, H, D]")
    T, H, D = y.shape
    _req(z.dtype == BF16 and z.dim() == 2 and z.shape[0] == T and z.shape[1] == H * D and z.stride(1) == 1,
         "z must be bf16 [T, H*D] (row stride free)")
    out = torch.empty((T, H * D), dtype=BF16, device=y.device)
    _lib.check(_lib.lib().skinny_gated_rmsnorm(y.data_ptr(), z.data_ptr(), z.stride(0), weight.data_ptr(), eps,
                                               out.data_ptr(), T, H, D, _lib.stream_of(y)), "gated_rmsnorm")
    return out


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up for the fused [T, 2F] gate|up projection output -> [T, F]."""
    _bf16_2d(gate_up, "gate_up")
    T, F2 = gate_up.shape
    F = F2 // 2
    out = torch.empty((T, F), dtype=BF16, device=gate_up.device)
    _lib.check(_lib.lib().skinny_silu_mul_bf16(gate_up.data_ptr(), gate_up.stride(0), out.data_ptr(), T, F,
                                               _lib.stream_of(gate_up)), "silu_mul")
    return out


def embed(ids: torch.Tensor, table: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """table[ids] for int32 ids on the GPU (ids must be in range; the host checks host-side ids)."""
    _req(ids.is_cuda and ids.dtype == torch.int32 and ids.dim() == 1 and ids.is_contiguous(), "ids: int32 [T] GPU")
    _bf16_2d(table, "table")
    V, H = table.shape
    T = ids.shape[0]
    y = torch.empty((T, H), dtype=BF16, device=ids.device) if out is None else out
    _lib.check(_lib.lib().skinny_embed_bf16(ids.data_ptr(), T, table.data_ptr(), V, H, y.data_ptr(),
                                            _lib.stream_of(ids)), "embed")
    return y


def dequant(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor) -> torch.Tensor:
    """MLX W4 g64 -> fp32 [N, K] (q*s + b in fp32)."""
    n, kp = w.shape
    k = kp * 8
    out = torch.empty((n, k), dtype=torch.float32, device=w.device)
    _lib.check(_lib.lib().skinny_w4g64_dequant(w.data_ptr(), scales.data_ptr(), biases.data_ptr(), out.data_ptr(), n, k,
                                               _lib.stream_of(w)), "dequant")
    return out


def qk_rope_store(qkv: torch.Tensor, n_q: int, n_kv: int, head_dim: int, q_norm, k_norm, eps: float,
                  pos: torch.Tensor, theta: float, k_cache: torch.Tensor, vt_cache: torch.Tensor,
                  tree: torch.Tensor | None = None) -> torch.Tensor:
    """Per-head q/k RMSNorm + RoPE; k, v into the caches at slots pos[0] + t; returns q [T, Hq, D].
    Token t is rotated to position pos[0] + t, or as the draft-tree descriptor `tree` says."""
    _bf16_2d(qkv, "qkv")
    T = qkv.shape[0]
    maxlen = k_cache.shape[1]
    q = torch.empty((T, n_q, head_dim), dtype=BF16, device=qkv.device)
    _lib.check(_lib.lib().skinny_qk_rope_store(qkv.data_ptr(), qkv.stride(0), T, n_q, n_kv, head_dim, _lib.ptr(q_norm),
                                               _lib.ptr(k_norm), eps, pos.data_ptr(), theta, _lib.ptr(tree),
                                               q.data_ptr(), k_cache.data_ptr(), vt_cache.data_ptr(), maxlen,
                                               _lib.stream_of(qkv)), "qk_rope_store")
    return q


def attn_workspace_bytes(n_kv: int, maxlen: int) -> int:
    return int(_lib.lib().skinny_attn_workspace_bytes(n_kv, maxlen))


def attn_workspace(n_kv: int, maxlen: int, device) -> torch.Tensor:
    """The attention workspace (chunk partials) for n_kv kv heads over maxlen cache slots. One
    workspace serves one stream's calls; calls on different streams need their own."""
    return torch.empty(max(attn_workspace_bytes(n_kv, maxlen) // 4, 1), dtype=torch.float32, device=device)


def attention(q: torch.Tensor, k_cache: torch.Tensor, vt_cache: torch.Tensor, pos: torch.Tensor, scale: float,
              workspace: torch.Tensor, tree: torch.Tensor | None = None) -> torch.Tensor:
    """GQA attention of q [T, Hq, D] over the cache (causal, or as the draft-tree descriptor
    `tree` says) -> [T, Hq*D] bf16."""
    T, Hq, D = q.shape
    Hkv, maxlen, _ = k_cache.shape
    out = torch.empty((T, Hq * D), dtype=BF16, device=q.device)
    _lib.check(_lib.lib().skinny_attention_bf16(q.data_ptr(), T, Hq, Hkv, D, k_cache.data_ptr(), vt_cache.data_ptr(),
                                                maxlen, pos.data_ptr(), scale, _lib.ptr(tree), workspace.data_ptr(),
                                                workspace.numel() * workspace.element_size(), out.data_ptr(),
                                                _lib.stream_of(q)), "attention")
    return out


def rope_table(theta: float, positions: int, device) -> torch.Tensor:
    """fp32 [positions, 64, 2]: (cos, sin) of rotate-half RoPE at every position."""
    table = torch.empty((positions, 64, 2), dtype=torch.float32, device=device)
    _lib.check(_lib.lib().skinny_rope_table(theta, positions, table.data_ptr(), _lib.stream_of(table)), "rope_table")
    return table


def rope_table_dim(theta: float, rotary_dim: int, positions: int, device) -> torch.Tensor:
    """fp32 [positions, rotary_dim / 2, 2] (cos, sin) of a RoPE over the first rotary_dim dims."""
    t = torch.empty((positions, rotary_dim // 2, 2), dtype=torch.float32, device=device)
    _lib.check(_lib.lib().skinny_rope_table_dim(theta, rotary_dim, positions, t.data_ptr(), _lib.stream_of(t)),
               "rope_table_dim")
    return t


def attn_general_workspace(n_q: int, n_kv: int, head_dim: int, maxlen: int, device) -> torch.Tensor:
    """Workspace of attention_general (normalised queries and chunk partials)."""
    nbytes = int(_lib.lib().skinny_attn_general_workspace_bytes(n_q, n_kv, head_dim, maxlen))
    return torch.empty(max((nbytes + 3) // 4, 64), dtype=torch.float32, device=device)


def attention_general(qkv: torch.Tensor, n_q: int, n_kv: int, head_dim: int, q_stride: int, k_offset: int,
                      v_offset: int, gate_offset: int | None, q_norm, k_norm, eps: float, rotary_dim: int,
                      table: torch.Tensor, pos: torch.Tensor, k_cache: torch.Tensor, vt_cache: torch.Tensor,
                      scale: float, workspace: torch.Tensor, tree: torch.Tensor | None = None) -> torch.Tensor:
    """Attention for head layouts the 128-dim kernels do not take (skinny_attention_general_bf16):
    head_dim 64/128/256, RoPE over the first rotary_dim dims (`table` from rope_table_dim), query
    head h at column h * q_stride of the raw q|k|v rows [T, ldq], key / value head j at k_offset /
    v_offset + j * head_dim, and with gate_offset the output multiplied by sigmoid of the gate at
    gate_offset + h * q_stride -> [T, Hq * D] bf16; the new keys and values go into the caches."""
    _bf16_2d(qkv, "qkv")
    T = qkv.shape[0]
    maxlen = k_cache.shape[1]
    _req(table.dim() == 3 and table.shape[1] * 2 == rotary_dim and table.dtype == torch.float32,
         f"table must be a rope_table_dim table for rotary_dim={rotary_dim}")
    out = torch.empty((T, n_q * head_dim), dtype=BF16, device=qkv.device)
    _lib.check(_lib.lib().skinny_attention_general_bf16(
        qkv.data_ptr(), qkv.stride(0), T, n_q, n_kv, head_dim, q_stride, k_offset, v_offset,
        -1 if gate_offset is None else gate_offset, _lib.ptr(q_norm), _lib.ptr(k_norm), eps, rotary_dim,
        table.data_ptr(), table.shape[0], pos.data_ptr(), _lib.ptr(tree), k_cache.data_ptr(), vt_cache.data_ptr(),
        maxlen, scale, workspace.data_ptr(), workspace.numel() * workspace.element_size(), out.data_ptr(),
        _lib.stream_of(qkv)), "attention_general")
    return out


def attention_fused(qkv: torch.Tensor, n_q: int, n_kv: int, head_dim: int, q_norm, k_norm, eps: float,
                    table: torch.Tensor, pos: torch.Tensor, k_cache: torch.Tensor, vt_cache: torch.Tensor,
                    scale: float, workspace: torch.Tensor, tree: torch.Tensor | None = None) -> torch.Tensor:
    """qk_rope_store + attention in one fewer launch: from raw q|k|v rows [T, (Hq+2Hkv)*D] ->
    [T, Hq*D] bf16; the new keys and values go into the caches."""
    _bf16_2d(qkv, "qkv")
    T = qkv.shape[0]
    maxlen = k_cache.shape[1]
    out = torch.empty((T, n_q * head_dim), dtype=BF16, device=qkv.device)
    _lib.check(_lib.lib().skinny_attention_fused_bf16(
        qkv.data_ptr(), qkv.stride(0), T, n_q, n_kv, head_dim, _lib.ptr(q_norm), _lib.ptr(k_norm), eps,
        table.data_ptr(), table.shape[0], pos.data_ptr(), _lib.ptr(tree), k_cache.data_ptr(), vt_cache.data_ptr(),
        maxlen, scale, workspace.data_ptr(), workspace.numel() * workspace.element_size(), out.data_ptr(),
        _lib.stream_of(qkv)), "attention_fused")
    return out


_QKV_ATTN_OK: dict = {}


def qkv_attention_supported(k: int, n: int, n_kv: int, maxlen: int) -> bool:
    """Whether qkv_attention_fused runs for a (K, N) projection over Hkv heads and a maxlen cache
    (a fused kernel for the table's tile, and the launch fits on the GPU at once); cached."""
    key = (k, n, n_kv, maxlen)
    if key not in _QKV_ATTN_OK:
        rc = _lib.lib().skinny_qkv_attention_supported(k, n, n_kv, maxlen)
        if rc < 0:
            _lib.check(rc, "qkv_attention_supported")
        _QKV_ATTN_OK[key] = rc == 1
    return _QKV_ATTN_OK[key]


def qkv_attention_fused(x: torch.Tensor, packed: torch.Tensor, n_q: int, n_kv: int, head_dim: int, q_norm, k_norm,
                        eps: float, table: torch.Tensor, pos: torch.Tensor, k_cache: torch.Tensor,
                        vt_cache: torch.Tensor, scale: float, workspace: torch.Tensor, handoff: torch.Tensor,
                        tree: torch.Tensor | None = None) -> torch.Tensor:
    """attention_fused(skinny_qmm(x, packed), ...) in one launch plus the chunk merge
    (skinny_qkv_attention_fused_bf16): x [T, K] bf16 rows, `packed` the q|k|v projection's
    skinny_w4g64_pack buffer. The q|k|v rows pass through `handoff` (int16 [>= T, >= N], every
    word -1 before the call and after it) -> [T, Hq*D] bf16; the new keys and values go into the
    caches."""
    _bf16_2d(x, "x")
    T, k = x.shape
    n = packed.shape[0]
    _req(handoff.dtype == torch.int16 and handoff.dim() == 2 and handoff.is_contiguous()
         and handoff.shape[0] >= T and handoff.shape[1] >= n, f"handoff must be contiguous int16 [>= {T}, >= {n}]")
    maxlen = k_cache.shape[1]
    out = torch.empty((T, n_q * head_dim), dtype=BF16, device=x.device)
    _lib.check(_lib.lib().skinny_qkv_attention_fused_bf16(
        x.data_ptr(), T, k, x.stride(0), packed.data_ptr(), n, handoff.data_ptr(), handoff.stride(0), n_q, n_kv,
        head_dim, _lib.ptr(q_norm), _lib.ptr(k_norm), eps, table.data_ptr(), table.shape[0], pos.data_ptr(),
        _lib.ptr(tree), k_cache.data_ptr(), vt_cache.data_ptr(), maxlen, scale, workspace.data_ptr(),
        workspace.numel() * workspace.element_size(), out.data_ptr(), _lib.stream_of(x)), "qkv_attention_fused")
    return out


def attention_fused_noalloc(qkv: torch.Tensor, n_q: int, n_kv: int, head_dim: int, q_norm, k_norm, eps: float,
                            table: torch.Tensor, pos: torch.Tensor, k_cache: torch.Tensor, vt_cache: torch.Tensor,
                            scale: float, tree: torch.Tensor | None = None,
                            out: torch.Tensor | None = None) -> torch.Tensor:
    """attention_fused with its chunk partials in the library's own device array instead of a
    workspace (skinny_attention_fused_noalloc_bf16): with `out` given, the call allocates nothing.
    At most n_kv * maxlen / 128 = 256 chunk pairs."""
    _bf16_2d(qkv, "qkv")
    T = qkv.shape[0]
    maxlen = k_cache.shape[1]
    if out is None:
        out = torch.empty((T, n_q * head_dim), dtype=BF16, device=qkv.device)
    _req(out.dtype == BF16 and tuple(out.shape) == (T, n_q * head_dim) and out.is_contiguous(),
         f"out must be contiguous bf16 [{T}, {n_q * head_dim}]")
    _lib.check(_lib.lib().skinny_attention_fused_noalloc_bf16(
        qkv.data_ptr(), qkv.stride(0), T, n_q, n_kv, head_dim, _lib.ptr(q_norm), _lib.ptr(k_norm), eps,
        table.data_ptr(), table.shape[0], pos.data_ptr(), _lib.ptr(tree), k_cache.data_ptr(), vt_cache.data_ptr(),
        maxlen, scale, out.data_ptr(), _lib.stream_of(qkv)), "attention_fused_noalloc")
    return out


def gdn_conv_silu(x: torch.Tensor, conv_state: torch.Tensor, weight: torch.Tensor,
                  window: torch.Tensor | None, parent: torch.Tensor | None = None) -> torch.Tensor:
    """silu(causal conv over [conv_state; x]); conv_state advanced in place; window keeps the input.
    With a draft tree's `parent` array, each token's window follows its ancestors instead."""
    _req(x.dtype == BF16 and x.dim() == 2 and x.stride(1) == 1, "x must be bf16 [T, C] rows")
    T, C = x.shape
    KW = weight.shape[1]
    out = torch.empty((T, C), dtype=BF16, device=x.device)
    _lib.check(_lib.lib().skinny_gdn_conv_silu(x.data_ptr(), x.stride(0), T, C, KW, conv_state.data_ptr(),
                                               weight.data_ptr(), out.data_ptr(), C, _lib.ptr(window), _lib.ptr(parent),
                                               _lib.stream_of(x)), "gdn_conv")
    return out


def gdn_recurrence(qkv: torch.Tensor, b: torch.Tensor, a: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor,
                   state: torch.Tensor, states_out: torch.Tensor | None, n_heads: int, dk: int,
                   dv: int, parent: torch.Tensor | None = None, record: torch.Tensor | None = None,
                   n_key_heads: int | None = None) -> torch.Tensor:
    """Gated delta rule over T tokens; state [H, Dv, Dk] fp32 advanced in place -> y fp32 [T, H, Dv].
    With a draft tree's `parent` array, each token continues from its parent's state, and the
    pass keeps either every node's state (states_out) or its update operands (`record`, fp32 of
    gdn_record_words(H) words, for gdn_commit_replay). qkv rows hold q and k of `n_key_heads`
    heads (default: n_heads), each shared by n_heads / n_key_heads value heads, then v of n_heads."""
    T = qkv.shape[0]
    _req(b.stride(0) == a.stride(0), "a and b must share a row stride")
    _req(record is None or (record.dtype == torch.float32 and record.is_contiguous()
                            and record.numel() >= gdn_record_words(n_heads)), "record too small")
    y = torch.empty((T, n_heads, dv), dtype=torch.float32, device=qkv.device)
    _lib.check(_lib.lib().skinny_gdn_recurrence(qkv.data_ptr(), qkv.stride(0), b.data_ptr(), a.data_ptr(), b.stride(0),
                                                A_log.data_ptr(), dt_bias.data_ptr(), state.data_ptr(),
                                                _lib.ptr(states_out), y.data_ptr(), _lib.ptr(parent), T, n_heads,
                                                n_key_heads or n_heads, dk, dv, _lib.ptr(record),
                                                _lib.stream_of(qkv)), "gdn_recurrence")
    return y


def gdn_recurrence_gated(qkv: torch.Tensor, b: torch.Tensor, a: torch.Tensor, A_log: torch.Tensor,
                         dt_bias: torch.Tensor, state: torch.Tensor, z: torch.Tensor, weight: torch.Tensor,
                         eps: float, n_heads: int, dk: int, dv: int, n_key_heads: int | None = None) -> torch.Tensor:
    """One token of gdn_recurrence (no per-token states, no draft tree) with gated_rmsnorm in the
    same launch: state [H, Dv, Dk] fp32 advanced in place -> rmsnorm(y) * weight * silu(z) bf16
    [1, H*Dv], bitwise gdn_recurrence followed by gated_rmsnorm."""
    _req(qkv.shape[0] == 1 and b.shape[0] == 1 and a.shape[0] == 1, "one token")
    _req(z.dtype == BF16 and z.dim() == 2 and z.shape[0] == 1 and z.shape[1] == n_heads * dv and z.stride(1) == 1,
         "z must be bf16 [1, H*Dv]")
    out = torch.empty((1, n_heads * dv), dtype=BF16, device=qkv.device)
    _lib.check(_lib.lib().skinny_gdn_recurrence_gated_bf16(qkv.data_ptr(), qkv.stride(0), b.data_ptr(), a.data_ptr(),
                                                           A_log.data_ptr(), dt_bias.data_ptr(), state.data_ptr(),
                                                           z.data_ptr(), weight.data_ptr(), eps, out.data_ptr(),
                                                           n_heads, n_key_heads or n_heads, dk, dv,
                                                           _lib.stream_of(qkv)),
               "gdn_recurrence_gated")
    return out


def gdn_record_words(n_heads: int) -> int:
    """fp32 words of one layer's draft-tree record (16 nodes)."""
    return int(_lib.lib().skinny_gdn_record_words(n_heads))


def gdn_select(keep: torch.Tensor, fed: int, state_all: torch.Tensor, states_all: torch.Tensor,
               conv_all: torch.Tensor, window_all: torch.Tensor) -> None:
    """Rollback of every GDN layer to `keep` (device int32) of `fed` tokens in one launch."""
    L = state_all.shape[0]
    state_elems = state_all[0].numel()
    conv_rows, C = conv_all.shape[1], conv_all.shape[2]
    _lib.check(_lib.lib().skinny_gdn_select(keep.data_ptr(), fed, L, state_all.data_ptr(), states_all.data_ptr(),
                                            state_elems, states_all[0].numel(), conv_all.data_ptr(),
                                            window_all.data_ptr(), conv_rows, C, window_all[0].numel(),
                                            _lib.stream_of(state_all)), "gdn_select")


def argmax_rows(logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """First-index argmax of each bf16 row -> int32 [rows]."""
    _bf16_2d(logits, "logits")
    rows, V = logits.shape
    pred = torch.empty((rows,), dtype=torch.int32, device=logits.device) if out is None else out
    _lib.check(_lib.lib().skinny_argmax_rows_bf16(logits.data_ptr(), rows, V, logits.stride(0), pred.data_ptr(),
                                                  _lib.stream_of(logits)), "argmax")
    return pred


def accept(pred: torch.Tensor, draft: torch.Tensor | None, out: torch.Tensor) -> torch.Tensor:
    """out[0] = n, out[1] = bonus pred[n], out[2] = keep = n + 1, for k = len(draft) drafts."""
    k = 0 if draft is None else draft.numel()
    _lib.check(_lib.lib().skinny_accept(pred.data_ptr(), _lib.ptr(draft), k, out.data_ptr(), _lib.stream_of(pred)),
               "accept")
    return out


def _int32_vec(t: torch.Tensor, name: str, n: int = 1) -> None:
    _req(t.is_cuda and t.dtype == torch.int32 and t.is_contiguous() and t.numel() >= n,
         f"{name} must be a contiguous int32 GPU tensor of at least {n} elements")


def spec_commit(result: torch.Tensor, pos: torch.Tensor, pred: torch.Tensor, tokens: torch.Tensor,
                count: torch.Tensor, nxt: torch.Tensor, path: bool = False) -> None:
    """After `accept` (or `tree_accept`, path=True) over fed = len(pred) verify rows, with
    keep = result[2]: pos += keep - fed, tokens[count : count + keep] = pred[:keep] (path: pred
    at the path's nodes result[3 : 3 + keep]; slots past len(tokens) dropped), count += keep,
    nxt[0] = the bonus result[1]. All device side."""
    fed = pred.numel()
    for t, name, n in ((result, "result", 3 + (fed if path else 0)), (pos, "pos", 1), (pred, "pred", fed),
                       (tokens, "tokens", 0), (count, "count", 1), (nxt, "next", 1)):
        _int32_vec(t, name, n)
    sel = result.data_ptr() + 12 if path else None
    _lib.check(_lib.lib().skinny_spec_commit(result.data_ptr(), fed, pos.data_ptr(), pred.data_ptr(), sel,
                                             tokens.data_ptr(), count.data_ptr(), tokens.numel(), nxt.data_ptr(),
                                             _lib.stream_of(pred)), "spec_commit")


def spec_select_row(result: torch.Tensor, pos: torch.Tensor, rows: torch.Tensor, out: torch.Tensor) -> None:
    """out[0] = rows[result[2] - 1] (bf16 [fed, H] rows) and pos += result[2] - fed, device side."""
    _bf16_2d(rows, "rows")
    fed, H = rows.shape
    _req(out.is_cuda and out.dtype == BF16 and out.is_contiguous() and out.numel() == H,
         f"spec_select_row: out must be {H} contiguous bf16 values")
    _int32_vec(result, "result", 3)
    _int32_vec(pos, "pos", 1)
    _lib.check(_lib.lib().skinny_spec_select_row(result.data_ptr(), fed, pos.data_ptr(), rows.data_ptr(),
                                                 rows.stride(0), H, out.data_ptr(), _lib.stream_of(rows)),
               "spec_select_row")


def gdn_commit(path: torch.Tensor, max_nodes: int, state_all: torch.Tensor, states_all: torch.Tensor,
               conv_all: torch.Tensor, window_all: torch.Tensor) -> None:
    """Every GDN layer to the accepted draft-tree path (path[0] = nodes kept, then the nodes)."""
    L = state_all.shape[0]
    conv_rows, C = conv_all.shape[1], conv_all.shape[2]
    _lib.check(_lib.lib().skinny_gdn_commit(path.data_ptr(), max_nodes, L, state_all.data_ptr(), states_all.data_ptr(),
                                            state_all[0].numel(), states_all[0].numel(), conv_all.data_ptr(),
                                            window_all.data_ptr(), conv_rows, C, window_all[0].numel(),
                                            _lib.stream_of(state_all)), "gdn_commit")


def gdn_commit_replay(path: torch.Tensor, n_heads: int, state_all: torch.Tensor, record_all: torch.Tensor,
                      conv_all: torch.Tensor, window_all: torch.Tensor) -> None:
    """gdn_commit from the tree pass's records (record_all [L, >= gdn_record_words(H)] fp32):
    every GDN layer's state advanced through the accepted path's nodes, bitwise the leaf's state."""
    L = state_all.shape[0]
    conv_rows, C = conv_all.shape[1], conv_all.shape[2]
    _lib.check(_lib.lib().skinny_gdn_commit_replay(path.data_ptr(), L, n_heads, state_all.data_ptr(),
                                                   record_all.data_ptr(), record_all[0].numel(), conv_all.data_ptr(),
                                                   window_all.data_ptr(), conv_rows, C, window_all[0].numel(),
                                                   _lib.stream_of(state_all)), "gdn_commit_replay")


def kv_commit(path: torch.Tensor, pos: torch.Tensor, pos_back: int, k_all: torch.Tensor, vt_all: torch.Tensor) -> None:
    """Every attention layer's accepted path into consecutive slots from pos[0] - pos_back
    (k_all, vt_all: [L, Hkv, ...])."""
    L, Hkv, maxlen, D = k_all.shape
    _lib.check(_lib.lib().skinny_kv_commit(path.data_ptr(), pos.data_ptr(), pos_back, k_all.data_ptr(), vt_all.data_ptr(),
                                           L, Hkv, maxlen, D, k_all[0].numel(), _lib.stream_of(k_all)), "kv_commit")


def tree_accept(pred: torch.Tensor, tokens: torch.Tensor, parent: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out = [n, bonus, n + 1, path nodes ...] of the greedy walk down the draft tree."""
    M = tokens.numel()
    _req(out.numel() >= 3 + M, "tree_accept: out too small")
    _lib.check(_lib.lib().skinny_tree_accept(pred.data_ptr(), tokens.data_ptr(), parent.data_ptr(), M, out.data_ptr(),
                                             _lib.stream_of(pred)), "tree_accept")
    return out


def topk_rows(logits: torch.Tensor, k: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """Indices of the k largest values per bf16 row (decreasing, ties by index) -> int32 [rows, k]."""
    _bf16_2d(logits, "logits")
    rows, V = logits.shape
    idx = torch.empty((rows, k), dtype=torch.int32, device=logits.device) if out is None else out
    _lib.check(_lib.lib().skinny_topk_rows_bf16(logits.data_ptr(), rows, V, logits.stride(0), k, idx.data_ptr(),
                                                _lib.stream_of(logits)), "topk")
    return idx


def quantized_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor) -> torch.Tensor:
    """The unpatched linear: x [..., K] . dequant(w)^T in fp32 (fp32 weights, fp32 GEMM), rounded
    once to x's dtype — the semantics of mx.quantized_matmul(transpose=True)."""
    k = x.shape[-1]
    wd = dequant(w, scales, biases)
    y = x.reshape(-1, k).float() @ wd.t()
    return y.to(x.dtype).reshape(*x.shape[:-1], w.shape[0])


def random_uniform(seed: int, counter: torch.Tensor, n: int, offset: int = 0, rng_stream: int = 0) -> torch.Tensor:
    """float32 [n]: the Philox uniforms of counters *counter + offset + i (device int64 counter)."""
    _req(counter.dtype == torch.int64 and counter.numel() >= 1, "counter must be a device int64 tensor")
    out = torch.empty((n,), dtype=torch.float32, device=counter.device)
    _lib.check(_lib.lib().skinny_random_uniform(seed & (2 ** 64 - 1), counter.data_ptr(), offset, n, rng_stream,
                                                out.data_ptr(), _lib.stream_of(counter)), "random_uniform")
    return out


def row_stats(logits: torch.Tensor, temperature: float, out: torch.Tensor | None = None) -> torch.Tensor:
    """float32 [rows, 2]: (max, sum exp((x - max) / T)) per bf16 row."""
    _bf16_2d(logits, "logits")
    rows, V = logits.shape
    stats = torch.empty((rows, 2), dtype=torch.float32, device=logits.device) if out is None else out
    _lib.check(_lib.lib().skinny_row_stats_bf16(logits.data_ptr(), rows, V, logits.stride(0), 1.0 / temperature,
                                                stats.data_ptr(), _lib.stream_of(logits)), "row_stats")
    return stats


def sample_rows(logits: torch.Tensor, temperature: float, seed: int, counter: torch.Tensor, offset: int = 0,
                rng_stream: int = 0, out: torch.Tensor | None = None) -> torch.Tensor:
    """int32 [rows]: a sample of softmax(row / T) per bf16 row (row r uses counter *counter + offset + r)."""
    _bf16_2d(logits, "logits")
    _req(counter.dtype == torch.int64, "counter must be a device int64 tensor")
    rows, V = logits.shape
    toks = torch.empty((rows,), dtype=torch.int32, device=logits.device) if out is None else out
    _lib.check(_lib.lib().skinny_sample_rows_bf16(logits.data_ptr(), rows, V, logits.stride(0), 1.0 / temperature,
                                                  seed & (2 ** 64 - 1), counter.data_ptr(), offset, rng_stream,
                                                  toks.data_ptr(), _lib.stream_of(logits)), "sample_rows")
    return toks


def spec_accept_sampled(target: torch.Tensor, stats_t: torch.Tensor, drafts: torch.Tensor, temperature: float,
                        seed: int, counter: torch.Tensor, out: torch.Tensor, draft: torch.Tensor | None = None,
                        stats_d: torch.Tensor | None = None) -> torch.Tensor:
    """out = [n accepted, emitted token, n + 1] of one speculative step with rejection sampling."""
    _bf16_2d(target, "target")
    K = drafts.numel()
    _req(target.shape[0] >= K + 1, "target needs K + 1 rows")
    _req(draft is None or (draft.shape[0] >= K and stats_d is not None), "draft rows need their stats")
    Vd = 0 if draft is None else draft.shape[1]
    _lib.check(_lib.lib().skinny_spec_accept_sampled(
        target.data_ptr(), target.stride(0), stats_t.data_ptr(), _lib.ptr(draft),
        0 if draft is None else draft.stride(0), _lib.ptr(stats_d), Vd, drafts.data_ptr(), K, target.shape[1],
        1.0 / temperature, seed & (2 ** 64 - 1), counter.data_ptr(), out.data_ptr(), _lib.stream_of(target)),
        "spec_accept_sampled")
    return out
