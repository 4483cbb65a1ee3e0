"""In-place patch of a decoder: W4 g64 linears run the gfx950 skinny kernel, and projections
that read the same input run as one wider matmul.

Call surface kept from the reference module (skinny_mlx/patch.py:22-115): `SKINNY_RANGE`,
`FUSE_GROUPS`, `SkinnyQuantizedLinear`, `FusedSliceLinear`, and
`patch_model(model, fuse=True)` returning {"fused_groups", "single", "heads"}.

How it works here:

* Routing by token count. A call with M tokens in SKINNY_RANGE runs the skinny kernel on the
  weights packed at patch time; M > 16 runs as 16-row pieces when 16 is in the range; anything
  else keeps the unpatched semantics (fp32 dequantise + GEMM, what mx.quantized_matmul computes
  for the reference outside its range, patch.py:30-35). The default range is 1..16 rather than
  the reference's 6..16: the skinny kernel is the only path whose output for a token does not
  depend on M, which is what makes a K-token verify reproduce single-token decoding exactly.
* Fusion. A module whose children named in one FUSE_GROUPS entry are all eligible gets one
  `_Projection` holding their weights concatenated along N; each child is replaced by a
  `FusedSliceLinear` that returns its column range of the projection's output. The projection
  remembers its last input — by identity AND torch's in-place version counter, since torch
  tensors, unlike MLX arrays, can change under the same identity — so the siblings that follow
  reuse one matmul and the model code stays untouched.
* gate_proj/up_proj are packed in the gate|up tile order of `skinny_glu`, whose epilogue can
  also apply the SwiGLU activation: models that ask the slices for `swiglu(x)` get silu(gate) * up
  from one launch, bitwise equal to the separate activation of the two slices.

Like the reference prototype, the MLX-format weights stay resident next to the packed ones
(the unpatched fallback reads them).
"""

from __future__ import annotations

import torch
from torch import nn

from . import kernels as K
from .model import QuantizedLinear
from .qmm import (GROUP, MAX_M, NORMIN_CONV, NORMIN_PLAIN, NORMIN_SWIGLU, gated_partial_supported, mlp_fused_buffers,
                  mlp_fused_supported, normin_supported, packed_k, repack_for_skinny, repack_gate_up, skinny_glu,
                  skinny_glu_normin, skinny_mlp_fused_partial, skinny_qmm, skinny_qmm_conv, skinny_qmm_conv_normin,
                  skinny_qmm_normin, skinny_qmm_partial, skinny_qmm_partial_gated)

SKINNY_RANGE = (1, 16)
# Token counts up to which a fused projection forms a kernels.NormIn input in its own launch, per
# kind; past them (and for kinds at 0) it takes the separate norm kernel, with the same bits. The
# Gated-DeltaNet input projection (conv epilogue) keeps the separate norm: folded, the hybrid
# one-token step measured 1.352-1.355 against 1.349-1.351 ms. From two tokens on the 4-wave norm-in
# tiles stage the rows by LDS-DMA: folded at M = 2 the 36-layer steps took 2.06 / 1.96 ms (dense /
# hybrid) against 1.46 / 1.44 ms.
NORMIN_TOKENS = {NORMIN_PLAIN: 1, NORMIN_SWIGLU: 1, NORMIN_CONV: 0}
FUSE_GROUPS = [
    ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a"),  # Gated DeltaNet mixer
    ("q_proj", "k_proj", "v_proj"),                          # full attention
    ("gate_proj", "up_proj"),                                # MLP
]
_GATE_UP = ("gate_proj", "up_proj")


def _skinny_ok(m: int) -> bool:
    """Whether an M-token call takes the skinny kernel (M > 16 runs as 16-row pieces)."""
    lo, hi = SKINNY_RANGE
    return lo <= m <= hi or (m > MAX_M and lo <= MAX_M <= hi)


def _tokens(x: torch.Tensor) -> int:
    return x.numel() // x.shape[-1]


def _eligible(m) -> bool:
    """A 4-bit, group-64 QuantizedLinear without bias whose shape the kernel tiles (reference
    eligibility: patch.py:80-81; the kernel adds N % 16 == 0 and K % 128 == 0)."""
    return (isinstance(m, QuantizedLinear) and m.bits == 4 and m.group_size == GROUP
            and getattr(m, "bias", None) is None and m.out_features % 16 == 0 and m.in_features % 128 == 0)


class SkinnyQuantizedLinear(nn.Module):
    """A patched single linear: packed weights for the skinny kernel plus the original ones."""

    def __init__(self, ql: QuantizedLinear):
        super().__init__()
        self.group_size, self.bits = ql.group_size, ql.bits
        self.in_features, self.out_features = ql.in_features, ql.out_features
        self.weight, self.scales, self.biases = ql.weight, ql.scales, ql.biases
        self.bias = getattr(ql, "bias", None)
        self.rweight = repack_for_skinny(ql.weight, ql.scales, ql.biases)

    def forward(self, x) -> torch.Tensor:
        if isinstance(x, K.NormIn):
            x = x.value()
        if _skinny_ok(_tokens(x)):
            y = skinny_qmm(x, self.rweight)
        else:
            y = K.quantized_matmul(x, self.weight, self.scales, self.biases)
        return y if self.bias is None else y + self.bias

    def partial(self, x: torch.Tensor):
        """The output as a kernels.PartialSum (split-K fp32 slices) when the skinny kernel runs
        and the linear has no bias, for a caller that adds it as a residual (kernels.rmsnorm);
        otherwise the ordinary output."""
        if self.bias is None and x.dim() == 2 and _skinny_ok(_tokens(x)):
            return skinny_qmm_partial(x, self.rweight)
        return self(x)

    def partial_gated(self, y: torch.Tensor, z: torch.Tensor, norm_w: torch.Tensor, eps: float):
        """partial(gated_rmsnorm(y, z, norm_w, eps)) with the Gated-DeltaNet output norm formed
        inside the projection's launch (bitwise the two launches), or None where that form does not
        apply: a token count outside the skinny range or past 16, a bias, no kernel for the tile."""
        m = y.shape[0]
        if (self.bias is not None or not 1 <= m <= MAX_M or not _skinny_ok(m)
                or not gated_partial_supported(packed_k(self.rweight), self.rweight.shape[0])):
            return None
        return skinny_qmm_partial_gated(y, z, norm_w, eps, self.rweight)


class _Projection:
    """Same-input linears concatenated along N, with a one-entry cache of the last result."""

    def __init__(self, linears: list[QuantizedLinear], gate_up: bool):
        self.gate_up = gate_up
        self.w = torch.cat([q.weight for q in linears])
        self.s = torch.cat([q.scales for q in linears])
        self.b = torch.cat([q.biases for q in linears])
        self.packed = (repack_gate_up if gate_up else repack_for_skinny)(self.w, self.s, self.b)
        edges = [0]
        for q in linears:
            edges.append(edges[-1] + q.out_features)
        self.columns = [slice(lo, hi) for lo, hi in zip(edges, edges[1:])]
        self._key = None
        self._out = None
        self._mlp_buffers = None  # (act, sync) of the fused MLP launch, made on its first call

    def mlp_partial(self, x, down):
        """The whole MLP — this gate|up projection with SwiGLU, then `down` as split-K slices
        (kernels.PartialSum) — in one launch (skinny_mlp_fused_partial), bitwise the two launches,
        where the fused instance applies: 2..16 tokens in the skinny range and the decoders' shapes.
        Otherwise None."""
        if not self.gate_up or not isinstance(x, torch.Tensor) or x.dim() != 2:
            return None
        rw = getattr(down, "rweight", None)
        if rw is None or getattr(down, "bias", None) is not None or not _skinny_ok(x.shape[0]):
            return None
        k, f, n = packed_k(self.packed), self.packed.shape[0] // 2, rw.shape[0]
        if not mlp_fused_supported(x.shape[0], k, f, n):
            return None
        if self._mlp_buffers is None:
            self._mlp_buffers = mlp_fused_buffers(f, x.device)
        return skinny_mlp_fused_partial(x, self.packed, rw, *self._mlp_buffers)

    def _normin(self, x, kind: int) -> bool:
        """Whether a kernels.NormIn input takes the norm-in form of `kind` (else its value())."""
        return (isinstance(x, K.NormIn) and _skinny_ok(x.shape[0]) and x.shape[0] <= NORMIN_TOKENS.get(kind, 0)
                and normin_supported(kind, x.shape[0], packed_k(self.packed), self.packed.shape[0], x.splits))

    def _compute(self, x) -> torch.Tensor:
        if isinstance(x, K.NormIn):
            if not self.gate_up and self._normin(x, NORMIN_PLAIN):
                return skinny_qmm_normin(x, self.packed)
            x = x.value()
        if not _skinny_ok(_tokens(x)):
            return K.quantized_matmul(x, self.w, self.s, self.b)
        if self.gate_up:
            return skinny_glu(x, self.packed, swiglu=False)
        return skinny_qmm(x, self.packed)

    def output(self, x) -> torch.Tensor:
        version = getattr(x, "_version", 0)
        if self._key is None or self._key[0] is not x or self._key[1] != version:
            self._key, self._out = (x, version), self._compute(x)
        return self._out

    def conv_output(self, x, c: int, conv_state: torch.Tensor, conv_w: torch.Tensor, window=None, parent=None):
        """The output with a Gated-DeltaNet mixer's conv + SiLU applied to its first `c` columns in
        the same launch (qmm.skinny_qmm_conv), or None where that form does not apply (a token count
        outside the skinny range, the gate|up layout)."""
        if self.gate_up or x.dim() != 2 or not 1 <= x.shape[0] <= MAX_M:
            return None
        if not _skinny_ok(x.shape[0]):
            return None
        if isinstance(x, K.NormIn):
            if self._normin(x, NORMIN_CONV):
                return skinny_qmm_conv_normin(x, self.packed, c, conv_state, conv_w, window, parent)
            x = x.value()
        return skinny_qmm_conv(x, self.packed, c, conv_state, conv_w, window, parent)

    def attention_output(self, x, attn: dict):
        """The attention over this q|k|v projection's rows in one launch with the projection
        (kernels.qkv_attention_fused; `attn` holds its attention arguments), or None where that
        form does not apply: a token count outside the skinny range or past 16, the gate|up
        layout, no fused kernel for the table's tile, or a launch too large to be resident."""
        if self.gate_up or x.dim() != 2 or not 1 <= x.shape[0] <= MAX_M or not _skinny_ok(x.shape[0]):
            return None
        handoff = attn["handoff"]
        if handoff is None or not K.qkv_attention_supported(packed_k(self.packed), self.packed.shape[0],
                                                            attn["n_kv"], attn["k_cache"].shape[1]):
            return None
        if isinstance(x, K.NormIn):
            x = x.value()
        return K.qkv_attention_fused(x, self.packed, attn["n_q"], attn["n_kv"], attn["head_dim"], attn["q_norm"],
                                     attn["k_norm"], attn["eps"], attn["table"], attn["pos"], attn["k_cache"],
                                     attn["vt_cache"], attn["scale"], attn["workspace"], handoff, attn["tree"])

    def swiglu(self, x) -> torch.Tensor:
        """silu(gate(x)) * up(x) in one launch (gate|up projections only)."""
        if not self.gate_up:
            raise TypeError("swiglu needs the gate|up projection")
        if isinstance(x, K.NormIn):
            if self._normin(x, NORMIN_SWIGLU):
                return skinny_glu_normin(x, self.packed)
            x = x.value()
        if _skinny_ok(_tokens(x)):
            return skinny_glu(x, self.packed, swiglu=True)
        return K.silu_mul(self.output(x).reshape(-1, self.w.shape[0])).reshape(*x.shape[:-1], -1)


class FusedSliceLinear(nn.Module):
    """One member of a fused projection: its columns of the shared result."""

    def __init__(self, projection: _Projection, index: int):
        super().__init__()
        self.projection = projection
        self.columns = projection.columns[index]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.projection.output(x)[..., self.columns]


def patch_model(model: nn.Module, fuse: bool = True) -> dict:
    """Patch `model` in place; returns counts of fused groups, single swaps and patched tied heads."""
    fused_groups = 0
    taken: set[int] = set()
    if fuse:
        plans = []
        for parent in model.modules():
            kids = dict(parent.named_children())
            for names in FUSE_GROUPS:
                members = [kids.get(n) for n in names]
                if all(_eligible(m) for m in members) and not any(id(m) in taken for m in members):
                    if names == _GATE_UP and (members[0].out_features != members[1].out_features
                                              or members[0].in_features != members[1].in_features):
                        continue
                    taken.update(id(m) for m in members)
                    plans.append((parent, names, members))
        for parent, names, members in plans:
            proj = _Projection(members, gate_up=names == _GATE_UP)
            for i, name in enumerate(names):
                setattr(parent, name, FusedSliceLinear(proj, i))
            fused_groups += 1
    singles = []
    for parent in model.modules():
        for name, child in parent.named_children():
            if _eligible(child) and id(child) not in taken:
                singles.append((parent, name, child))
    for parent, name, child in singles:
        setattr(parent, name, SkinnyQuantizedLinear(child))
    # The decoders here keep bf16 embeddings and an untied W4 lm_head, which is patched (and
    # counted) as a single linear; the reference's tied 4-bit embedding head
    # (patch.py:84-87, 111-114) has no counterpart, so "heads" stays 0.
    return {"fused_groups": fused_groups, "single": len(singles), "heads": 0}
