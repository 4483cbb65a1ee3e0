"""Drop-in patch for the decoders: skinny qmm for every W4 g64 linear + horizontal fusion.

Same call surface as the reference module (skinny_mlx/patch.py:22-115): `SKINNY_RANGE`,
`FUSE_GROUPS`, `SkinnyQuantizedLinear`, `FusedSliceLinear`, `patch_model(model, fuse=True)`
returning {"fused_groups", "single", "heads"}.

1. Skinny routing. Token counts M in SKINNY_RANGE run the gfx950 skinny kernel on weights
   packed once at patch time; the reference keeps M = 1..5 on MLX's qmv (patch.py:3-4), here
   M = 1..16 all take the skinny kernel so that a token's output is bitwise the same for any M
   (speculative verify then reproduces single-token decoding exactly). Outside the range the
   unpatched semantics run (fp32 dequantise + GEMM); M > 16 inside the range runs in 16-row pieces.
2. Horizontal fusion. Projections that read the same input (GDN qkv/z/b/a, attention q/k/v,
   MLP gate/up) are concatenated along N at patch time and run as one matmul; siblings return
   slices of the cached result, matched by input identity (patch.py:52-77), so model code is
   untouched. The fused GDN projection is N = 6144 + 2048 + 16 + 16 = 8224.

Like the reference prototype, both layouts stay resident (originals + packed).
"""

from __future__ import annotations

import torch
from torch import nn

from .model import QuantizedLinear
from .qmm import GROUP, repack_for_skinny, skinny_qmm

SKINNY_RANGE = (1, 16)
FUSE_GROUPS = [
    ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a"),  # Gated DeltaNet mixer
    ("q_proj", "k_proj", "v_proj"),                          # full attention
    ("gate_proj", "up_proj"),                                # MLP
]


def _fallback(x: torch.Tensor, w, s, b) -> torch.Tensor:
    from . import kernels as K

    return K.quantized_matmul(x, w, s, b)


def _qmm(x: torch.Tensor, w, s, b, rw) -> torch.Tensor:
    """Route by token count (reference patch.py:30-35)."""
    k = x.shape[-1]
    m = x.numel() // k
    lo, hi = SKINNY_RANGE
    # M > 16 runs as 16-row pieces, so it takes the skinny kernel whenever 16 is in range
    if lo <= m <= hi or (m > 16 and lo <= 16 <= hi):
        return skinny_qmm(x.reshape(m, k), rw).reshape(*x.shape[:-1], -1)
    return _fallback(x, w, s, b)


class SkinnyQuantizedLinear(nn.Module):
    def __init__(self, ql: QuantizedLinear):
        super().__init__()
        self.group_size, self.bits = ql.group_size, ql.bits
        self.in_features, self.out_features = ql.in_features, ql.out_features
        self.weight, self.scales, self.biases = ql.weight, ql.scales, ql.biases
        self.rweight = repack_for_skinny(ql.weight, ql.scales, ql.biases)
        self.bias = getattr(ql, "bias", None)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = _qmm(x, self.weight, self.scales, self.biases, self.rweight)
        return y + self.bias if self.bias is not None else y


class _FusedGroup:
    """Concatenated weights of same-input projections + a one-entry result cache."""

    def __init__(self, qls: list[QuantizedLinear]):
        self.group_size, self.bits = qls[0].group_size, qls[0].bits
        self.w = torch.cat([q.weight for q in qls])
        self.s = torch.cat([q.scales for q in qls])
        self.b = torch.cat([q.biases for q in qls])
        self.rw = repack_for_skinny(self.w, self.s, self.b)
        sizes = [q.weight.shape[0] for q in qls]
        self.bounds = [(sum(sizes[:i]), sum(sizes[: i + 1])) for i in range(len(sizes))]
        self.x = self.y = None

    def output(self, x: torch.Tensor) -> torch.Tensor:
        if self.x is not x:  # strong ref held, so identity can't be recycled
            self.x, self.y = x, _qmm(x, self.w, self.s, self.b, self.rw)
        return self.y


class FusedSliceLinear(nn.Module):
    def __init__(self, group: _FusedGroup, idx: int):
        super().__init__()
        self._group, (self._lo, self._hi) = group, group.bounds[idx]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self._group.output(x)[..., self._lo:self._hi]


def _ok(m) -> bool:
    """Eligible: a 4-bit, group-64 QuantizedLinear without bias (reference patch.py:80-81)."""
    return (isinstance(m, QuantizedLinear) and m.bits == 4 and m.group_size == GROUP
            and getattr(m, "bias", None) is None and m.out_features % 16 == 0 and m.in_features % 128 == 0)


def patch_model(model: nn.Module, fuse: bool = True) -> dict:
    """Patch in place. Returns counts of fused groups, single swaps, and patched tied heads."""
    stats = {"fused_groups": 0, "single": 0, "heads": 0}
    fused_ids = set()
    if fuse:
        for _, parent in list(model.named_modules()):
            children = dict(parent.named_children())
            for names in FUSE_GROUPS:
                if all(_ok(children.get(n)) for n in names):
                    group = _FusedGroup([children[n] for n in names])
                    for i, n in enumerate(names):
                        fused_ids.add(id(children[n]))
                        setattr(parent, n, FusedSliceLinear(group, i))
                    stats["fused_groups"] += 1
    for _, parent in list(model.named_modules()):
        for n, child in list(parent.named_children()):
            if _ok(child) and id(child) not in fused_ids:
                setattr(parent, n, SkinnyQuantizedLinear(child))
                stats["single"] += 1
    # The decoders here keep bf16 embeddings and an untied W4 lm_head (counted under
    # "single"); the reference's tied 4-bit embedding head (patch.py:84-87, 111-114) has no
    # counterpart to patch, so "heads" stays 0.
    return stats
