"""Replay-free rollback for hybrid (Gated DeltaNet + attention) caches.

Same call surface as the reference (skinny_mlx/rollback.py:19-73): `HybridRollback.for_model(
model)`, `.record()` right before the verify forward, `.rollback(cache, fed, keep)` after it.

Speculative verify feeds `fed` tokens; only the first `keep` are accepted. Attention KV
caches just trim. The reference records the GDN recurrence inputs and re-runs the
recurrence over the accepted prefix (rollback.py:4-9, 64-68). Here the recording forward
stores every per-token state S_1..S_fed of every GDN layer in HBM (plus the conv inputs),
and rollback selects S_keep and the conv window rows keep .. keep+2 on the device, for all
layers in one launch — no replay. The selected state is bitwise the state a forward over
only the first `keep` tokens would have produced (the recurrence is token-sequential).
"""

from __future__ import annotations

import torch

from . import kernels as K
from .cache import KVCache, PromptCache


class HybridRollback:
    @classmethod
    def for_model(cls, model) -> "HybridRollback":
        """One instance per model (reference rollback.py:20-25)."""
        if getattr(model, "_skinny_rollback", None) is None:
            model._skinny_rollback = cls(model)
        return model._skinny_rollback

    def __init__(self, model):
        self.model = model
        self.layers = model.layers
        self.gdn_idx = [i for i, l in enumerate(self.layers) if getattr(l, "is_linear", False)]
        self._keep = None

    @property
    def recording(self) -> bool:
        return self.model.recorder.recording

    def record(self) -> None:
        """Arm recording: the next forward keeps every GDN layer's per-token states and conv
        inputs. Call it immediately before the verify pass."""
        self.model.recorder.recording = True

    def rollback(self, cache: PromptCache, fed: int, keep: int, keep_device: torch.Tensor | None = None) -> None:
        """Shrink `cache` from the `fed` tokens of the last verify pass to its first `keep`.

        keep == fed changes nothing; otherwise 1 <= keep < fed. `keep_device` may hold the same
        count on the device already (the acceptance kernel's output), which saves an upload."""
        self.model.recorder.recording = False
        if keep == fed:
            return
        if not (1 <= keep < fed):
            raise ValueError(f"rollback: keep={keep} must be in [1, fed={fed})")
        if self.gdn_idx:
            gb = cache.shared.gdn
            if gb.recorded != fed:
                raise RuntimeError(f"rollback: the last recording forward fed {gb.recorded} tokens, not {fed}")
            if keep_device is None:
                if self._keep is None or self._keep.device != gb.state.device:
                    self._keep = torch.zeros(1, dtype=torch.int32, device=gb.state.device)
                self._keep.fill_(keep)
                keep_device = self._keep
            K.gdn_select(keep_device, fed, gb.state, gb.states, gb.conv, gb.window)
        for li, c in enumerate(cache):
            if isinstance(c, KVCache):
                c.trim(fed - keep)
