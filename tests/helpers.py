"""Shared helpers for the tests: seeded synthetic inputs and tensor <-> numpy bit views."""

import numpy as np
import torch

from skinny_mlx.qmm import random_w4g64


def bits16(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor (any device) -> numpy uint16 bit patterns."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def u32(t: torch.Tensor) -> np.ndarray:
    """int32 packed words (any device) -> numpy uint32."""
    return t.detach().cpu().contiguous().numpy().view(np.uint32)


def qmm_case(m: int, n: int, k: int, seed: int = 0):
    """Seeded CPU inputs of the benchmark distributions: x ~ N(0,1) bf16, q ~ U{0..15},
    s = |N(0, 0.02)| bf16, b = -8 s."""
    g = torch.Generator().manual_seed(seed)
    w, s, b = random_w4g64(n, k, generator=g)
    x = torch.randn((m, k), generator=g).to(torch.bfloat16)
    return x, w, s, b


def state_numpy(model) -> dict:
    """Model buffers as numpy for the oracle: bf16 -> uint16 bits, packs -> uint32, fp32 -> fp64."""
    out = {}
    for name, t in model.state_dict().items():
        t = t.detach().cpu().contiguous()
        if t.dtype == torch.bfloat16:
            out[name] = t.view(torch.int16).numpy().view(np.uint16)
        elif t.dtype == torch.int32:
            out[name] = t.numpy().view(np.uint32)
        else:
            out[name] = t.double().numpy()
    return out


def model_cfg(model) -> dict:
    import dataclasses

    return dataclasses.asdict(model.args)


def near_tie_ok(ref_logits: np.ndarray, got_logits: np.ndarray, ulps: int = 2) -> bool:
    """Argmax agreement per row, except where the reference's top-1 / top-2 gap is at most
    `ulps` bf16 ulps of the top logit (the near-tie exception of the path's contract)."""
    for r, g in zip(ref_logits, got_logits):
        a, b = int(np.argmax(r)), int(np.argmax(g))
        if a == b:
            continue
        top = r[a]
        ulp = 2.0 ** (np.floor(np.log2(abs(top))) - 7) if top != 0 else 2.0 ** -133
        if r[a] - r[b] > ulps * ulp:
            return False
    return True
