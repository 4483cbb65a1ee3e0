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
