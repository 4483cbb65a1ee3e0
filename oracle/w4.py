"""MLX affine W4 g64 format and dequant+matmul, restated in numpy (oracle; tests only).

Reference arithmetic:
  * packing: eight 4-bit codes per little-endian uint32, element i at bits 4i — the
    extraction `(a >> (4*i)) & 0xF` of skinny_mlx/qmm.py:104;
  * dequant: w[n,k] = q[n,k]*s[n,k//64] + b[n,k//64] with 64-wide groups along K
    (qmm.py:8-9, 19; patch.py:80-81 accepts only bits=4, group_size=64);
  * result: y = x . dequant(w)^T, the semantics of mx.quantized_matmul(transpose=True)
    that the reference's kernel is checked against (qmm.py:183-186);
  * error metric: max|got - ref| / max|ref| (qmm.py:185).

Pins (tests/test_oracle_w4.py): hand-computed pack/unpack known answers, round trips,
closed forms (one-hot x gives a dequantized column; q=8 with b=-8s gives 0; q=0, b=0 gives
0; x=1 gives the row sums), and bf16 rounding checked against torch's own conversion.

The fragment relayout at the bottom is this build's own format (not the reference's Metal
order); it is pinned by a round trip, the per-word nibble multiset, and an emulation of the
kernel's lane read-out that must reproduce the MLX unpack.
"""

from __future__ import annotations

import numpy as np

GROUP = 64


# --- bf16 as uint16 bit patterns ------------------------------------------------------------

def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """uint16 bf16 bit patterns -> float32 (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> uint16 bf16 bits, round to nearest even; NaN stays a quiet NaN."""
    u = np.ascontiguousarray(np.asarray(x, dtype=np.float32)).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round float values to the nearest bf16, returned as float32."""
    return bf16_to_f32(f32_to_bf16(x))


# --- MLX packing ----------------------------------------------------------------------------

def pack_mlx(q: np.ndarray) -> np.ndarray:
    """uint8 codes [N, K] (0..15) -> uint32 packs [N, K/8], element i at bits 4i."""
    q = np.asarray(q)
    n, k = q.shape
    if k % 8:
        raise ValueError("K must be a multiple of 8")
    if q.min(initial=0) < 0 or q.max(initial=0) > 15:
        raise ValueError("codes must be in 0..15")
    q8 = q.astype(np.uint32).reshape(n, k // 8, 8)
    out = np.zeros((n, k // 8), dtype=np.uint32)
    for i in range(8):
        out |= q8[:, :, i] << np.uint32(4 * i)
    return out


def unpack_mlx(w: np.ndarray) -> np.ndarray:
    """uint32 packs [N, K/8] -> uint8 codes [N, K] (reference qmm.py:104 order)."""
    a = np.asarray(w).view(np.uint32) if np.asarray(w).dtype != np.uint32 else np.asarray(w)
    n, kp = a.shape
    q = np.stack([((a >> np.uint32(4 * i)) & np.uint32(0xF)).astype(np.uint8) for i in range(8)], axis=-1)
    return q.reshape(n, kp * 8)


def as_u32(w) -> np.ndarray:
    """View int32/uint32 words (numpy or CPU torch) as a uint32 numpy array."""
    a = w.numpy() if hasattr(w, "numpy") else np.asarray(w)
    return a.view(np.uint32)


def dequant(w: np.ndarray, s_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    """float64 [N, K] = q*s + b, s and b broadcast over their 64-wide group."""
    q = unpack_mlx(as_u32(w)).astype(np.float64)
    s = bf16_to_f32(s_bits).astype(np.float64)
    b = bf16_to_f32(b_bits).astype(np.float64)
    n, k = q.shape
    if s.shape != (n, k // GROUP) or b.shape != (n, k // GROUP):
        raise ValueError("scales/biases must be [N, K/64]")
    return (q.reshape(n, k // GROUP, GROUP) * s[:, :, None] + b[:, :, None]).reshape(n, k)


def qmm(x_bits: np.ndarray, w: np.ndarray, s_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    """float64 [M, N] = x . dequant(w)^T with bf16 x given as bit patterns."""
    x = bf16_to_f32(x_bits).astype(np.float64)
    return x @ dequant(w, s_bits, b_bits).T


def qmm_affine(x_bits, w, s_bits, b_bits) -> np.ndarray:
    """The same product through the reference's affine identity (qmm.py:8-9):
    sum_g [ s_g * sum_{k in g} x q + b_g * sum_{k in g} x ]."""
    x = bf16_to_f32(x_bits).astype(np.float64)
    q = unpack_mlx(as_u32(w)).astype(np.float64)
    s = bf16_to_f32(s_bits).astype(np.float64)
    b = bf16_to_f32(b_bits).astype(np.float64)
    m, k = x.shape
    n = q.shape[0]
    G = k // GROUP
    xg = x.reshape(m, G, GROUP)
    qg = q.reshape(n, G, GROUP)
    xq = np.einsum("mgk,ngk->mng", xg, qg)
    xs = xg.sum(-1)
    return np.einsum("mng,ng->mn", xq, s) + np.einsum("mg,ng->mn", xs, b)


def rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    """max|got - ref| / max|ref| (reference qmm.py:185)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.abs(ref).max()
    return float(np.abs(got - ref).max() / den) if den > 0 else float(np.abs(got - ref).max())


# --- fragment relayout (this build's format) --------------------------------------------------

def relayout_frag(w: np.ndarray) -> np.ndarray:
    """MLX packs [N, K/8] -> fragment order [N/16][K/64][64 lanes][2 words], reshaped [N, K/8].

    Lane l of tile t, group g, word h holds row 16t + l%16 and columns 64g + 32h + 8(l//16) + e,
    e = 0..7, with element e = 2i at bits 4i and e = 2i+1 at bits 16 + 4i.
    """
    q = unpack_mlx(as_u32(w))
    n, k = q.shape
    if n % 16 or k % GROUP:
        raise ValueError("N must be a multiple of 16 and K of 64")
    T, G = n // 16, k // GROUP
    # k = 64g + 32h + 8quad + e ; row = 16t + r
    q6 = q.reshape(T, 16, G, 2, 4, 8).astype(np.uint32)       # [t, r, g, h, quad, e]
    q6 = q6.transpose(0, 2, 4, 1, 3, 5)                          # [t, g, quad, r, h, e]
    word = np.zeros(q6.shape[:-1], dtype=np.uint32)
    for i in range(4):
        word |= q6[..., 2 * i] << np.uint32(4 * i)
        word |= q6[..., 2 * i + 1] << np.uint32(16 + 4 * i)
    # lane = quad*16 + r  -> [t, g, lane, h]
    return np.ascontiguousarray(word.reshape(T, G, 64, 2)).reshape(n, k // 8)


def unrelayout_frag(wf: np.ndarray) -> np.ndarray:
    """Inverse of relayout_frag."""
    a = as_u32(wf)
    n, kp = a.shape
    k = kp * 8
    T, G = n // 16, k // GROUP
    word = a.reshape(T, G, 4, 16, 2)                              # [t, g, quad, r, h]
    e = np.zeros(word.shape + (8,), dtype=np.uint8)
    for i in range(4):
        e[..., 2 * i] = (word >> np.uint32(4 * i)) & 0xF
        e[..., 2 * i + 1] = (word >> np.uint32(16 + 4 * i)) & 0xF
    q = e.transpose(0, 3, 1, 4, 2, 5).reshape(n, k)              # [t, r, g, h, quad, e]
    return pack_mlx(q)


def lane_operands(wf: np.ndarray, t: int, g: int) -> np.ndarray:
    """Emulates the kernel's read-out of one (tile, group): the B-operand values each lane
    feeds to the two MFMAs after `(w >> 4i) & 0x000F000F | 0x43004300`, decoded as bf16.

    Returns float32 [2 (k half), 64 lanes, 8] holding 128 + q for row 16t + l%16 and columns
    64g + 32h + 8(l//16) + 0..7.
    """
    a = as_u32(wf)
    n, kp = a.shape
    G = kp * 8 // GROUP
    frag = a.reshape(n // 16, G, 64, 2)[t, g]                    # [lane, h]
    out = np.zeros((2, 64, 8), dtype=np.float32)
    for h in range(2):
        w = frag[:, h]
        for i in range(4):
            pair = ((w >> np.uint32(4 * i)) & np.uint32(0x000F000F)) | np.uint32(0x43004300)
            lo = (pair & np.uint32(0xFFFF)).astype(np.uint16)
            hi = (pair >> np.uint32(16)).astype(np.uint16)
            out[h, :, 2 * i] = bf16_to_f32(lo)
            out[h, :, 2 * i + 1] = bf16_to_f32(hi)
    return out
