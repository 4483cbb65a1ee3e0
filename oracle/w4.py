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

The fragment packing at the bottom is skinny_mlx's own format (not the reference's Metal
order); it is pinned by a round trip, the per-tile nibble multiset, and an emulation of the
kernel's lane read-out (nibbles, scales, biases) that must reproduce the MLX values.
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


# --- fragment packing (skinny_mlx's format) ----------------------------------------------------

BLOCK_WORDS = 288  # per (16-row tile, group pair): 256 nibble words + 16 rows x (scales, biases)


def _frag_nibble_words(q: np.ndarray) -> np.ndarray:
    """codes [N, K] -> nibble words [T, P, 64 lanes, 4]: word 2j+h of lane l holds row 16t + l%16,
    columns 128p + 64j + 32h + 8(l//16) + e with e < 4 in bits 8e..8e+3, e+4 in bits 8e+4..8e+7."""
    n, k = q.shape
    T, P = n // 16, k // (2 * GROUP)
    q7 = q.reshape(T, 16, P, 2, 2, 4, 8).astype(np.uint32)      # [t, r, p, j, h, quad, e]
    q7 = q7.transpose(0, 2, 5, 1, 3, 4, 6)                        # [t, p, quad, r, j, h, e]
    word = np.zeros(q7.shape[:-1], dtype=np.uint32)
    for b in range(4):
        word |= q7[..., b] << np.uint32(8 * b)
        word |= q7[..., b + 4] << np.uint32(8 * b + 4)
    return word.reshape(T, P, 64, 4)                              # lane = quad*16 + r


def pack_frag(w: np.ndarray, s_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    """MLX (packs [N, K/8], scales, biases [N, K/64] bf16 bits) -> packed uint32 [N, K/8 + K/64].

    N/16 x K/128 blocks of 288 words; block (t, p): words 0..255 are the nibble words
    (lane l, word 2j+h at 4l + 2j + h), words 256 + 2r and 257 + 2r hold row 16t + r's
    scales and biases of groups 2p (low 16 bits) and 2p+1 (high 16 bits).
    """
    q = unpack_mlx(as_u32(w))
    n, k = q.shape
    if n % 16 or k % (2 * GROUP):
        raise ValueError("N must be a multiple of 16 and K of 128")
    T, P = n // 16, k // (2 * GROUP)
    out = np.zeros((T, P, BLOCK_WORDS), dtype=np.uint32)
    out[:, :, :256] = _frag_nibble_words(q).reshape(T, P, 256)
    for src, off in ((np.asarray(s_bits, np.uint16), 0), (np.asarray(b_bits, np.uint16), 1)):
        pairs = src.reshape(T, 16, P, 2).astype(np.uint32)        # [t, r, p, group-in-pair]
        out[:, :, 256 + off::2] = (pairs[..., 0] | (pairs[..., 1] << np.uint32(16))).transpose(0, 2, 1)
    return out.reshape(n, k // 8 + k // GROUP)


def relayout_frag(w: np.ndarray) -> np.ndarray:
    """MLX packs [N, K/8] -> the nibbles alone in fragment order, uint32 [N, K/8] (the
    one-argument repack_for_skinny(w)): block (t, p) of 256 words = words 0..255 of
    pack_frag's block."""
    q = unpack_mlx(as_u32(w))
    n, k = q.shape
    if n % 16 or k % (2 * GROUP):
        raise ValueError("N must be a multiple of 16 and K of 128")
    return _frag_nibble_words(q).reshape(n, k // 8)


def unpack_frag(wf: np.ndarray):
    """Inverse of pack_frag: (packs uint32 [N, K/8], scales, biases uint16 [N, K/64])."""
    a = as_u32(wf)
    n, words = a.shape
    k = words // 9 * 64
    T, P = n // 16, k // (2 * GROUP)
    blk = a.reshape(T, P, BLOCK_WORDS)
    word = blk[:, :, :256].reshape(T, P, 4, 16, 2, 2)             # [t, p, quad, r, j, h]
    e = np.zeros(word.shape + (8,), dtype=np.uint8)
    for b in range(4):
        e[..., b] = (word >> np.uint32(8 * b)) & 0xF
        e[..., b + 4] = (word >> np.uint32(8 * b + 4)) & 0xF
    q = e.transpose(0, 3, 1, 4, 5, 2, 6).reshape(n, k)             # [t, r, p, j, h, quad, e]
    sb = []
    for off in (0, 1):
        pw = blk[:, :, 256 + off::2].transpose(0, 2, 1)             # [t, r, p]
        lo = (pw & np.uint32(0xFFFF)).astype(np.uint16)
        hi = (pw >> np.uint32(16)).astype(np.uint16)
        sb.append(np.stack([lo, hi], axis=-1).reshape(n, k // GROUP))
    return pack_mlx(q), sb[0], sb[1]


def _perm(src0: np.ndarray, src1: np.ndarray, sel: int) -> np.ndarray:
    """v_perm_b32 for selector bytes 0..7: byte k of the result is byte sel.k of the 8-byte
    value {src0 (bytes 4-7) : src1 (bytes 0-3)}."""
    both = (src0.astype(np.uint64) << np.uint64(32)) | src1.astype(np.uint64)
    out = np.zeros_like(src1, dtype=np.uint32)
    for k in range(4):
        b = (sel >> (8 * k)) & 0xFF
        out |= (((both >> np.uint64(8 * b)) & np.uint64(0xFF)).astype(np.uint32)) << np.uint32(8 * k)
    return out


def lane_operands(wf: np.ndarray, t: int, g: int) -> np.ndarray:
    """Emulates the kernel's read-out of one (tile, group): the B-operand values each lane
    feeds to the group's two MFMAs, built as in the kernel from lo = w & 0x0F0F0F0F,
    hi = (w >> 4) & 0x0F0F0F0F and v_perm_b32 against 0x43434343, decoded as bf16.

    Returns float32 [2 (k half), 64 lanes, 8] holding 128 + q for row 16t + l%16 and columns
    64g + 32h + 8(l//16) + 0..7.
    """
    a = as_u32(wf)
    n, words = a.shape
    P = words // 9 * 64 // (2 * GROUP)
    frag = a.reshape(n // 16, P, BLOCK_WORDS)[t, g // 2, :256].reshape(64, 4)   # [lane, word]
    c43 = np.full(64, 0x43434343, dtype=np.uint32)
    out = np.zeros((2, 64, 8), dtype=np.float32)
    for h in range(2):
        w = frag[:, 2 * (g % 2) + h]
        lo = w & np.uint32(0x0F0F0F0F)
        hi = (w >> np.uint32(4)) & np.uint32(0x0F0F0F0F)
        pairs = [_perm(c43, lo, 0x04010400), _perm(c43, lo, 0x04030402),
                 _perm(c43, hi, 0x04010400), _perm(c43, hi, 0x04030402)]
        for v, pair in enumerate(pairs):
            out[h, :, 2 * v] = bf16_to_f32((pair & np.uint32(0xFFFF)).astype(np.uint16))
            out[h, :, 2 * v + 1] = bf16_to_f32((pair >> np.uint32(16)).astype(np.uint16))
    return out


def lane_scale_bias(wf: np.ndarray, t: int, g: int) -> np.ndarray:
    """Emulates the kernel's scale/bias read: float32 [16 rows, 2] = (s, b) of group g for rows
    16t + r, taken from the block's words 256 + 2r (+1) as the kernel does (low half for an even
    group, high half for an odd one)."""
    a = as_u32(wf)
    n, words = a.shape
    P = words // 9 * 64 // (2 * GROUP)
    blk = a.reshape(n // 16, P, BLOCK_WORDS)[t, g // 2]
    out = np.zeros((16, 2), dtype=np.float32)
    for r in range(16):
        for c in range(2):
            wv = blk[256 + 2 * r + c]
            out[r, c] = bf16_to_f32(np.uint16((wv >> 16) if g % 2 else (wv & 0xFFFF)))
    return out
