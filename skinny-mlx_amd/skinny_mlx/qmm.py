"""Skinny W4A16 affine group-64 quantized matmul for 1..16 tokens per weight read.

Same call surface as the reference module (skinny_mlx/qmm.py:19-152): `GROUP`,
`repack_for_skinny(w)`, `config_for(m, k)`, `CONFIG_OVERRIDE`, `skinny_qmm(x, w, scales, biases)`.
Tensors are torch tensors on the ROCm device instead of MLX arrays; the packed format is MLX's
(`w` [N, K/8] as 32-bit words, eight 4-bit codes each, element i at bits 4i; `scales`/`biases`
[N, K/64] bf16), so the same bytes drop in.

The work is done by hand-written gfx950 kernels in libskinny_hip.so (csrc/qmm.hip):
`skinny_w4g64_pack` reorders the nibbles once at load into MFMA-fragment order, with the
scales and biases moved beside them, and `skinny_qmm_w4g64_bf16` computes
y = x . dequant(w)^T with bf16 MFMA and fp32 accumulation. There is no fallback path:
without the library every call raises.

The reference's two-call sequence works unchanged: `rw = repack_for_skinny(w)` relays the
nibbles alone ([N, K/8] words, like the reference's result), and `skinny_qmm(x, rw, scales,
biases)` completes that relayout with the scales and biases into the kernel's packed blocks on its
first call and keeps the result on `rw`, rebuilt whenever any of the three tensors is replaced or
changed in place (torch's version counter). `repack_for_skinny(w, scales, biases)` builds the packed
blocks directly (what the patched modules hold); `skinny_qmm` then checks that the scales and biases
it is given are the ones packed.

Differences from the reference, by design:
  * bf16 activations go straight into the MFMA (the reference casts to fp16, qmm.py:136);
  * the tile depends on (K, N) only, never on M (the reference's RF/SK change with M,
    qmm.py:123), so each token's output is bitwise identical for every M = 1..16;
  * M > 16 runs in 16-row chunks (the reference hands M outside 6..16 to mx.quantized_matmul).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

GROUP = 64
MAX_M = 16

# The tile forced for every skinny_qmm call when set; used by tile sweeps (reference qmm.py:129,
# 201-213). Either the reference's pair (rf, sk) — rf 16-row tiles per wave, sk waves per workgroup
# splitting K, the wave-X kernel with a 2-deep ring — or this library's (kind, rf, waves, ns).
CONFIG_OVERRIDE: tuple[int, int] | tuple[int, int, int, int] | None = None
# (splits, kind, rf, waves, ns) forced for every skinny_qmm call when set: splits >= 2 takes the
# split-K kernel with that tile, splits = 1 the unsplit one (split-K sweeps).
SPLITK_OVERRIDE: tuple[int, int, int, int, int] | None = None
# (splits, kind, rf, waves, ns) forced for every split-K residual projection (skinny_qmm_partial)
# when set.
PARTIAL_OVERRIDE: tuple[int, int, int, int, int] | None = None

_TILES: dict[tuple[int, int], object] = {}

def _check_words(w: torch.Tensor, name: str) -> None:
    if w.dtype not in (torch.int32, torch.uint32):
        raise ValueError(f"{name} must hold 32-bit words (int32/uint32), got {w.dtype}")
    if w.dim() != 2 or not w.is_contiguous():
        raise ValueError(f"{name} must be a contiguous 2-D tensor")
    if not w.is_cuda:
        raise ValueError(f"{name} must be on the GPU")


def packed_k(w: torch.Tensor) -> int:
    """K of a repack_for_skinny(w, scales, biases) result ([N, K/8 + K/64] words)."""
    _check_words(w, "w")
    words = w.shape[1]
    if words % 9:
        raise ValueError(f"w has {words} words per row: not a repack_for_skinny(w, scales, biases) result "
                         "([N, K/8 + K/64])")
    return words // 9 * 64


# Marks a repack_for_skinny(w) result (the nibbles alone), which has the shape of MLX's packs.
_NIBBLES = "skinny-w4g64-nibbles"


def _ident(t: torch.Tensor) -> tuple:
    """Identity of a tensor's contents for the packed-weight caches: storage address, shape and
    torch's in-place version counter."""
    return (t.data_ptr(), tuple(t.shape), t._version)


def _check_sb(t: torch.Tensor, name: str, n: int, k: int) -> None:
    if t.dtype != torch.bfloat16 or tuple(t.shape) != (n, k // GROUP) or not t.is_contiguous() or not t.is_cuda:
        raise ValueError(f"{name} must be contiguous bf16 [{n}, {k // GROUP}] on the GPU")


def repack_for_skinny(w: torch.Tensor, scales: torch.Tensor | None = None,
                      biases: torch.Tensor | None = None) -> torch.Tensor:
    """One-time load-time relayout of MLX 4-bit weights for the gfx950 kernel.

    `w` is MLX's packs, [N, K/8] 32-bit words (eight codes per word, element i at bits 4i).

    * `repack_for_skinny(w)` — the reference's call (qmm.py:96-115): the same nibbles in MFMA
      fragment order, int32 [N, K/8] (per (16-row tile, pair of groups) 64 lanes x 16 bytes, each
      lane holding exactly its four MFMA operands). `skinny_qmm(x, rw, scales, biases)` adds the
      scales and biases on its first call.
    * `repack_for_skinny(w, scales, biases)` — the kernel's packed blocks directly, int32
      [N, K/8 + K/64]: after each 1 KB of nibbles, the 16 rows' scales and biases of the two groups
      (`scales`/`biases` [N, K/64] bf16), so one wave stage is two contiguous loads.
    """
    _check_words(w, "w")
    n, kp = w.shape
    k = kp * 8
    if n % 16 or k % (2 * GROUP):
        raise ValueError(f"N={n} must be a multiple of 16 and K={k} of {2 * GROUP}")
    if scales is None and biases is None:
        out = torch.empty((n, kp), dtype=torch.int32, device=w.device)
        _lib.check(_lib.lib().skinny_w4g64_relayout(w.data_ptr(), out.data_ptr(), n, k, _lib.stream_of(w)),
                   "repack_for_skinny")
        out._skinny_layout = _NIBBLES
        return out
    if scales is None or biases is None:
        raise ValueError("pass both scales and biases, or neither")
    _check_sb(scales, "scales", n, k)
    _check_sb(biases, "biases", n, k)
    out = torch.empty((n, k // 8 + k // GROUP), dtype=torch.int32, device=w.device)
    _lib.check(_lib.lib().skinny_w4g64_pack(w.data_ptr(), scales.data_ptr(), biases.data_ptr(), out.data_ptr(), n, k,
                                            _lib.stream_of(w)), "repack_for_skinny")
    out._skinny_packed_from = (_ident(scales), _ident(biases))
    return out


def packed_weights(w: torch.Tensor, k: int, scales: torch.Tensor | None = None,
                   biases: torch.Tensor | None = None) -> torch.Tensor:
    """The kernel's packed blocks for a skinny_qmm call with K = k.

    A repack_for_skinny(w) relayout is completed with `scales` and `biases` (required) by one
    device pass, and the result is kept on the relayout until one of the three tensors changes:
    the first call per weight allocates, so it must not be inside a graph capture. A packed
    buffer is returned as it is, after checking that `scales`/`biases`, when given, are the
    tensors it was packed from and have not changed since."""
    _check_words(w, "w")
    n, words = w.shape
    if words * 8 == k:
        if getattr(w, "_skinny_layout", None) != _NIBBLES:
            raise ValueError(f"w [{n}, {words}] holds MLX packs, not a relayout: pass repack_for_skinny(w)")
        if scales is None or biases is None:
            raise ValueError("a repack_for_skinny(w) relayout needs skinny_qmm(x, w, scales, biases)")
        _check_sb(scales, "scales", n, k)
        _check_sb(biases, "biases", n, k)
        key = (_ident(w), _ident(scales), _ident(biases))
        cached = getattr(w, "_skinny_full", None)
        if cached is not None and cached[0] == key:
            return cached[1]
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("skinny_qmm: call it once with these weights before graph capture (its first call "
                               "completes the relayout with the scales and biases, which allocates)")
        full = torch.empty((n, k // 8 + k // GROUP), dtype=torch.int32, device=w.device)
        _lib.check(_lib.lib().skinny_w4g64_attach(w.data_ptr(), scales.data_ptr(), biases.data_ptr(), full.data_ptr(),
                                                  n, k, _lib.stream_of(w)), "skinny_qmm")
        w._skinny_full = (key, full)
        return full
    if packed_k(w) != k:
        raise ValueError(f"x has K={k}, weights have K={packed_k(w)}")
    src = getattr(w, "_skinny_packed_from", None)
    for t, name, i in ((scales, "scales", 0), (biases, "biases", 1)):
        if t is None:
            continue
        if tuple(t.shape) != (n, k // GROUP):
            raise ValueError(f"{name} shape {tuple(t.shape)} does not match the packed weights [{n}, {k // GROUP}]")
        if src is not None and _ident(t) != src[i]:
            raise ValueError(f"{name} are not the tensor packed into w (or changed since): repack the weights")
    return w


def unrepack(wf: torch.Tensor):
    """Inverse of repack_for_skinny: MLX packs [N, K/8] int32 for a relayout; (packs, scales,
    biases [N, K/64] bf16) for packed blocks."""
    _check_words(wf, "w")
    n = wf.shape[0]
    if getattr(wf, "_skinny_layout", None) == _NIBBLES:
        k = wf.shape[1] * 8
        w = torch.empty((n, k // 8), dtype=torch.int32, device=wf.device)
        _lib.check(_lib.lib().skinny_w4g64_unrelayout(wf.data_ptr(), w.data_ptr(), n, k, _lib.stream_of(wf)),
                   "unrepack")
        return w
    k = packed_k(wf)
    w = torch.empty((n, k // 8), dtype=torch.int32, device=wf.device)
    s = torch.empty((n, k // GROUP), dtype=torch.bfloat16, device=wf.device)
    b = torch.empty_like(s)
    _lib.check(_lib.lib().skinny_w4g64_unpack(wf.data_ptr(), w.data_ptr(), s.data_ptr(), b.data_ptr(), n, k,
                                              _lib.stream_of(wf)), "unrepack")
    return w, s, b


_WAVE_X = 1  # SKINNY_QMM_WAVE_X
_OVERRIDE_NS = 2  # ring depth of a tile given as the reference's (rf, sk) pair


def override_tile():
    """CONFIG_OVERRIDE as a library tile, or None when unset. The reference's pair (rf, sk)
    (qmm.py:118-129: RF row fragments per simdgroup, SK simdgroups splitting K per threadgroup)
    becomes the wave-X tile with rf 16-row tiles per wave and sk waves per workgroup."""
    if not CONFIG_OVERRIDE:
        return None
    cfg = tuple(int(v) for v in CONFIG_OVERRIDE)
    if len(cfg) == 2:
        return _lib.QmmTile(_WAVE_X, cfg[0], cfg[1], _OVERRIDE_NS)
    if len(cfg) == 4:
        return _lib.QmmTile(*cfg)
    raise ValueError(f"CONFIG_OVERRIDE must be (rf, sk) or (kind, rf, waves, ns), got {CONFIG_OVERRIDE!r}")


def config_for(m: int, k: int, n: int | None = None) -> tuple[int, ...]:
    """The tile skinny_qmm takes.

    * `config_for(m, k)` — the reference's call (qmm.py:118-126): the pair (rf, sk), rf 16-row
      tiles per wave and sk waves splitting K in a workgroup. CONFIG_OVERRIDE when it is set (in
      the form it was given); otherwise the tile the library takes for a square K x K weight,
      since this library keys its tiles by (K, N) and N is not given.
    * `config_for(m, k, n)` — (kind, rf, waves, ns) for a (K, N) weight: CONFIG_OVERRIDE as a
      library tile, else the library's measured table or rule.

    `m` is accepted for call-compatibility and ignored: the tile never depends on M, which is
    what keeps every token's output bitwise the same for M = 1..16.
    """
    del m
    if n is None:
        if CONFIG_OVERRIDE:
            return tuple(CONFIG_OVERRIDE)
        t = _table_tile(k, k)
        return (t.rf, t.waves)
    forced = override_tile()
    if forced is not None:
        return forced.as_tuple()
    return _table_tile(k, n).as_tuple()


def _table_tile(k: int, n: int):
    """The library table's QmmTile for (K, N), cached."""
    t = _TILES.get((k, n))
    if t is None:
        t = _lib.QmmTile()
        _lib.check(_lib.lib().skinny_qmm_pick_tile(k, n, ctypes.byref(t)), "config_for")
        _TILES[(k, n)] = t
    return t


def skinny_qmm(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor | None = None,
               biases: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """x [..., K] @ dequant(w)[N, K]^T -> [..., N] in bf16 (fp32 accumulation).

    The reference's call (qmm.py:132): `w` is `repack_for_skinny(w)` and `scales`/`biases` are
    MLX's [N, K/64] bf16 (see packed_weights for the one-time completion), or `w` is
    `repack_for_skinny(w, scales, biases)`, which carries them, and they may be omitted. x is
    cast to bf16 if needed. `out` may supply a bf16 [M, N] buffer.
    """
    k = x.shape[-1]
    w = packed_weights(w, k, scales, biases)
    n = w.shape[0]
    lead = x.shape[:-1]
    x2 = x.reshape(-1, k)
    if x2.dtype != torch.bfloat16:
        x2 = x2.to(torch.bfloat16)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 != 0 or x2.data_ptr() % 16 != 0:
        x2 = x2.contiguous()
    m = x2.shape[0]
    if out is None:
        y = torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    else:
        if out.dtype != torch.bfloat16 or tuple(out.shape) != (m, n) or out.stride(-1) != 1:
            raise ValueError("out must be bf16 [M, N] with unit inner stride")
        y = out
    L = _lib.lib()
    stream = _lib.stream_of(x2)
    splits, tile = _plain_config(k, n)
    if splits > 1:
        ws = splitk_workspace(x2.device, n, splits, stream)
        for m0 in range(0, m, MAX_M):
            mc = min(MAX_M, m - m0)
            xc, yc = x2[m0:m0 + mc], y[m0:m0 + mc]
            _lib.check(L.skinny_qmm_w4g64_splitk_bf16(xc.data_ptr(), mc, k, x2.stride(0), w.data_ptr(), n,
                                                      yc.data_ptr(), y.stride(0), ws.data_ptr(),
                                                      ws.numel() * ws.element_size(), splits, ctypes.byref(tile),
                                                      stream), "skinny_qmm")
        return y.reshape(*lead, n)
    for m0 in range(0, m, MAX_M):
        mc = min(MAX_M, m - m0)
        xc, yc = x2[m0:m0 + mc], y[m0:m0 + mc]
        _lib.check(L.skinny_qmm_w4g64_bf16(xc.data_ptr(), mc, k, x2.stride(0), w.data_ptr(), n, yc.data_ptr(),
                                           y.stride(0), ctypes.byref(tile), stream), "skinny_qmm")
    return y.reshape(*lead, n)


_SPLITK: dict[tuple[int, int], tuple] = {}
_SPLITK_WS: dict = {}


def _plain_config(k: int, n: int):
    """(splits, tile) skinny_qmm launches for (K, N): the split-K table's entry, else one split with
    the unsplit table's tile; the overrides win."""
    if SPLITK_OVERRIDE:
        return SPLITK_OVERRIDE[0], _lib.QmmTile(*SPLITK_OVERRIDE[1:])
    forced = override_tile()
    if forced is not None:
        return 1, forced
    cfg = _SPLITK.get((k, n))
    if cfg is None:
        splits = ctypes.c_int(0)
        tile = _lib.QmmTile()
        _lib.check(_lib.lib().skinny_qmm_splitk_pick(k, n, ctypes.byref(splits), ctypes.byref(tile)), "splitk_pick")
        cfg = _SPLITK[(k, n)] = (splits.value, tile)
    return cfg


_SPLITK_WS_MIN_WORDS = 4 + 16 * 16384 * 3  # the header and three slices of N = 16384


def splitk_workspace(device, n: int, splits: int, stream: int | None = None) -> torch.Tensor:
    """The split-K workspace of (device, stream), every word 0xFFFFFFFF (the kernel's "not yet
    written", restored by every call). Calls on one stream are ordered, so they share it; calls on
    different streams, which may overlap, each have their own, so skinny_qmm needs no shared state
    between streams.

    It is allocated (filled by a torch fill kernel, on that stream) on the stream's first split-K
    call, or grown when a call needs more. Inside a graph capture that allocation comes from the
    graph's memory pool and its fill is recorded ahead of the matmul, so every replay starts from
    a filled buffer; eager calls on the same stream later use the same buffer."""
    key_dev = torch.device(device)
    if key_dev.type == "cuda" and key_dev.index is None:
        key_dev = torch.device("cuda", torch.cuda.current_device())
    if stream is None:
        stream = torch.cuda.current_stream(key_dev).cuda_stream
    key = (key_dev, int(stream))
    need = int(_lib.lib().skinny_qmm_splitk_workspace_bytes(n, splits))
    ws = _SPLITK_WS.get(key)
    if ws is None or ws.numel() * 4 < need:
        ws = _SPLITK_WS[key] = torch.full((max(need // 4, _SPLITK_WS_MIN_WORDS),), -1, dtype=torch.int32,
                                          device=key_dev).view(torch.float32)
    return ws


def splitk_workspace_failed(device=None) -> bool:
    """Whether a split-K call on `device` (all devices when None) gave up waiting for a slice and
    marked its workspace: such a workspace makes every later call on its stream write NaN rows
    until reset_splitk_workspaces(). Reads device memory (synchronises its streams)."""
    for (dev, _), ws in list(_SPLITK_WS.items()):
        if device is not None and dev != torch.device(device):
            continue
        if int(ws[:1].view(torch.int32).item()) != -1:
            return True
    return False


def reset_splitk_workspaces() -> None:
    """Drop every split-K workspace; the next split-K call on each stream allocates a fresh one."""
    _SPLITK_WS.clear()


def partial_config(k: int, n: int) -> tuple[int, _lib.QmmTile]:
    """(splits, tile) of the split-K form for (K, N): the measured table, else a rule
    (PARTIAL_OVERRIDE: (splits, kind, rf, waves, ns) for every shape)."""
    if PARTIAL_OVERRIDE:
        return PARTIAL_OVERRIDE[0], _lib.QmmTile(*PARTIAL_OVERRIDE[1:])
    key = (k, n)
    cfg = _PARTIAL.get(key)
    if cfg is None:
        splits = ctypes.c_int(0)
        tile = _lib.QmmTile()
        _lib.check(_lib.lib().skinny_qmm_partial_pick(k, n, ctypes.byref(splits), ctypes.byref(tile)), "partial_pick")
        cfg = _PARTIAL[key] = (splits.value, tile)
    return cfg


_PARTIAL: dict = {}


def skinny_qmm_partial(x: torch.Tensor, w: torch.Tensor):
    """The split-K form of skinny_qmm for 1..16 tokens: a kernels.PartialSum of fp32 slices
    [splits, M, N] whose ordered sum, rounded to bf16, is the product. For a projection whose
    output only feeds a residual RMSNorm, which adds the slices itself."""
    from .kernels import PartialSum

    k = packed_k(w)
    n = w.shape[0]
    x2 = x.reshape(-1, k)
    if x2.dtype != torch.bfloat16:
        x2 = x2.to(torch.bfloat16)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 != 0 or x2.data_ptr() % 16 != 0:
        x2 = x2.contiguous()
    m = x2.shape[0]
    if not 1 <= m <= MAX_M:
        raise ValueError(f"skinny_qmm_partial takes 1..{MAX_M} tokens, got {m}")
    splits, tile = partial_config(k, n)
    parts = torch.empty((splits, m, n), dtype=torch.float32, device=x.device)
    _lib.check(_lib.lib().skinny_qmm_w4g64_partial_f32(x2.data_ptr(), m, k, x2.stride(0), w.data_ptr(), n,
                                                       parts.data_ptr(), n, splits, ctypes.byref(tile),
                                                       _lib.stream_of(x2)), "skinny_qmm_partial")
    return PartialSum(parts)


_GATED_OK: dict = {}


def gated_partial_supported(k: int, n: int) -> bool:
    """Whether skinny_qmm_partial_gated has a kernel for the (K, N) split-K tile; cached."""
    if (k, n) not in _GATED_OK:
        _GATED_OK[(k, n)] = _lib.lib().skinny_qmm_gated_partial_supported(k, n) == 1
    return _GATED_OK[(k, n)]


def skinny_qmm_partial_gated(y: torch.Tensor, z: torch.Tensor, norm_w: torch.Tensor, eps: float, w: torch.Tensor):
    """skinny_qmm_partial(gated_rmsnorm(y, z, norm_w, eps), w) in one launch, bitwise: y fp32
    [M, H, 128] (or [M, H*128]), z bf16 [M, H*128] rows; the Gated-DeltaNet output norm is formed
    per head inside the split-K projection (skinny_qmm_w4g64_gated_partial_f32)."""
    from .kernels import PartialSum

    k = packed_k(w)
    n = w.shape[0]
    m = y.shape[0]
    y2 = y.reshape(m, -1)
    if not 1 <= m <= MAX_M:
        raise ValueError(f"skinny_qmm_partial_gated takes 1..{MAX_M} tokens, got {m}")
    if y2.dtype != torch.float32 or y2.shape[1] != k or y2.stride(1) != 1:
        raise ValueError(f"y must be fp32 [{m}, {k}] rows")
    if z.dtype != torch.bfloat16 or z.dim() != 2 or tuple(z.shape) != (m, k) or z.stride(1) != 1:
        raise ValueError(f"z must be bf16 [{m}, {k}] rows")
    splits, _ = partial_config(k, n)
    parts = torch.empty((splits, m, n), dtype=torch.float32, device=y.device)
    _lib.check(_lib.lib().skinny_qmm_w4g64_gated_partial_f32(y2.data_ptr(), y2.stride(0), z.data_ptr(), z.stride(0),
                                                             norm_w.data_ptr(), eps, m, k, w.data_ptr(), n,
                                                             parts.data_ptr(), n, _lib.stream_of(y2)),
               "skinny_qmm_partial_gated")
    return PartialSum(parts)


def _rows(x: torch.Tensor, k: int) -> torch.Tensor:
    if x.shape[-1] != k:
        raise ValueError(f"x has K={x.shape[-1]}, weights have K={k}")
    x2 = x.reshape(-1, k)
    if x2.dtype != torch.bfloat16:
        x2 = x2.to(torch.bfloat16)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 != 0 or x2.data_ptr() % 16 != 0:
        x2 = x2.contiguous()
    if not 1 <= x2.shape[0] <= MAX_M:
        raise ValueError(f"takes 1..{MAX_M} tokens, got {x2.shape[0]}")
    return x2


# ---------------------------------------------------------------------------------------------
# Norm-in forms: the projection of a kernels.NormIn, the RMSNorm formed inside the matmul.

NORMIN_PLAIN, NORMIN_SWIGLU, NORMIN_CONV = 0, 1, 2
_NORMIN_OK: dict = {}


def _normin_tile(kind: int, k: int, n: int):
    """The tile of the plain form the norm-in form of `kind` must share (so both give the same
    bits), or None where there is no such unsplit tile."""
    if kind == NORMIN_PLAIN:
        splits, tile = _plain_config(k, n)
        return tile if splits == 1 else None
    if kind == NORMIN_SWIGLU:
        return glu_tile(k, n // 2)
    return _lib.QmmTile(0, 0, 0, 0)  # the conv form: the library's default on both paths


def normin_supported(kind: int, m: int, k: int, n: int, splits: int) -> bool:
    """Whether the norm-in form of `kind` runs for these sizes: the tile the plain form takes has
    a norm-in kernel and the rows fit its LDS."""
    tile = _normin_tile(kind, k, n)
    if tile is None:
        return False
    key = (kind, m, k, n, splits, tile.as_tuple())
    ok = _NORMIN_OK.get(key)
    if ok is None:
        t = None if tile.kind == 0 else ctypes.byref(tile)
        ok = _NORMIN_OK[key] = bool(_lib.lib().skinny_qmm_normin_supported(kind, m, k, n, splits, t))
    return ok


def _normin_args(nx, w: torch.Tensor):
    k = packed_k(w)
    if nx.shape[-1] != k:
        raise ValueError(f"input has K={nx.shape[-1]}, weights have K={k}")
    return nx.shape[0], k


def skinny_qmm_normin(nx, w: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """skinny_qmm of nx.value() for a kernels.NormIn, the norm formed in the same launch; bitwise
    skinny_qmm(nx.value(), w). nx.h_out receives the new residual stream."""
    m, k = _normin_args(nx, w)
    n = w.shape[0]
    y = torch.empty((m, n), dtype=torch.bfloat16, device=nx.device) if out is None else out
    ni = nx.abi()
    tile = _normin_tile(NORMIN_PLAIN, k, n)
    if tile is None:
        raise ValueError(f"({k}, {n}) takes split-K, which has no norm-in form")
    _lib.check(_lib.lib().skinny_qmm_w4g64_normin_bf16(ctypes.byref(ni), m, k, w.data_ptr(), n, y.data_ptr(),
                                                       y.stride(0), ctypes.byref(tile), _lib.stream_of(nx.h)),
               "skinny_qmm_normin")
    return y


def skinny_glu_normin(nx, w: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """skinny_glu(nx.value(), w, swiglu=True) for a kernels.NormIn, the norm formed in the same
    launch (bitwise)."""
    m, k = _normin_args(nx, w)
    f = w.shape[0] // 2
    y = torch.empty((m, f), dtype=torch.bfloat16, device=nx.device) if out is None else out
    ni = nx.abi()
    _lib.check(_lib.lib().skinny_qmm_w4g64_glu_normin_bf16(ctypes.byref(ni), m, k, w.data_ptr(), f, y.data_ptr(),
                                                           y.stride(0), ctypes.byref(glu_tile(k, f)),
                                                           _lib.stream_of(nx.h)), "skinny_glu_normin")
    return y


def skinny_qmm_conv_normin(nx, w: torch.Tensor, c: int, conv_state: torch.Tensor, conv_w: torch.Tensor,
                           window: torch.Tensor | None = None, parent: torch.Tensor | None = None) -> torch.Tensor:
    """skinny_qmm_conv(nx.value(), ...) for a kernels.NormIn, the norm formed in the same launch
    (bitwise)."""
    m, k = _normin_args(nx, w)
    n = w.shape[0]
    kw = _check_conv(c, conv_state, conv_w, window, m)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=nx.device)
    ni = nx.abi()
    _lib.check(_lib.lib().skinny_qmm_w4g64_conv_normin_bf16(
        ctypes.byref(ni), m, k, w.data_ptr(), n, y.data_ptr(), y.stride(0), c, conv_state.data_ptr(),
        conv_w.data_ptr(), kw, _lib.ptr(window), _lib.ptr(parent), None, _lib.stream_of(nx.h)), "skinny_qmm_conv_normin")
    return y


def _check_conv(c: int, conv_state: torch.Tensor, conv_w: torch.Tensor, window, m: int) -> int:
    kw = conv_w.shape[1]
    if conv_state.dtype != torch.bfloat16 or tuple(conv_state.shape) != (kw - 1, c) or not conv_state.is_contiguous():
        raise ValueError(f"conv_state must be contiguous bf16 [{kw - 1}, {c}]")
    if conv_w.dtype != torch.bfloat16 or conv_w.shape[0] != c or not conv_w.is_contiguous():
        raise ValueError(f"conv_w must be contiguous bf16 [{c}, KW]")
    if window is not None and (window.dtype != torch.bfloat16 or window.shape[-1] != c or window.shape[0] < kw - 1 + m):
        raise ValueError(f"window must be bf16 with >= {kw - 1 + m} rows of {c}")
    return kw


def skinny_qmm_conv(x: torch.Tensor, w: torch.Tensor, c: int, conv_state: torch.Tensor, conv_w: torch.Tensor,
                    window: torch.Tensor | None = None, parent: torch.Tensor | None = None,
                    tile: tuple[int, int, int, int] | None = None) -> torch.Tensor:
    """skinny_qmm for 1..16 tokens with a Gated-DeltaNet mixer's causal conv + SiLU applied to the
    first `c` output columns in the same launch: bitwise kernels.gdn_conv_silu of skinny_qmm's
    output there (conv_state [KW-1, c] advanced in place, `window` recorded, a draft tree's
    `parent` followed), the plain product in the other columns. `tile` (kind, rf, waves, ns)
    overrides the library's choice."""
    k = packed_k(w)
    n = w.shape[0]
    x2 = _rows(x, k)
    m = x2.shape[0]
    kw = _check_conv(c, conv_state, conv_w, window, m)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=x2.device)
    _lib.check(_lib.lib().skinny_qmm_w4g64_conv_bf16(x2.data_ptr(), m, k, x2.stride(0), w.data_ptr(), n, y.data_ptr(), n,
                                                     c, conv_state.data_ptr(), conv_w.data_ptr(), kw, _lib.ptr(window),
                                                     _lib.ptr(parent), ctypes.byref(_lib.QmmTile(*tile)) if tile else None,
                                                     _lib.stream_of(x2)), "skinny_qmm_conv")
    return y


# ---------------------------------------------------------------------------------------------
# The MLP sublayer (gate|up + SwiGLU, then down) in one launch.

_MLP_OK: dict = {}


def mlp_fused_supported(m: int, k: int, f: int, n: int) -> bool:
    """Whether skinny_mlp_fused_partial runs for m tokens over a K -> 2F -> N MLP (the library's
    fused instance: the decoders' gate|up tile in its one-wave form and the down projection's
    split-K tile); cached."""
    key = (m, k, f, n)
    if key not in _MLP_OK:
        _MLP_OK[key] = _lib.lib().skinny_mlp_fused_supported(m, k, f, n) == 1
    return _MLP_OK[key]


def mlp_fused_buffers(f: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    """(act, sync) of skinny_mlp_fused_partial: the [16, F] bf16 SwiGLU rows and the zeroed
    arrival counters (every call leaves them zero)."""
    words = int(_lib.lib().skinny_mlp_fused_sync_bytes(f)) // 4
    return (torch.empty((MAX_M, f), dtype=torch.bfloat16, device=device),
            torch.zeros((max(words, 1),), dtype=torch.int32, device=device))


def skinny_mlp_fused_partial(x: torch.Tensor, w_gate_up: torch.Tensor, w_down: torch.Tensor, act: torch.Tensor,
                             sync: torch.Tensor):
    """skinny_qmm_partial(skinny_glu(x, w_gate_up, swiglu=True), w_down) in one launch
    (skinny_mlp_fused_partial_f32), bitwise the two launches: a kernels.PartialSum of the down
    projection's fp32 slices. The SwiGLU rows pass through `act`, the hand-off through `sync`
    (mlp_fused_buffers); calls sharing them must be ordered (one stream)."""
    from .kernels import PartialSum

    k = packed_k(w_gate_up)
    f = w_gate_up.shape[0] // 2
    n = w_down.shape[0]
    x2 = _rows(x, k)
    m = x2.shape[0]
    if act.dtype != torch.bfloat16 or act.shape[0] < m or act.shape[1] != f or not act.is_contiguous():
        raise ValueError(f"act must be contiguous bf16 [>= {m}, {f}]")
    if packed_k(w_down) != f:
        raise ValueError(f"w_down has K={packed_k(w_down)}, the MLP's width is {f}")
    parts = torch.empty((3, m, n), dtype=torch.float32, device=x2.device)
    _lib.check(_lib.lib().skinny_mlp_fused_partial_f32(x2.data_ptr(), m, k, x2.stride(0), w_gate_up.data_ptr(), f,
                                                       w_down.data_ptr(), n, act.data_ptr(), parts.data_ptr(),
                                                       sync.data_ptr(), sync.numel() * sync.element_size(),
                                                       _lib.stream_of(x2)), "skinny_mlp_fused_partial")
    return PartialSum(parts)


# ---------------------------------------------------------------------------------------------
# Fused gate|up projection with the SwiGLU activation in the matmul epilogue.

_GLU_TILES: dict[tuple[int, int], object] = {}


def glu_tile(k: int, f: int) -> _lib.QmmTile:
    """The tile skinny_glu and skinny_glu_normin take for (K, F): the library's table or rule."""
    tile = _GLU_TILES.get((k, f))
    if tile is None:
        tile = _lib.QmmTile()
        _lib.check(_lib.lib().skinny_qmm_glu_pick_tile(k, f, ctypes.byref(tile)), "skinny_glu")
        _GLU_TILES[(k, f)] = tile
    return tile


def gate_up_order(f: int) -> torch.Tensor:
    """Row order of the gate|up layout: 16-row tiles alternate gate rows 16j.. and up rows
    16j.. of the concatenated [gate; up] (2F rows), so one wave of the kernel holds both halves
    of 16 activations."""
    if f % 16:
        raise ValueError(f"F={f} must be a multiple of 16")
    j = torch.arange(f // 16).repeat_interleave(16) * 16 + torch.arange(16).repeat(f // 16)
    return torch.stack([j.view(-1, 16), (j + f).view(-1, 16)], dim=1).reshape(-1)


def repack_gate_up(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor) -> torch.Tensor:
    """Pack a concatenated [gate; up] W4 g64 weight (MLX format, 2F rows) in the gate|up
    layout that skinny_glu reads."""
    order = gate_up_order(w.shape[0] // 2).to(w.device)
    return repack_for_skinny(w[order].contiguous(), scales[order].contiguous(), biases[order].contiguous())


def skinny_glu(x: torch.Tensor, w: torch.Tensor, swiglu: bool, out: torch.Tensor | None = None) -> torch.Tensor:
    """x [..., K] against a repack_gate_up() weight: swiglu=False -> [..., 2F] = [gate | up]
    (the unfused column order); swiglu=True -> [..., F] = silu(gate) * up, bitwise what
    the activation kernel makes of the swiglu=False result."""
    k = packed_k(w)
    f = w.shape[0] // 2
    if x.shape[-1] != k:
        raise ValueError(f"x has K={x.shape[-1]}, weights have K={k}")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, k)
    if x2.dtype != torch.bfloat16:
        x2 = x2.to(torch.bfloat16)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 != 0 or x2.data_ptr() % 16 != 0:
        x2 = x2.contiguous()
    m = x2.shape[0]
    width = f if swiglu else 2 * f
    if out is None:
        y = torch.empty((m, width), dtype=torch.bfloat16, device=x.device)
    else:
        if out.dtype != torch.bfloat16 or tuple(out.shape) != (m, width) or out.stride(-1) != 1:
            raise ValueError(f"out must be bf16 [M, {width}] with unit inner stride")
        y = out
    tile = glu_tile(k, f)
    L = _lib.lib()
    stream = _lib.stream_of(x2)
    for m0 in range(0, m, MAX_M):
        mc = min(MAX_M, m - m0)
        _lib.check(L.skinny_qmm_w4g64_glu_bf16(x2[m0:].data_ptr(), mc, k, x2.stride(0), w.data_ptr(), f,
                                               y[m0:].data_ptr(), y.stride(0), int(swiglu), ctypes.byref(tile),
                                               stream), "skinny_glu")
    return y.reshape(*lead, width)


# ---------------------------------------------------------------------------------------------
# Synthetic W4 g64 weights in MLX's format (benchmark shapes use these; see bench.py).

def random_w4g64(n: int, k: int, generator: torch.Generator | None = None, device="cpu",
                 scale_std: float = 0.02):
    """(w packs int32 [N, K/8], scales bf16 [N, K/64], biases bf16 [N, K/64]).

    Each 32-bit word is uniform, i.e. eight independent codes q ~ Uniform{0..15}; scales are
    |N(0, scale_std)| rounded to bf16 and biases are -8*scale (exact in bf16), so the
    dequantized weights are centred on zero.
    """
    if k % GROUP or n <= 0:
        raise ValueError(f"bad shape N={n} K={k}")
    w = torch.randint(-2 ** 31, 2 ** 31, (n, k // 8), dtype=torch.int32, generator=generator, device=device)
    s = (torch.randn((n, k // GROUP), generator=generator, device=device) * scale_std).abs().to(torch.bfloat16)
    b = (s.float() * -8.0).to(torch.bfloat16)
    return w, s, b


def nbytes_w4g64(n: int, k: int) -> int:
    """Bytes of packs + scales + biases of one [N, K] W4 g64 weight (reference qmm.py:173)."""
    return n * k // 2 + 2 * 2 * n * (k // GROUP)
