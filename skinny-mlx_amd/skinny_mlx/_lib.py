"""ctypes boundary to libskinny_hip.so (the HIP kernels of this package).

The library exposes a plain C ABI (include/skinny_hip.h): device pointers, sizes and a
hipStream_t, returning 0 or a negative code with a thread-local message. This module
loads it once, declares every signature, and turns error codes into exceptions:
argument errors (-1) raise ValueError, launch/runtime errors raise RuntimeError.

torch is imported first on purpose: the library's NEEDED libamdhip64.so.7 then binds to
the HIP runtime torch already loaded, so torch streams and pointers are shared with it.

There is no fallback: if the library is missing, every entry point raises.
"""

from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must load the HIP runtime before the library)

LIB_NAME = "libskinny_hip.so"
# SKINNY_HIP_LIB names another build of the same library (the host-only sanitizer build the CPU
# tests load); unset, the in-tree build next to this file.
LIB_PATH = os.environ.get("SKINNY_HIP_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
ABI_VERSION = 19

_c_void_p = ctypes.c_void_p
_c_int = ctypes.c_int
_c_size_t = ctypes.c_size_t
_c_float = ctypes.c_float
_c_u64 = ctypes.c_uint64
_c_i64 = ctypes.c_int64


class QmmTile(ctypes.Structure):
    """skinny_qmm_tile of include/skinny_hip.h."""

    _fields_ = [("kind", ctypes.c_int), ("rf", ctypes.c_int), ("waves", ctypes.c_int), ("ns", ctypes.c_int)]

    def as_tuple(self) -> tuple:
        return (self.kind, self.rf, self.waves, self.ns)


_tile_p = ctypes.POINTER(QmmTile)


class NormIn(ctypes.Structure):
    """skinny_norm_in of include/skinny_hip.h."""

    _fields_ = [("h", ctypes.c_void_p), ("parts", ctypes.c_void_p), ("splits", ctypes.c_int),
                ("weight", ctypes.c_void_p), ("eps", ctypes.c_float), ("h_out", ctypes.c_void_p)]


_normin_p = ctypes.POINTER(NormIn)

# name -> (restype, argtypes). Every symbol declared in include/skinny_hip.h is listed.
SIGNATURES: dict[str, tuple] = {
    "skinny_abi_version": (_c_int, []),
    "skinny_last_error": (ctypes.c_char_p, []),
    "skinny_w4g64_pack": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_void_p]),
    "skinny_w4g64_unpack": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_void_p]),
    "skinny_w4g64_relayout": (_c_int, [_c_void_p, _c_void_p, _c_int, _c_int, _c_void_p]),
    "skinny_w4g64_unrelayout": (_c_int, [_c_void_p, _c_void_p, _c_int, _c_int, _c_void_p]),
    "skinny_w4g64_attach": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_void_p]),
    "skinny_qmm_w4g64_bf16": (
        _c_int,
        [_c_void_p, _c_int, _c_int, _c_int, _c_void_p, _c_int, _c_void_p, _c_int, _tile_p, _c_void_p],
    ),
    "skinny_qmm_pick_tile": (_c_int, [_c_int, _c_int, _tile_p]),
    "skinny_qmm_w4g64_glu_bf16": (
        _c_int, [_c_void_p, _c_int, _c_int, _c_int, _c_void_p, _c_int, _c_void_p, _c_int, _c_int, _tile_p, _c_void_p]),
    "skinny_qmm_glu_pick_tile": (_c_int, [_c_int, _c_int, _tile_p]),
    "skinny_stream_read": (_c_int, [_c_void_p, _c_size_t, _c_void_p, _c_int, _c_void_p]),
    "skinny_stream_read_chunked": (_c_int, [_c_void_p, _c_size_t, _c_void_p, _c_int, _c_int, _c_void_p]),
    "skinny_rmsnorm_bf16": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_float, _c_void_p, _c_void_p, _c_int, _c_int,
                                     _c_void_p]),
    "skinny_mtp_input_bf16": (_c_int, [_c_void_p, _c_int, _c_void_p, _c_int, _c_void_p, _c_int, _c_void_p, _c_void_p,
                                       _c_float, _c_void_p, _c_int, _c_void_p]),
    "skinny_gated_rmsnorm": (_c_int, [_c_void_p, _c_void_p, _c_int, _c_void_p, _c_float, _c_void_p, _c_int, _c_int,
                                      _c_int, _c_void_p]),
    "skinny_silu_mul_bf16": (_c_int, [_c_void_p, _c_int, _c_void_p, _c_int, _c_int, _c_void_p]),
    "skinny_embed_bf16": (_c_int, [_c_void_p, _c_int, _c_void_p, _c_int, _c_int, _c_void_p, _c_void_p]),
    "skinny_w4g64_dequant": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_void_p]),
    "skinny_qk_rope_store": (_c_int, [_c_void_p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_void_p, _c_void_p, _c_float,
                                      _c_void_p, _c_float, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int,
                                      _c_void_p]),
    "skinny_attn_workspace_bytes": (_c_size_t, [_c_int, _c_int]),
    "skinny_attention_bf16": (_c_int, [_c_void_p, _c_int, _c_int, _c_int, _c_int, _c_void_p, _c_void_p, _c_int,
                                       _c_void_p, _c_float, _c_void_p, _c_void_p, _c_size_t, _c_void_p, _c_void_p]),
    "skinny_kv_commit": (_c_int, [_c_void_p, _c_void_p, _c_int, _c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_int,
                                  _c_size_t, _c_void_p]),
    "skinny_gdn_conv_silu": (_c_int, [_c_void_p, _c_int, _c_int, _c_int, _c_int, _c_void_p, _c_void_p, _c_void_p,
                                      _c_int, _c_void_p, _c_void_p, _c_void_p]),
    "skinny_gdn_recurrence": (_c_int, [_c_void_p, _c_int, _c_void_p, _c_void_p, _c_int, _c_void_p, _c_void_p,
                                       _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_int,
                                       _c_int, _c_void_p, _c_void_p]),
    "skinny_gdn_record_words": (_c_size_t, [_c_int]),
    "skinny_gdn_recurrence_gated_bf16": (_c_int, [_c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                                  _c_void_p, _c_void_p, _c_void_p, _c_float, _c_void_p,
                                                  _c_int, _c_int, _c_int, _c_int, _c_void_p]),
    "skinny_gdn_commit_replay": (_c_int, [_c_void_p, _c_int, _c_int, _c_void_p, _c_void_p, _c_size_t, _c_void_p,
                                          _c_void_p, _c_int, _c_int, _c_size_t, _c_void_p]),
    "skinny_gdn_commit": (_c_int, [_c_void_p, _c_int, _c_int, _c_void_p, _c_void_p, _c_size_t, _c_size_t, _c_void_p,
                                   _c_void_p, _c_int, _c_int, _c_size_t, _c_void_p]),
    "skinny_gdn_select": (_c_int, [_c_void_p, _c_int, _c_int, _c_void_p, _c_void_p, _c_size_t, _c_size_t, _c_void_p,
                                   _c_void_p, _c_int, _c_int, _c_size_t, _c_void_p]),
    "skinny_argmax_rows_bf16": (_c_int, [_c_void_p, _c_int, _c_int, _c_int, _c_void_p, _c_void_p]),
    "skinny_accept": (_c_int, [_c_void_p, _c_void_p, _c_int, _c_void_p, _c_void_p]),
    "skinny_tree_accept": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_int, _c_void_p, _c_void_p]),
    "skinny_spec_commit": (_c_int, [_c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int,
                                    _c_void_p, _c_void_p]),
    "skinny_spec_select_row": (_c_int, [_c_void_p, _c_int, _c_void_p, _c_void_p, _c_int, _c_int, _c_void_p, _c_void_p]),
    "skinny_topk_rows_bf16": (_c_int, [_c_void_p, _c_int, _c_int, _c_int, _c_int, _c_void_p, _c_void_p]),
    "skinny_qmm_w4g64_partial_f32": (_c_int, [_c_void_p, _c_int, _c_int, _c_int, _c_void_p, _c_int, _c_void_p, _c_int,
                                              _c_int, _tile_p, _c_void_p]),
    "skinny_qmm_partial_pick": (_c_int, [_c_int, _c_int, ctypes.POINTER(_c_int), _tile_p]),
    "skinny_qmm_w4g64_splitk_bf16": (_c_int, [_c_void_p, _c_int, _c_int, _c_int, _c_void_p, _c_int, _c_void_p, _c_int,
                                              _c_void_p, _c_size_t, _c_int, _tile_p, _c_void_p]),
    "skinny_qmm_splitk_workspace_bytes": (_c_size_t, [_c_int, _c_int]),
    "skinny_qmm_splitk_pick": (_c_int, [_c_int, _c_int, ctypes.POINTER(_c_int), _tile_p]),
    "skinny_qmm_normin_supported": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int, _tile_p]),
    "skinny_qmm_w4g64_normin_bf16": (_c_int, [_normin_p, _c_int, _c_int, _c_void_p, _c_int, _c_void_p, _c_int, _tile_p,
                                              _c_void_p]),
    "skinny_qmm_w4g64_glu_normin_bf16": (_c_int, [_normin_p, _c_int, _c_int, _c_void_p, _c_int, _c_void_p, _c_int,
                                                  _tile_p, _c_void_p]),
    "skinny_qmm_w4g64_conv_normin_bf16": (_c_int, [_normin_p, _c_int, _c_int, _c_void_p, _c_int, _c_void_p, _c_int,
                                                   _c_int, _c_void_p, _c_void_p, _c_int, _c_void_p, _c_void_p,
                                                   _tile_p, _c_void_p]),
    "skinny_qmm_w4g64_conv_bf16": (_c_int, [_c_void_p, _c_int, _c_int, _c_int, _c_void_p, _c_int, _c_void_p, _c_int,
                                            _c_int, _c_void_p, _c_void_p, _c_int, _c_void_p, _c_void_p, _tile_p,
                                            _c_void_p]),
    "skinny_rmsnorm_partials_bf16": (_c_int, [_c_void_p, _c_void_p, _c_int, _c_size_t, _c_int, _c_void_p, _c_float,
                                              _c_void_p, _c_void_p, _c_int, _c_int, _c_void_p]),
    "skinny_attention_fused_bf16": (_c_int, [_c_void_p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_void_p, _c_void_p,
                                             _c_float, _c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                             _c_int, _c_float, _c_void_p, _c_size_t, _c_void_p, _c_void_p]),
    "skinny_qmm_w4g64_gated_partial_f32": (_c_int, [_c_void_p, _c_int, _c_void_p, _c_int, _c_void_p, _c_float, _c_int,
                                                    _c_int, _c_void_p, _c_int, _c_void_p, _c_int, _c_void_p]),
    "skinny_qmm_gated_partial_supported": (_c_int, [_c_int, _c_int]),
    "skinny_qkv_attention_fused_bf16": (_c_int, [_c_void_p, _c_int, _c_int, _c_int, _c_void_p, _c_int, _c_void_p, _c_int,
                                                 _c_int, _c_int, _c_int, _c_void_p, _c_void_p, _c_float, _c_void_p,
                                                 _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_float,
                                                 _c_void_p, _c_size_t, _c_void_p, _c_void_p]),
    "skinny_qkv_attention_supported": (_c_int, [_c_int, _c_int, _c_int, _c_int]),
    "skinny_attention_fused_noalloc_bf16": (_c_int, [_c_void_p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_void_p,
                                                     _c_void_p, _c_float, _c_void_p, _c_int, _c_void_p, _c_void_p,
                                                     _c_void_p, _c_void_p, _c_int, _c_float, _c_void_p, _c_void_p]),
    "skinny_rope_table": (_c_int, [_c_float, _c_int, _c_void_p, _c_void_p]),
    "skinny_mlp_fused_partial_f32": (_c_int, [_c_void_p, _c_int, _c_int, _c_int, _c_void_p, _c_int, _c_void_p, _c_int,
                                              _c_void_p, _c_void_p, _c_void_p, _c_size_t, _c_void_p]),
    "skinny_mlp_fused_supported": (_c_int, [_c_int, _c_int, _c_int, _c_int]),
    "skinny_mlp_fused_sync_bytes": (_c_size_t, [_c_int]),
    "skinny_rope_table_dim": (_c_int, [_c_float, _c_int, _c_int, _c_void_p, _c_void_p]),
    "skinny_attention_general_bf16": (_c_int, [_c_void_p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                               _c_int, _c_int, _c_void_p, _c_void_p, _c_float, _c_int, _c_void_p,
                                               _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_float,
                                               _c_void_p, _c_size_t, _c_void_p, _c_void_p]),
    "skinny_attn_general_workspace_bytes": (_c_size_t, [_c_int, _c_int, _c_int, _c_int]),
    "skinny_random_uniform": (_c_int, [_c_u64, _c_void_p, _c_i64, _c_int, _c_int, _c_void_p, _c_void_p]),
    "skinny_row_stats_bf16": (_c_int, [_c_void_p, _c_int, _c_int, _c_int, _c_float, _c_void_p, _c_void_p]),
    "skinny_sample_rows_bf16": (_c_int, [_c_void_p, _c_int, _c_int, _c_int, _c_float, _c_u64, _c_void_p, _c_i64,
                                         _c_int, _c_void_p, _c_void_p]),
    "skinny_spec_accept_sampled": (_c_int, [_c_void_p, _c_int, _c_void_p, _c_void_p, _c_int, _c_void_p, _c_int,
                                            _c_void_p, _c_int, _c_int, _c_float, _c_u64, _c_void_p, _c_void_p,
                                            _c_void_p]),
}

_lib = None


class SkinnyLaunchError(RuntimeError):
    """A HIP launch or runtime failure reported by the library."""


def lib() -> ctypes.CDLL:
    """The loaded library (raises ImportError when it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                "(or `make -C skinny-mlx_amd/csrc`). There is no CPU fallback.")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        ver = handle.skinny_abi_version()
        if ver != ABI_VERSION:
            raise ImportError(f"{LIB_PATH}: ABI version {ver}, expected {ABI_VERSION}")
        _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    """Raise for a non-zero return code of an ABI call."""
    if rc == 0:
        return
    msg = lib().skinny_last_error().decode(errors="replace")
    if rc == -1:
        raise ValueError(f"{what}: {msg}")
    raise SkinnyLaunchError(f"{what} (code {rc}): {msg}")


def stream_of(t: torch.Tensor) -> int:
    """hipStream_t (as int) of torch's current stream on t's device."""
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
