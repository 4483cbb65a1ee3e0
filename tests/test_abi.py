"""The C-ABI library loads, exports every symbol include/skinny_hip.h declares, and rejects
bad arguments on the host before any device work (no GPU needed)."""

import ctypes
import os
import re

import pytest

from skinny_mlx import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "skinny_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(skinny_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = declared_functions()
    assert len(names) >= 6
    for name in names:
        assert hasattr(L, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert L.skinny_abi_version() == _lib.ABI_VERSION


def _expect_einval(rc, fragment):
    assert rc == -1
    assert fragment in _lib.lib().skinny_last_error().decode()


def test_qmm_argument_validation_on_host():
    L = _lib.lib()
    dummy = ctypes.c_void_p(4096)  # never dereferenced: validation fails before any launch
    _expect_einval(L.skinny_qmm_w4g64_bf16(dummy, 0, 2560, 2560, dummy, 9728, dummy, 9728,
                                           0, 0, 0, None), "M=0")
    _expect_einval(L.skinny_qmm_w4g64_bf16(dummy, 17, 2560, 2560, dummy, 9728, dummy, 9728,
                                           0, 0, 0, None), "M=17")
    _expect_einval(L.skinny_qmm_w4g64_bf16(dummy, 8, 2496, 2560, dummy, 9728, dummy, 9728,
                                           0, 0, 0, None), "K=2496")
    _expect_einval(L.skinny_qmm_w4g64_bf16(dummy, 8, 2560, 2560, dummy, 9720, dummy, 9728,
                                           0, 0, 0, None), "N=9720")
    _expect_einval(L.skinny_qmm_w4g64_bf16(None, 8, 2560, 2560, dummy, 9728, dummy, 9728,
                                           0, 0, 0, None), "null")
    _expect_einval(L.skinny_qmm_w4g64_bf16(ctypes.c_void_p(4098), 8, 2560, 2560, dummy, 9728, dummy,
                                           9728, 0, 0, 0, None), "aligned")
    _expect_einval(L.skinny_qmm_w4g64_bf16(dummy, 8, 2560, 2560, dummy, 9728, dummy, 9728,
                                           3, 4, 2, None), "tile")


def test_pack_argument_validation_on_host():
    L = _lib.lib()
    d, o = ctypes.c_void_p(4096), ctypes.c_void_p(8192)
    _expect_einval(L.skinny_w4g64_pack(d, d, d, o, 24, 128, None), "N=24")
    _expect_einval(L.skinny_w4g64_pack(d, d, d, o, 32, 192, None), "K=192")
    _expect_einval(L.skinny_w4g64_pack(d, d, d, d, 32, 128, None), "in-place")
    _expect_einval(L.skinny_w4g64_unpack(None, d, d, d, 32, 128, None), "null")


def test_pick_tile_depends_on_k_and_n_only():
    from skinny_mlx.qmm import config_for

    for k, n in ((2560, 9728), (2560, 6144), (4096, 2560), (2560, 19456), (9728, 2560), (2560, 151936)):
        tiles = {config_for(m, k, n) for m in range(1, 17)}
        assert len(tiles) == 1
        rf, sk, ns = tiles.pop()
        assert (n // 16) % rf == 0 and 1 <= sk <= min(16, k // 128) and 2 <= ns <= 5


def test_check_maps_codes_to_exceptions():
    with pytest.raises(ValueError):
        _lib.check(_lib.lib().skinny_w4g64_pack(None, None, None, None, 16, 128, None), "x")
