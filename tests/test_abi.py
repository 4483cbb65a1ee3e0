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

    def call(x=dummy, m=8, k=2560, ldx=2560, n=9728, tile=None):
        t = None if tile is None else ctypes.byref(_lib.QmmTile(*tile))
        return L.skinny_qmm_w4g64_bf16(x, m, k, ldx, dummy, n, dummy, n, t, None)

    _expect_einval(call(m=0), "M=0")
    _expect_einval(call(m=17), "M=17")
    _expect_einval(call(k=2496, ldx=2496), "K=2496")
    _expect_einval(call(n=9720), "N=9720")
    _expect_einval(call(x=None), "null")
    _expect_einval(call(x=ctypes.c_void_p(4098)), "aligned")
    _expect_einval(call(ldx=2552), "ldx")
    _expect_einval(call(tile=(1, 3, 4, 2)), "rf=3")
    _expect_einval(call(tile=(3, 1, 4, 2)), "kind")
    _expect_einval(call(tile=(2, 1, 16, 4)), "slab waves=16")
    _expect_einval(call(k=4096, ldx=4096, tile=(2, 1, 4, 4)), "slab")
    _expect_einval(call(tile=(1, 1, 4, 6)), "unsupported")
    _expect_einval(call(tile=(1, 4, 4, 4)), "unsupported")
    _expect_einval(call(tile=(1, 1, 32, 2)), "waves=32")
    _expect_einval(call(n=9712, tile=(1, 2, 4, 2)), "not divisible")


def test_pack_argument_validation_on_host():
    L = _lib.lib()
    d, o = ctypes.c_void_p(4096), ctypes.c_void_p(8192)
    _expect_einval(L.skinny_w4g64_pack(d, d, d, o, 24, 128, None), "N=24")
    _expect_einval(L.skinny_w4g64_pack(d, d, d, o, 32, 192, None), "K=192")
    _expect_einval(L.skinny_w4g64_pack(d, d, d, d, 32, 128, None), "in-place")
    _expect_einval(L.skinny_w4g64_unpack(None, d, d, d, 32, 128, None), "null")


def test_pick_tile_depends_on_k_and_n_only():
    from skinny_mlx.qmm import config_for

    L = _lib.lib()
    for k, n in ((2560, 9728), (2560, 6144), (4096, 2560), (2560, 19456), (9728, 2560), (2560, 151936),
                 (2560, 8224), (2560, 32768), (5120, 2560), (2048, 2560)):
        tiles = {config_for(m, k, n) for m in range(1, 17)}
        assert len(tiles) == 1
        tile = tiles.pop()
        kind, rf, waves, ns = tile
        assert kind in (1, 2) and (n // 16) % rf == 0, tile
        # the table's tiles pass the library's own validation
        rc = L.skinny_qmm_w4g64_bf16(ctypes.c_void_p(4096), 8, k, k, ctypes.c_void_p(4096), n, None, n,
                                     ctypes.byref(_lib.QmmTile(*tile)), None)
        assert rc == -1 and "null" in L.skinny_last_error().decode(), tile


def test_check_maps_codes_to_exceptions():
    with pytest.raises(ValueError):
        _lib.check(_lib.lib().skinny_w4g64_pack(None, None, None, None, 16, 128, None), "x")


def test_folded_norm_entry_points_validate_on_host():
    L = _lib.lib()
    d = ctypes.c_void_p(4096)
    t = ctypes.byref(_lib.QmmTile(1, 2, 4, 3))

    def resnorm(m=8, splits=2, part=d, counters=d, out_v=ctypes.c_void_p(8192), out_xw=ctypes.c_void_p(12288), tile=t):
        return L.skinny_qmm_w4g64_resnorm_bf16(d, m, 9728, 9728, d, 2560, ctypes.c_void_p(8192), 2560, d, out_v, 2560,
                                               out_xw, 2560, d, part, 2560, counters, splits, tile, None)

    _expect_einval(resnorm(m=0), "M=0")
    _expect_einval(resnorm(splits=5), "splits=5")
    _expect_einval(resnorm(part=None), "slice buffer")
    _expect_einval(resnorm(counters=None), "slice buffer")
    _expect_einval(resnorm(out_xw=ctypes.c_void_p(8192)), "alias")
    _expect_einval(resnorm(tile=None), "splits must be 0")
    _expect_einval(resnorm(tile=ctypes.byref(_lib.QmmTile(2, 1, 4, 4))), "wave-X")
    scaled = L.skinny_qmm_w4g64_scaled_bf16
    _expect_einval(scaled(d, 8, 8192, 8192, d, 256, d, 256, d, 1e-6, None, None), "exceeds")
    _expect_einval(scaled(d, 8, 2560, 2560, d, 256, d, 256, ctypes.c_void_p(4100), 1e-6, None, None), "16-byte")
    _expect_einval(L.skinny_qmm_w4g64_glu_scaled_bf16(d, 8, 2560, 2560, d, 1024, d, 1024, 2, d, 1e-6, None, None),
                   "swiglu=2")
    _expect_einval(L.skinny_rms_prep_bf16(d, 2560, d, ctypes.c_void_p(8192), 2560, d, 17, 2560, None), "rows=17")
    _expect_einval(L.skinny_rms_prep_bf16(d, 2560, d, d, 2560, d, 8, 2560, None), "alias")
    n = ctypes.c_int(0)
    assert L.skinny_qmm_resnorm_counters(2560, ctypes.byref(n)) == 0 and n.value == 160


def test_resnorm_config_stays_within_the_built_tiles():
    """The residual-norm epilogue is built for waves <= 8 and ring depths <= 4 (<= 3 with rf = 4);
    its default configuration is one split with the plain table's tile, clamped to that range."""
    from skinny_mlx import qmm as Q

    for k, n in ((9728, 2560), (4096, 2560), (2048, 2560), (256, 256), (2560, 9728), (2560, 151936)):
        splits, t = Q.resnorm_config(k, n)
        assert splits == 1 and t.kind == 1, (k, n)
        assert t.waves <= min(8, k // 128) and t.ns <= (3 if t.rf == 4 else 4) and (n // 16) % t.rf == 0, (k, n)
