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


def test_config_for_takes_the_reference_forms():
    """config_for(m, k) (the reference's two-argument call, qmm.py:118) gives a pair (rf, sk);
    CONFIG_OVERRIDE = (rf, sk) (qmm.py:129, 208) becomes the wave-X tile (rf, sk waves, ring 2),
    which the library accepts for every pair the reference sweeps; the library's own 4-tuple form
    stays accepted; anything else is refused."""
    from skinny_mlx import qmm as Q

    L = _lib.lib()
    assert Q.CONFIG_OVERRIDE is None
    for k in (2560, 4096, 9728, 9216):
        rf, sk = Q.config_for(8, k)
        assert Q.config_for(1, k) == Q.config_for(16, k) == (rf, sk)
        assert Q.config_for(8, k, k)[1:3] == (rf, sk)  # the tile of a square K x K weight
    try:
        for rf in (1, 2, 4):
            for sk in (1, 2, 4, 8):
                Q.CONFIG_OVERRIDE = (rf, sk)
                assert Q.config_for(8, 2560) == (rf, sk)
                for k, n in ((2560, 9728), (9728, 2560), (2560, 9216), (9216, 2560), (2560, 7680)):
                    tile = Q.config_for(16, k, n)
                    assert tile == (1, rf, sk, 2)
                    assert Q._plain_config(k, n)[0] == 1
                    rc = L.skinny_qmm_w4g64_bf16(ctypes.c_void_p(4096), 8, k, k, ctypes.c_void_p(4096), n, None, n,
                                                 ctypes.byref(_lib.QmmTile(*tile)), None)
                    assert rc == -1 and "null" in L.skinny_last_error().decode(), (tile, k, n)
        Q.CONFIG_OVERRIDE = (1, 2, 4, 3)
        assert Q.config_for(8, 2560, 9728) == (1, 2, 4, 3) and Q.config_for(8, 2560) == (1, 2, 4, 3)
        Q.CONFIG_OVERRIDE = (1, 2, 4)
        with pytest.raises(ValueError):
            Q.config_for(8, 2560, 9728)
    finally:
        Q.CONFIG_OVERRIDE = None


def test_host_queries_over_many_shapes():
    """Every pure-host query of the library (tile tables and rules, workspace sizes, support
    predicates) over a grid of shapes, valid and invalid: each returns a defined result (0 or the
    argument-error code, a sane tile) and never touches memory it should not. Run under the
    sanitizer build as well (tests/test_sanitized_host.py)."""
    L = _lib.lib()
    ks = (-128, 0, 64, 128, 256, 2048, 2560, 4096, 9728, 12288, 1 << 20)
    ns = (-16, 0, 8, 16, 256, 2560, 6144, 8224, 19456, 151936, 1 << 24)
    for k in ks:
        for n in ns:
            t = _lib.QmmTile()
            splits = ctypes.c_int(0)
            for rc, what in ((L.skinny_qmm_pick_tile(k, n, ctypes.byref(t)), "pick"),
                             (L.skinny_qmm_splitk_pick(k, n, ctypes.byref(splits), ctypes.byref(t)), "splitk"),
                             (L.skinny_qmm_partial_pick(k, n, ctypes.byref(splits), ctypes.byref(t)), "partial"),
                             (L.skinny_qmm_glu_pick_tile(k, n // 2, ctypes.byref(t)), "glu")):
                assert rc in (0, -1), (what, k, n, rc)
                if rc == 0:
                    assert t.rf in (1, 2, 4) and 1 <= t.waves <= 16 and 2 <= t.ns <= 8, (what, k, n, t.as_tuple())
            assert L.skinny_qmm_gated_partial_supported(k, n) in (0, 1)
            for kind in (0, 1, 2, 7):
                for m in (0, 1, 4, 5):
                    assert L.skinny_qmm_normin_supported(kind, m, k, n, 3, None) in (0, 1, -1)
        for sp in (-1, 0, 1, 2, 4, 5):
            L.skinny_qmm_splitk_workspace_bytes(k, sp)
        for h in (0, 1, 8, 16):
            L.skinny_attn_workspace_bytes(h, max(k, 0))
    for h in (-1, 0, 1, 16, 64):
        L.skinny_gdn_record_words(h)
    # a message longer than the thread-local buffer is cut, not overrun
    t = _lib.QmmTile(1, 3, 1 << 30, 2)
    rc = L.skinny_qmm_w4g64_bf16(ctypes.c_void_p(4096), 8, 2560, 2560, ctypes.c_void_p(4096), 9728,
                                 ctypes.c_void_p(4096), 9728, ctypes.byref(t), None)
    assert rc == -1 and len(L.skinny_last_error()) < 512


def test_check_maps_codes_to_exceptions():
    with pytest.raises(ValueError):
        _lib.check(_lib.lib().skinny_w4g64_pack(None, None, None, None, 16, 128, None), "x")


def test_normin_entry_points_validate_on_host():
    L = _lib.lib()
    d = ctypes.c_void_p(4096)
    parts = ctypes.c_void_p(1 << 20)

    def ni(h=d, p=parts, splits=3, w=d, h_out=ctypes.c_void_p(8192)):
        return ctypes.byref(_lib.NormIn(h, p, splits, w, 1e-6, h_out))

    def plain(n=ni(), m=1, k=2560, n_=6144, tile=None):
        return L.skinny_qmm_w4g64_normin_bf16(n, m, k, d, n_, ctypes.c_void_p(1 << 22), n_, tile, None)

    _expect_einval(plain(m=0), "M=0")
    _expect_einval(plain(m=5), "M=5")
    _expect_einval(plain(n=ni(h=None)), "null")
    _expect_einval(plain(n=ni(p=None)), "slices exactly")
    _expect_einval(plain(n=ni(splits=0)), "slices exactly")
    _expect_einval(plain(n=ni(splits=5)), "splits=5")
    _expect_einval(plain(n=ni(h_out=d)), "must not alias")
    _expect_einval(plain(n=ni(h=ctypes.c_void_p(4100))), "misaligned")
    _expect_einval(plain(n_=151936), "no norm-in kernel")  # the lm_head's slab tile
    _expect_einval(plain(m=4, n=ni(splits=4)), "exceed")
    _expect_einval(plain(tile=ctypes.byref(_lib.QmmTile(1, 2, 8, 3))), "no norm-in kernel")
    _expect_einval(L.skinny_qmm_w4g64_glu_normin_bf16(ni(), 1, 2560, d, 9720, d, 9728, None, None), "F=9720")
    _expect_einval(L.skinny_qmm_w4g64_conv_normin_bf16(ni(), 1, 2560, d, 8224, d, 8224, 6144, None, d, 4, None, None,
                                                       None, None), "null")
    _expect_einval(L.skinny_qmm_w4g64_conv_normin_bf16(ni(), 1, 2560, d, 8224, d, 8224, 6144, d, d, 3, None, None,
                                                       None, None), "kernel width")
    _expect_einval(L.skinny_qmm_w4g64_conv_normin_bf16(ni(), 2, 2560, d, 8224, d, 8224, 6144, d, d, 4, None, d,
                                                       None, None), "window")


def test_spec_loop_entry_points_validate_on_host():
    L = _lib.lib()
    d = ctypes.c_void_p(4096)
    _expect_einval(L.skinny_spec_commit(None, 4, d, d, None, d, d, 8, d, None), "null")
    _expect_einval(L.skinny_spec_commit(d, 4, d, d, d, d, d, 8, None, None), "null")
    _expect_einval(L.skinny_spec_commit(d, 0, d, d, None, d, d, 8, d, None), "fed=0")
    _expect_einval(L.skinny_spec_commit(d, 65, d, d, None, d, d, 8, d, None), "fed=65")
    _expect_einval(L.skinny_spec_commit(d, 4, d, d, None, d, d, -1, d, None), "cap=-1")
    _expect_einval(L.skinny_spec_select_row(d, 4, None, d, 64, 64, d, None), "null")
    _expect_einval(L.skinny_spec_select_row(d, 0, d, d, 64, 64, d, None), "fed=0")
    _expect_einval(L.skinny_spec_select_row(d, 4, d, d, 32, 64, d, None), "bad shape")


def test_qkv_attention_entry_point_validates_on_host():
    L = _lib.lib()
    d = ctypes.c_void_p(4096)

    def call(x=d, m=1, k=2560, ldx=2560, n=6144, ld=6144, hq=32, hkv=8, dim=128, maxlen=4096, ws_bytes=1 << 30):
        return L.skinny_qkv_attention_fused_bf16(x, m, k, ldx, d, n, d, ld, hq, hkv, dim, None, None, 1e-6, d, 4096, d,
                                                 None, d, d, maxlen, 0.088, d, ws_bytes, d, None)

    _expect_einval(call(x=None), "null")
    _expect_einval(call(dim=64), "head dim")
    _expect_einval(call(n=6160), "N=6160")
    _expect_einval(call(m=0), "M=0")
    _expect_einval(call(m=17), "M=17")
    _expect_einval(call(ldx=2552), "ldx")
    _expect_einval(call(ld=6136), "ld_handoff")
    _expect_einval(call(maxlen=4000), "maxlen")
    _expect_einval(call(ws_bytes=16), "workspace")
    _expect_einval(L.skinny_qkv_attention_supported(2560, 6150, 8, 4096), "bad shape")


def test_normin_supported_covers_the_decoder_consumers():
    from skinny_mlx import qmm as Q

    assert Q.normin_supported(Q.NORMIN_PLAIN, 1, 2560, 6144, 3)
    assert Q.normin_supported(Q.NORMIN_SWIGLU, 1, 2560, 19456, 3)
    assert Q.normin_supported(Q.NORMIN_CONV, 1, 2560, 8224, 3)
    assert Q.normin_supported(Q.NORMIN_PLAIN, 1, 256, 768, 0)    # the test decoders
    assert Q.normin_supported(Q.NORMIN_SWIGLU, 1, 256, 1024, 3)
    assert not Q.normin_supported(Q.NORMIN_PLAIN, 5, 2560, 6144, 3)     # M > 4
    assert not Q.normin_supported(Q.NORMIN_PLAIN, 1, 2560, 151936, 0)   # the lm_head's slab tile
    assert not Q.normin_supported(Q.NORMIN_PLAIN, 4, 2560, 6144, 4)     # past the LDS budget
    assert not Q.normin_supported(Q.NORMIN_CONV, 1, 2560, 6144, 3)      # no conv instance for that tile


def test_gdn_record_entry_points_validate_on_host():
    L = _lib.lib()
    d = ctypes.c_void_p(4096)
    words = L.skinny_gdn_record_words(16)
    assert words == 16 * 16 * 2 * 128 + 16 * 16 * 2 + 16 * 16 * 128 // 2
    _expect_einval(L.skinny_gdn_commit_replay(None, 27, 16, d, d, words, d, d, 3, 6144, 19 * 6144, None), "null")
    _expect_einval(L.skinny_gdn_commit_replay(d, 27, 16, d, d, words - 4, d, d, 3, 6144, 19 * 6144, None), "bad sizes")
    _expect_einval(L.skinny_gdn_commit_replay(d, 27, 16, d, d, words, d, d, 3, 6144, 18 * 6144, None), "window")
    # a record belongs to a draft tree
    _expect_einval(L.skinny_gdn_recurrence(d, 6144, d, d, 32, d, d, d, None, d, None, 4, 16, 16, 128, 128, d, None),
                   "record")
    # key heads shared by value heads: the value-head count must be a multiple, and the row must hold
    # q and k of the key heads and v of the value heads
    _expect_einval(L.skinny_gdn_recurrence(d, 8192, d, d, 32, d, d, d, None, d, None, 4, 32, 12, 128, 128, None,
                                           None), "Hk=12")
    _expect_einval(L.skinny_gdn_recurrence(d, 8190, d, d, 32, d, d, d, None, d, None, 4, 32, 16, 128, 128, None,
                                           None), "ldq=8190")


def test_gated_partial_entry_point_validates_on_host():
    L = _lib.lib()
    d = ctypes.c_void_p(4096)

    def call(y=d, ldy=2048, ldz=8224, m=1, k=2048, n=2560, ldp=2560):
        return L.skinny_qmm_w4g64_gated_partial_f32(y, ldy, d, ldz, d, 1e-6, m, k, d, n, d, ldp, None)

    _expect_einval(call(y=None), "null")
    _expect_einval(call(m=0), "M=0")
    _expect_einval(call(m=17), "M=17")
    _expect_einval(call(k=2112), "K=2112")
    _expect_einval(call(ldy=2046), "ldy=2046")
    _expect_einval(call(ldz=2044), "ldz=2044")
    _expect_einval(call(y=ctypes.c_void_p(4100)), "misaligned")
    _expect_einval(call(k=512, n=256, ldy=512, ldz=512, ldp=256), "no gated-norm-in kernel")
    from skinny_mlx import qmm as Q

    assert Q.gated_partial_supported(2048, 2560) and Q.gated_partial_supported(256, 256)
    assert not Q.gated_partial_supported(512, 256)


def test_head_gated_recurrence_entry_point_validates_on_host():
    L = _lib.lib()
    d = ctypes.c_void_p(4096)

    def call(qkv=d, ldq=6144, state=d, z=ctypes.c_void_p(8192), out=d, h=16, dk=128, dv=128):
        return L.skinny_gdn_recurrence_gated_bf16(qkv, ldq, d, d, d, d, state, z, d, 1e-6, out, h, h, dk, dv, None)

    _expect_einval(call(qkv=None), "null pointer")
    _expect_einval(call(out=None), "null pointer")
    _expect_einval(call(dk=64), "head dims 64x128")
    _expect_einval(call(h=0), "H=0")
    _expect_einval(call(ldq=6143), "ldq=6143")
    _expect_einval(call(state=ctypes.c_void_p(4100)), "state must be 16-byte aligned")
    _expect_einval(call(qkv=ctypes.c_void_p(4104)), "qkv row must be 16-byte aligned")
    _expect_einval(call(out=ctypes.c_void_p(8192)), "out must not alias z")


def test_general_attention_entry_point_validates_on_host():
    """skinny_attention_general_bf16 (head dims 64/128/256, partial RoPE, strided query heads, an
    output gate) rejects layouts that do not fit before any launch."""
    L = _lib.lib()
    d = ctypes.c_void_p(4096)
    Hq, Hkv, D = 16, 4, 256
    ldq = (2 * Hq + 2 * Hkv) * D
    need = L.skinny_attn_general_workspace_bytes(Hq, Hkv, D, 4096)
    assert need > 0 and L.skinny_attn_general_workspace_bytes(0, Hkv, D, 4096) == 0

    def call(m=8, hq=Hq, hkv=Hkv, dim=D, qs=2 * D, koff=2 * Hq * D, voff=(2 * Hq + Hkv) * D, goff=D, rd=64,
             maxlen=4096, positions=4096, ws=need, ld=ldq, q=d):
        return L.skinny_attention_general_bf16(q, ld, m, hq, hkv, dim, qs, koff, voff, goff, d, d, 1e-6, rd, d,
                                               positions, d, None, d, d, maxlen, 0.0625, ctypes.c_void_p(1 << 20), ws,
                                               d, None)

    _expect_einval(call(q=None), "null")
    _expect_einval(call(dim=192, qs=384), "head dim 192")
    _expect_einval(call(hq=15), "not a multiple")
    _expect_einval(call(m=17), "M=17")
    _expect_einval(call(m=16, hq=32, hkv=4, ld=(2 * 32 + 8) * D, koff=64 * D, voff=68 * D), "query rows")
    _expect_einval(call(rd=63), "rotary_dim=63")
    _expect_einval(call(rd=512), "rotary_dim=512")
    _expect_einval(call(goff=ldq - D), "do not fit")
    _expect_einval(call(voff=ldq - D), "do not fit")
    _expect_einval(call(maxlen=4000), "maxlen")
    _expect_einval(call(positions=2048), "RoPE table")
    _expect_einval(call(ws=need - 4), "workspace")
    _expect_einval(L.skinny_rope_table_dim(1e7, 63, 16, d, None), "rotary_dim=63")


def test_fused_mlp_entry_point_validates_on_host():
    """skinny_mlp_fused_partial_f32 takes 2..16 tokens at the decoders' MLP shape and a hand-off
    buffer of skinny_mlp_fused_sync_bytes(F); anything else is rejected before a launch."""
    L = _lib.lib()
    d = ctypes.c_void_p(4096)
    need = L.skinny_mlp_fused_sync_bytes(9728)
    assert need >= (9728 // 128 + 1) * 4 and L.skinny_mlp_fused_sync_bytes(100) == 0
    assert L.skinny_mlp_fused_supported(8, 2560, 9728, 2560) == 1
    assert L.skinny_mlp_fused_supported(1, 2560, 9728, 2560) == 0   # one token: the norm-in gate|up form
    assert L.skinny_mlp_fused_supported(8, 256, 512, 256) == 0      # no fused instance for those tiles

    def call(m=8, k=2560, f=9728, n=2560, ldx=2560, sync_bytes=need, x=d):
        return L.skinny_mlp_fused_partial_f32(x, m, k, ldx, d, f, d, n, d, d, d, sync_bytes, None)

    _expect_einval(call(x=None), "null")
    _expect_einval(call(m=1), "M=1")
    _expect_einval(call(m=17), "M=17")
    _expect_einval(call(k=2048, ldx=2048), "one-wave form")
    _expect_einval(call(f=9680), "bad shape")
    _expect_einval(call(ldx=2552), "ldx=2552")
    _expect_einval(call(sync_bytes=need - 4), "sync of")
