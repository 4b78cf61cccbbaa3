"""C-ABI checks that need no GPU: the library loads, exports every entry point
declared in include/*.h, and rejects invalid calls on the host before
anything is launched (the reference's CPU-forcible failure cases)."""
import ctypes
import os
import re

import pytest

import qwfn_kv as K

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FAKE = 0x7F0000000000          # never dereferenced: validation fails first


def declared_symbols():
    syms = set()
    for name in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if name.endswith(".h"):
            hdr = open(os.path.join(ROOT, "include", name)).read()
            hdr = re.sub(r"/\*.*?\*/", "", hdr, flags=re.S)
            syms |= set(re.findall(r"\b(qwfn_[a-z0-9_]+)\s*\(", hdr))
    return sorted(syms)


def test_library_exports_header_symbols():
    L = K.load()
    syms = declared_symbols()
    assert len(syms) >= 10
    for s in syms:
        assert hasattr(L, s), s
    assert set(K.EXPORTS) == set(syms)
    assert L.qwfn_abi_version() == 2


def _err(rc, code, needle):
    assert rc == code, (rc, K.load().qwfn_last_error())
    assert needle in K.load().qwfn_last_error().decode()


def q8(ne0, n, nb1=None):
    return K.tensor(FAKE, K.TYPE_Q8_0, (ne0, n), (34, nb1 or ne0 // 32 * 34))


def f32(ne0, n):
    return K.tensor(FAKE, K.TYPE_F32, (ne0, n), (4, ne0 * 4))


def i32(n):
    return K.tensor(FAKE, K.TYPE_I32, (n,), (4,))


def test_set_rows_validation():
    L = K.load()
    r = ctypes.byref
    _err(L.qwfn_set_rows_q8_0(r(q8(512, 64)), r(f32(500, 1)), r(i32(1)), 1, None), K.EINVAL, "multiple of 32")
    _err(L.qwfn_set_rows_q8_0(r(q8(512, 64)), r(f32(512, 2)), r(i32(3)), 1, None), K.EINVAL, "idx")
    bad = K.tensor(FAKE, K.TYPE_F16, (512, 1), (2, 1024))
    _err(L.qwfn_set_rows_q8_0(r(q8(512, 64)), r(bad), r(i32(1)), 1, None), K.EINVAL, "f32")
    _err(L.qwfn_set_rows_q8_0(r(q8(512, 64)), r(f32(512, 1)), r(i32(1)), 7, None), K.EINVAL, "variant")
    _err(L.qwfn_set_rows_q8_0(r(q8(256, 64)), r(f32(512, 1)), r(i32(1)), 1, None), K.EINVAL, "ne[0]")
    mis = K.tensor(FAKE + 1, K.TYPE_Q8_0, (512, 64), (34, 544))
    _err(L.qwfn_set_rows_q8_0(r(mis), r(f32(512, 1)), r(i32(1)), 1, None), K.EALIGN, "aligned")


def test_cpy_validation():
    L = K.load()
    r = ctypes.byref
    _err(L.qwfn_cpy_f32_q8_0(r(f32(512, 3)), r(q8(512, 2)), 1, None), K.EINVAL, "ne[1]")
    _err(L.qwfn_cpy_f32_q8_0(r(f32(512, 3)), r(q8(512, 3, nb1=100)), 1, None), K.EINVAL, "overlap")


def test_fused_kv_append_validation():
    """The fused K+V entry points check each pair like the single calls, and the K and V
    sources must have the same shape."""
    L = K.load()
    r = ctypes.byref
    _err(L.qwfn_set_rows_q8_0_kv(r(q8(512, 64)), r(f32(512, 2)), r(q8(512, 64)), r(f32(512, 3)), r(i32(2)), 1, None),
         K.EINVAL, "idx")
    _err(L.qwfn_set_rows_q8_0_kv(r(q8(512, 64)), r(f32(512, 2)), r(q8(512, 64)), r(f32(500, 2)), r(i32(2)), 1, None),
         K.EINVAL, "multiple of 32")
    _err(L.qwfn_cpy_f32_q8_0_kv(r(f32(512, 3)), r(q8(512, 3)), r(f32(256, 3)), r(q8(256, 3)), 1, None),
         K.EINVAL, "same shape")
    _err(L.qwfn_cpy_f32_q8_0_kv(r(f32(512, 3)), r(q8(512, 3)), r(f32(512, 3)), r(q8(512, 2)), 1, None),
         K.EINVAL, "ne[1]")


def test_get_rows_and_gather_validation():
    L = K.load()
    r = ctypes.byref
    src = K.tensor(FAKE, K.TYPE_I32, (136, 100), (4, 544))
    dst = K.tensor(FAKE, K.TYPE_I32, (136, 5), (4, 544))
    _err(L.qwfn_get_rows_i32(r(src), r(i32(4)), r(dst), None), K.EINVAL, "dst")
    srcq = K.tensor(FAKE, K.TYPE_Q8_0, (256, 100), (34, 544))
    _err(L.qwfn_get_rows_i32(r(srcq), r(i32(5)), r(dst), None), K.EINVAL, "i32")
    _err(L.qwfn_kv_gather_segments(FAKE, 544, 100, 2, 272, 272, 2, FAKE, 10, FAKE, 272, 2720, None),
         K.EALIGN, "multiples of 4")
    _err(L.qwfn_kv_gather_segments(FAKE, 544, 100, 0, 272, 276, 2, FAKE, 10, FAKE, 276, 2760, None),
         K.ERANGE, "past the source row")
    G2 = L.qwfn_kv_gather_segments_kv
    _err(G2(FAKE, None, 544, 100, 0, 272, 272, 2, FAKE, 10, FAKE, FAKE + 8192, 272, 2720, None), K.EINVAL, "NULL")
    _err(G2(FAKE, FAKE, 544, 100, 2, 272, 272, 2, FAKE, 10, FAKE, FAKE + 8192, 272, 2720, None),
         K.EALIGN, "multiples of 4")
    _err(G2(FAKE, FAKE, 544, 100, 0, 272, 276, 2, FAKE, 10, FAKE, FAKE + 8192, 276, 2760, None),
         K.ERANGE, "past the source row")
    _err(G2(FAKE, FAKE, 544, 100, 0, 272, 272, 2, FAKE, 10, FAKE, FAKE + 4096, 272, 2720, None),
         K.EINVAL, "overlap")


def _fa_views(hd=256, T=1, nh=16, nh_kv=2, n_kv=100, qtype=K.TYPE_F32):
    q = K.tensor(FAKE, qtype, (hd, T, nh, 1), (4, nh * hd * 4, hd * 4, T * nh * hd * 4))
    k = K.tensor(FAKE, K.TYPE_Q8_0, (hd, n_kv, nh_kv, 1), (34, hd // 32 * 34 * nh_kv, hd // 32 * 34, 1 << 20))
    o = K.tensor(FAKE, K.TYPE_F32, (hd, nh, T, 1), (4, hd * 4, hd * nh * 4, hd * nh * T * 4))
    return q, k, o


def test_flash_attn_validation():
    L = K.load()
    r = ctypes.byref
    q, k, o = _fa_views()
    _err(L.qwfn_flash_attn_ext_q8_0(r(q), r(k), r(k), None, 0.0625, 8.0, 0.0, r(o), 1, None, 0, None),
         K.ENOTSUP, "max_bias")
    _err(L.qwfn_flash_attn_ext_q8_0(r(q), r(k), r(k), None, 0.0625, 0.0, 30.0, r(o), 1, None, 0, None),
         K.ENOTSUP, "softcap")
    q2, k2, o2 = _fa_views(hd=128)
    _err(L.qwfn_flash_attn_ext_q8_0(r(q2), r(k2), r(k2), None, 0.0625, 0.0, 0.0, r(o2), 1, None, 0, None),
         K.ENOTSUP, "head size")
    q3, k3, o3 = _fa_views(nh=15)
    _err(L.qwfn_flash_attn_ext_q8_0(r(q3), r(k3), r(k3), None, 0.0625, 0.0, 0.0, r(o3), 1, None, 0, None),
         K.EINVAL, "multiple of n_head_kv")
    m = K.tensor(FAKE, K.TYPE_F16, (50, 1, 1, 1), (2, 100, 100, 100))
    _err(L.qwfn_flash_attn_ext_q8_0(r(q), r(k), r(k), r(m), 0.0625, 0.0, 0.0, r(o), 1, None, 0, None),
         K.EINVAL, "mask")
    kmis = K.tensor(FAKE, K.TYPE_Q8_0, (256, 100, 2, 1), (34, 550, 272, 1 << 20))
    _err(L.qwfn_flash_attn_ext_q8_0(r(q), r(kmis), r(kmis), None, 0.0625, 0.0, 0.0, r(o), 1, None, 0, None),
         K.EALIGN, "16-byte")
    q4, k4, o4 = _fa_views(qtype=K.TYPE_F16)
    _err(L.qwfn_flash_attn_ext_q8_0(r(q4), r(k4), r(k4), None, 0.0625, 0.0, 0.0, r(o4), 1, None, 0, None),
         K.EINVAL, "f32")


def test_restore_validation():
    L = K.load()
    vp = ctypes.c_void_p
    S = (vp * 2)(FAKE, None)
    B = (ctypes.c_size_t * 2)(16, 16)
    D = (vp * 2)(FAKE, FAKE)
    _err(L.qwfn_state_restore(S, B, D, 2, 1, 0, None), K.EINVAL, "source part 1")
    _err(L.qwfn_state_restore(S, B, D, 2, 0, 0, None), K.EINVAL, "n_slots")
    _err(L.qwfn_state_restore(S, B, D, 2, 1, 5, None), K.EINVAL, "source kind")


def test_fused_append_attention_validation():
    L = K.load()
    r = ctypes.byref
    q4, k4, o4 = _fa_views()
    src = K.tensor(FAKE, K.TYPE_F32, (512, 3), (4, 2048))
    call = lambda sk, sv, first, q=q4, k=k4: L.qwfn_flash_attn_ext_q8_0_append(
        r(q), r(k), r(k), None, 0.0625, 0.0, 0.0, r(o4), 1, None, 0, r(sk), r(sv), first, None)
    _err(call(src, src, 10 ** 9), K.ERANGE, "inside the attended keys")
    _err(call(src, src, -1), K.ERANGE, "inside the attended keys")
    _err(call(K.tensor(FAKE, K.TYPE_F32, (256, 3), (4, 1024)), src, 0), K.EINVAL, "every KV head")
    _err(call(K.tensor(FAKE, K.TYPE_F32, (512, 65), (4, 2048)), K.tensor(FAKE, K.TYPE_F32, (512, 65), (4, 2048)), 0),
         K.ENOTSUP, "1 to 64")
    _err(call(K.tensor(FAKE + 4, K.TYPE_F32, (512, 3), (4, 2048)), src, 0), K.EALIGN, "16-byte")
    _err(call(src, K.tensor(FAKE, K.TYPE_F32, (512, 2), (4, 2048)), 0), K.EINVAL, "same shape")
    _err(call(K.tensor(FAKE, K.TYPE_F16, (512, 3), (2, 1024)), src, 0), K.EINVAL, "f32")


def test_ragged_batch_validation():
    L = K.load()
    r = ctypes.byref
    q4, k4, o4 = _fa_views()
    seq = (ctypes.c_int64 * 1)(101)
    _err(L.qwfn_flash_attn_ext_q8_0_seq(r(q4), r(k4), r(k4), None, 0.0625, 0.0, 0.0, r(o4), 1, None, 0, seq, None),
         K.ERANGE, "[0, n_kv]")
    _err(L.qwfn_flash_attn_ext_q8_0_seq(r(q4), r(k4), r(k4), None, 0.0625, 0.0, 0.0, r(o4), 1, None, 0, None, None),
         K.EINVAL, "NULL")
    B = 17
    q = K.tensor(FAKE, K.TYPE_F32, (256, 1, 16, B), (4, 16 * 1024, 1024, 16 * 1024))
    k = K.tensor(FAKE, K.TYPE_Q8_0, (256, 100, 2, B), (34, 544, 272, 1 << 20))
    o = K.tensor(FAKE, K.TYPE_F32, (256, 16, 1, B), (4, 1024, 16 * 1024, 16 * 1024))
    seq = (ctypes.c_int64 * B)(*([50] * B))
    _err(L.qwfn_flash_attn_ext_q8_0_seq(r(q), r(k), r(k), None, 0.0625, 0.0, 0.0, r(o), 1, None, 0, seq, None),
         K.ENOTSUP, "at most 16")
    assert L.qwfn_fattn_workspace_size_seq(r(q4), r(k4), r(k4), None, None) == 0


def test_cells_attention_validation():
    L = K.load()
    r = ctypes.byref
    q, k, o = _fa_views()
    n = (ctypes.c_int64 * 2)(8, 5)

    def call(qq, kk, cells, counts, stride, pos0=50):
        return L.qwfn_flash_attn_ext_q8_0_cells(r(qq), r(kk), r(kk), cells, counts, stride, pos0, 0.0625, r(o), 1,
                                                None, 0, None)
    _err(call(q, k, None, n, 8), K.EINVAL, "NULL")
    _err(call(q, k, FAKE, None, 8), K.EINVAL, "NULL")
    _err(call(q, k, FAKE + 4, n, 8), K.EALIGN, "16-byte")
    _err(call(q, k, FAKE, n, 6), K.EALIGN, "cell_stride")
    _err(call(q, k, FAKE, n, -4), K.EALIGN, "cell_stride")
    _err(call(q, k, FAKE, (ctypes.c_int64 * 2)(9, 5), 8), K.ERANGE, "[0, cell_stride]")
    _err(call(q, k, FAKE, (ctypes.c_int64 * 2)(-1, 5), 0), K.ERANGE, "[0, cell_stride]")
    _err(call(q, k, FAKE, n, 8, -1), K.EINVAL, "pos0")
    q9, k9, _ = _fa_views(nh=18, nh_kv=9)
    _err(call(q9, k9, FAKE, (ctypes.c_int64 * 9)(*([4] * 9)), 4), K.ENOTSUP, "1 to 8 KV heads")
    q5, k5, _ = _fa_views(T=5)
    _err(call(q5, k5, FAKE, n, 8), K.ENOTSUP, "at most 32 query rows")
    big = K.tensor(FAKE, K.TYPE_Q8_0, (256, 1 << 22, 2, 1), (34, 544, 272, 1 << 20))
    _err(call(q, big, FAKE, n, 8), K.ENOTSUP, "2 GiB")
    # sizing is host-only: one 512-cell split per block at most, partials when there are several splits
    assert L.qwfn_fattn_workspace_size_cells(r(q5), r(k5), r(k5), n, 8) == 0
    one = L.qwfn_fattn_workspace_size_cells(r(q), r(k), r(k), (ctypes.c_int64 * 2)(4000, 3000), 4000)
    assert one >= 2 * 8 * 8 * 256 * 4


def test_qsa_pool_validation():
    L = K.load()
    cfg = K.qsa_pool_cfg()
    assert (cfg.idx_dim, cfg.n_dims, list(cfg.sections), cfg.freq_base, cfg.rms_eps) == (128, 64, [11, 11, 10, 0],
                                                                                        1e7, pytest.approx(1e-6))
    r = ctypes.byref
    _err(L.qwfn_qsa_pool_rebuild(FAKE, 100, 64, 0, FAKE, FAKE, 10, r(cfg), None), K.EINVAL, "ratio")
    _err(L.qwfn_qsa_pool_rebuild(FAKE, 100, 640, 32, FAKE, FAKE, 10, r(cfg), None), K.ERANGE, "index cache")
    _err(L.qwfn_qsa_pool_rebuild(FAKE, 1000, 640, 32, FAKE, FAKE, 10, r(cfg), None), K.ERANGE, "pool rows")
    _err(L.qwfn_qsa_pool_rebuild(FAKE, 1000, -1, 32, FAKE, FAKE, 10, r(cfg), None), K.EINVAL, "n_past")
    bad = K.qsa_pool_cfg(n_dims=65)
    _err(L.qwfn_qsa_pool_rebuild(FAKE, 1000, 64, 32, FAKE, FAKE, 10, r(bad), None), K.EINVAL, "n_dims")
    bad = K.qsa_pool_cfg(idx_dim=512)
    _err(L.qwfn_qsa_pool_rebuild(FAKE, 1000, 64, 32, FAKE, FAKE, 10, r(bad), None), K.ENOTSUP, "idx_dim")
    bad = K.qsa_pool_cfg(sections=[0, 0, 0, 0])
    _err(L.qwfn_qsa_pool_rebuild(FAKE, 1000, 64, 32, FAKE, FAKE, 10, r(bad), None), K.EINVAL, "sections")
    _err(L.qwfn_qsa_pool_decode(FAKE, 100, FAKE, None, FAKE, 32, FAKE, FAKE, FAKE, FAKE, 10, r(cfg), None),
         K.EINVAL, "NULL")
    _err(L.qwfn_qsa_pool_decode(FAKE + 1, 100, None, None, FAKE, 32, FAKE, FAKE, FAKE, FAKE, 10, r(cfg), None),
         K.EALIGN, "alignment")
    d = K.tensor(FAKE, K.TYPE_F16, (128, 10), (2, 256))
    s = K.tensor(FAKE, K.TYPE_F32, (128, 2), (4, 512))
    i = K.tensor(FAKE, K.TYPE_I32, (2,), (4,))
    _err(L.qwfn_set_rows_f16(r(d), r(s), r(K.tensor(FAKE, K.TYPE_I32, (3,), (4,))), None), K.EINVAL, "idx [n]")
    _err(L.qwfn_set_rows_f16(r(s), r(s), r(i), None), K.EINVAL, "f16")
