"""ctypes binding of the CPU oracle (liboracle.so). TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg import
this module, and only to check results. The product library never loads it.

The C sources restate ggml-cpu semantics for the q8_0 KV-cache path; see the
header of oracle.c for the ggml functions and reference call sites they follow.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

Q8_REF = 0
Q8_X86 = 1
QK8_0 = 32
Q8_0_BLOCK_BYTES = 34


class View(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p),
                ("ne", ctypes.c_int64 * 4),
                ("nb", ctypes.c_size_t * 4)]


_lib = None


def build(force: bool = False) -> str:
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE, "-B" if force else "liboracle.so"], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        vp, i64, u64, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint64, ctypes.c_size_t
        L.oracle_splitmix64.argtypes = [ctypes.POINTER(u64)]
        L.oracle_splitmix64.restype = u64
        L.oracle_rng_seed.argtypes = [vp, u64]
        L.oracle_rng_next.argtypes = [vp]
        L.oracle_rng_next.restype = u64
        L.oracle_stream_key.argtypes = [u64, u64, u64, u64]
        L.oracle_stream_key.restype = u64
        L.oracle_fill_normal.argtypes = [u64, vp, i64, ctypes.c_double]
        L.oracle_fill_uniform.argtypes = [u64, vp, i64]
        L.oracle_fp32_to_fp16.argtypes = [ctypes.c_float]
        L.oracle_fp32_to_fp16.restype = ctypes.c_uint16
        L.oracle_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        L.oracle_fp16_to_fp32.restype = ctypes.c_float
        L.oracle_quantize_row_q8_0.argtypes = [vp, vp, i64, ctypes.c_int]
        L.oracle_dequantize_row_q8_0.argtypes = [vp, vp, i64]
        L.oracle_vec_dot_q8_0_q8_0.argtypes = [i64, vp, vp, ctypes.c_int]
        L.oracle_vec_dot_q8_0_q8_0.restype = ctypes.c_float
        L.oracle_set_rows_q8_0.argtypes = [vp, sz, i64, vp, sz, i64, vp, i64, ctypes.c_int]
        L.oracle_cpy_f32_q8_0.argtypes = [vp, sz, i64, i64, vp, sz, i64, i64, ctypes.c_int]
        L.oracle_get_rows.argtypes = [vp, sz, i64, sz, vp, i64, vp, sz]
        L.oracle_flash_attn_ext_q8_0.argtypes = [ctypes.POINTER(View)] * 4 + [
            ctypes.c_float, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.oracle_attn_f64.argtypes = [ctypes.POINTER(View)] * 4 + [ctypes.c_double, vp, ctypes.c_int]
        L.oracle_rms_norm_f32.argtypes = [vp, vp, i64, ctypes.c_float]
        L.oracle_rope_multi_f32.argtypes = [vp, vp, i64, ctypes.c_int, vp, vp, ctypes.c_int, ctypes.c_float]
        L.oracle_set_rows_f16.argtypes = [vp, i64, i64, vp, vp, i64]
        L.oracle_kv_produce_q8_0.argtypes = [vp, i64, i64, vp, vp, i64, vp, vp, vp, ctypes.c_int, ctypes.c_float,
                                             ctypes.c_float, vp, vp, vp, vp, ctypes.c_int, ctypes.c_int]
        L.oracle_fp32_to_bf16.argtypes = [ctypes.c_float]
        L.oracle_fp32_to_bf16.restype = ctypes.c_uint16
        L.oracle_bf16_to_fp32.argtypes = [ctypes.c_uint16]
        L.oracle_bf16_to_fp32.restype = ctypes.c_float
        L.oracle_gated_delta_net.argtypes = [vp, i64, vp, i64, vp, i64, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64,
                                             i64, ctypes.c_float]
        L.oracle_qsa_pool_blocks.argtypes = [vp, i64, vp, i64, i64, vp, vp, vp, ctypes.c_float, ctypes.c_float,
                                             ctypes.c_int, vp]
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


# ------------------------------------------------------------------ PRNG

def stream_key(seed: int, a: int = 0, b: int = 0, c: int = 0) -> int:
    return int(lib().oracle_stream_key(seed, a, b, c))


def normal(key: int, n: int, stddev: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().oracle_fill_normal(key, _p(out), n, stddev)
    return out


def uniform(key: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().oracle_fill_uniform(key, _p(out), n)
    return out


def splitmix64_stream(state: int, n: int) -> list[int]:
    s = ctypes.c_uint64(state)
    return [int(lib().oracle_splitmix64(ctypes.byref(s))) for _ in range(n)]


def xoshiro_stream(seed: int, n: int) -> list[int]:
    st = (ctypes.c_uint64 * 4)()
    lib().oracle_rng_seed(st, seed)
    return [int(lib().oracle_rng_next(st)) for _ in range(n)]


# ------------------------------------------------------------------ q8_0

def fp32_to_fp16_bits(x: np.ndarray) -> np.ndarray:
    f = lib().oracle_fp32_to_fp16
    return np.array([f(float(v)) for v in np.asarray(x, np.float32).ravel()], dtype=np.uint16)


def fp16_bits_to_fp32(h: np.ndarray) -> np.ndarray:
    f = lib().oracle_fp16_to_fp32
    return np.array([f(int(v)) for v in np.asarray(h, np.uint16).ravel()], dtype=np.float32)


def quantize(x: np.ndarray, variant: int = Q8_X86) -> np.ndarray:
    """F32 [..., k] -> q8_0 bytes [..., k/32*34] (uint8)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    assert k % QK8_0 == 0
    out = np.empty(x.shape[:-1] + (k // QK8_0 * Q8_0_BLOCK_BYTES,), dtype=np.uint8)
    lib().oracle_quantize_row_q8_0(_p(x), _p(out), x.size, variant)
    return out


def dequantize(y: np.ndarray) -> np.ndarray:
    y = np.ascontiguousarray(y, dtype=np.uint8)
    nbytes = y.shape[-1]
    assert nbytes % Q8_0_BLOCK_BYTES == 0
    k = nbytes // Q8_0_BLOCK_BYTES * QK8_0
    out = np.empty(y.shape[:-1] + (k,), dtype=np.float32)
    lib().oracle_dequantize_row_q8_0(_p(y), _p(out), out.size)
    return out


def vec_dot(x: np.ndarray, y: np.ndarray, variant: int = Q8_X86) -> float:
    x = np.ascontiguousarray(x, np.uint8)
    y = np.ascontiguousarray(y, np.uint8)
    n = x.size // Q8_0_BLOCK_BYTES * QK8_0
    return float(lib().oracle_vec_dot_q8_0_q8_0(n, _p(x), _p(y), variant))


def set_rows(cache: np.ndarray, src: np.ndarray, idx: np.ndarray, variant: int = Q8_X86) -> None:
    """In place on a uint8 cache [n_rows, row_bytes]; src F32 [n, ne0]; idx I32 [n]."""
    src = np.ascontiguousarray(src, np.float32)
    idx = np.ascontiguousarray(idx, np.int32)
    rc = lib().oracle_set_rows_q8_0(_p(cache), cache.strides[0], cache.shape[0], _p(src), src.strides[0],
                                    src.shape[1], _p(idx), idx.size, variant)
    if rc:
        raise ValueError(f"oracle set_rows failed ({rc})")


def cpy(cache: np.ndarray, src: np.ndarray, first_row: int, variant: int = Q8_X86) -> None:
    src = np.ascontiguousarray(src, np.float32)
    rc = lib().oracle_cpy_f32_q8_0(_p(cache), cache.strides[0], first_row, cache.shape[0], _p(src),
                                   src.strides[0], src.shape[1], src.shape[0], variant)
    if rc:
        raise ValueError(f"oracle cpy failed ({rc})")


def get_rows(src: np.ndarray, idx: np.ndarray, row_bytes: int | None = None, col_off: int = 0) -> np.ndarray:
    """Copy row_bytes bytes (from byte col_off) of each indexed row of a uint8 [rows, stride] array."""
    idx = np.ascontiguousarray(idx, np.int32)
    rb = src.shape[1] - col_off if row_bytes is None else row_bytes
    dst = np.zeros((idx.size, rb), dtype=np.uint8)
    base = src[:, col_off:]
    rc = lib().oracle_get_rows(base.ctypes.data, src.strides[0], src.shape[0], rb, _p(idx), idx.size,
                               _p(dst), dst.strides[0])
    if rc:
        raise ValueError(f"oracle get_rows failed ({rc})")
    return dst


# ------------------------------------------------------------------ attention

def view(data: np.ndarray, ne, nb) -> View:
    v = View()
    v.data = data.ctypes.data
    for i in range(4):
        v.ne[i] = int(ne[i]) if i < len(ne) else 1
    last = 0
    for i in range(4):
        if i < len(nb):
            v.nb[i] = int(nb[i])
            last = v.nb[i] * v.ne[i]
        else:
            v.nb[i] = last
            last = v.nb[i] * v.ne[i]
    return v


NATIVE_PATH = os.path.join(HERE, "liboracle_native.so")
_native = None


def native_lib():
    """The same C source built with -march=native (`make -C oracle native`): a separate
    library used only to time the CPU baseline; the tests check against lib()."""
    global _native
    if _native is None:
        # built on first use in each process, for the host it runs on (a build
        # shipped from another machine might use instructions this CPU lacks)
        subprocess.run(["make", "-B", "-s", "-C", HERE, "liboracle_native.so"], check=True)
        L = ctypes.CDLL(NATIVE_PATH)
        L.oracle_flash_attn_ext_q8_0.argtypes = lib().oracle_flash_attn_ext_q8_0.argtypes
        L.oracle_flash_attn_ext_q8_0.restype = lib().oracle_flash_attn_ext_q8_0.restype
        _native = L
    return _native


def flash_attn_ext(qv: View, kv: View, vv: View, mv: View | None, scale: float, out_shape,
                   q_variant: int = Q8_X86, dot_variant: int = Q8_X86, n_threads: int = 1,
                   native: bool = False) -> np.ndarray:
    dst = np.zeros(out_shape, dtype=np.float32)
    L = native_lib() if native else lib()
    rc = L.oracle_flash_attn_ext_q8_0(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv),
                                      ctypes.byref(mv) if mv is not None else None, scale, _p(dst),
                                      q_variant, dot_variant, n_threads)
    if rc:
        raise ValueError(f"oracle flash_attn_ext failed ({rc})")
    return dst


def attn_f64(qv: View, kv: View, vv: View, mv: View | None, scale: float, out_shape,
             quantize_q: int = 0) -> np.ndarray:
    dst = np.zeros(out_shape, dtype=np.float64)
    rc = lib().oracle_attn_f64(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv),
                               ctypes.byref(mv) if mv is not None else None, scale, _p(dst), quantize_q)
    if rc:
        raise ValueError(f"oracle attn_f64 failed ({rc})")
    return dst


def cache_views(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, n_kv: int, n_head_kv: int, hd: int):
    """ggml views for the reference's layout.

    q: F32 [T, n_head, hd] (the projection's natural order; the graph permutes it
    to [hd, T, n_head], qwfn_graph.cpp:466); kc/vc: uint8 caches [n_ctx, row_bytes]
    token-major, KV head h at byte 34*(hd/32)*h (qwfn_graph.cpp:461-464).
    """
    T, nh, _ = q.shape
    seg = hd // QK8_0 * Q8_0_BLOCK_BYTES
    qv = view(q, (hd, T, nh, 1), (4, nh * hd * 4, hd * 4, T * nh * hd * 4))
    kv = view(kc, (hd, n_kv, n_head_kv, 1), (Q8_0_BLOCK_BYTES, kc.strides[0], seg, kc.strides[0] * n_kv))
    vv = view(vc, (hd, n_kv, n_head_kv, 1), (Q8_0_BLOCK_BYTES, vc.strides[0], seg, vc.strides[0] * n_kv))
    return qv, kv, vv


def mask_view(mask_f16_bits: np.ndarray) -> View:
    """mask: uint16 F16 bits [T, n_kv] (ggml [n_kv, T])."""
    T, n_kv = mask_f16_bits.shape
    return view(mask_f16_bits, (n_kv, T, 1, 1), (2, mask_f16_bits.strides[0], mask_f16_bits.strides[0] * T,
                                                 mask_f16_bits.strides[0] * T))


F16_NEG_INF = 0xFC00
F16_ZERO = 0x0000


def causal_mask(T: int, n_past: int, n_kv: int | None = None) -> np.ndarray:
    """F16 bits [T, n_kv]: query i sees rows <= n_past + i (qwfn_engine.cpp:2093-2098, :1261-1271)."""
    n_kv = n_past + T if n_kv is None else n_kv
    m = np.full((T, n_kv), F16_NEG_INF, dtype=np.uint16)
    for i in range(T):
        m[i, :min(n_kv, n_past + i + 1)] = F16_ZERO
    return m


# ------------------------------------------------------- QSA index producer

IMROPE_SECTIONS = (11, 11, 10, 0)     # qwfn_hparams.h:36
ROPE_FREQ_BASE = 10000000.0           # qwfn_hparams.h:34
ROPE_DIM = 64                         # qwfn_hparams.h:35
RMS_EPS = 1e-6                        # qwfn_hparams.h:26


def rms_norm(x: np.ndarray, eps: float = RMS_EPS) -> np.ndarray:
    """ggml_rms_norm over the last axis (float32); qwfn_graph.cpp:124-126, :443, :295."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    n = x.shape[-1]
    xf, yf = x.reshape(-1, n), y.reshape(-1, n)
    for i in range(xf.shape[0]):
        lib().oracle_rms_norm_f32(_p(xf[i]), _p(yf[i]), n, eps)
    return y


def rope_multi(x: np.ndarray, pos, n_dims: int = ROPE_DIM, sections=IMROPE_SECTIONS, imrope: bool = True,
               freq_base: float = ROPE_FREQ_BASE) -> np.ndarray:
    """ggml_rope_multi (IMROPE) of one or more heads (last axis) at one position (t, h, w, e);
    qwfn_graph.cpp:128-131, :297-299, :911-913."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    n = x.shape[-1]
    p4 = np.ascontiguousarray(np.broadcast_to(np.asarray(pos, np.int32), (4,)))
    sec = np.ascontiguousarray(np.asarray(sections, np.int32))
    xf, yf = x.reshape(-1, n), y.reshape(-1, n)
    for i in range(xf.shape[0]):
        lib().oracle_rope_multi_f32(_p(xf[i]), _p(yf[i]), n, n_dims, _p(p4), _p(sec), int(imrope), freq_base)
    return y


def set_rows_f16(dst_bits: np.ndarray, src: np.ndarray, idx: np.ndarray) -> None:
    """ggml_set_rows F32 -> F16 (qwfn_graph.cpp:543, the raw indexer key):
    dst_bits uint16 [rows, ne0] in place, row idx[i] = fp16(src[i])."""
    src = np.ascontiguousarray(src, np.float32)
    idx = np.ascontiguousarray(idx, np.int32)
    rc = lib().oracle_set_rows_f16(_p(dst_bits), dst_bits.shape[0], dst_bits.shape[1], _p(src), _p(idx), len(idx))
    if rc:
        raise IndexError("set_rows_f16: index out of range")


def qsa_pool_blocks(ic_bits: np.ndarray, members: np.ndarray, r: int, k_norm_w: np.ndarray, pos4: np.ndarray,
                    n_dims: int = ROPE_DIM, sections=IMROPE_SECTIONS, eps: float = RMS_EPS,
                    freq_base: float = ROPE_FREQ_BASE) -> np.ndarray:
    """qsa_pool_blocks (qwfn_graph.cpp:282-301; decode :544-549, rebuild qwfn_engine.cpp:1121-1145):
    pooled F16 bits [n_blk, idx_dim] from members [n_blk * r] rows of ic_bits (uint16 [rows, idx_dim]),
    pos4 [n_blk, 4] int32 (t, h, w, e)."""
    ic_bits = np.ascontiguousarray(ic_bits, np.uint16)
    members = np.ascontiguousarray(members, np.int32)
    n_blk = len(members) // r
    out = np.zeros((n_blk, ic_bits.shape[1]), np.uint16)
    w = np.ascontiguousarray(k_norm_w, np.float32)
    p4 = np.ascontiguousarray(pos4, np.int32).reshape(-1)
    sec = np.ascontiguousarray(np.asarray(sections, np.int32))
    lib().oracle_qsa_pool_blocks(_p(ic_bits), ic_bits.shape[1], _p(members), r, n_blk, _p(w), _p(p4), _p(sec),
                                 eps, freq_base, n_dims, _p(out))
    return out


def fp32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """F32 -> BF16 bits, round to nearest even (the conversion of ggml_mul_mat's src1 for BF16 weights)."""
    L = lib()
    return np.array([L.oracle_fp32_to_bf16(float(v)) for v in np.asarray(x, np.float32).ravel()],
                    np.uint16).reshape(np.shape(x))


def kv_produce(cur: np.ndarray, wk_bits: np.ndarray, wv_bits: np.ndarray, k_norm_w: np.ndarray, pos: np.ndarray,
               variant: int = Q8_X86, n_dims: int = ROPE_DIM, sections=IMROPE_SECTIONS, freq_base: float = ROPE_FREQ_BASE,
               eps: float = RMS_EPS, w_bf16: bool = False):
    """The K/V producer (qwfn_graph.cpp:441-451, then the append of :370-384 / :623-624):
    cur f32 [T, E]; w*_bits uint16 [kv_dim, E] (F16 bits, or BF16 bits with w_bf16); pos int32 [4*T].
    Returns (k_rows, v_rows, k_f32, v_f32): q8_0 rows uint8 [T, kv_dim/32*34] and the float rows
    before quantisation [T, kv_dim]."""
    cur = np.ascontiguousarray(cur, np.float32)
    T, E = cur.shape
    kv_dim = wk_bits.shape[0]
    rb = kv_dim // QK8_0 * Q8_0_BLOCK_BYTES
    k_rows = np.zeros((T, rb), np.uint8)
    v_rows = np.zeros((T, rb), np.uint8)
    k_f = np.zeros((T, kv_dim), np.float32)
    v_f = np.zeros((T, kv_dim), np.float32)
    sec = np.ascontiguousarray(np.asarray(sections, np.int32))
    lib().oracle_kv_produce_q8_0(_p(cur), E, T, _p(np.ascontiguousarray(wk_bits, np.uint16)),
                                 _p(np.ascontiguousarray(wv_bits, np.uint16)), kv_dim,
                                 _p(np.ascontiguousarray(k_norm_w, np.float32)), _p(np.ascontiguousarray(pos, np.int32)),
                                 _p(sec), n_dims, freq_base, eps, _p(k_rows), _p(v_rows), _p(k_f), _p(v_f), variant,
                                 1 if w_bf16 else 0)
    return k_rows, v_rows, k_f, v_f


def gated_delta_net(q: np.ndarray, k: np.ndarray, v: np.ndarray, g: np.ndarray, beta: np.ndarray, state: np.ndarray,
                    n_snap: int = 0, scale: float | None = None):
    """The gated delta rule of ggml_gated_delta_net (qwfn_graph.cpp:240-278, snapshots :210-238; an op of
    the reference's ggml fork, parity unpinned beyond the fp64 brute force and closed forms):
    q, k f32 [T, n_k, dk]; v [T, n_v, dv]; g, beta [T, n_v]; state [n_v, dk, dv] (not modified).
    Returns (out [T, n_v, dv], final state, snapshots [n_snap, n_v, dk, dv])."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    T, n_k, dk = q.shape
    n_v, dv = v.shape[1], v.shape[2]
    st = np.ascontiguousarray(state, np.float32).copy()
    out = np.zeros((T, n_v, dv), np.float32)
    snap = np.zeros((max(n_snap, 1), n_v, dk, dv), np.float32)
    scale = float(1.0 / np.sqrt(dk)) if scale is None else scale
    lib().oracle_gated_delta_net(_p(q), n_k * dk, _p(k), n_k * dk, _p(v), n_v * dv,
                                 _p(np.ascontiguousarray(g, np.float32)), _p(np.ascontiguousarray(beta, np.float32)),
                                 _p(st), _p(out), _p(snap) if n_snap else None, n_snap, T, n_k, n_v, dk, dv, scale)
    return out, st, snap[:n_snap]
