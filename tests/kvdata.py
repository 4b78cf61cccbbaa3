"""Seeded synthetic inputs for the q8_0 KV-cache path, shared by tests and smoke.

Every tensor comes from the oracle's SplitMix64-seeded xoshiro256** stream,
keyed by (config seed, layer, tensor kind, extra), so CPU and GPU see identical
bytes. Shapes follow the reference's attention layers: n_head_kv = 2, head size
256, a token-major q8_0 cache row of 544 bytes (qwfn_state.cpp:48-91).
"""
from __future__ import annotations

import numpy as np

from oracle import oracle as O

HD = 256
SEG = HD // 32 * 34          # 272 bytes per KV head per row
K_KIND, V_KIND, Q_KIND, SCORE_KIND, STATE_KIND = 1, 2, 3, 4, 5


def normal(seed: int, layer: int, kind: int, n: int, extra: int = 0, std: float = 1.0) -> np.ndarray:
    return O.normal(O.stream_key(seed, layer, kind, extra), n, std)


def outlier_channels(seed: int, layer: int, n_head_kv: int, hd: int = HD, n: int = 4) -> np.ndarray:
    """n distinct channels per KV head, drawn without replacement from [0, hd)."""
    out = np.zeros((n_head_kv, n), dtype=np.int64)
    for h in range(n_head_kv):
        u = O.uniform(O.stream_key(seed, layer, 99, h), hd)
        out[h] = np.argsort(u, kind="stable")[:n]
    return out


def kv_rows(seed: int, layer: int, kind: int, n_rows: int, first_row: int = 0, n_head_kv: int = 2,
            hd: int = HD, outliers: bool = False) -> np.ndarray:
    """F32 [n_rows, n_head_kv*hd] K or V rows ~N(0,1); row r drawn from its own stream."""
    kv_dim = n_head_kv * hd
    # one stream per block of 1024 rows keeps generation of a row range cheap
    out = np.empty((n_rows, kv_dim), dtype=np.float32)
    r = 0
    while r < n_rows:
        g = (first_row + r) // 1024
        g0 = g * 1024
        lo = first_row + r - g0
        cnt = min(1024 - lo, n_rows - r)
        blk = normal(seed, layer, kind, 1024 * kv_dim, extra=g).reshape(1024, kv_dim)
        out[r:r + cnt] = blk[lo:lo + cnt]
        r += cnt
    if outliers:
        ch = outlier_channels(seed, layer, n_head_kv, hd)
        for h in range(n_head_kv):
            out[:, h * hd + ch[h]] *= 8.0
    return out


def q_rows(seed: int, layer: int, T: int, n_head: int, hd: int = HD, batch: int = 1) -> np.ndarray:
    """F32 Q, [batch, T, n_head, hd] ~N(0,1)."""
    return normal(seed, layer, Q_KIND, batch * T * n_head * hd).reshape(batch, T, n_head, hd)


def make_cache(rows_f32: np.ndarray, n_ctx: int, variant: int = O.Q8_X86, first_row: int = 0) -> np.ndarray:
    """uint8 [n_ctx, row_bytes] cache with rows quantised at first_row.. (others zero)."""
    kv_dim = rows_f32.shape[1]
    cache = np.zeros((n_ctx, kv_dim // 32 * 34), dtype=np.uint8)
    cache[first_row:first_row + rows_f32.shape[0]] = O.quantize(rows_f32, variant)
    return cache


def oracle_attn(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, n_kv: int, n_head_kv: int,
                mask: np.ndarray | None, scale: float, variant: int = O.Q8_X86, threads: int = 8,
                native: bool = False) -> np.ndarray:
    """ggml-cpu flash_attn_ext over a token-major cache. q [T, nh, hd]; mask F16 bits [T, n_kv] or None.
    Returns [T, nh, hd] float32. native: the -march=native build of the same C (CPU timing only)."""
    T, nh, hd = q.shape
    q = np.ascontiguousarray(q, np.float32)
    qv, kv, vv = O.cache_views(q, kc, vc, n_kv, n_head_kv, hd)
    mv = O.mask_view(mask) if mask is not None else None
    return O.flash_attn_ext(qv, kv, vv, mv, scale, (T, nh, hd), variant, variant, threads, native=native)


def oracle_attn_f64(q, kc, vc, n_kv, n_head_kv, mask, scale, quantize_q: int = 2) -> np.ndarray:
    T, nh, hd = q.shape
    q = np.ascontiguousarray(q, np.float32)
    qv, kv, vv = O.cache_views(q, kc, vc, n_kv, n_head_kv, hd)
    mv = O.mask_view(mask) if mask is not None else None
    return O.attn_f64(qv, kv, vv, mv, scale, (T, nh, hd), quantize_q)


def selection_lists(seed: int = 4, n_ctx: int = 65536, blocks: int = 1024, bsz: int = 64, top: int = 128,
                    tail: int = 512, n_head_kv: int = 2) -> list[np.ndarray]:
    """Sparse selection per KV head: the top-`top` of `blocks` blocks of `bsz`
    positions by seeded uniform scores (ties to the lower block) united with
    the last `tail` positions; ascending int32 cell lists."""
    lists = []
    for h in range(n_head_kv):
        u = O.uniform(O.stream_key(seed, 0, SCORE_KIND, h), blocks)
        order = np.argsort(-u, kind="stable")[:top]
        pos = (order[:, None] * bsz + np.arange(bsz)[None, :]).reshape(-1)
        lists.append(np.union1d(pos, np.arange(n_ctx - tail, n_ctx)).astype(np.int32))
    return lists


def oracle_attn_cells(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, lists, pos0: int, scale: float,
                      variant: int = O.Q8_X86) -> np.ndarray:
    """ggml-cpu attention of query t (position pos0 + t) over the cache rows that
    KV head h's list names (repeats count), those at most pos0 + t and inside
    the cache: the gathered copy with its cell mask. q [T, nh, hd]; a query row
    that sees no cell is 0."""
    T, nh, hd = q.shape
    nh_kv = len(lists)
    g = nh // nh_kv
    seg = hd // 32 * 34
    out = np.zeros((T, nh, hd), np.float32)
    for h in range(nh_kv):
        lst = np.asarray(lists[h], np.int64)
        for t in range(T):
            sel = lst[(lst >= 0) & (lst < kc.shape[0]) & (lst <= pos0 + t)]
            if len(sel) == 0:
                continue
            kh = np.ascontiguousarray(kc[sel][:, h * seg:(h + 1) * seg])
            vh = np.ascontiguousarray(vc[sel][:, h * seg:(h + 1) * seg])
            out[t, h * g:(h + 1) * g] = oracle_attn(q[t:t + 1, h * g:(h + 1) * g], kh, vh, len(sel), 1, None, scale,
                                                    variant)[0]
    return out


def err_stats(got: np.ndarray, ref: np.ndarray) -> tuple[float, float]:
    d = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    return float(d.max()), float(d.mean())


MAX_ABS_TOL = 2e-3      # tolerance of the attention outputs vs ggml-cpu semantics
MEAN_ABS_TOL = 1e-3
