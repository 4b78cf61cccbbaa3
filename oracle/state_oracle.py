"""CPU restatement of the reference's per-sequence state bookkeeping and step
inputs. TEST INFRASTRUCTURE ONLY: imported by tests/ and nothing else.

Each function follows the reference file:line named in its docstring:

* state layout and summary       qwfn_state.cpp:48-91, :154-173
* snapshot part list             qwfn_engine.cpp:988-999 (snapshot_parts)
* rollback bookkeeping           qwfn_engine.cpp:2033-2035, :3629-3660
* decode sparse-attention inputs qwfn_engine.cpp:1072-1105 (qsa_decode_prepare),
                                 :3582-3614 (qsa_decode_prepare_k),
                                 :1107-1125 (qsa_pool_rebuild), :672-684 (init_qsa_tables)
* masks                          qwfn_engine.cpp:1261-1271, :2093-2098, :3415-3421;
                                 qwfn_graph.cpp:668-675, :681-693 (cell mask, padding)
* saved-sequence pool            tools/qwfn_server.cpp:767-793, :1380-1424
* prefill sparse-attention inputs qwfn_engine.cpp:1276-1320 (fill_chunk_qsa);
                                 qwfn_graph.cpp:388-414 (qsa_mask)

How each is pinned (tests/test_state_cpu.py): the layout and summary by the
summary line the reference's own runs logged at 73728 positions and by the
sizes in qwfn_state.h:4-8; the part list by closed-form byte counts; the bias
window by its equality with the full rebuild after every decode position; the
three causal-mask builders by their agreement with each other; the cell mask's
ggml op chain (float arithmetic) by the integer comparison it reduces to; the
pool by scripted cases whose outcomes follow from the server's rules (count
and byte caps, replacement of an equal sequence, strict extension, the split
conditions) and by the invariants the server asserts; the prefill chunk's
tables and bias by the per-block closed form (whole block ending at or before
the query: 0; the block holding it mid-block, or the partial tail block at or
before it: 1e9; a block wholly after it: -1e9); the selection mask by its
limits (every cell selected: the causal mask; none: all -inf) and the set of
zeros it must hold (selected and causally visible).
"""
from __future__ import annotations

import numpy as np

TYPE_F32, TYPE_F16, TYPE_Q8_0 = 0, 1, 8
K, V, IDX, RS, CONV, PLE_CONV = range(6)
TYPE_NAME = {TYPE_F32: "f32", TYPE_F16: "f16", TYPE_Q8_0: "q8_0"}
F16_ZERO, F16_NEG_INF = 0x0000, 0xFC00


def config_default(n_ctx: int) -> dict:
    """The model's hyper-parameters (qwfn_hparams.h:16-80 comments)."""
    return dict(n_ctx=n_ctx, n_layer=48, full_attention_interval=4, n_head_kv=2, n_embd_head_k=256,
                n_embd_head_v=256, idx_key_len=128, ssm_d_state=128, ssm_n_group=16, ssm_dt_rank=48,
                ssm_d_conv=4, hc_count=4, n_embd=2560, ple_n_head=16, ple_conv_kernel=4, ple_ngram_size=3,
                type_k=TYPE_Q8_0, type_v=TYPE_Q8_0, type_idx=TYPE_F16, kv_host=0, idx_host=0, n_rollback=0)


def is_attn_layer(cfg: dict, il: int) -> bool:
    """qwfn_hparams.h:85-87."""
    fai = cfg["full_attention_interval"]
    return fai > 0 and (il + 1) % fai == 0


def row_size(typ: int, n: int) -> int:
    """ggml_row_size: q8_0 is 34 bytes per 32 values."""
    if typ == TYPE_Q8_0:
        assert n % 32 == 0
        return n // 32 * 34
    return n * (2 if typ == TYPE_F16 else 4)


def declare_tensors(cfg: dict) -> list[dict]:
    """state::declare_tensors (qwfn_state.cpp:48-91): the tensors in declaration
    order with kind, layer, type, ne and nbytes."""
    n_ctx = cfg["n_ctx"]
    kv_dim = cfg["n_embd_head_k"] * cfg["n_head_kv"]
    v_dim = cfg["n_embd_head_v"] * cfg["n_head_kv"]
    hv = cfg["ssm_d_state"]
    conv_dim = hv * cfg["ssm_n_group"] * 2 + hv * cfg["ssm_dt_rank"]
    hc_dim = cfg["hc_count"] * cfg["n_embd"]
    out = []

    def add(kind, il, typ, ne):
        ne = list(ne) + [1] * (4 - len(ne))
        nbytes = row_size(typ, ne[0]) * ne[1] * ne[2] * ne[3]
        out.append(dict(kind=kind, il=il, type=typ, ne=ne, nbytes=nbytes))

    for il in range(cfg["n_layer"]):
        if is_attn_layer(cfg, il):
            add(K, il, cfg["type_k"], [kv_dim * n_ctx])
            add(V, il, cfg["type_v"], [v_dim * n_ctx])
            add(IDX, il, cfg["type_idx"], [cfg["idx_key_len"] * n_ctx])
        else:
            add(RS, il, TYPE_F32, [hv, hv, cfg["ssm_dt_rank"]])
            add(CONV, il, TYPE_F32, [cfg["ssm_d_conv"] - 1, conv_dim])
    if cfg["ple_n_head"] > 0:
        hist = (cfg["ple_conv_kernel"] - 1) * cfg["ple_ngram_size"]
        add(PLE_CONV, 0, TYPE_F32, [hist, hc_dim])
    return out


def summary(cfg: dict, device_bytes: int, host_bytes: int = 0) -> str:
    """state::summary (qwfn_state.cpp:154-173). ostream's default double format
    is printf's %g."""
    kv = ix = rs = cv = 0
    for t in declare_tensors(cfg):
        if t["kind"] in (K, V):
            kv += t["nbytes"]
        elif t["kind"] == IDX:
            ix += t["nbytes"]
        elif t["kind"] == RS:
            rs += t["nbytes"]
        else:
            cv += t["nbytes"]
    s = (f"state @ {cfg['n_ctx']} ctx: KV {'%g' % (kv / 1e9)} GB ({TYPE_NAME[cfg['type_k']]}), "
         f"indexer {'%g' % (ix / 1e9)} GB, deltanet {'%g' % (rs / 1e6)} MB (constant), "
         f"conv {'%g' % (cv / 1e6)} MB  =>  total {'%g' % (device_bytes / 1e9)} GB on the device")
    if host_bytes:
        s += f" + {'%g' % (host_bytes / 1e9)} GB in pinned host memory"
    return s


def snapshot_parts(cfgs: list[dict], n_past: int) -> list[tuple[int, int, int, int]]:
    """snapshot_parts (qwfn_engine.cpp:990-999) over the states in order:
    (state index, kind, layer, bytes). Positional caches keep
    min(nbytes, n * row bytes), with row bytes = ggml_row_size(type, ne0 / n_ctx);
    recurrent tensors are whole."""
    out = []
    for si, cfg in enumerate(cfgs):
        ts = declare_tensors(cfg)
        by_layer = {}
        for t in ts:
            by_layer.setdefault((t["il"], t["kind"]), t)
        for il in range(cfg["n_layer"]):
            for kind in (K, V, IDX):
                t = by_layer.get((il, kind))
                if t is not None:
                    rb = row_size(t["type"], t["ne"][0] // cfg["n_ctx"])
                    out.append((si, kind, il, min(t["nbytes"], n_past * rb)))
            for kind in (RS, CONV):
                t = by_layer.get((il, kind))
                if t is not None:
                    out.append((si, kind, il, t["nbytes"]))
        for t in ts:
            if t["kind"] == PLE_CONV:
                out.append((si, PLE_CONV, 0, t["nbytes"]))
    return out


def rollback_depth_after_step(T: int, verified: bool, n_snap: int) -> int:
    """eval_batch (qwfn_engine.cpp:2033): depth = min(T-1, rb_nsnap_) after a
    verified decode step of T >= 2 positions with rollback snapshots, else 0."""
    return min(T - 1, n_snap) if (verified and T >= 2 and n_snap > 0) else 0


def rollback_ok(n_back: int, depth: int) -> bool:
    """rollback_n's guard (qwfn_engine.cpp:3630)."""
    return 1 <= n_back <= depth


# ------------------------------------------------------------ decode QSA inputs

def _window(bias: np.ndarray, n_past: int, ratio: int) -> None:
    """The bias window of qwfn_engine.cpp:1093-1096 (and :3604-3607)."""
    nb_max = bias.shape[0]
    b_last = n_past // ratio
    n_bid = (n_past + 1) // ratio
    b = max(0, b_last - 1)
    while b <= b_last + 1 and b < nb_max:
        bias[b] = 0.0 if b < n_bid else (1e9 if b == b_last else -np.inf)
        b += 1


def qsa_decode_prepare(bias: np.ndarray, n_past: int, ratio: int) -> dict:
    """qsa_decode_prepare (qwfn_engine.cpp:1072-1105) without the pool rebuild:
    the per-token inputs, and the bias with this token's window applied in place."""
    b_last = n_past // ratio
    out = dict(write_idx=np.array([n_past], np.int32),
               member_idx=np.array([b_last * ratio + m for m in range(ratio)], np.int32),
               blk_pos=np.array([b_last * ratio] * 4, np.int32),
               blk_idx=np.array([b_last], np.int32),
               npast_f=np.array([n_past], np.float32))
    _window(bias, n_past, ratio)
    out["bias"] = bias
    return out


def qsa_decode_prepare_k(prev_bias: np.ndarray, n_past2: int, ratio: int) -> dict:
    """qsa_decode_prepare_k (qwfn_engine.cpp:3582-3614): the previous position's
    bias copied, then this position's window on top."""
    return qsa_decode_prepare(prev_bias.astype(np.float32).copy(), n_past2, ratio)


def qsa_bucket(n_past: int, ratio: int, nb_max: int) -> int:
    """qwfn_engine.cpp:1099-1101 (and :3608-3611)."""
    b_last = n_past // ratio
    nb = (b_last + 1 + 255) // 256 * 256
    return min(max(nb, 768), nb_max)


def qsa_pool_rebuild_bias(nb_max: int, n_past: int, ratio: int) -> np.ndarray:
    """The full rewrite of qsa_pool_rebuild (qwfn_engine.cpp:1115-1120)."""
    b_last = n_past // ratio
    n_bid = (n_past + 1) // ratio
    full = np.full(nb_max, -np.inf, np.float32)
    for b in range(min(n_bid, nb_max)):
        full[b] = 0.0
    if b_last < nb_max:
        full[b_last] = 0.0 if b_last < n_bid else 1e9
    return full


def qsa_reset_bias(nb_max: int) -> np.ndarray:
    """engine::reset / init_qsa_tables: -inf everywhere (qwfn_engine.cpp:1062-1064, :682-683)."""
    return np.full(nb_max, -np.inf, np.float32)


def qsa_tables(nb_max: int, ratio: int, n_ctx: int, n_whole: int):
    """init_qsa_tables (qwfn_engine.cpp:676-681) and the block positions of
    qsa_pool_rebuild (:1121-1124)."""
    blk_cells = np.array([b * ratio + k for b in range(nb_max) for k in range(ratio)], np.int32)
    cell_pos = np.arange(n_ctx, dtype=np.float32)
    bpa = np.zeros(4 * n_whole, np.int32)
    for sec in range(4):
        for b in range(n_whole):
            bpa[sec * n_whole + b] = b * ratio
    return blk_cells, cell_pos, bpa


# ------------------------------------------------------------------- masks

def attn_inputs_mask(n_past_c: int, Tc: int) -> np.ndarray:
    """build_attn_inputs (qwfn_engine.cpp:1261-1271): per row a run of zeros of
    length min(n_kv, n_past_c + i + 1), then -inf."""
    n_kv = n_past_c + Tc
    m = np.empty((Tc, n_kv), np.uint16)
    for i in range(Tc):
        vis = min(n_kv, n_past_c + i + 1)
        m[i, :vis] = F16_ZERO
        m[i, vis:] = F16_NEG_INF
    return m


def step_inputs_mask(n_past: int, T: int) -> np.ndarray:
    """build_step_inputs (qwfn_engine.cpp:2093-2098): all -inf, then j <= n_past + i set to 0."""
    n_kv = n_past + T
    m = np.full((T, n_kv), F16_NEG_INF, np.uint16)
    for i in range(T):
        for j in range(n_past + i + 1):
            m[i, j] = F16_ZERO
    return m


def mtp_mask(pos: int, n: int) -> np.ndarray:
    """mtp_mask (qwfn_engine.cpp:3415-3421): all 0, then j > pos + i set to -inf."""
    n_kv = pos + n
    m = np.zeros((n, n_kv), np.uint16)
    for i in range(n):
        for j in range(pos + i + 1, n_kv):
            m[i, j] = F16_NEG_INF
    return m


def _f16_bits(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        return x.astype(np.float16).view(np.uint16)


def cell_mask(cells: np.ndarray, n_past: int, n_pad: int) -> tuple[np.ndarray, np.ndarray]:
    """The decode cell mask as the reference's ggml op chain computes it
    (qwfn_graph.cpp:668-675, :685-693), in float32: cp = cell_pos[cell] (= the
    cell as a float, qwfn_engine.cpp:679-680), ok = step((cp - n_past) * -1 + 0.5),
    mask = f16(ok * 1e30 - 1e30), padded with ok = 0; and the padded cell list
    concat(cells, cells[:n_pad - n_cells])."""
    cells = np.asarray(cells, np.int32)
    n = cells.shape[0]
    assert n <= n_pad <= 2 * n
    cp = cells.astype(np.float32)
    dpos = cp - np.float32(n_past)
    ok = ((dpos * np.float32(-1.0) + np.float32(0.5)) > 0).astype(np.float32)
    ok = np.concatenate([ok, np.zeros(n_pad - n, np.float32)])
    mask = _f16_bits(ok * np.float32(1e30) - np.float32(1e30))
    gcells = np.concatenate([cells, cells[:n_pad - n]])
    return mask, gcells


# ------------------------------------------------------- saved-sequence pool

class SnapPool:
    """The server's saved sequences (tools/qwfn_server.cpp:767-793) and the
    decisions around them (restore_or_reset :1380-1400, shared_prefix_split
    :1401-1424). Entries are (tokens, n_past, bytes), least recently used first."""

    def __init__(self, cap: int, max_entries: int = 4):
        self.cap, self.max_entries = cap, max_entries
        self.saved: list[tuple[tuple, int, int]] = []

    def save_seq(self, tok, n_past: int, nbytes: int) -> bool:
        """save_seq (:771-780): a snapshot larger than the cap is not kept; an
        equal token sequence is replaced; the oldest go first."""
        if nbytes > self.cap:
            return False
        tok = tuple(tok)
        for k, e in enumerate(self.saved):
            if e[0] == tok:
                del self.saved[k]
                break
        self.saved.append((tok, n_past, nbytes))
        total = sum(e[2] for e in self.saved)
        while len(self.saved) > self.max_entries or total > self.cap:
            total -= self.saved[0][2]
            del self.saved[0]
        assert len(self.saved) <= self.max_entries and total <= self.cap
        return True

    def best_saved(self, tok, has_images: bool = False) -> int:
        """best_saved (:782-793): the longest saved sequence the prompt strictly extends."""
        if has_images:
            return -1
        tok = tuple(tok)
        best = -1
        for k, (t, _, _) in enumerate(self.saved):
            if len(t) < len(tok) and tok[:len(t)] == t and (best < 0 or len(t) > len(self.saved[best][0])):
                best = k
        return best

    def load(self, k: int):
        """snapshot_load of entry k, then most recently used last (:1395)."""
        e = self.saved[k]
        self.saved = self.saved[:k] + self.saved[k + 1:] + [e]
        return e

    def restore_or_reset(self, consumed, consumed_bytes: int, consumed_has_images: bool, prompt,
                         prompt_has_images: bool = False) -> int:
        """restore_or_reset (:1380-1400): the restored token count, 0 after a reset."""
        if len(consumed) >= 2048 and not consumed_has_images:
            self.save_seq(consumed, len(consumed), consumed_bytes)
        best = self.best_saved(prompt, prompt_has_images)
        if best >= 0:
            return len(self.load(best)[0])
        return 0

    def shared_prefix_split(self, prompt, n_consumed: int, has_images: bool = False) -> int:
        """shared_prefix_split (:1406-1424)."""
        if has_images or n_consumed >= 2048:
            return 0
        prompt = tuple(prompt)
        L = 0
        for t, _, _ in self.saved:
            m = min(len(t), len(prompt))
            l = 0
            while l < m and t[l] == prompt[l]:
                l += 1
            L = max(L, l)
        have = any(len(t) == L and prompt[:L] == t for t, _, _ in self.saved)
        return L if (L >= 2048 and L + 16 < len(prompt) and L >= n_consumed + 2 and not have) else 0


# ------------------------------------------------- sparse block selection

def qsa_scores(pool_f16: np.ndarray, q: np.ndarray, bias: np.ndarray) -> np.ndarray:
    """qsa_dec_cells' scores (qwfn_graph.cpp:570-576) for one query: ggml's F16
    mul_mat rounds the F32 query to f16 and accumulates the products in f32
    (here in f64, the order-free sum); relu; the sum over indexer heads; the bias."""
    k = pool_f16.astype(np.float64)                       # [n_blocks, 128]
    q16 = q.astype(np.float16).astype(np.float64)         # [n_heads, 128]
    d = k @ q16.T                                         # [n_blocks, n_heads]
    return np.maximum(d, 0.0).sum(axis=1) + bias.astype(np.float64)


def qsa_top_k(score: np.ndarray, k: int) -> np.ndarray:
    """ggml_top_k (qwfn_graph.cpp:577): the k best blocks, best first; equal
    scores keep the lower block first (the order a stable descending sort gives)."""
    return np.argsort(-score, kind="stable")[:k].astype(np.int32)


def qsa_cells(top: np.ndarray, blk_cells: np.ndarray, ratio: int) -> np.ndarray:
    """get_rows(blk_cells, top) reshaped to [k * ratio] (qwfn_graph.cpp:578-579)."""
    return np.concatenate([blk_cells[b * ratio:(b + 1) * ratio] for b in top]).astype(np.int32)


# ------------------------------------------------- prefill sparse-attention inputs

def fill_chunk_qsa(n_past_c: int, Tc: int, ratio: int) -> dict:
    """engine::fill_chunk_qsa (qwfn_engine.cpp:1276-1320) step by step: n_kv =
    n_past_c + Tc keys in n_blocks = ceil(n_kv / ratio) blocks (ai.qsa.n_blocks,
    :1247), n_bid whole ones; cell_blk [n_kv], blk_cells [n_blocks * ratio],
    blk_pos [4 * n_blocks] and the bias [Tc, n_blocks] (row i for query
    n_past_c + i): filled 0 / 1e9 / -inf around tail_b, the dead block set to
    1e9, then positive entries of blocks wholly after the query set to -1e9."""
    n_kv = n_past_c + Tc
    n_blocks = (n_kv + ratio - 1) // ratio
    n_bid = n_kv // ratio
    have_dead = n_bid < n_blocks
    dead = n_bid if have_dead else n_blocks - 1
    cb = np.empty(n_kv, np.int32)
    cb[:n_bid * ratio] = np.arange(n_bid * ratio) // ratio
    cb[n_bid * ratio:] = dead
    bc = np.zeros(ratio * n_blocks, np.int32)
    bp = np.zeros(4 * n_blocks, np.int32)
    bc[:n_bid * ratio] = np.arange(n_bid * ratio)
    for sec in range(4):
        bp[sec * n_blocks:sec * n_blocks + n_bid] = np.arange(n_bid) * ratio
    if n_bid < n_blocks:
        bc[n_bid * ratio:(n_bid + 1) * ratio] = np.minimum(n_bid * ratio + np.arange(ratio), n_kv - 1)
        for sec in range(4):
            bp[sec * n_blocks + n_bid] = n_bid * ratio
    bi = np.empty((Tc, n_blocks), np.float32)
    blocks = np.arange(n_blocks)
    for i in range(Tc):
        row = bi[i]
        q = n_past_c + i
        tail_b = min(n_bid, (q + 1) // ratio)
        row[:tail_b] = 0.0
        row[tail_b:n_bid] = 1e9
        row[n_bid:] = -np.inf
        if have_dead:
            row[dead] = 1e9
        flip = (blocks >= tail_b) & (row > 0.0) & (blocks * ratio > q)
        row[flip] = -1e9
    return dict(n_blocks=n_blocks, cell_blk=cb, blk_cells=bc, blk_pos=bp, bias=bi)


def qsa_mask(cells: np.ndarray, causal_bits: np.ndarray, n_kv: int, row_len: int) -> np.ndarray:
    """graph_builder::qsa_mask (qwfn_graph.cpp:388-414): an F16 [n_kv, T] tensor
    filled with -inf, 0 written at each query's selected cells (ggml_set_rows
    of an F32 zero: +0), then the causal mask added in place (ggml's F16 add:
    f16(f32(a) + f32(b))). cells: int32 [T, width]; causal_bits: uint16
    [T, >= n_kv]. Returned as uint16 rows of row_len values, the padding past
    n_kv -inf as the kernel writes it."""
    cells = np.asarray(cells, np.int64)
    T = cells.shape[0]
    sel = np.full((T, n_kv), -np.inf, np.float32)
    for t in range(T):
        sel[t, cells[t]] = 0.0
    causal = np.ascontiguousarray(causal_bits[:, :n_kv]).view(np.float16).astype(np.float32)
    with np.errstate(invalid="ignore"):
        out = _f16_bits(sel + causal)
    res = np.full((T, row_len), F16_NEG_INF, np.uint16)
    res[:, :n_kv] = out
    return res


def visible_cells(cells_row: np.ndarray, n_kv: int, pos: int) -> np.ndarray:
    """The keys a query at position pos of a QSA-on prefill chunk sees: the zero entries
    of qsa_mask (qwfn_graph.cpp:388-414) over the chunk's causal row (0 at keys <= pos,
    -inf after, qwfn_engine.cpp:1261-1270), ascending. cells_row: the query's selected
    cells, all in [0, n_kv)."""
    causal = np.full((1, n_kv), F16_NEG_INF, np.uint16)
    causal[0, :min(n_kv, pos + 1)] = F16_ZERO
    m = qsa_mask(np.asarray(cells_row, np.int64)[None], causal, n_kv, n_kv)
    return np.flatnonzero(m[0] == F16_ZERO).astype(np.int32)
