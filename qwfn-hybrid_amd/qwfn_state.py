"""Python mirror of the reference's state interface over libqwfn_kv.so
(include/qwfn_state.h). Every operation runs in the HIP library; PyTorch only
supplies caller-owned device buffers and the current stream.

  State            qwfn::state (qwfn_state.h:39-92): init, k_cache, v_cache,
                   idx_cache, rs_state, rs_conv, ple_conv, reset, bytes,
                   summary, n_ctx; plus the engine's position bookkeeping
                   (n_past, rollback depth, rollback_n, qwfn_engine.cpp:3629-3660)
  snapshot_*       engine::snapshot_save / snapshot_load (qwfn_engine.cpp:988-1053)
  causal_mask_f16, cell_mask_f16
                   the masks of qwfn_engine.cpp:1261-1271, :2093-2098,
                   :3415-3421 and qwfn_graph.cpp:668-693
  QsaDecodeInputs  qsa_decode_inputs and qsa_decode_prepare(_k)
                   (qwfn_graph.h:71-84, qwfn_engine.cpp:1072-1105, :3582-3614)
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import qwfn_kv as K

STATE_K, STATE_V, STATE_IDX, STATE_RS, STATE_CONV, STATE_PLE_CONV = range(6)
MEM_DEVICE, MEM_HOST = 0, 1
LAYOUT_ONLY = -1


def config(n_ctx: int, **overrides) -> K.StateConfig:
    """The model's configuration (qwfn_state_config_default) with overrides."""
    c = K.StateConfig()
    K.load().qwfn_state_config_default(ctypes.byref(c), n_ctx)
    for k, v in overrides.items():
        if not hasattr(c, k):
            raise KeyError(k)
        setattr(c, k, int(v))
    return c


class State:
    """qwfn::state: owns the caches and recurrent state of one sequence."""

    def __init__(self):
        self._h = ctypes.c_void_p(None)

    def init(self, cfg: K.StateConfig, device: int = 0) -> tuple[bool, str]:
        """state::init: (True, "") or (False, message), as bool + std::string& err."""
        if self._h:
            raise RuntimeError("state initialised once")
        L = K.load()
        rc = L.qwfn_state_create(ctypes.byref(cfg), device, ctypes.byref(self._h))
        if rc != K.OK:
            return False, L.qwfn_last_error().decode(errors="replace")
        return True, ""

    def close(self):
        if self._h:
            K.load().qwfn_state_destroy(self._h)
            self._h = ctypes.c_void_p(None)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self):
        return self._h

    # -- tensors (null for the wrong layer kind, as in qwfn_state.cpp:123-148)
    def tensor(self, kind: int, il: int = 0, slot: int = -1) -> K.Tensor | None:
        t = K.Tensor()
        rc = K.load().qwfn_state_tensor(self._h, kind, il, slot, ctypes.byref(t))
        if rc < 0:
            K.check(rc)
        return t if rc == 1 else None

    def k_cache(self, il: int):
        return self.tensor(STATE_K, il)

    def v_cache(self, il: int):
        return self.tensor(STATE_V, il)

    def idx_cache(self, il: int):
        return self.tensor(STATE_IDX, il)

    def rs_state(self, il: int):
        return self.tensor(STATE_RS, il)

    def rs_conv(self, il: int):
        return self.tensor(STATE_CONV, il)

    def ple_conv(self):
        return self.tensor(STATE_PLE_CONV, 0)

    def rollback_slot(self, kind: int, il: int, slot: int):
        """The image of a recurrent tensor in rollback slot `slot` (the state slot+1 tokens back)."""
        return self.tensor(kind, il, slot)

    # -- sizes
    def bytes(self) -> int:
        return int(K.load().qwfn_state_bytes(self._h))

    def host_bytes(self) -> int:
        return int(K.load().qwfn_state_host_bytes(self._h))

    def rollback_bytes(self) -> int:
        return int(K.load().qwfn_state_rollback_bytes(self._h))

    def n_ctx(self) -> int:
        return int(K.load().qwfn_state_n_ctx(self._h))

    def summary(self) -> str:
        L = K.load()
        n = L.qwfn_state_summary(self._h, None, 0)
        K.check(min(n, 0))
        buf = ctypes.create_string_buffer(n + 1)
        L.qwfn_state_summary(self._h, buf, n + 1)
        return buf.value.decode()

    # -- bookkeeping
    def n_past(self) -> int:
        return int(K.load().qwfn_state_n_past(self._h))

    def rollback_depth(self) -> int:
        return int(K.load().qwfn_state_rollback_depth(self._h))

    def step_done(self, T: int, verified: bool = False):
        K.check(K.load().qwfn_state_step_done(self._h, T, int(verified)))

    def reset(self, stream=None):
        K.check(K.load().qwfn_state_reset(self._h, K._stream(stream)))

    def rollback_n(self, n_back: int, stream=None) -> tuple[bool, str]:
        """engine::rollback_n: (True, "") or (False, message)."""
        L = K.load()
        rc = L.qwfn_state_rollback(self._h, n_back, K._stream(stream))
        if rc != K.OK:
            return False, L.qwfn_last_error().decode(errors="replace")
        return True, ""


def _handles(states):
    return (ctypes.c_void_p * len(states))(*[s.handle for s in states])


def snapshot_parts(states, n_past: int) -> list[tuple[int, int]]:
    """(address, bytes) of each snapshot part, in snapshot_parts order."""
    L = K.load()
    H = _handles(states)
    n = ctypes.c_int32(0)
    K.check(L.qwfn_snapshot_parts(H, len(states), n_past, None, 0, ctypes.byref(n)))
    P = (K.Part * max(1, n.value))()
    K.check(L.qwfn_snapshot_parts(H, len(states), n_past, P, n.value, ctypes.byref(n)))
    return [(P[i].data or 0, int(P[i].bytes)) for i in range(n.value)]


@dataclass
class Snapshot:
    """engine::state_snapshot: n_past and one blob per part (torch uint8 tensors)."""
    n_past: int = 0
    blobs: list = field(default_factory=list)

    def bytes(self) -> int:
        return sum(int(b.numel()) for b in self.blobs)


def snapshot_save(states, where: int = MEM_HOST, stream=None, sync: bool = True) -> Snapshot:
    """engine::snapshot_save into pinned host blobs (MEM_HOST) or device blobs."""
    import torch
    parts = snapshot_parts(states, states[0].n_past())
    dev = torch.device("cuda")
    blobs = [torch.empty(b, dtype=torch.uint8, device=dev) if where == MEM_DEVICE
             else torch.empty(b, dtype=torch.uint8, pin_memory=True) for _, b in parts]
    D = (ctypes.c_void_p * max(1, len(blobs)))(*[b.data_ptr() if b.numel() else None for b in blobs])
    B = (ctypes.c_size_t * max(1, len(blobs)))(*[b.numel() for b in blobs])
    n_past = ctypes.c_int32(0)
    H = _handles(states)
    K.check(K.load().qwfn_snapshot_save(H, len(states), D, B, len(blobs), where, ctypes.byref(n_past),
                                        K._stream(stream)))
    if sync:
        torch.cuda.current_stream().synchronize() if stream is None else stream.synchronize()
    return Snapshot(int(n_past.value), blobs)


def snapshot_load(states, snap: Snapshot, stream=None) -> tuple[bool, str]:
    """engine::snapshot_load: (False, message) on a part count or size mismatch
    (the states are reset either way)."""
    L = K.load()
    if not snap.blobs:
        kind = MEM_HOST
    else:
        kind = MEM_DEVICE if snap.blobs[0].is_cuda else MEM_HOST
    S = (ctypes.c_void_p * max(1, len(snap.blobs)))(*[b.data_ptr() if b.numel() else None for b in snap.blobs])
    B = (ctypes.c_size_t * max(1, len(snap.blobs)))(*[b.numel() for b in snap.blobs])
    rc = L.qwfn_snapshot_load(_handles(states), len(states), snap.n_past, S, B, len(snap.blobs), kind,
                              K._stream(stream))
    if rc != K.OK:
        if rc != K.ESIZE:
            K.check(rc)
        return False, L.qwfn_last_error().decode(errors="replace")
    return True, ""


# ------------------------------------------------------------------- masks

def causal_mask_f16(mask, n_kv: int, T: int, n_past: int, stream=None):
    """mask: a CUDA uint16/float16 tensor [T, row]; key j of row i is visible iff j <= n_past + i."""
    row_stride = mask.stride(0) * mask.element_size() if mask.dim() == 2 else n_kv * 2
    K.check(K.load().qwfn_causal_mask_f16(mask.data_ptr(), n_kv, T, n_past, row_stride, K._stream(stream)))


def cell_mask_f16(cells, n_past: int, n_pad: int, mask, gcells=None, stream=None):
    K.check(K.load().qwfn_cell_mask_f16(cells.data_ptr(), cells.numel(), n_pad, n_past, mask.data_ptr(),
                                        gcells.data_ptr() if gcells is not None else None, K._stream(stream)))


def _dev_check(name, **tensors):
    for k, t in tensors.items():
        if t is not None and not t.is_cuda:
            raise ValueError(f"{name}: {k} must be device memory")


def qsa_chunk_inputs(n_past_c: int, Tc: int, ratio: int, cell_blk=None, blk_cells=None, blk_pos=None, bias=None,
                     stream=None) -> int:
    """engine::fill_chunk_qsa on the device; returns n_blocks = ceil((n_past_c + Tc) / ratio).
    cell_blk: i32 [n_kv]; blk_cells: i32 [n_blocks * ratio]; blk_pos: i32 [4 * n_blocks];
    bias: f32 [Tc, >= n_blocks] with contiguous rows. Any may be None."""
    import torch
    n_kv = n_past_c + Tc
    nb = -(-n_kv // ratio)
    _dev_check("qsa_chunk_inputs", cell_blk=cell_blk, blk_cells=blk_cells, blk_pos=blk_pos, bias=bias)
    for name, t, n in (("cell_blk", cell_blk, n_kv), ("blk_cells", blk_cells, nb * ratio), ("blk_pos", blk_pos, 4 * nb)):
        if t is not None and (t.dtype != torch.int32 or not t.is_contiguous() or t.numel() < n):
            raise ValueError(f"qsa_chunk_inputs: {name} must be contiguous i32 with at least {n} entries")
    if bias is not None and (bias.dtype != torch.float32 or bias.dim() != 2 or bias.shape[0] < Tc
                             or bias.shape[1] < nb or bias.stride(1) != 1):
        raise ValueError("qsa_chunk_inputs: bias must be f32 [Tc, >= n_blocks] with contiguous rows")
    p = lambda t: t.data_ptr() if t is not None else None
    K.check(K.load().qwfn_qsa_chunk_inputs(n_past_c, Tc, ratio, p(cell_blk), p(blk_cells), p(blk_pos), p(bias),
                                           bias.stride(0) * 4 if bias is not None else 0, K._stream(stream)))
    return nb


def qsa_mask_f16(cells, causal, n_kv: int, mask, stream=None):
    """graph_builder::qsa_mask on the device: cells i32 [T, width] (contiguous rows), causal
    f16 [T, >= n_kv] and mask f16 [T, row] (2-byte elements, contiguous rows); row t of mask
    becomes causal where selected, -inf elsewhere (padding included)."""
    import torch
    _dev_check("qsa_mask_f16", cells=cells, causal=causal, mask=mask)
    f16 = (torch.float16,) + ((torch.uint16,) if hasattr(torch, "uint16") else ())
    if cells.dtype != torch.int32 or cells.dim() != 2 or cells.stride(1) != 1:
        raise ValueError("qsa_mask_f16: cells must be i32 [T, width] with contiguous rows")
    for name, t in (("causal", causal), ("mask", mask)):
        if t.dim() != 2 or t.dtype not in f16 or t.stride(1) != 1 or t.shape[1] < n_kv or t.shape[0] < cells.shape[0]:
            raise ValueError(f"qsa_mask_f16: {name} must be f16 [T, >= n_kv] with contiguous rows")
    T = cells.shape[0]
    K.check(K.load().qwfn_qsa_mask_f16(cells.data_ptr(), cells.shape[1], cells.stride(0) * 4, causal.data_ptr(),
                                       causal.stride(0) * 2, n_kv, T, mask.data_ptr(), mask.stride(0) * 2,
                                       K._stream(stream)))


def qsa_visible_cells(cells, n_kv: int, n_past: int, lists, counts, stream=None):
    """The keys each query of a QSA-on prefill chunk sees: row t of lists (i32 [T, >= width],
    contiguous rows) gets the distinct cells of cells row t (i32 [T, width]) at most n_past
    + t, ascending, and counts[t] (i32 [T]) their number."""
    import torch
    _dev_check("qsa_visible_cells", cells=cells, lists=lists, counts=counts)
    for name, t in (("cells", cells), ("lists", lists)):
        if t.dtype != torch.int32 or t.dim() != 2 or t.stride(1) != 1:
            raise ValueError(f"qsa_visible_cells: {name} must be i32 [T, width] with contiguous rows")
    T, width = cells.shape
    if lists.shape[0] < T or lists.shape[1] < width:
        raise ValueError("qsa_visible_cells: lists must be at least [T, width]")
    if counts.dtype != torch.int32 or counts.dim() != 1 or counts.shape[0] < T or not counts.is_contiguous():
        raise ValueError("qsa_visible_cells: counts must be a contiguous i32 [T]")
    K.check(K.load().qwfn_qsa_visible_cells(cells.data_ptr(), width, cells.stride(0) * 4, n_kv, T, n_past,
                                            lists.data_ptr(), lists.stride(0) * 4, counts.data_ptr(),
                                            K._stream(stream)))


# ------------------------------------------- decode-time sparse-attention inputs

class QsaDecodeInputs:
    """qsa_decode_inputs (qwfn_graph.h:71-84): the per-token device tensors."""

    def __init__(self, ratio: int, n_blocks_max: int, device="cuda"):
        import torch
        self.ratio, self.n_blocks_max = ratio, n_blocks_max
        self.bias = torch.full((n_blocks_max,), float("-inf"), dtype=torch.float32, device=device)
        self.write_idx = torch.zeros(1, dtype=torch.int32, device=device)
        self.member_idx = torch.zeros(ratio, dtype=torch.int32, device=device)
        self.blk_pos = torch.zeros(4, dtype=torch.int32, device=device)
        self.blk_idx = torch.zeros(1, dtype=torch.int32, device=device)
        self.npast_f = torch.zeros(1, dtype=torch.float32, device=device)
        self.n_bucket = 0

    def _c(self) -> K.QsaInputs:
        q = K.QsaInputs()
        q.bias, q.write_idx, q.member_idx = self.bias.data_ptr(), self.write_idx.data_ptr(), self.member_idx.data_ptr()
        q.blk_pos, q.blk_idx, q.npast_f = self.blk_pos.data_ptr(), self.blk_idx.data_ptr(), self.npast_f.data_ptr()
        q.ratio, q.n_blocks_max = self.ratio, self.n_blocks_max
        return q

    def bucket(self, n_past: int) -> int:
        return int(K.load().qwfn_qsa_bucket(n_past, self.ratio, self.n_blocks_max))

    def prepare(self, n_past: int, prev: "QsaDecodeInputs | None" = None, stream=None):
        """qsa_decode_prepare (prev None) or qsa_decode_prepare_k (prev = the previous position's inputs)."""
        q = self._c()
        K.check(K.load().qwfn_qsa_decode_prepare(ctypes.byref(q), prev.bias.data_ptr() if prev is not None else None,
                                                 n_past, K._stream(stream)))
        nb = self.bucket(n_past)
        self.n_bucket = nb if prev is None else max(prev.n_bucket, nb)
        if prev is not None:
            prev.n_bucket = self.n_bucket

    def rebuild_bias(self, n_past: int, stream=None):
        """qsa_pool_rebuild's bias rewrite; n_past = -1 resets it to -inf."""
        K.check(K.load().qwfn_qsa_bias_rebuild(self.bias.data_ptr(), self.n_blocks_max, n_past, self.ratio,
                                               K._stream(stream)))


def qsa_decode_prepare_steps(qds, n_past: int, stream=None):
    """The inputs of positions n_past .. n_past + T - 1 in one launch: the same as qds[0].prepare(n_past)
    followed by qds[t].prepare(n_past + t, prev=qds[t - 1])."""
    arr = (K.QsaInputs * len(qds))(*[q._c() for q in qds])
    K.check(K.load().qwfn_qsa_decode_prepare_steps(arr, len(qds), n_past, K._stream(stream)))
    nb = max(q.bucket(n_past + t) for t, q in enumerate(qds))
    for q in qds:
        q.n_bucket = nb


def qsa_decode_prepare_pool_steps(qds, n_past: int, ic, k_raw, k_norm_w, pool, cfg=None, stream=None):
    """qsa_decode_prepare_steps(qds, n_past) then qwfn_kv.qsa_pool_decode_steps(ic, k_raw, qds, k_norm_w, pool)
    in one launch, the pooling's indices in their closed forms."""
    cfg = cfg or K.qsa_pool_cfg()
    T = len(qds)
    K._check_pool_args("qsa_decode_prepare_pool_steps", cfg, ic, pool, k_norm_w,
                       k_raw=k_raw[0] if k_raw is not None else None)
    if k_raw is not None and (k_raw.dim() != 2 or k_raw.shape[0] != T or k_raw.stride(1) != 1):
        raise ValueError("qsa_decode_prepare_pool_steps: k_raw must be [T, idx_dim] with contiguous rows")
    arr = (K.QsaInputs * T)(*[q._c() for q in qds])
    K.check(K.load().qwfn_qsa_decode_prepare_pool_steps(arr, T, n_past, ic.data_ptr(), ic.shape[0],
                                                        k_raw.data_ptr() if k_raw is not None else None,
                                                        k_raw.stride(0) * 4 if k_raw is not None else 0,
                                                        k_norm_w.data_ptr(), pool.data_ptr(), pool.shape[0],
                                                        ctypes.byref(cfg), K._stream(stream)))
    nb = max(q.bucket(n_past + t) for t, q in enumerate(qds))
    for q in qds:
        q.n_bucket = nb


def qsa_tables(blk_cells, ratio: int, cell_pos=None, blk_pos_all=None, n_whole: int = 0, stream=None):
    n_blocks_max = blk_cells.numel() // ratio if blk_cells is not None else 0
    K.check(K.load().qwfn_qsa_tables(blk_cells.data_ptr() if blk_cells is not None else None, n_blocks_max, ratio,
                                     cell_pos.data_ptr() if cell_pos is not None else None,
                                     cell_pos.numel() if cell_pos is not None else 0,
                                     blk_pos_all.data_ptr() if blk_pos_all is not None else None, n_whole,
                                     K._stream(stream)))


# ------------------------------------------------------- saved-sequence pool

def _i32(seq):
    seq = list(seq)
    return (ctypes.c_int32 * max(1, len(seq)))(*seq), len(seq)


class SnapPool:
    """The server's saved sequences (tools/qwfn_server.cpp:767-793) in HBM."""

    def __init__(self, cap_bytes: int, max_entries: int = 4, device: int = 0):
        self._h = ctypes.c_void_p(None)
        K.check(K.load().qwfn_snap_pool_create(cap_bytes, max_entries, device, ctypes.byref(self._h)))

    def close(self):
        if self._h:
            K.load().qwfn_snap_pool_destroy(self._h)
            self._h = ctypes.c_void_p(None)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def count(self) -> int:
        return int(K.load().qwfn_snap_pool_count(self._h))

    def bytes(self) -> int:
        return int(K.load().qwfn_snap_pool_bytes(self._h))

    def entry(self, k: int) -> tuple[list[int], int, int]:
        """(tokens, n_past, bytes) of entry k, least recently used first."""
        L = K.load()
        n, npast, b = ctypes.c_int32(0), ctypes.c_int32(0), ctypes.c_size_t(0)
        K.check(L.qwfn_snap_pool_entry(self._h, k, ctypes.byref(n), ctypes.byref(npast), ctypes.byref(b), None, 0))
        tok = (ctypes.c_int32 * max(1, n.value))()
        K.check(L.qwfn_snap_pool_entry(self._h, k, None, None, None, tok, n.value))
        return list(tok[:n.value]), int(npast.value), int(b.value)

    def save_seq(self, states, tok, stream=None) -> bool:
        T, n = _i32(tok)
        rc = K.load().qwfn_snap_pool_save(self._h, _handles(states), len(states), T, n, K._stream(stream))
        if rc < 0:
            K.check(rc)
        return rc == 1

    def best_saved(self, tok, has_images: bool = False) -> int:
        T, n = _i32(tok)
        return int(K.load().qwfn_snap_pool_best(self._h, T, n, int(has_images)))

    def load(self, k: int, states, stream=None) -> tuple[bool, str]:
        L = K.load()
        rc = L.qwfn_snap_pool_load(self._h, k, _handles(states), len(states), K._stream(stream))
        if rc != K.OK:
            if rc != K.ESIZE:
                K.check(rc)
            return False, L.qwfn_last_error().decode(errors="replace")
        return True, ""

    def shared_prefix_split(self, prompt, n_consumed: int, has_images: bool = False) -> int:
        T, n = _i32(prompt)
        return int(K.load().qwfn_snap_pool_split(self._h, T, n, n_consumed, int(has_images)))

    def restore_or_reset(self, states, consumed, prompt, consumed_has_images: bool = False,
                         prompt_has_images: bool = False, stream=None) -> int:
        C, nc = _i32(consumed)
        P, n_p = _i32(prompt)
        out = ctypes.c_int32(0)
        K.check(K.load().qwfn_snap_pool_restore_or_reset(self._h, _handles(states), len(states), C, nc,
                                                         int(consumed_has_images), P, n_p, int(prompt_has_images),
                                                         ctypes.byref(out), K._stream(stream)))
        return int(out.value)


# ------------------------------------------------- sparse block selection

def qsa_select_cells(pool, q, bias, k_blocks: int, blk_cells, ratio: int, cells, top=None, ws=None, stream=None):
    """qsa_dec_cells for T queries. pool: f16 [n_blocks, 128] (CUDA, uint16 or float16);
    q: f32 [T, n_heads, 128]; bias: f32 [T, n_blocks]; blk_cells: i32 [>= n_blocks * ratio];
    cells: i32 [T, k_blocks * ratio]; top: optional i32 [T, k_blocks]."""
    import torch
    L = K.load()
    n_blocks = pool.shape[0]
    T = q.shape[0]
    # the C ABI takes raw device pointers and rows at a stride with contiguous
    # elements; what it cannot see (device, dtype, sizes) is checked here
    f16_types = (torch.float16,) + ((torch.uint16,) if hasattr(torch, "uint16") else ())
    if pool.dim() != 2 or pool.shape[1] != 128 or pool.stride(1) != 1 or pool.dtype not in f16_types:
        raise ValueError("qsa_select_cells: pool must be [n_blocks, 128] f16 rows")
    if q.dim() != 3 or q.dtype != torch.float32 or q.shape[2] != 128 or q.stride(2) != 1 or q.stride(1) != 128:
        raise ValueError("qsa_select_cells: q must be f32 [T, n_heads, 128] with contiguous heads")
    if bias.dim() != 2 or bias.dtype != torch.float32 or bias.shape[0] != T or bias.shape[1] < n_blocks \
            or bias.stride(1) != 1:
        raise ValueError("qsa_select_cells: bias must be f32 [T, >= n_blocks] rows")
    if blk_cells.dtype != torch.int32 or not blk_cells.is_contiguous() or blk_cells.numel() < n_blocks * ratio:
        raise ValueError("qsa_select_cells: blk_cells must be contiguous i32 with n_blocks * ratio entries")
    if cells.dtype != torch.int32 or not cells.is_contiguous() or cells.numel() < T * k_blocks * ratio:
        raise ValueError("qsa_select_cells: cells must be contiguous i32 [T, k_blocks * ratio]")
    if top is not None and (top.dtype != torch.int32 or not top.is_contiguous() or top.numel() < T * k_blocks):
        raise ValueError("qsa_select_cells: top must be contiguous i32 [T, k_blocks]")
    for name, t in (("pool", pool), ("q", q), ("bias", bias), ("blk_cells", blk_cells), ("cells", cells),
                    ("top", top), ("ws", ws)):
        if t is not None and (not t.is_cuda or t.device != pool.device):
            raise ValueError(f"qsa_select_cells: {name} must be a GPU tensor on the pool's device")
    need = int(L.qwfn_qsa_select_workspace_size(n_blocks, T))
    if ws is None:
        ws = torch.empty(need, dtype=torch.uint8, device=pool.device)
    elif ws.numel() * ws.element_size() < need or ws.data_ptr() % 256 or not ws.is_contiguous():
        raise ValueError(f"qsa_select_cells: ws must be a contiguous 256-byte aligned buffer of >= {need} bytes")
    K.check(L.qwfn_qsa_select_cells(pool.data_ptr(), pool.stride(0) * pool.element_size(), n_blocks, q.data_ptr(),
                                    q.shape[1], q.stride(0) * 4, bias.data_ptr(), bias.stride(0) * 4, T, k_blocks,
                                    blk_cells.data_ptr(), ratio, cells.data_ptr(),
                                    top.data_ptr() if top is not None else None, ws.data_ptr(), ws.numel() * ws.element_size(),
                                    K._stream(stream)))
