"""Python binding of libqwfn_kv.so (the C ABI declared in include/qwfn_kv.h).

The binding only marshals descriptors: every operation runs in the HIP library.
PyTorch supplies device memory and the current stream. Loading fails loudly
when the library has not been built; there is no fallback.

Tensors follow ggml conventions (ne = element counts, nb = byte strides). The
helpers below build the views the reference engine builds over its per-layer
caches (qwfn_state.cpp:48-91, qwfn_graph.cpp:461-464): a cache is a uint8
[n_ctx, row_bytes] array, token-major, KV head h at byte h * 272.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libqwfn_kv.so")

TYPE_F32, TYPE_F16, TYPE_Q8_0, TYPE_I32, TYPE_BF16 = 0, 1, 8, 26, 30
Q8_REF, Q8_X86 = 0, 1
SRC_DEVICE, SRC_HOST = 0, 1

QK8_0 = 32
Q8_0_BLOCK = 34

OK, EINVAL, ERANGE, EALIGN, ENOTSUP, EDEVICE, ENOMEM, ESIZE = 0, -1, -2, -3, -4, -5, -6, -7

DEVERR_SET_ROWS_INDEX = 1
DEVERR_GET_ROWS_INDEX = 2

# attention kernel families (qwfn_fattn_force_kernel)
FA_KERNEL_AUTO, FA_KERNEL_VD, FA_KERNEL_DEC, FA_KERNEL_GENERAL, FA_KERNEL_PRE, FA_KERNEL_VS = 0, 1, 2, 3, 4, 5


def last_kernel() -> str:
    """The attention kernel instantiation this thread's last attention call launched."""
    return load().qwfn_fattn_last_kernel().decode()


# split-merge paths (qwfn_fattn_force_merge, qwfn_fattn_last_merge)
FA_MERGE_AUTO, FA_MERGE_FUSED, FA_MERGE_KERNEL, FA_MERGE_NONE = 0, 1, 2, 3


def last_merge() -> int:
    """How this thread's last attention call merged its key splits (FA_MERGE_*)."""
    return int(load().qwfn_fattn_last_merge())


class forced_merge:
    """Context manager: later attention calls in this process merge their key splits
    by path `mode` (FA_MERGE_*) while it is active."""
    def __init__(self, mode: int):
        self.mode = mode

    def __enter__(self):
        load().qwfn_fattn_force_merge(self.mode)
        return self

    def __exit__(self, *exc):
        load().qwfn_fattn_force_merge(FA_MERGE_AUTO)
        return False


class forced_kernel:
    """Context manager: later attention calls in this process use kernel family `kind`
    (FA_KERNEL_*) while it is active."""
    def __init__(self, kind: int):
        self.kind = kind

    def __enter__(self):
        load().qwfn_fattn_force_kernel(self.kind)
        return self

    def __exit__(self, *exc):
        load().qwfn_fattn_force_kernel(FA_KERNEL_AUTO)
        return False


class QwfnError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"qwfn error {code}: {msg}")
        self.code = code


class Tensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p),
                ("type", ctypes.c_int32),
                ("pad_", ctypes.c_int32),
                ("ne", ctypes.c_int64 * 4),
                ("nb", ctypes.c_size_t * 4)]


class StateConfig(ctypes.Structure):
    """qwfn_state_config (include/qwfn_state.h)."""
    _fields_ = [(n, ctypes.c_uint32) for n in (
        "n_ctx", "n_layer", "full_attention_interval", "n_head_kv", "n_embd_head_k", "n_embd_head_v",
        "idx_key_len", "ssm_d_state", "ssm_n_group", "ssm_dt_rank", "ssm_d_conv", "hc_count", "n_embd",
        "ple_n_head", "ple_conv_kernel", "ple_ngram_size")] + [
        ("type_k", ctypes.c_int32), ("type_v", ctypes.c_int32), ("type_idx", ctypes.c_int32),
        ("kv_host", ctypes.c_uint32), ("idx_host", ctypes.c_uint32), ("n_rollback", ctypes.c_uint32)]


class Part(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("bytes", ctypes.c_size_t)]


class QsaInputs(ctypes.Structure):
    """qwfn_qsa_inputs: device addresses of the per-token decode inputs."""
    _fields_ = [("bias", ctypes.c_void_p), ("write_idx", ctypes.c_void_p), ("member_idx", ctypes.c_void_p),
                ("blk_pos", ctypes.c_void_p), ("blk_idx", ctypes.c_void_p), ("npast_f", ctypes.c_void_p),
                ("ratio", ctypes.c_int32), ("pad_", ctypes.c_int32), ("n_blocks_max", ctypes.c_int64)]


class RopeCfg(ctypes.Structure):
    """qwfn_rope_cfg: rope and norm constants of the attention layers."""
    _fields_ = [("n_dims", ctypes.c_int32), ("sections", ctypes.c_int32 * 4), ("freq_base", ctypes.c_float),
                ("rms_eps", ctypes.c_float)]


def rope_cfg(n_dims: int = 64, sections=(11, 11, 10, 0), freq_base: float = 1e7, rms_eps: float = 1e-6) -> RopeCfg:
    c = RopeCfg()
    c.n_dims = n_dims
    for i in range(4):
        c.sections[i] = int(sections[i])
    c.freq_base, c.rms_eps = freq_base, rms_eps
    return c


class QsaPoolCfg(ctypes.Structure):
    """qwfn_qsa_pool_cfg: the indexer key geometry and rope / norm constants."""
    _fields_ = [("idx_dim", ctypes.c_int32), ("n_dims", ctypes.c_int32), ("sections", ctypes.c_int32 * 4),
                ("freq_base", ctypes.c_float), ("rms_eps", ctypes.c_float)]


EXPORTS = [
    "qwfn_abi_version", "qwfn_last_error", "qwfn_init", "qwfn_device_status",
    "qwfn_set_rows_q8_0", "qwfn_cpy_f32_q8_0", "qwfn_set_rows_q8_0_kv", "qwfn_cpy_f32_q8_0_kv", "qwfn_get_rows_i32", "qwfn_kv_gather_segments", "qwfn_kv_gather_segments_kv",
    "qwfn_fattn_workspace_size", "qwfn_fattn_force_splits", "qwfn_fattn_force_kernel", "qwfn_fattn_last_kernel", "qwfn_fattn_force_merge", "qwfn_fattn_last_merge", "qwfn_flash_attn_ext_q8_0", "qwfn_flash_attn_ext_q8_0_noalloc", "qwfn_flash_attn_ext_q8_0_append",
    "qwfn_fattn_workspace_size_seq", "qwfn_flash_attn_ext_q8_0_seq", "qwfn_state_restore",
    "qwfn_fattn_workspace_size_cells", "qwfn_flash_attn_ext_q8_0_cells", "qwfn_kv_produce_q8_0",
    "qwfn_fattn_workspace_size_query_cells", "qwfn_flash_attn_ext_q8_0_query_cells",
    "qwfn_flash_attn_ext_q8_0_query_cells_dev", "qwfn_qsa_visible_cells",
    "qwfn_flash_attn_ext_q8_0_gated",
    # include/qwfn_state.h
    "qwfn_state_config_default", "qwfn_state_create", "qwfn_state_destroy", "qwfn_state_tensor",
    "qwfn_state_bytes", "qwfn_state_host_bytes", "qwfn_state_rollback_bytes", "qwfn_state_n_ctx",
    "qwfn_state_summary", "qwfn_state_n_past", "qwfn_state_rollback_depth", "qwfn_state_step_done",
    "qwfn_state_reset", "qwfn_state_rollback", "qwfn_snapshot_parts", "qwfn_snapshot_save", "qwfn_snapshot_load",
    "qwfn_causal_mask_f16", "qwfn_cell_mask_f16", "qwfn_qsa_chunk_inputs", "qwfn_qsa_mask_f16",
    "qwfn_qsa_bucket", "qwfn_qsa_decode_prepare", "qwfn_qsa_decode_prepare_steps", "qwfn_qsa_pool_decode_steps",
    "qwfn_qsa_decode_prepare_pool_steps",
    "qwfn_qsa_bias_rebuild", "qwfn_qsa_tables",
    "qwfn_snap_pool_create", "qwfn_snap_pool_destroy", "qwfn_snap_pool_count", "qwfn_snap_pool_bytes",
    "qwfn_snap_pool_entry", "qwfn_snap_pool_save", "qwfn_snap_pool_best", "qwfn_snap_pool_load",
    "qwfn_snap_pool_split", "qwfn_snap_pool_restore_or_reset",
    "qwfn_qsa_select_workspace_size", "qwfn_qsa_select_cells",
    "qwfn_qsa_pool_cfg_default", "qwfn_set_rows_f16", "qwfn_qsa_pool_decode", "qwfn_qsa_pool_rebuild",
    "qwfn_gated_delta_net",
]

_lib = None


def load(path: str = LIB_PATH):
    """Load the HIP library; raise if it is missing (no fallback exists)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"libqwfn_kv.so not built ({path}); run __graft_entry__.build()")
    L = ctypes.CDLL(path)
    vp, i32, i64, sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t
    T = ctypes.POINTER(Tensor)
    L.qwfn_abi_version.restype = ctypes.c_int
    L.qwfn_last_error.restype = ctypes.c_char_p
    L.qwfn_init.argtypes = [ctypes.c_int]
    L.qwfn_device_status.argtypes = [vp, ctypes.POINTER(ctypes.c_uint32)]
    L.qwfn_set_rows_q8_0.argtypes = [T, T, T, ctypes.c_int, vp]
    L.qwfn_cpy_f32_q8_0.argtypes = [T, T, ctypes.c_int, vp]
    L.qwfn_set_rows_q8_0_kv.argtypes = [T, T, T, T, T, ctypes.c_int, vp]
    L.qwfn_cpy_f32_q8_0_kv.argtypes = [T, T, T, T, ctypes.c_int, vp]
    L.qwfn_get_rows_i32.argtypes = [T, T, T, vp]
    L.qwfn_kv_gather_segments.argtypes = [vp, sz, i64, sz, sz, sz, i32, vp, i64, vp, sz, sz, vp]
    L.qwfn_kv_gather_segments_kv.argtypes = [vp, vp, sz, i64, sz, sz, sz, i32, vp, i64, vp, vp, sz, sz, vp]
    L.qwfn_fattn_workspace_size.argtypes = [T, T, T, T]
    L.qwfn_fattn_workspace_size.restype = sz
    L.qwfn_flash_attn_ext_q8_0_noalloc.argtypes = [T, T, T, T, ctypes.c_float, ctypes.c_float, ctypes.c_float, T,
                                                   ctypes.c_int, vp]
    L.qwfn_fattn_force_splits.argtypes = [i32]
    L.qwfn_fattn_force_splits.restype = None
    L.qwfn_fattn_force_kernel.argtypes = [i32]
    L.qwfn_fattn_force_kernel.restype = None
    L.qwfn_fattn_last_kernel.argtypes = []
    L.qwfn_fattn_last_kernel.restype = ctypes.c_char_p
    L.qwfn_fattn_force_merge.argtypes = [i32]
    L.qwfn_fattn_force_merge.restype = None
    L.qwfn_fattn_last_merge.argtypes = []
    L.qwfn_fattn_last_merge.restype = i32
    L.qwfn_flash_attn_ext_q8_0.argtypes = [T, T, T, T, ctypes.c_float, ctypes.c_float, ctypes.c_float, T,
                                           ctypes.c_int, vp, sz, vp]
    PL = ctypes.POINTER(i64)
    L.qwfn_fattn_workspace_size_seq.argtypes = [T, T, T, T, PL]
    L.qwfn_fattn_workspace_size_seq.restype = sz
    L.qwfn_flash_attn_ext_q8_0_seq.argtypes = [T, T, T, T, ctypes.c_float, ctypes.c_float, ctypes.c_float, T,
                                               ctypes.c_int, vp, sz, PL, vp]
    L.qwfn_flash_attn_ext_q8_0_append.argtypes = [T, T, T, T, ctypes.c_float, ctypes.c_float, ctypes.c_float, T,
                                                  ctypes.c_int, vp, sz, T, T, i64, vp]
    L.qwfn_fattn_workspace_size_cells.argtypes = [T, T, T, PL, i64]
    L.qwfn_fattn_workspace_size_cells.restype = sz
    L.qwfn_flash_attn_ext_q8_0_cells.argtypes = [T, T, T, vp, PL, i64, i64, ctypes.c_float, T, ctypes.c_int, vp, sz, vp]
    L.qwfn_fattn_workspace_size_query_cells.argtypes = [T, T, T, PL, i64]
    L.qwfn_fattn_workspace_size_query_cells.restype = sz
    L.qwfn_flash_attn_ext_q8_0_query_cells_dev.argtypes = [T, T, T, vp, vp, i64, i64, ctypes.c_float, T, T, ctypes.c_int,
                                                          vp]
    L.qwfn_qsa_visible_cells.argtypes = [vp, i64, sz, i64, i64, i64, vp, sz, vp, vp]
    L.qwfn_flash_attn_ext_q8_0_query_cells.argtypes = [T, T, T, vp, PL, i64, i64, ctypes.c_float, T, T, ctypes.c_int,
                                                       vp, sz, vp]
    L.qwfn_kv_produce_q8_0.argtypes = [T, T, T, vp, vp, ctypes.POINTER(RopeCfg), T, T, i64, ctypes.c_int, vp]
    L.qwfn_flash_attn_ext_q8_0_gated.argtypes = [T, T, T, T, ctypes.c_float, ctypes.c_float, ctypes.c_float, T, T,
                                                 ctypes.c_int, vp, sz, vp]
    L.qwfn_state_restore.argtypes = [ctypes.POINTER(vp), ctypes.POINTER(sz), ctypes.POINTER(vp), i32, i32, i32, vp]
    # include/qwfn_state.h
    u32, PV, PS = ctypes.c_uint32, ctypes.POINTER(vp), ctypes.POINTER(sz)
    L.qwfn_state_config_default.argtypes = [ctypes.POINTER(StateConfig), u32]
    L.qwfn_state_config_default.restype = None
    L.qwfn_state_create.argtypes = [ctypes.POINTER(StateConfig), ctypes.c_int, PV]
    L.qwfn_state_destroy.argtypes = [vp]
    L.qwfn_state_destroy.restype = None
    L.qwfn_state_tensor.argtypes = [vp, i32, u32, i32, T]
    for f in ("qwfn_state_bytes", "qwfn_state_host_bytes", "qwfn_state_rollback_bytes"):
        getattr(L, f).argtypes = [vp]
        getattr(L, f).restype = sz
    L.qwfn_state_n_ctx.argtypes = [vp]
    L.qwfn_state_n_ctx.restype = u32
    L.qwfn_state_summary.argtypes = [vp, ctypes.c_char_p, sz]
    L.qwfn_state_n_past.argtypes = [vp]
    L.qwfn_state_n_past.restype = i32
    L.qwfn_state_rollback_depth.argtypes = [vp]
    L.qwfn_state_rollback_depth.restype = i32
    L.qwfn_state_step_done.argtypes = [vp, i32, i32]
    L.qwfn_state_reset.argtypes = [vp, vp]
    L.qwfn_state_rollback.argtypes = [vp, i32, vp]
    L.qwfn_snapshot_parts.argtypes = [PV, i32, i32, ctypes.POINTER(Part), i32, ctypes.POINTER(i32)]
    L.qwfn_snapshot_save.argtypes = [PV, i32, PV, PS, i32, i32, ctypes.POINTER(i32), vp]
    L.qwfn_snapshot_load.argtypes = [PV, i32, i32, PV, PS, i32, i32, vp]
    L.qwfn_causal_mask_f16.argtypes = [vp, i64, i64, i64, sz, vp]
    L.qwfn_cell_mask_f16.argtypes = [vp, i64, i64, i32, vp, vp, vp]
    L.qwfn_qsa_chunk_inputs.argtypes = [i64, i64, i32, vp, vp, vp, vp, sz, vp]
    L.qwfn_qsa_mask_f16.argtypes = [vp, i64, sz, vp, sz, i64, i64, vp, sz, vp]
    L.qwfn_qsa_bucket.argtypes = [i32, i32, i64]
    L.qwfn_qsa_bucket.restype = i64
    L.qwfn_qsa_decode_prepare.argtypes = [ctypes.POINTER(QsaInputs), vp, i32, vp]
    L.qwfn_qsa_decode_prepare_steps.argtypes = [ctypes.POINTER(QsaInputs), i32, i32, vp]
    L.qwfn_qsa_bias_rebuild.argtypes = [vp, i64, i32, i32, vp]
    L.qwfn_qsa_tables.argtypes = [vp, i64, i32, vp, i64, vp, i64, vp]
    PI = ctypes.POINTER(i32)
    L.qwfn_snap_pool_create.argtypes = [sz, i32, ctypes.c_int, PV]
    L.qwfn_snap_pool_destroy.argtypes = [vp]
    L.qwfn_snap_pool_destroy.restype = None
    L.qwfn_snap_pool_count.argtypes = [vp]
    L.qwfn_snap_pool_count.restype = i32
    L.qwfn_snap_pool_bytes.argtypes = [vp]
    L.qwfn_snap_pool_bytes.restype = sz
    L.qwfn_snap_pool_entry.argtypes = [vp, i32, PI, PI, ctypes.POINTER(sz), PI, i32]
    L.qwfn_snap_pool_save.argtypes = [vp, PV, i32, PI, i32, vp]
    L.qwfn_snap_pool_best.argtypes = [vp, PI, i32, i32]
    L.qwfn_snap_pool_best.restype = i32
    L.qwfn_snap_pool_load.argtypes = [vp, i32, PV, i32, vp]
    L.qwfn_snap_pool_split.argtypes = [vp, PI, i32, i32, i32]
    L.qwfn_snap_pool_split.restype = i32
    L.qwfn_snap_pool_restore_or_reset.argtypes = [vp, PV, i32, PI, i32, i32, PI, i32, i32, PI, vp]
    L.qwfn_qsa_pool_cfg_default.argtypes = [ctypes.POINTER(QsaPoolCfg)]
    L.qwfn_qsa_pool_cfg_default.restype = None
    L.qwfn_set_rows_f16.argtypes = [T, T, T, vp]
    L.qwfn_qsa_pool_decode.argtypes = [vp, i64, vp, vp, vp, i32, vp, vp, vp, vp, i64, ctypes.POINTER(QsaPoolCfg), vp]
    L.qwfn_qsa_pool_decode_steps.argtypes = [vp, i64, vp, sz, ctypes.POINTER(QsaInputs), i32, vp, vp, i64,
                                             ctypes.POINTER(QsaPoolCfg), vp]
    L.qwfn_qsa_decode_prepare_pool_steps.argtypes = [ctypes.POINTER(QsaInputs), i32, i32, vp, i64, vp, sz, vp, vp, i64,
                                                     ctypes.POINTER(QsaPoolCfg), vp]
    L.qwfn_qsa_pool_rebuild.argtypes = [vp, i64, i64, i32, vp, vp, i64, ctypes.POINTER(QsaPoolCfg), vp]
    L.qwfn_gated_delta_net.argtypes = [vp, i64, vp, i64, vp, i64, vp, vp, i32, i32, i32, i32, ctypes.c_float, vp, vp,
                                       vp, sz, i32, vp]
    L.qwfn_qsa_select_workspace_size.argtypes = [i64, i32]
    L.qwfn_qsa_select_workspace_size.restype = sz
    L.qwfn_qsa_select_cells.argtypes = [vp, sz, i64, vp, i32, sz, vp, sz, i32, i32, vp, i32, vp, vp, vp, sz, vp]
    for name in EXPORTS:
        if name not in ("qwfn_state_config_default", "qwfn_state_destroy", "qwfn_snap_pool_destroy",
                        "qwfn_fattn_force_splits", "qwfn_fattn_force_kernel", "qwfn_fattn_last_kernel",
                        "qwfn_fattn_force_merge", "qwfn_fattn_last_merge"):
            getattr(L, name).restype = getattr(L, name).restype or ctypes.c_int
    L.qwfn_last_error.restype = ctypes.c_char_p
    L.qwfn_fattn_last_kernel.restype = ctypes.c_char_p
    L.qwfn_fattn_workspace_size.restype = sz
    L.qwfn_fattn_workspace_size_seq.restype = sz
    L.qwfn_fattn_workspace_size_cells.restype = sz
    L.qwfn_qsa_select_workspace_size.restype = sz
    _lib = L
    return L


def check(rc: int) -> int:
    if rc != OK:
        raise QwfnError(rc, load().qwfn_last_error().decode(errors="replace"))
    return rc


def tensor(ptr: int, typ: int, ne, nb) -> Tensor:
    t = Tensor()
    t.data = ptr
    t.type = typ
    ne = list(ne) + [1] * (4 - len(ne))
    nb = list(nb)
    while len(nb) < 4:
        nb.append(nb[-1] * ne[len(nb) - 1])
    for i in range(4):
        t.ne[i] = int(ne[i])
        t.nb[i] = int(nb[i])
    return t


def _stream(stream) -> int | None:
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    return int(stream) if not hasattr(stream, "cuda_stream") else stream.cuda_stream


# --------------------------------------------------------------------- views

def row_bytes(kv_dim: int) -> int:
    return kv_dim // QK8_0 * Q8_0_BLOCK


def cache_rows_view(cache, n_rows: int | None = None, first_row: int = 0) -> Tensor:
    """q8_0 [kv_dim, n_rows] view of a uint8 [n_ctx, row_bytes] cache starting at first_row."""
    n_ctx, rb = cache.shape
    n = n_ctx - first_row if n_rows is None else n_rows
    kv_dim = rb // Q8_0_BLOCK * QK8_0
    return tensor(cache.data_ptr() + first_row * cache.stride(0), TYPE_Q8_0, (kv_dim, n), (Q8_0_BLOCK, cache.stride(0)))


def cache_attn_view(cache, n_kv: int, n_head_kv: int, hd: int = 256, batch: int = 1, batch_stride: int = 0) -> Tensor:
    """ggml view [hd, n_kv, n_head_kv, batch] of a token-major cache (nb1 = row, nb2 = head segment)."""
    seg = hd // QK8_0 * Q8_0_BLOCK
    rs = cache.stride(0) if cache.dim() == 2 else cache.stride(-2)
    return tensor(cache.data_ptr(), TYPE_Q8_0, (hd, n_kv, n_head_kv, batch),
                  (Q8_0_BLOCK, rs, seg, batch_stride or rs * n_kv))


def f32_view(t) -> Tensor:
    """Contiguous torch float32 tensor in ggml order (reversed torch dims)."""
    assert t.dtype.itemsize == 4
    dims = list(t.shape)[::-1]
    strides = [s * 4 for s in list(t.stride())[::-1]]
    return tensor(t.data_ptr(), TYPE_F32, dims, strides)


def q_view(q) -> Tensor:
    """Q in the projection's natural order, torch [B, T, n_head, hd] (or [T, n_head, hd]),
    as the graph's permuted view [hd, T, n_head, B] (qwfn_graph.cpp:466, :697)."""
    if q.dim() == 3:
        q = q.unsqueeze(0)
    B, T, nh, hd = q.shape
    s = q.stride()
    return tensor(q.data_ptr(), TYPE_F32, (hd, T, nh, B), (4, s[1] * 4, s[2] * 4, s[0] * 4))


def mask_view(mask) -> Tensor:
    """F16 mask, torch [T, n_kv] (or [B|1, H|1, T, n_kv]) -> ggml [n_kv, T, H, B]."""
    if mask.dim() == 2:
        mask = mask.unsqueeze(0).unsqueeze(0)
    B, H, T, n = mask.shape
    s = mask.stride()
    return tensor(mask.data_ptr(), TYPE_F16, (n, T, H, B), (2, s[2] * 2, s[1] * 2, s[0] * 2))


def out_view(out) -> Tensor:
    """Output torch [B, T, n_head, hd] float32 contiguous = ggml [hd, n_head, T, B]."""
    if out.dim() == 3:
        out = out.unsqueeze(0)
    B, T, nh, hd = out.shape
    return tensor(out.data_ptr(), TYPE_F32, (hd, nh, T, B), (4, hd * 4, hd * nh * 4, hd * nh * T * 4))


# --------------------------------------------------------------------- ops

def set_rows_q8_0(cache, src, idx, variant: int = Q8_X86, stream=None, n_rows: int | None = None):
    """cache uint8 [n_ctx, rb]; src float32 [n, kv_dim]; idx int32 [n] (device)."""
    L = load()
    dst = cache_rows_view(cache, n_rows)
    s = tensor(src.data_ptr(), TYPE_F32, (src.shape[1], src.shape[0]), (4, src.stride(0) * 4))
    i = tensor(idx.data_ptr(), TYPE_I32, (idx.shape[0],), (4,))
    return check(L.qwfn_set_rows_q8_0(ctypes.byref(dst), ctypes.byref(s), ctypes.byref(i), variant, _stream(stream)))


def cpy_f32_q8_0(src, cache, first_row: int, variant: int = Q8_X86, stream=None):
    L = load()
    s = tensor(src.data_ptr(), TYPE_F32, (src.shape[1], src.shape[0]), (4, src.stride(0) * 4))
    dst = cache_rows_view(cache, src.shape[0], first_row)
    return check(L.qwfn_cpy_f32_q8_0(ctypes.byref(s), ctypes.byref(dst), variant, _stream(stream)))


def set_rows_q8_0_kv(kcache, ksrc, vcache, vsrc, idx, variant: int = Q8_X86, stream=None, n_rows: int | None = None):
    """The K and the V set_rows of one layer in one launch (same idx)."""
    L = load()
    dk, dv = cache_rows_view(kcache, n_rows), cache_rows_view(vcache, n_rows)
    sk = tensor(ksrc.data_ptr(), TYPE_F32, (ksrc.shape[1], ksrc.shape[0]), (4, ksrc.stride(0) * 4))
    sv = tensor(vsrc.data_ptr(), TYPE_F32, (vsrc.shape[1], vsrc.shape[0]), (4, vsrc.stride(0) * 4))
    i = tensor(idx.data_ptr(), TYPE_I32, (idx.shape[0],), (4,))
    return check(L.qwfn_set_rows_q8_0_kv(ctypes.byref(dk), ctypes.byref(sk), ctypes.byref(dv), ctypes.byref(sv),
                                         ctypes.byref(i), variant, _stream(stream)))


def cpy_f32_q8_0_kv(ksrc, kcache, vsrc, vcache, first_row: int, variant: int = Q8_X86, stream=None):
    """The K and the V cpy of one append in one launch."""
    L = load()
    sk = tensor(ksrc.data_ptr(), TYPE_F32, (ksrc.shape[1], ksrc.shape[0]), (4, ksrc.stride(0) * 4))
    sv = tensor(vsrc.data_ptr(), TYPE_F32, (vsrc.shape[1], vsrc.shape[0]), (4, vsrc.stride(0) * 4))
    dk = cache_rows_view(kcache, ksrc.shape[0], first_row)
    dv = cache_rows_view(vcache, vsrc.shape[0], first_row)
    return check(L.qwfn_cpy_f32_q8_0_kv(ctypes.byref(sk), ctypes.byref(dk), ctypes.byref(sv), ctypes.byref(dv),
                                        variant, _stream(stream)))


def get_rows_i32(cache, idx, out, stream=None):
    """Raw row gather: cache uint8 [n_ctx, rb] viewed as I32 words; out uint8 [n, rb]."""
    L = load()
    rb = cache.shape[1]
    src = tensor(cache.data_ptr(), TYPE_I32, (rb // 4, cache.shape[0]), (4, cache.stride(0)))
    i = tensor(idx.data_ptr(), TYPE_I32, (idx.shape[0],), (4,))
    dst = tensor(out.data_ptr(), TYPE_I32, (rb // 4, out.shape[0]), (4, out.stride(0)))
    return check(L.qwfn_get_rows_i32(ctypes.byref(src), ctypes.byref(i), ctypes.byref(dst), _stream(stream)))


def gather_segments(cache, idx, out, seg_off: int, seg_stride: int, seg_bytes: int, stream=None):
    """idx int32 [n_seg, n_idx]; out uint8 [n_seg, n_idx, seg_bytes]."""
    L = load()
    n_seg, n_idx = idx.shape
    return check(L.qwfn_kv_gather_segments(cache.data_ptr(), cache.stride(0), cache.shape[0], seg_off, seg_stride,
                                           seg_bytes, n_seg, idx.data_ptr(), n_idx, out.data_ptr(), out.stride(1),
                                           out.stride(0), _stream(stream)))


def gather_segments_kv(kcache, vcache, idx, out_k, out_v, seg_off: int, seg_stride: int, seg_bytes: int, stream=None):
    """gather_segments of the K and the V cache with the same idx, one launch; the caches share their
    geometry, as do out_k and out_v."""
    L = load()
    n_seg, n_idx = idx.shape
    if kcache.shape != vcache.shape or kcache.stride() != vcache.stride() or out_k.shape != out_v.shape \
            or out_k.stride() != out_v.stride():
        raise ValueError("gather_segments_kv: K and V caches (and outputs) must share shape and strides")
    return check(L.qwfn_kv_gather_segments_kv(kcache.data_ptr(), vcache.data_ptr(), kcache.stride(0), kcache.shape[0],
                                              seg_off, seg_stride, seg_bytes, n_seg, idx.data_ptr(), n_idx,
                                              out_k.data_ptr(), out_v.data_ptr(), out_k.stride(1), out_k.stride(0),
                                              _stream(stream)))


def flash_attn_ext(qv: Tensor, kv: Tensor, vv: Tensor, mv: Tensor | None, scale: float, ov: Tensor,
                   variant: int = Q8_X86, ws=None, stream=None, max_bias: float = 0.0, softcap: float = 0.0):
    L = load()
    ws_ptr = ws.data_ptr() if ws is not None else None
    ws_bytes = ws.numel() * ws.element_size() if ws is not None else 0
    return check(L.qwfn_flash_attn_ext_q8_0(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv),
                                            ctypes.byref(mv) if mv is not None else None, scale, max_bias, softcap,
                                            ctypes.byref(ov), variant, ws_ptr, ws_bytes, _stream(stream)))


def flash_attn_ext_seq(qv: Tensor, kv: Tensor, vv: Tensor, mv: Tensor | None, scale: float, ov: Tensor, seq_n_kv,
                       variant: int = Q8_X86, ws=None, stream=None):
    """Batched attention where sequence b attends its first seq_n_kv[b] keys."""
    L = load()
    n = (ctypes.c_int64 * len(seq_n_kv))(*[int(x) for x in seq_n_kv])
    ws_ptr = ws.data_ptr() if ws is not None else None
    ws_bytes = ws.numel() * ws.element_size() if ws is not None else 0
    return check(L.qwfn_flash_attn_ext_q8_0_seq(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv),
                                                ctypes.byref(mv) if mv is not None else None, scale, 0.0, 0.0,
                                                ctypes.byref(ov), variant, ws_ptr, ws_bytes, n, _stream(stream)))


def fattn_workspace_size_seq(qv: Tensor, kv: Tensor, vv: Tensor, mv: Tensor | None, seq_n_kv) -> int:
    n = (ctypes.c_int64 * len(seq_n_kv))(*[int(x) for x in seq_n_kv])
    return int(load().qwfn_fattn_workspace_size_seq(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv),
                                                    ctypes.byref(mv) if mv is not None else None, n))


def flash_attn_ext_cells(qv: Tensor, kv: Tensor, vv: Tensor, cells, n_cells, pos0: int, scale: float, ov: Tensor,
                         variant: int = Q8_X86, ws=None, stream=None, shared: bool = False):
    """Attention of KV head h's query heads over the cache rows cells[h, :n_cells[h]]
    (cells: device int32 [n_head_kv, stride]; shared: every head reads row 0, the
    reference's one list); query t sees a row at most pos0 + t."""
    L = load()
    n = (ctypes.c_int64 * len(n_cells))(*[int(x) for x in n_cells])
    ws_ptr = ws.data_ptr() if ws is not None else None
    ws_bytes = ws.numel() * ws.element_size() if ws is not None else 0
    if str(cells.dtype) != "torch.int32" or cells.dim() != 2 or cells.stride(1) != 1:
        raise ValueError("cells must be an int32 [n_head_kv, stride] tensor with contiguous rows")
    return check(L.qwfn_flash_attn_ext_q8_0_cells(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv), cells.data_ptr(),
                                                  n, 0 if shared else cells.stride(0), pos0, scale, ctypes.byref(ov),
                                                  variant, ws_ptr,
                                                  ws_bytes, _stream(stream)))


def flash_attn_ext_query_cells(qv: Tensor, kv: Tensor, vv: Tensor, cells, n_cells, pos0: int, scale: float,
                               ov: Tensor, gate=None, variant: int = Q8_X86, ws=None, stream=None):
    """Attention of query position t over the cache rows cells[t, :n_cells[t]] (cells:
    device int32 [T, stride] with contiguous rows, read by every KV head; a [1, stride]
    list serves every position), the rows at most pos0 + t; times sigmoid(gate) when
    gate (a torch f32 tensor laid out as the output) is given."""
    L = load()
    gv = out_view(gate) if gate is not None else None
    n = (ctypes.c_int64 * len(n_cells))(*[int(x) for x in n_cells])
    ws_ptr = ws.data_ptr() if ws is not None else None
    ws_bytes = ws.numel() * ws.element_size() if ws is not None else 0
    if str(cells.dtype) != "torch.int32" or cells.dim() != 2 or cells.stride(1) != 1 or not cells.is_cuda:
        raise ValueError("cells must be a device int32 [T, stride] tensor with contiguous rows")
    stride = 0 if cells.shape[0] == 1 else cells.stride(0)
    return check(L.qwfn_flash_attn_ext_q8_0_query_cells(
        ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv), cells.data_ptr(), n, stride, pos0, scale,
        ctypes.byref(gv) if gv is not None else None, ctypes.byref(ov), variant, ws_ptr, ws_bytes, _stream(stream)))


def flash_attn_ext_query_cells_dev(qv: Tensor, kv: Tensor, vv: Tensor, cells, counts, pos0: int, scale: float,
                                   ov: Tensor, gate=None, variant: int = Q8_X86, stream=None):
    """Attention of query position t over the cache rows cells[t, :counts[t]] (cells: device
    int32 [T, stride] with contiguous rows, stride a multiple of 4; counts: device int32
    [T]), the rows at most pos0 + t; times sigmoid(gate) when gate (a torch f32 tensor laid
    out as the output) is given. No workspace."""
    L = load()
    gv = out_view(gate) if gate is not None else None
    for name, x in (("cells", cells), ("counts", counts)):
        if str(x.dtype) != "torch.int32" or not x.is_cuda:
            raise ValueError(f"{name} must be a device int32 tensor")
    if cells.dim() != 2 or cells.stride(1) != 1 or counts.dim() != 1 or not counts.is_contiguous():
        raise ValueError("cells must be [T, stride] with contiguous rows and counts a contiguous [T]")
    return check(L.qwfn_flash_attn_ext_q8_0_query_cells_dev(
        ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv), cells.data_ptr(), counts.data_ptr(), cells.stride(0),
        pos0, scale, ctypes.byref(gv) if gv is not None else None, ctypes.byref(ov), variant, _stream(stream)))


def fattn_workspace_size_query_cells(qv: Tensor, kv: Tensor, vv: Tensor, n_cells, cell_stride: int) -> int:
    n = (ctypes.c_int64 * len(n_cells))(*[int(x) for x in n_cells])
    return int(load().qwfn_fattn_workspace_size_query_cells(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv), n,
                                                            cell_stride))


def fattn_workspace_size_cells(qv: Tensor, kv: Tensor, vv: Tensor, n_cells, cell_stride: int) -> int:
    n = (ctypes.c_int64 * len(n_cells))(*[int(x) for x in n_cells])
    return int(load().qwfn_fattn_workspace_size_cells(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv), n,
                                                      cell_stride))


def flash_attn_ext_append(qv: Tensor, kv: Tensor, vv: Tensor, mv: Tensor | None, scale: float, ov: Tensor,
                          ksrc, vsrc, first_row: int, variant: int = Q8_X86, ws=None, stream=None):
    """K/V append (ksrc, vsrc: torch f32 [n, 256 * n_head_kv]) at first_row, then attention, one launch."""
    L = load()
    ws_ptr = ws.data_ptr() if ws is not None else None
    ws_bytes = ws.numel() * ws.element_size() if ws is not None else 0
    sk, sv = f32_view(ksrc), f32_view(vsrc)
    return check(L.qwfn_flash_attn_ext_q8_0_append(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv),
                                                   ctypes.byref(mv) if mv is not None else None, scale, 0.0, 0.0,
                                                   ctypes.byref(ov), variant, ws_ptr, ws_bytes, ctypes.byref(sk),
                                                   ctypes.byref(sv), first_row, _stream(stream)))


def fattn_workspace_size(qv: Tensor, kv: Tensor, vv: Tensor, mv: Tensor | None = None) -> int:
    return int(load().qwfn_fattn_workspace_size(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv),
                                                ctypes.byref(mv) if mv is not None else None))


def state_restore(srcs, nbytes, dsts, n_slots: int, src_kind: int = SRC_DEVICE, stream=None):
    """srcs: list of n_parts pointers; dsts: list of n_slots*n_parts pointers (slot-major)."""
    L = load()
    n_parts = len(srcs)
    S = (ctypes.c_void_p * max(1, n_parts))(*srcs)
    B = (ctypes.c_size_t * max(1, n_parts))(*nbytes)
    Dd = (ctypes.c_void_p * max(1, len(dsts)))(*dsts)
    return check(L.qwfn_state_restore(S, B, Dd, n_parts, n_slots, src_kind, _stream(stream)))


def device_status(stream=None) -> int:
    L = load()
    f = ctypes.c_uint32(0)
    check(L.qwfn_device_status(_stream(stream), ctypes.byref(f)))
    return int(f.value)


def qsa_pool_cfg(**overrides) -> QsaPoolCfg:
    c = QsaPoolCfg()
    load().qwfn_qsa_pool_cfg_default(ctypes.byref(c))
    for k, v in overrides.items():
        if k == "sections":
            for i in range(4):
                c.sections[i] = int(v[i])
        else:
            setattr(c, k, v)
    return c


def set_rows_f16(dst, src, idx, stream=None):
    """ggml_set_rows F32 -> F16: dst torch f16/uint16 [rows, ne0], src f32 [n, ne0], idx i32 [n] (device)."""
    d = tensor(dst.data_ptr(), TYPE_F16, (dst.shape[1], dst.shape[0]), (2, dst.stride(0) * 2))
    sv = tensor(src.data_ptr(), TYPE_F32, (src.shape[1], src.shape[0]), (4, src.stride(0) * 4))
    iv = tensor(idx.data_ptr(), TYPE_I32, (idx.shape[0],), (4,))
    return check(load().qwfn_set_rows_f16(ctypes.byref(d), ctypes.byref(sv), ctypes.byref(iv), _stream(stream)))


def _check_pool_args(name, cfg, ic, pool, k_norm_w, k_raw=None, **i32):
    """What the C ABI cannot see: the caches are 2-byte rows packed at idx_dim (the kernels
    index row * idx_dim), everything lives on one device, the vectors are contiguous."""
    import torch
    two = (torch.float16, torch.int16) + ((torch.uint16,) if hasattr(torch, "uint16") else ())
    dev_ = ic.device
    for nm, t in (("ic", ic), ("pool", pool)):
        if t.dim() != 2 or t.dtype not in two or t.shape[1] != cfg.idx_dim or t.stride(1) != 1 \
                or t.stride(0) != cfg.idx_dim:
            raise ValueError(f"{name}: {nm} must be a 2-byte [rows, {cfg.idx_dim}] tensor with rows packed at idx_dim")
    vecs = [("k_norm_w", k_norm_w, torch.float32), ("k_raw", k_raw, torch.float32)]
    vecs += [(k, v, torch.int32) for k, v in i32.items()]
    for nm, t, dt in vecs:
        if t is not None and (t.dtype != dt or not t.is_contiguous()):
            raise ValueError(f"{name}: {nm} must be contiguous {dt}")
    for nm, t in [("ic", ic), ("pool", pool)] + [(n, t) for n, t, _ in vecs]:
        if t is not None and (not t.is_cuda or t.device != dev_):
            raise ValueError(f"{name}: {nm} must be on {dev_}")


def qsa_pool_decode(ic, k_raw, write_idx, member_idx, ratio: int, blk_pos, blk_idx, k_norm_w, pool, cfg=None,
                    stream=None):
    """qsa_dec_index: ic / pool torch f16 or uint16 [rows, idx_dim] (device), k_raw f32 [idx_dim] or None,
    the i32 decode inputs on the device."""
    cfg = cfg or qsa_pool_cfg()
    _check_pool_args("qsa_pool_decode", cfg, ic, pool, k_norm_w, k_raw=k_raw, write_idx=write_idx,
                     member_idx=member_idx, blk_pos=blk_pos, blk_idx=blk_idx)
    return check(load().qwfn_qsa_pool_decode(ic.data_ptr(), ic.shape[0], k_raw.data_ptr() if k_raw is not None else None,
                                             write_idx.data_ptr(), member_idx.data_ptr(), ratio, blk_pos.data_ptr(),
                                             blk_idx.data_ptr(), k_norm_w.data_ptr(), pool.data_ptr(), pool.shape[0],
                                             ctypes.byref(cfg), _stream(stream)))


def qsa_pool_decode_steps(ic, k_raw, qds, k_norm_w, pool, cfg=None, stream=None):
    """qsa_dec_index for a step's T positions in one launch: k_raw f32 [T, idx_dim] (rows may be strided) or None;
    qds: the positions' QsaDecodeInputs (qwfn_state), as prepared."""
    cfg = cfg or qsa_pool_cfg()
    T = len(qds)
    _check_pool_args("qsa_pool_decode_steps", cfg, ic, pool, k_norm_w, k_raw=k_raw[0] if k_raw is not None else None,
                     write_idx=qds[0].write_idx, member_idx=qds[0].member_idx, blk_pos=qds[0].blk_pos,
                     blk_idx=qds[0].blk_idx)
    if k_raw is not None and (k_raw.dim() != 2 or k_raw.shape[0] != T or k_raw.stride(1) != 1):
        raise ValueError("qsa_pool_decode_steps: k_raw must be [T, idx_dim] with contiguous rows")
    arr = (QsaInputs * T)(*[q._c() for q in qds])
    return check(load().qwfn_qsa_pool_decode_steps(ic.data_ptr(), ic.shape[0],
                                                   k_raw.data_ptr() if k_raw is not None else None,
                                                   k_raw.stride(0) * 4 if k_raw is not None else 0, arr, T,
                                                   k_norm_w.data_ptr(), pool.data_ptr(), pool.shape[0],
                                                   ctypes.byref(cfg), _stream(stream)))


def qsa_pool_rebuild(ic, n_past: int, ratio: int, k_norm_w, pool, cfg=None, stream=None):
    """Every whole block's pooled key: ic / pool torch f16 or uint16 [rows, idx_dim] (device)."""
    cfg = cfg or qsa_pool_cfg()
    _check_pool_args("qsa_pool_rebuild", cfg, ic, pool, k_norm_w)
    return check(load().qwfn_qsa_pool_rebuild(ic.data_ptr(), ic.shape[0], n_past, ratio, k_norm_w.data_ptr(),
                                              pool.data_ptr(), pool.shape[0], ctypes.byref(cfg), _stream(stream)))


def kv_produce(cur, wk, wv, k_norm_w, pos, kcache, vcache, first_row: int, variant: int = Q8_X86, rope=None,
               stream=None):
    """K/V producer: cur torch f32 [T, n_embd]; wk, wv torch f16 or bf16 [kv_dim, n_embd]; k_norm_w f32 [256];
    pos i32 [4 * T]; caches uint8 [n_rows, kv_dim/32*34] (all on the device)."""
    T, E = cur.shape
    kv_dim = wk.shape[0]
    cv = tensor(cur.data_ptr(), TYPE_F32, (E, T), (4, cur.stride(0) * 4))
    import torch
    wt = TYPE_BF16 if wk.dtype == torch.bfloat16 else TYPE_F16
    if wv.dtype != wk.dtype or wk.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("kv_produce: wk and wv must both be float16 or both bfloat16")
    wkv = tensor(wk.data_ptr(), wt, (E, kv_dim), (2, wk.stride(0) * 2))
    wvv = tensor(wv.data_ptr(), wt, (E, kv_dim), (2, wv.stride(0) * 2))
    kcv = tensor(kcache.data_ptr(), TYPE_Q8_0, (kv_dim, kcache.shape[0]), (34, kcache.stride(0)))
    vcv = tensor(vcache.data_ptr(), TYPE_Q8_0, (kv_dim, vcache.shape[0]), (34, vcache.stride(0)))
    rope = rope or rope_cfg()
    return check(load().qwfn_kv_produce_q8_0(ctypes.byref(cv), ctypes.byref(wkv), ctypes.byref(wvv),
                                             k_norm_w.data_ptr(), pos.data_ptr(), ctypes.byref(rope), ctypes.byref(kcv),
                                             ctypes.byref(vcv), first_row, variant, _stream(stream)))


def flash_attn_ext_gated(qv: Tensor, kv: Tensor, vv: Tensor, mv: Tensor | None, scale: float, ov: Tensor, gate,
                         variant: int = Q8_X86, ws=None, stream=None):
    """Attention times sigmoid(gate): gate a torch f32 tensor laid out as the output."""
    L = load()
    gv = out_view(gate)
    ws_ptr = ws.data_ptr() if ws is not None else None
    ws_bytes = ws.numel() * ws.element_size() if ws is not None else 0
    return check(L.qwfn_flash_attn_ext_q8_0_gated(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv),
                                                  ctypes.byref(mv) if mv is not None else None, scale, 0.0, 0.0,
                                                  ctypes.byref(ov), ctypes.byref(gv), variant, ws_ptr, ws_bytes,
                                                  _stream(stream)))


def gated_delta_net(q, k, v, g, beta, state, out, n_k: int, snap=None, n_snap: int = 0, scale: float | None = None,
                    stream=None):
    """The gated delta rule over T tokens. q, k: torch f32 [T, >= n_k*128] (token stride = row stride);
    v: [T, >= n_v*128]; g, beta: [T, n_v]; state [n_v, 128, 128] in place; out [T, n_v, 128];
    snap [>= n_snap, n_v, 128, 128] or None."""
    T = q.shape[0]
    n_v, hd = state.shape[0], state.shape[1]
    scale = 1.0 / hd ** 0.5 if scale is None else scale
    return check(load().qwfn_gated_delta_net(q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), v.data_ptr(),
                                             v.stride(0), g.data_ptr(), beta.data_ptr(), T, n_k, n_v, hd, scale,
                                             state.data_ptr(), out.data_ptr(),
                                             snap.data_ptr() if snap is not None else None,
                                             snap.stride(0) * 4 if snap is not None else 0, n_snap, _stream(stream)))
