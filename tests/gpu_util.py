"""Helpers for the GPU parity tests: move numpy inputs to the device, call the
HIP library through its C ABI, and bring results back."""
from __future__ import annotations

import sys

import numpy as np


def say(msg: str) -> None:
    """Name the case before a GPU step (so a fault is attributable)."""
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def dev(a: np.ndarray):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t) -> np.ndarray:
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def gpu_attn(K, q: np.ndarray, kc: np.ndarray, vc: np.ndarray, n_kv: int, nh_kv: int, mask: np.ndarray | None,
             scale: float, variant: int = 1, ws: bool = False) -> np.ndarray:
    """q [T, nh, hd] or [B, T, nh, hd]; kc/vc uint8 [n_ctx, rb] (or [B, n_ctx, rb]); mask uint16 F16 bits
    [T, n_kv] / [B|1, H|1, T, n_kv] or None. Returns float32 shaped like q."""
    import torch
    q4 = q if q.ndim == 4 else q[None]
    B, T, nh, hd = q4.shape
    qd = dev(q4.astype(np.float32))
    kd, vd = dev(kc), dev(vc)
    if kc.ndim == 3:
        kb, n_ctx, rb = kc.shape
        kv = K.tensor(kd.data_ptr(), K.TYPE_Q8_0, (hd, n_kv, nh_kv, kb), (34, rb, hd // 32 * 34, n_ctx * rb))
        vv = K.tensor(vd.data_ptr(), K.TYPE_Q8_0, (hd, n_kv, nh_kv, kb), (34, rb, hd // 32 * 34, n_ctx * rb))
    else:
        kv = K.cache_attn_view(kd, n_kv, nh_kv, hd)
        vv = K.cache_attn_view(vd, n_kv, nh_kv, hd)
    md = None
    mv = None
    if mask is not None:
        md = dev(mask.view(np.float16))
        mv = K.mask_view(md)
    out = torch.full((B, T, nh, hd), float("nan"), dtype=torch.float32, device="cuda")
    wst = None
    if ws:
        n = K.fattn_workspace_size(K.q_view(qd), kv, vv, mv)
        wst = torch.empty(max(n, 256), dtype=torch.uint8, device="cuda")
    K.flash_attn_ext(K.q_view(qd), kv, vv, mv, scale, K.out_view(out), variant, ws=wst)
    o = host(out)
    return o if q.ndim == 4 else o[0]
