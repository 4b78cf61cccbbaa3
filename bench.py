"""Benchmark of the q8_0 KV-cache hot path on one MI355X.

Workload (default, the MTP verify decode step): 12 full-attention layers,
n_head 16, n_head_kv 2, head size 256, a q8_0 K/V cache at depth 16384 per
layer (K/V ~N(0,1), 4 outlier channels per KV head scaled x8). One step =
for every layer: append 3 new K and V rows (set_rows F32 -> q8_0 at
16384..16386), then flash attention of 3 F32 query tokens (1 + 2 drafts,
causal among them) over the 16387 cached rows, read straight from the raw
q8_0 cache. Inputs are resident in HBM before timing starts. Three independent
12-layer cache sets are rotated step by step (642 MB) so the 256 MB Infinity
Cache cannot serve a repeated layer.

Reported: µs per layer and the achieved algorithmic HBM throughput (GB/s) of
the whole step, replayed from a HIP graph (value) and launched eagerly; the
attention op's own event-timed roofline; and the ggml-cpu flash_attn_ext
semantics (the oracle) timed on this host's cores over one layer.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "qwfn-hybrid_amd"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "decode-attn µs/layer + achieved HBM GB/s (% peak) over q8_0 KV at 16K/64K ctx"
HBM_PEAK_GBS = 8000.0
ROW = 544                     # q8_0 row of K (or V) per token: 2 KV heads x 272 bytes


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--depth", type=int, default=16384)
    ap.add_argument("--T", type=int, default=3)
    ap.add_argument("--layers", type=int, default=12)
    ap.add_argument("--sets", type=int, default=3, help="independent cache sets rotated per step")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="bound on the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--separate-append", action="store_true",
                    help="append K/V with its own launch before the attention launch (default: fused into it)")
    ap.add_argument("--long-depth", type=int, default=65536,
                    help="also time the attention op alone at this depth (0: skip)")
    ap.add_argument("--no-rows", action="store_true",
                    help="skip the per-row measurements (append, gather, restore, batch decode, prefill)")
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="also run one device copy of this many MiB (counter calibration)")
    return ap.parse_args()


def cpu_model() -> str | None:
    """The host CPU: model name, family / model / stepping, and the widest x86 vector
    extension it reports (what a -march=native build can use)."""
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k = k.strip()
            if k in ("model name", "cpu family", "model", "stepping", "flags") and k not in info:
                info[k] = v.strip()
            if len(info) == 5:
                break
    except OSError:
        return None
    if "model name" not in info:
        return None
    flags = set(info.get("flags", "").split())
    vec = next((f for f in ("avx512f", "avx2", "avx", "sse4_2") if f in flags), "none")
    return (f"{info['model name']} (family {info.get('cpu family', '?')}, model {info.get('model', '?')}, "
            f"stepping {info.get('stepping', '?')}; widest vector ISA: {vec})")


def timed(torch, fn, reps: int) -> float:
    """Average µs per call of fn(k) over reps back-to-back calls on the current stream."""
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    fn(0)                                        # warm-up
    torch.cuda.synchronize()
    e0.record(stream)
    for k in range(reps):
        fn(k)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps


def timed_graph(torch, fn, per_graph: int, reps: int) -> float:
    """Average µs per call of fn(k) with per_graph calls captured in one HIP graph and the
    graph replayed reps times: for launches shorter than the host's per-call cost."""
    stream = torch.cuda.current_stream()
    fn(0)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            for k in range(per_graph):
                fn(k)
    stream.wait_stream(side)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * per_graph)


def measure_state_rows(K, torch, np, dev, gbs) -> dict:
    """The state rows on the model's own state (48 layers, 73728 positions, 2 rollback
    slots): reset of the recurrent region, an MTP-verify rollback, snapshot save and
    load of an 8192-position prefix with device blobs (and save into pinned host
    blobs), the 512-query causal mask of a prefill chunk, and one decode step's
    sparse-attention inputs and cell mask."""
    import ctypes
    import qwfn_state as S
    rows = {}
    frac = lambda b, us: round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
    st = S.State()
    ok, err = st.init(S.config(73728, n_rollback=2), 0)
    if not ok:
        raise RuntimeError(err)
    rec = st.rollback_bytes() // 2
    us = timed(torch, lambda k: st.reset(), 10)
    rows["state_reset"] = {"us_per_op": round(us, 1), "bytes_written": rec, "GBs": gbs(rec, us), "frac": frac(rec, us)}

    def rollback(k):
        # alternate the two slots: one slot image read every time would stay in the 256 MB cache
        st.step_done(3, verified=True)
        ok_, err_ = st.rollback_n(1 + (k & 1))
        if not ok_:
            raise RuntimeError(err_)
    us = timed(torch, rollback, 10)
    rows["state_rollback"] = {"us_per_op": round(us, 1), "bytes_read": rec, "bytes_written": rec,
                              "GBs": gbs(2 * rec, us), "frac": frac(2 * rec, us)}

    st.reset()
    st.step_done(8192)
    parts = S.snapshot_parts([st], 8192)
    snap_b = sum(b for _, b in parts)
    blobs = [torch.empty(max(b, 1), dtype=torch.uint8, device=dev) for _, b in parts]
    H = (ctypes.c_void_p * 1)(st.handle)
    P = (ctypes.c_void_p * len(parts))(*[x.data_ptr() for x in blobs])
    B = (ctypes.c_size_t * len(parts))(*[b for _, b in parts])
    L = K.load()
    stream = lambda: K._stream(None)
    us = timed(torch, lambda k: K.check(L.qwfn_snapshot_save(H, 1, P, B, len(parts), S.MEM_DEVICE, None, stream())), 10)
    rows["snapshot_save_device"] = {"us_per_op": round(us, 1), "positions": 8192, "parts": len(parts),
                                    "bytes": snap_b, "GBs": gbs(2 * snap_b, us), "frac": frac(2 * snap_b, us)}
    us = timed(torch, lambda k: K.check(L.qwfn_snapshot_load(H, 1, 8192, P, B, len(parts), S.MEM_DEVICE, stream())), 10)
    moved = 2 * snap_b + rec                       # the load resets the recurrent region first
    rows["snapshot_load_device"] = {"us_per_op": round(us, 1), "bytes": snap_b, "GBs": gbs(moved, us),
                                    "frac": frac(moved, us)}
    hb = [torch.empty(max(b, 1), dtype=torch.uint8, pin_memory=True) for _, b in parts]
    PH = (ctypes.c_void_p * len(parts))(*[x.data_ptr() for x in hb])
    us = timed(torch, lambda k: K.check(L.qwfn_snapshot_save(H, 1, PH, B, len(parts), S.MEM_HOST, None, stream())), 3)
    rows["snapshot_save_pinned_host"] = {"us_per_op": round(us, 1), "bytes": snap_b, "host_link_GBs": gbs(snap_b, us)}
    del blobs, hb
    # the server's switch between two conversations of 8192 positions (restore_or_reset):
    # the current one is set aside in the HBM pool and the other restored
    pool = S.SnapPool(1024 << 20, 4, 0)
    convs = [[7] * 8192, [9] * 8192]
    pool.save_seq([st], convs[1])

    held = [0]                                     # the conversation the state holds
    ctoks = [(ctypes.c_int32 * 8192)(*c) for c in convs]
    ptoks = [(ctypes.c_int32 * 8193)(*(c + [1])) for c in convs]
    n_out = ctypes.c_int32(0)

    def switch(k):
        cur = held[0]
        K.check(L.qwfn_snap_pool_restore_or_reset(pool._h, H, 1, ctoks[cur], 8192, 0, ptoks[1 - cur], 8193, 0,
                                                  ctypes.byref(n_out), stream()))
        if n_out.value != 8192:
            raise RuntimeError("pool: the conversation was not restored")
        held[0] = 1 - cur
    us = timed(torch, switch, 10)
    moved = 4 * snap_b + rec                       # save (read + write), reset, load (read + write)
    rows["pool_switch_conversation"] = {"us_per_op": round(us, 1), "positions": 8192, "GBs": gbs(moved, us),
                                        "frac": frac(moved, us)}
    pool.close()
    st.close()

    T, d0 = 512, 16384
    mask = torch.empty((T, d0 + T), dtype=torch.float16, device=dev)
    us = timed_graph(torch, lambda k: S.causal_mask_f16(mask, d0 + T, T, d0), 16, 10)
    rows["causal_mask_512_at_16k"] = {"us_per_op": round(us, 2), "bytes_written": mask.numel() * 2,
                                      "GBs": gbs(mask.numel() * 2, us), "frac": frac(mask.numel() * 2, us)}
    del mask
    nb_max = 73728 // 4
    qd, qk = S.QsaDecodeInputs(4, nb_max), S.QsaDecodeInputs(4, nb_max)
    cells = torch.randint(0, 65536, (2052,), dtype=torch.int32, device=dev)
    cmask = torch.empty(2304, dtype=torch.float16, device=dev)
    gcells = torch.empty(2304, dtype=torch.int32, device=dev)

    def decode_inputs(k):
        qd.prepare(65533 + (k & 1))
        qk.prepare(65534 + (k & 1), prev=qd)
        S.cell_mask_f16(cells, 65533, 2304, cmask, gcells)
    us = timed_graph(torch, decode_inputs, 16, 10)
    # the decode step's block selection (qsa_dec_cells) for a 3-position verify step at
    # 73728 positions: 18432 pooled f16 keys scored against 4 indexer heads, top 513
    nb, kb = 73728 // 4, 513
    gsel = torch.Generator(device=dev)
    gsel.manual_seed(7)
    pool = (torch.randn((nb, 128), generator=gsel, device=dev) * 0.5).to(torch.float16)
    qsel = torch.randn((3, 4, 128), generator=gsel, device=dev)
    bsel = torch.zeros((3, nb), dtype=torch.float32, device=dev)
    bcells = torch.arange(nb * 4, dtype=torch.int32, device=dev)
    csel = torch.empty((3, kb * 4), dtype=torch.int32, device=dev)
    wsel = torch.empty(K.load().qwfn_qsa_select_workspace_size(nb, 3), dtype=torch.uint8, device=dev)
    us_sel = timed_graph(torch, lambda k: S.qsa_select_cells(pool, qsel, bsel, kb, bcells, 4, csel, ws=wsel), 8, 10)
    # compulsory bytes: the pool once, the bias rows, the cells written
    sel_bytes = nb * 128 * 2 + 3 * nb * 4 + 3 * kb * 4 * 4
    rows["qsa_select_cells"] = {"us_per_call": round(us_sel, 2), "blocks": nb, "k_blocks": kb, "queries": 3,
                                "bytes": sel_bytes, "GBs": gbs(sel_bytes, us_sel), "frac": frac(sel_bytes, us_sel)}
    del pool, qsel, bsel, bcells, csel, wsel
    rows["decode_step_inputs"] = {"us_per_step": round(us, 2), "launches": 3,
                                  "what": "qsa_decode_prepare, qsa_decode_prepare_k (18432-block bias), cell mask 2052->2304"}

    # ---- the QSA index producer: one decode step's raw key + pooled block key, and the
    #      pool rebuild after a 65536-position prefill (16384 blocks of 4) ----
    n_ctx, ratio = 73728, 4
    ic = (torch.randn((n_ctx, 128), generator=gsel, device=dev)).to(torch.float16)
    kpool = torch.zeros((n_ctx // ratio, 128), dtype=torch.float16, device=dev)
    knw = torch.rand(128, generator=gsel, device=dev) + 0.5
    kraw = torch.randn(128, generator=gsel, device=dev)
    us = timed_graph(torch, lambda k: K.qsa_pool_decode(ic, kraw, qd.write_idx, qd.member_idx, ratio, qd.blk_pos,
                                                         qd.blk_idx, knw, kpool), 16, 10)
    rows["qsa_pool_decode"] = {"us_per_call": round(us, 2), "ratio": ratio,
                               "what": "raw key F16 set_rows + mean-pool, RMS norm, IMROPE of its block (one launch)"}
    n_past = 65536
    us = timed(torch, lambda k: K.qsa_pool_rebuild(ic, n_past, ratio, knw, kpool), 20)
    rb = n_past * 128 * 2 + (n_past // ratio) * 128 * 2
    rows["qsa_pool_rebuild_64k"] = {"us_per_call": round(us, 2), "blocks": n_past // ratio, "bytes": rb,
                                    "GBs": gbs(rb, us), "frac": frac(rb, us)}
    del ic, kpool

    # ---- the K/V producer of a 3-token verify step (F16 weights 2 x 512 x 2560) ----
    E, kv_dim, T3 = 2560, 512, 3
    wk = (torch.randn((kv_dim, E), generator=gsel, device=dev) * 0.02).to(torch.float16)
    wv = (torch.randn((kv_dim, E), generator=gsel, device=dev) * 0.02).to(torch.float16)
    hid = torch.randn((T3, E), generator=gsel, device=dev)
    kpos = torch.arange(16384, 16384 + T3, dtype=torch.int32, device=dev).repeat(4)
    kcp = torch.zeros((16400, 544), dtype=torch.uint8, device=dev)
    vcp = torch.zeros((16400, 544), dtype=torch.uint8, device=dev)
    knw256 = torch.rand(256, generator=gsel, device=dev) + 0.5
    us = timed_graph(torch, lambda k: K.kv_produce(hid, wk, wv, knw256, kpos, kcp, vcp, 16384), 16, 10)
    pb = 2 * kv_dim * E * 2 + T3 * E * 4 + 2 * T3 * 544
    rows["kv_produce_T3"] = {"us_per_call": round(us, 2), "bytes": pb, "GBs": gbs(pb, us), "frac": frac(pb, us),
                             "what": "attn_k/attn_v projections + K RMS norm + IMROPE + q8_0 append, two launches"}
    del wk, wv, kcp, vcp

    # ---- one DeltaNet layer's recurrent update for a 3-token verify step with 2
    #      rollback snapshots (48 value heads of 128: 3.1 MB of state) ----
    conv = torch.randn((T3, 10240), generator=gsel, device=dev)
    conv[:, :4096] = torch.nn.functional.normalize(conv[:, :4096].view(T3, 32, 128), dim=-1).view(T3, 4096)
    dg = -torch.rand((T3, 48), generator=gsel, device=dev)
    db = torch.rand((T3, 48), generator=gsel, device=dev)
    dstates = [torch.randn((48, 128, 128), generator=gsel, device=dev) * 0.05 for _ in range(8)]
    dout = torch.empty((T3, 48, 128), dtype=torch.float32, device=dev)
    dsnap = torch.empty((2, 48, 128, 128), dtype=torch.float32, device=dev)
    us = timed_graph(torch, lambda k: K.gated_delta_net(conv[:, :2048], conv[:, 2048:4096], conv[:, 4096:], dg, db,
                                                        dstates[k % 8], dout, 16, dsnap, 2), 16, 10)
    sb = 48 * 128 * 128 * 4
    db_ = 2 * sb + 2 * sb + T3 * 10240 * 4 + T3 * 48 * 128 * 4
    rows["gated_delta_net_T3"] = {"us_per_call": round(us, 2), "bytes": db_, "GBs": gbs(db_, us), "frac": frac(db_, us),
                                  "what": "state read + written, 2 rollback snapshots written, q/k/v/out"}
    del conv, dstates, dsnap
    torch.cuda.empty_cache()
    return rows


def measure_qsa_step_rows(K, torch, np, dev, gen, n_layers: int = 12) -> dict:
    """The reference's default verify step with QSA on (qwfn_engine.cpp:2259-2280 ->
    qwfn_graph.cpp:653-705) for one attention layer, T = 3 positions at 73700 of a
    73728-position context (18432 pooled blocks of 4), composed as
    tests/test_gpu_qsa_verify_step.py composes it: prepare / prepare_k x3, pool decode x3,
    one top-513 selection for the 3 queries, the K/V producer (F16 weights), one gated
    attention launch over the 3 lists of 2052 cells and its merge. 12 layers' states (index
    cache, pool, K/V caches, weights: 1.3 GB) are rotated so each layer's reads come from
    HBM; one step of the 12 layers is captured in a HIP graph and replayed. Also the
    attention alone at the reference's shape: 3 per-position lists (one launch) and one
    shared list at T = 1 (decode)."""
    import qwfn_state as S
    rows = {}
    n_ctx, ratio, nbm, T, nh, nh_kv, kb, E = 73728, 4, 18432, 3, 24, 2, 513, 2560
    n_past, nc = 73700, 513 * 4
    frac = lambda b, us: round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
    gbs = lambda b, us: round(b / (us * 1e-6) / 1e9, 1)

    def cache():
        c = torch.randint(-100, 100, (n_ctx, ROW), dtype=torch.int8, device=dev, generator=gen).view(torch.uint8)
        c.view(-1, 34)[:, 0] = 0x1F
        c.view(-1, 34)[:, 1] = 0x21
        return c
    layers = []
    for _ in range(n_layers):
        kc, vc = cache(), cache()
        layers.append(dict(
            ic=torch.randn((n_ctx, 128), generator=gen, device=dev).to(torch.float16),
            pool=(torch.randn((nbm, 128), generator=gen, device=dev) * 0.5).to(torch.float16),
            kc=kc, vc=vc,
            kv=K.tensor(kc.data_ptr(), K.TYPE_Q8_0, (256, n_ctx, nh_kv, 1), (34, ROW, 272, n_ctx * ROW)),
            vv=K.tensor(vc.data_ptr(), K.TYPE_Q8_0, (256, n_ctx, nh_kv, 1), (34, ROW, 272, n_ctx * ROW)),
            wk=(torch.randn((512, E), generator=gen, device=dev) * 0.02).to(torch.float16),
            wv=(torch.randn((512, E), generator=gen, device=dev) * 0.02).to(torch.float16),
            knw=torch.rand(256, generator=gen, device=dev) + 0.5,
            knw_idx=torch.rand(128, generator=gen, device=dev) + 0.5))
    bias = torch.empty((T, nbm), dtype=torch.float32, device=dev)
    qds = []
    for t in range(T):
        qd = S.QsaDecodeInputs(ratio, nbm)
        qd.bias = bias[t]
        qds.append(qd)
    qds[0].rebuild_bias(n_past)
    blk_cells = torch.empty(nbm * ratio, dtype=torch.int32, device=dev)
    S.qsa_tables(blk_cells, ratio)
    k_raw = torch.randn((T, 128), generator=gen, device=dev)
    q_idx = torch.randn((T, 4, 128), generator=gen, device=dev)
    cur = torch.randn((T, E), generator=gen, device=dev)
    pos = torch.arange(n_past, n_past + T, dtype=torch.int32, device=dev).repeat(4)
    cells = torch.empty((T, nc), dtype=torch.int32, device=dev)
    wsel = torch.empty(K.load().qwfn_qsa_select_workspace_size(nbm, T), dtype=torch.uint8, device=dev)
    q = torch.randn((1, T, nh, 256), generator=gen, device=dev)
    gate = torch.randn((1, T, nh, 256), generator=gen, device=dev)
    out = torch.empty((1, T, nh, 256), dtype=torch.float32, device=dev)
    q1, out1 = q[:, :1].contiguous(), torch.empty((1, 1, nh, 256), dtype=torch.float32, device=dev)
    aws = torch.empty(max(256, K.fattn_workspace_size_query_cells(K.q_view(q), layers[0]["kv"], layers[0]["vv"],
                                                                  [nc] * T, nc),
                          K.fattn_workspace_size_cells(K.q_view(q1), layers[0]["kv"], layers[0]["vv"], [nc, nc], 0)),
                      dtype=torch.uint8, device=dev)

    def tail(L):
        S.qsa_select_cells(L["pool"], q_idx, bias, kb, blk_cells, ratio, cells, ws=wsel)
        K.kv_produce(cur, L["wk"], L["wv"], L["knw"], pos, L["kc"], L["vc"], n_past)
        K.flash_attn_ext_query_cells(K.q_view(q), L["kv"], L["vv"], cells, [nc] * T, n_past, 1 / 16, K.out_view(out),
                                     gate=gate, ws=aws)

    def step_chained(k):
        # the reference's order: prepare and pool decode one position a call
        L = layers[k % n_layers]
        for t in range(T):
            qds[t].prepare(n_past + t, prev=qds[t - 1] if t else None)
        for t in range(T):
            K.qsa_pool_decode(L["ic"], k_raw[t], qds[t].write_idx, qds[t].member_idx, ratio, qds[t].blk_pos,
                              qds[t].blk_idx, L["knw_idx"], L["pool"])
        tail(L)

    def step_two(k):
        # the step's positions batched: one prepare launch, one pool-decode launch
        L = layers[k % n_layers]
        S.qsa_decode_prepare_steps(qds, n_past)
        K.qsa_pool_decode_steps(L["ic"], k_raw, qds, L["knw_idx"], L["pool"])
        tail(L)

    def step(k):
        # the step's preparation and pooling in one launch
        L = layers[k % n_layers]
        S.qsa_decode_prepare_pool_steps(qds, n_past, L["ic"], k_raw, L["knw_idx"], L["pool"])
        tail(L)
    us_chained = timed_graph(torch, step_chained, n_layers, 10)
    us_two = timed_graph(torch, step_two, n_layers, 10)
    us = timed_graph(torch, step, n_layers, 10)
    lists = cells.cpu().numpy()
    union = int(np.unique(lists).size)
    # compulsory bytes per layer: the pool once (select), the bias rows, the K/V weights
    # (producer), the K/V rows of the union of the three lists, the produced rows, q / gate / out
    step_bytes = (nbm * 128 * 2 + T * nbm * 4 + 2 * 512 * E * 2 + union * ROW + 2 * T * ROW + 3 * T * nh * 256 * 4)
    rows["qsa_verify_step_T3"] = {
        "us_per_layer": round(us, 2), "bytes_per_layer": step_bytes, "GBs": gbs(step_bytes, us),
        "frac": frac(step_bytes, us), "blocks": nbm, "k_blocks": kb, "cells_per_position": nc,
        "union_cells": union, "launches_per_layer": 1 + 2 + 2 + 2,
        "us_per_layer_prepare_then_pool": round(us_two, 2),
        "us_per_layer_positions_one_a_call": round(us_chained, 2),
        "what": "the 3 positions' inputs and index pooling (one launch), select (3 queries), K/V produce, gated "
                "query-cells attention + merge; us_per_layer_prepare_then_pool: the inputs and the pooling in a "
                "launch each; us_per_layer_positions_one_a_call: prepare x3 and pool decode x3 as the reference "
                "issues them"}

    # ---- the attention alone at the reference's decode shape ----
    sel = cells.clone()

    def attn3(k):
        L = layers[k % n_layers]
        K.flash_attn_ext_query_cells(K.q_view(q), L["kv"], L["vv"], sel, [nc] * T, n_past, 1 / 16, K.out_view(out),
                                     gate=gate, ws=aws)
    us = timed_graph(torch, attn3, n_layers, 10)
    ab = union * ROW + 3 * T * nh * 256 * 4
    rows["query_cells_2052_T3"] = {"us_per_launch": round(us, 3), "union_cells": union, "bytes": ab,
                                   "GBs": gbs(ab, us), "frac": frac(ab, us),
                                   "entry": "qwfn_flash_attn_ext_q8_0_query_cells (3 lists of 2052, gated) + merge"}
    sel1 = sel[:1].contiguous()

    def attn1(k):
        L = layers[k % n_layers]
        K.flash_attn_ext_cells(K.q_view(q1), L["kv"], L["vv"], sel1, [nc, nc], n_past, 1 / 16, K.out_view(out1),
                               ws=aws, shared=True)
    us = timed_graph(torch, attn1, n_layers, 10)
    ab1 = nc * ROW + 2 * nh * 256 * 4
    rows["shared_cells_2052_T1"] = {"us_per_launch": round(us, 3), "cells": nc, "bytes": ab1, "GBs": gbs(ab1, us),
                                    "frac": frac(ab1, us),
                                    "entry": "qwfn_flash_attn_ext_q8_0_cells (one list shared by both KV heads) + merge"}
    del layers
    torch.cuda.empty_cache()
    return rows


def measure_rows(K, torch, np, dev, gen) -> dict:
    """The other rows of the path on their own workloads: append of a 512-row prefill chunk,
    the per-KV-head sparse gather at 64K, snapshot restore into 4 slots, batch-4 ragged decode
    and a 512-query causal prefill chunk. Synthetic seeded inputs; each timed back to back
    with HIP events after a warm-up."""
    rows = {}
    kv_dim, nh, nh_kv, hd = 512, 16, 2, 256
    gbs = lambda b, us: round(b / (us * 1e-6) / 1e9, 1)

    # ---- append: cpy of a 512-row F32 chunk of K and of V into the q8_0 caches
    #      (one launch), and the decode step's 3-row set_rows of K and V ----
    n_ctx, d0, T = 16384 + 512, 16384, 512
    caches = [torch.zeros((n_ctx, ROW), dtype=torch.uint8, device=dev) for _ in range(8)]
    srcs = [torch.randn((T, kv_dim), generator=gen, device=dev) for _ in range(8)]
    us = timed_graph(torch, lambda k: K.cpy_f32_q8_0_kv(srcs[k % 8], caches[(k * 3) % 8], srcs[(k + 1) % 8],
                                                        caches[(k * 3 + 1) % 8], d0), 64, 10)
    b = 2 * T * (kv_dim * 4 + ROW)
    rows["append_kv_512"] = {"us_per_launch": round(us, 3), "bytes_per_launch": b, "GBs": gbs(b, us),
                             "frac": round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    idx = torch.arange(d0, d0 + 3, dtype=torch.int32, device=dev)
    us = timed_graph(torch, lambda k: K.set_rows_q8_0_kv(caches[k % 8], srcs[k % 8][:3], caches[(k + 1) % 8],
                                                         srcs[(k + 1) % 8][:3], idx), 64, 10)
    rows["append_kv_3_rows"] = {"us_per_launch": round(us, 3), "bytes_per_launch": 2 * 3 * (kv_dim * 4 + ROW)}
    del caches, srcs

    # ---- sparse selection at 64K: per KV head, top-128 of 1024 blocks of 64 positions by
    #      uniform scores plus the last 512 positions. (i) attention of 3 queries over the
    #      selected cells with the gather fused in (qwfn_flash_attn_ext_q8_0_cells): 32 list
    #      variants rotated over 4 caches, so the touched lines (32 x 9.4 MB) exceed the
    #      Infinity Cache; (ii) the materialised per-head gather of the 272-byte half rows ----
    n_ctx, Tq = 65536, 3
    sets, n_lists = 4, 32
    kvs = []
    for _ in range(sets):
        kc = torch.randint(-100, 100, (n_ctx, ROW), dtype=torch.int8, device=dev, generator=gen).view(torch.uint8)
        vc = torch.randint(-100, 100, (n_ctx, ROW), dtype=torch.int8, device=dev, generator=gen).view(torch.uint8)
        for c in (kc, vc):                       # valid fp16 scales (0x211F ~ 0.0101)
            c.view(-1, 34)[:, 0] = 0x1F
            c.view(-1, 34)[:, 1] = 0x21
        kvs.append((kc, vc))
    rng = np.random.default_rng(4)

    def selection():
        out = []
        for h in range(nh_kv):
            sc = rng.random(1024)
            top = np.argsort(-sc, kind="stable")[:128]
            out.append(np.unique(np.concatenate([(top[:, None] * 64 + np.arange(64)).ravel(),
                                                 np.arange(n_ctx - 512, n_ctx)])))
        return out
    sel = [selection() for _ in range(n_lists)]
    stride = (max(len(x) for ls in sel for x in ls) + 3) // 4 * 4
    cells = []
    for ls in sel:
        c = np.zeros((nh_kv, stride), np.int32)
        for h, x in enumerate(ls):
            c[h, :len(x)] = x
        cells.append((torch.from_numpy(c).to(dev), [len(x) for x in ls]))
    sq = torch.randn((1, Tq, nh, hd), generator=gen, device=dev)
    sout = torch.zeros((1, Tq, nh, hd), dtype=torch.float32, device=dev)
    sviews = [(K.tensor(kc.data_ptr(), K.TYPE_Q8_0, (hd, n_ctx, nh_kv, 1), (34, ROW, 272, n_ctx * ROW)),
               K.tensor(vc.data_ptr(), K.TYPE_Q8_0, (hd, n_ctx, nh_kv, 1), (34, ROW, 272, n_ctx * ROW)))
              for kc, vc in kvs]
    sws = torch.empty(max(256, max(K.fattn_workspace_size_cells(K.q_view(sq), sviews[0][0], sviews[0][1], n, stride)
                                   for _, n in cells)), dtype=torch.uint8, device=dev)

    def sparse(k):
        kv, vv = sviews[k % sets]
        c, n = cells[k % n_lists]
        K.flash_attn_ext_cells(K.q_view(sq), kv, vv, c, n, n_ctx - Tq, 1 / 16, K.out_view(sout), ws=sws)
    for k in range(n_lists):
        sparse(k)
    us = timed(torch, sparse, 4 * n_lists)
    n_sel = float(np.mean([sum(n) for _, n in cells]))
    b = n_sel * 272 * 2 + n_sel * 4 + 2 * Tq * nh * hd * 4
    rows["sparse_64k_cells_attention"] = {
        "us_per_launch": round(us, 3), "cells_per_head": cells[0][1], "T": Tq,
        "bytes_per_launch": int(b), "GBs": gbs(b, us), "frac": round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "entry": "qwfn_flash_attn_ext_q8_0_cells (gather fused into k_fa_dec)"}

    lists = sel[0]
    m = max(len(x) for x in lists)
    idx = torch.from_numpy(np.stack([np.concatenate([x, np.repeat(x[-1:], m - len(x))]) for x in lists])
                           .astype(np.int32)).to(dev)
    gk = torch.zeros((nh_kv, m, 272), dtype=torch.uint8, device=dev)
    gv = torch.zeros((nh_kv, m, 272), dtype=torch.uint8, device=dev)

    def gather(k):
        kc, vc = kvs[k % sets]
        K.gather_segments_kv(kc, vc, idx, gk, gv, 0, 272, 272)

    def gather_two(k):
        kc, vc = kvs[k % sets]
        K.gather_segments(kc, idx, gk, 0, 272, 272)
        K.gather_segments(vc, idx, gv, 0, 272, 272)
    us_two = timed_graph(torch, gather_two, 16, 10)
    us = timed_graph(torch, gather, 16, 10)
    moved = sum(len(x) for x in lists) * 272 * 2
    rows["gather_64k"] = {"us_per_op": round(us, 3), "positions_per_head": [len(x) for x in lists],
                          "bytes_read": moved, "bytes_written": moved, "GBs": gbs(2 * moved, us),
                          "frac": round(2 * moved / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                          "us_per_op_two_launches": round(us_two, 3),
                          "entry": "qwfn_kv_gather_segments_kv (K and V in one launch); us_per_op_two_launches: "
                                   "qwfn_kv_gather_segments for K, then for V"}
    del kvs, gk, gv, sws

    # ---- snapshot restore: 12 layers x 8192 rows of K and V + 36 DeltaNet states
    #      [32,128,128] f32 into 4 slots, from device memory and from pinned host memory ----
    n_layers, n_dn, keep, slot_rows = 12, 36, 8192, 73728
    parts_b = [keep * ROW] * (2 * n_layers) + [32 * 128 * 128 * 4] * n_dn
    src = [torch.randint(0, 256, (pb,), dtype=torch.uint8, device=dev, generator=gen) for pb in parts_b]
    kv_dst = [torch.empty((4, slot_rows, ROW), dtype=torch.uint8, device=dev) for _ in range(2 * n_layers)]
    dn_dst = [torch.empty((4, 32 * 128 * 128 * 4), dtype=torch.uint8, device=dev) for _ in range(n_dn)]
    dsts = []
    for sl in range(4):
        dsts += [kv_dst[i][sl].data_ptr() for i in range(2 * n_layers)] + [dn_dst[i][sl].data_ptr() for i in range(n_dn)]
    src_ptrs = [x.data_ptr() for x in src]
    us = timed(torch, lambda k: K.state_restore(src_ptrs, parts_b, dsts, 4, K.SRC_DEVICE), 10)
    per_slot = sum(parts_b)
    rows["restore_device"] = {"us_per_op": round(us, 1), "bytes_per_slot": per_slot, "slots": 4,
                              "bytes_written": 4 * per_slot, "GBs_written": gbs(4 * per_slot, us)}
    host = [torch.empty((pb,), dtype=torch.uint8, pin_memory=True) for pb in parts_b]
    for h_, d_ in zip(host, src):
        h_.copy_(d_.cpu())
    host_ptrs = [x.data_ptr() for x in host]
    us = timed(torch, lambda k: K.state_restore(host_ptrs, parts_b, dsts, 4, K.SRC_HOST), 5)
    rows["restore_pinned_host"] = {"us_per_op": round(us, 1), "bytes_per_slot": per_slot, "slots": 4,
                                   "host_link_GBs": gbs(per_slot, us)}
    del src, kv_dst, dn_dst, host

    rows.update(measure_state_rows(K, torch, np, dev, gbs))
    rows.update(measure_qsa_step_rows(K, torch, np, dev, gen))

    # ---- batch-4 ragged decode: one query per slot at depths 8192..65536 (mask [n_kv,1,1,4]) ----
    depths = [8192, 16384, 32768, 65536]
    n_kv = max(depths)
    bsets = 2
    bc = []
    for _ in range(bsets):
        kc = torch.randint(0, 256, (4, n_kv, ROW), dtype=torch.uint8, device=dev, generator=gen)
        vc = torch.randint(0, 256, (4, n_kv, ROW), dtype=torch.uint8, device=dev, generator=gen)
        for c in (kc, vc):                       # valid fp16 scales: re-quantise a few rows' worth
            c.view(-1, 34)[:, 0] = 0x20
            c.view(-1, 34)[:, 1] = 0x14
        bc.append((kc, vc))
    mask_np = np.full((4, 1, 1, n_kv), 0xFC00, np.uint16)
    for s_, dp in enumerate(depths):
        mask_np[s_, 0, 0, :dp] = 0
    bmask = torch.from_numpy(mask_np.view(np.float16)).to(dev)
    bq = torch.randn((4, 1, nh, hd), generator=gen, device=dev)
    bout = torch.zeros((4, 1, nh, hd), dtype=torch.float32, device=dev)
    bviews = [(K.cache_attn_view(kc, n_kv, nh_kv, batch=4, batch_stride=n_kv * ROW),
               K.cache_attn_view(vc, n_kv, nh_kv, batch=4, batch_stride=n_kv * ROW)) for kc, vc in bc]
    bmv = K.mask_view(bmask)
    bws = torch.empty(max(256, K.fattn_workspace_size(K.q_view(bq), bviews[0][0], bviews[0][1], bmv)),
                      dtype=torch.uint8, device=dev)
    us = timed(torch, lambda k: K.flash_attn_ext(K.q_view(bq), bviews[k % bsets][0], bviews[k % bsets][1], bmv,
                                                1 / 16, K.out_view(bout), ws=bws), 20)
    b = sum(depths) * 2 * ROW
    rows["batch4_decode_mask_only"] = {"depths": depths, "us_per_launch": round(us, 3), "bytes_per_launch": b,
                                       "GBs": gbs(b, us), "frac": round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    # the same batch with the depths given per sequence (qwfn_flash_attn_ext_q8_0_seq)
    sws = torch.empty(max(256, K.fattn_workspace_size_seq(K.q_view(bq), bviews[0][0], bviews[0][1], None, depths)),
                      dtype=torch.uint8, device=dev)
    us = timed(torch, lambda k: K.flash_attn_ext_seq(K.q_view(bq), bviews[k % bsets][0], bviews[k % bsets][1], None,
                                                    1 / 16, K.out_view(bout), depths, ws=sws), 20)
    rows["batch4_decode"] = {"depths": depths, "us_per_launch": round(us, 3), "bytes_per_launch": b,
                             "GBs": gbs(b, us), "frac": round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                             "entry": "qwfn_flash_attn_ext_q8_0_seq"}
    del bc, bws, sws

    # ---- prefill chunk: 512 causal queries at depths 0, 4096 and 16384 through the same op ----
    for d0 in (0, 4096, 16384):
        T = 512
        n_kv = d0 + T
        kc = torch.randint(-100, 100, (n_kv, ROW), dtype=torch.int8, device=dev, generator=gen).view(torch.uint8)
        vc = torch.randint(-100, 100, (n_kv, ROW), dtype=torch.int8, device=dev, generator=gen).view(torch.uint8)
        for c in (kc, vc):
            c.view(-1, 34)[:, 0] = 0x1F
            c.view(-1, 34)[:, 1] = 0x21
        pm = np.full((T, n_kv), 0xFC00, np.uint16)
        for i in range(T):
            pm[i, :d0 + i + 1] = 0
        pmask = torch.from_numpy(pm.view(np.float16)).to(dev)
        pq = torch.randn((1, T, nh, hd), generator=gen, device=dev)
        pout = torch.zeros((1, T, nh, hd), dtype=torch.float32, device=dev)
        pk, pv, pmv = K.cache_attn_view(kc, n_kv, nh_kv), K.cache_attn_view(vc, n_kv, nh_kv), K.mask_view(pmask)
        pws = torch.empty(max(256, K.fattn_workspace_size(K.q_view(pq), pk, pv, pmv)), dtype=torch.uint8, device=dev)
        us = timed(torch, lambda k: K.flash_attn_ext(K.q_view(pq), pk, pv, pmv, 1 / 16, K.out_view(pout), ws=pws), 20)
        flops = 4 * nh * hd * (T * d0 + T * (T + 1) // 2)      # causal count, QK^T and PV
        rows[f"prefill_512_at_{d0}"] = {"us_per_launch": round(us, 1), "flops": flops,
                                        "TFLOPs": round(flops / (us * 1e-6) / 1e12, 2),
                                        "frac_of_f16_mfma_peak": round(flops / (us * 1e-6) / 2.5e15, 4)}
        del kc, vc, pws
    torch.cuda.empty_cache()
    rows.update(measure_qsa_prefill_row(K, torch, np, dev, gen))
    rows.update(measure_qsa_prefill_row(K, torch, np, dev, gen, d0=65536))
    return rows


def measure_qsa_prefill_row(K, torch, np, dev, gen, d0: int = 16384) -> dict:
    """The reference's default prefill with QSA on (qwfn_graph.cpp:313-414, :466) for a
    512-query chunk at depth d0 (16384: 4224 blocks of 4), 16 heads over 2 KV heads: the
    chunk's block tables and bias, the pooled keys of its blocks, each query's top 513
    blocks (indexer: 4 heads of 128), the causal and the selection masks, and flash
    attention over the selection mask; also the attention alone, and the same keys as
    lists (qwfn_qsa_visible_cells, then k_fa_qc). As the GPU test composes it."""
    import qwfn_state as S
    T, ratio, nh, nh_kv, hd, kb = 512, 4, 16, 2, 256, 513
    n_kv = d0 + T
    nb = n_kv // ratio
    row = (n_kv + 63) // 64 * 64

    def cache():
        c = torch.randint(-100, 100, (n_kv, ROW), dtype=torch.int8, device=dev, generator=gen).view(torch.uint8)
        c.view(-1, 34)[:, 0] = 0x1F
        c.view(-1, 34)[:, 1] = 0x21
        return c
    kc, vc = cache(), cache()
    ic = torch.randn((n_kv, 128), generator=gen, device=dev).to(torch.float16)
    knw = torch.rand(128, generator=gen, device=dev) + 0.5
    q_idx = torch.randn((T, 4, 128), generator=gen, device=dev)
    bc = torch.empty(nb * ratio, dtype=torch.int32, device=dev)
    bp = torch.empty(4 * nb, dtype=torch.int32, device=dev)
    bias = torch.empty((T, nb), dtype=torch.float32, device=dev)
    pool = torch.empty((nb, 128), dtype=torch.float16, device=dev)
    cells = torch.empty((T, kb * ratio), dtype=torch.int32, device=dev)
    wsel = torch.empty(K.load().qwfn_qsa_select_workspace_size(nb, T), dtype=torch.uint8, device=dev)
    causal = torch.empty((T, row), dtype=torch.float16, device=dev)
    qmask = torch.empty((T, row), dtype=torch.float16, device=dev)
    pq = torch.randn((1, T, nh, hd), generator=gen, device=dev)
    pout = torch.empty((1, T, nh, hd), dtype=torch.float32, device=dev)
    pk, pv, pmv = K.cache_attn_view(kc, n_kv, nh_kv), K.cache_attn_view(vc, n_kv, nh_kv), K.mask_view(qmask)
    pws = torch.empty(max(256, K.fattn_workspace_size(K.q_view(pq), pk, pv, pmv)), dtype=torch.uint8, device=dev)

    def chain(k):
        S.qsa_chunk_inputs(d0, T, ratio, None, bc, bp, bias)
        K.qsa_pool_rebuild(ic, n_kv, ratio, knw, pool)
        S.qsa_select_cells(pool, q_idx, bias, kb, bc, ratio, cells, ws=wsel)
        S.causal_mask_f16(causal, n_kv, T, d0)
        S.qsa_mask_f16(cells, causal, n_kv, qmask)
        K.flash_attn_ext(K.q_view(pq), pk, pv, pmv, 1 / 16, K.out_view(pout), ws=pws)
    us_chain = timed(torch, chain, 5)
    us_attn = timed(torch, lambda k: K.flash_attn_ext(K.q_view(pq), pk, pv, pmv, 1 / 16, K.out_view(pout), ws=pws), 5)
    # the same keys as lists: each query's visible cells (no causal or selection mask),
    # then attention over them
    lists = torch.empty((T, kb * ratio), dtype=torch.int32, device=dev)
    counts = torch.empty((T,), dtype=torch.int32, device=dev)
    lout = torch.empty((1, T, nh, hd), dtype=torch.float32, device=dev)

    def chain_lists(k):
        S.qsa_chunk_inputs(d0, T, ratio, None, bc, bp, bias)
        K.qsa_pool_rebuild(ic, n_kv, ratio, knw, pool)
        S.qsa_select_cells(pool, q_idx, bias, kb, bc, ratio, cells, ws=wsel)
        S.qsa_visible_cells(cells, n_kv, d0, lists, counts)
        K.flash_attn_ext_query_cells_dev(K.q_view(pq), pk, pv, lists, counts, d0, 1 / 16, K.out_view(lout))
    us_lists = timed(torch, chain_lists, 5)
    us_lattn = timed(torch, lambda k: K.flash_attn_ext_query_cells_dev(K.q_view(pq), pk, pv, lists, counts, d0, 1 / 16,
                                                                        K.out_view(lout)), 5)
    lerr = float((lout - pout).abs().max().item())
    visible = int((qmask[:, :n_kv] == 0).sum().item())
    flops = 4 * nh * hd * visible                               # QK^T and PV over the visible keys
    return {f"prefill_512_at_{d0}_qsa": {
        "us_per_layer": round(us_chain, 1), "us_attention": round(us_attn, 1), "us_inputs": round(us_chain - us_attn, 1),
        "blocks": nb, "k_blocks": kb, "visible_keys_per_query": round(visible / T, 1), "flops": flops,
        "TFLOPs": round(flops / (us_attn * 1e-6) / 1e12, 2),
        "frac_of_f16_mfma_peak": round(flops / (us_attn * 1e-6) / 2.5e15, 4),
        "us_per_layer_lists": round(us_lists, 1), "us_attention_lists": round(us_lattn, 1),
        "lists_gathered_bytes": int(counts.sum().item()) * nh_kv * 2 * 272,
        "lists_max_abs_diff_vs_mask": lerr,
        "what": f"chunk tables + pool of {nb} blocks + top-513 select for 512 queries + causal and selection masks "
                "+ k_fa_pre over the selection mask; _lists: the same selection, visible cells, k_fa_qc"}}


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this path has no multi-GPU form to run (asked for --gpus {args.gpus}); "
              "across GPUs it would shard by KV head and by key-position range, each GPU running these kernels on "
              "its share and the split partials merged across GPUs.",
              file=sys.stderr)
        return 2
    import numpy as np
    import torch

    import qwfn_kv as K

    torch.manual_seed(2)
    dev = torch.device("cuda:0")
    K.check(K.load().qwfn_init(0))
    L, T, depth, nh, nh_kv, hd = args.layers, args.T, args.depth, 16, 2, 256
    n_kv = depth + T
    n_ctx = (n_kv + 15) // 16 * 16
    kv_dim = nh_kv * hd
    gen = torch.Generator(device=dev)
    gen.manual_seed(2)

    # ---- synthetic caches: N(0,1) rows, 4 outlier channels per KV head x8, quantised by the library ----
    t0 = time.time()
    ch = torch.stack([torch.randperm(hd, generator=gen, device=dev)[:4] + h * hd for h in range(nh_kv)]).flatten()
    scale_vec = torch.ones(kv_dim, device=dev)
    scale_vec[ch] = 8.0
    caches = []   # [set][layer] -> (kc, vc)
    chunk = 4096
    for s in range(args.sets):
        layer_caches = []
        for _ in range(L):
            kc = torch.zeros((n_ctx, ROW), dtype=torch.uint8, device=dev)
            vc = torch.zeros((n_ctx, ROW), dtype=torch.uint8, device=dev)
            for c in (kc, vc):
                for r0 in range(0, depth, chunk):
                    n = min(chunk, depth - r0)
                    x = torch.randn((n, kv_dim), generator=gen, device=dev) * scale_vec
                    K.cpy_f32_q8_0(x, c, r0)
            layer_caches.append((kc, vc))
        caches.append(layer_caches)
    newk = [(torch.randn((T, kv_dim), generator=gen, device=dev) * scale_vec) for _ in range(L)]
    newv = [(torch.randn((T, kv_dim), generator=gen, device=dev) * scale_vec) for _ in range(L)]
    q = [torch.randn((1, T, nh, hd), generator=gen, device=dev) for _ in range(L)]
    idx = torch.arange(depth, depth + T, dtype=torch.int32, device=dev)
    mask_np = np.full((T, n_kv), 0xFC00, np.uint16)
    for i in range(T):
        mask_np[i, :depth + i + 1] = 0
    mask = torch.from_numpy(mask_np.view(np.float16)).to(dev)
    out = [torch.zeros((1, T, nh, hd), dtype=torch.float32, device=dev) for _ in range(L)]
    torch.cuda.synchronize()
    log(f"[bench] caches ready: {args.sets} sets x {L} layers x {n_kv} rows ({time.time() - t0:.1f}s)")

    qv = [K.q_view(x) for x in q]
    ov = [K.out_view(x) for x in out]
    mv = K.mask_view(mask)
    views = [[(K.cache_attn_view(kc, n_kv, nh_kv), K.cache_attn_view(vc, n_kv, nh_kv)) for kc, vc in st]
             for st in caches]
    ws_bytes = K.fattn_workspace_size(qv[0], views[0][0][0], views[0][0][1], mv)
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=dev)
    scale = 1.0 / 16.0

    def attn(s, l):
        kv, vv = views[s][l]
        K.flash_attn_ext(qv[l], kv, vv, mv, scale, ov[l], ws=ws)

    def step(s):
        for l in range(L):
            kc, vc = caches[s][l]
            if args.separate_append:
                K.set_rows_q8_0_kv(kc, newk[l], vc, newv[l], idx)   # the layer's K and V set_rows, one launch
                attn(s, l)
            else:                                                  # append + attention in one launch
                kv, vv = views[s][l]
                K.flash_attn_ext_append(qv[l], kv, vv, mv, scale, ov[l], newk[l], newv[l], n_kv - T, ws=ws)

    # algorithmic bytes: every cached K/V row read once, the appended rows
    # (F32 in, q8_0 out), Q and output, and the F16 mask.
    attn_bytes = n_kv * 2 * ROW + 2 * T * nh * hd * 4 + T * n_kv * 2
    append_bytes = 2 * T * (kv_dim * 4 + ROW)
    step_bytes = L * (attn_bytes + append_bytes)

    # ---- warmup (also allocates every lazily created resource) ----
    for w in range(max(1, args.warmup)):
        step(w % args.sets)
    torch.cuda.synchronize()
    log("[bench] warmup done")

    # quick parity check of one layer against the oracle (host side, small)
    parity = None
    try:
        import kvdata as KD
        kc, vc = caches[0][0]
        if args.separate_append:
            K.set_rows_q8_0_kv(kc, newk[0], vc, newv[0], idx)
            attn(0, 0)
        else:
            kv0, vv0 = views[0][0]
            K.flash_attn_ext_append(qv[0], kv0, vv0, mv, scale, ov[0], newk[0], newv[0], n_kv - T, ws=ws)
        torch.cuda.synchronize()
        got = out[0].cpu().numpy()[0]
        ref = KD.oracle_attn(q[0].cpu().numpy()[0], kc.cpu().numpy(), vc.cpu().numpy(), n_kv, nh_kv, mask_np,
                             scale, threads=min(16, len(os.sched_getaffinity(0))))
        parity = KD.err_stats(got, ref)
        log(f"[bench] parity vs oracle (layer 0): max abs {parity[0]:.2e} mean abs {parity[1]:.2e}")
    except Exception as e:  # the oracle only checks results; never part of the timed work
        log(f"[bench] parity check skipped: {e}")

    stream = torch.cuda.current_stream()

    # ---- eager timing ----
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for k in range(args.steps):
        step(k % args.sets)
    e1.record(stream)
    torch.cuda.synchronize()
    eager_ms = e0.elapsed_time(e1) / args.steps
    log(f"[bench] eager: {eager_ms * 1e3 / L:.2f} us/layer")

    # ---- attention op alone (roofline of the dominant kernel), eager, same stream ----
    torch.cuda.synchronize()
    e0.record(stream)
    n_att = 0
    for k in range(args.steps):
        for l in range(L):
            attn(k % args.sets, l)
            n_att += 1
    e1.record(stream)
    torch.cuda.synchronize()
    attn_us = e0.elapsed_time(e1) * 1e3 / n_att
    log(f"[bench] attention op: {attn_us:.2f} us/launch")

    # ---- HIP graph replay: one graph per cache set, 12 layers each ----
    graph_ms = None
    if not args.no_graph:
        graphs = []
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            for s in range(args.sets):
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=side):
                    step(s)
                graphs.append(g)
        stream.wait_stream(side)
        for s in range(args.sets):
            graphs[s].replay()
        torch.cuda.synchronize()
        e0.record(stream)
        for k in range(args.steps):
            graphs[k % args.sets].replay()
        e1.record(stream)
        torch.cuda.synchronize()
        graph_ms = e0.elapsed_time(e1) / args.steps
        log(f"[bench] graph: {graph_ms * 1e3 / L:.2f} us/layer")

    # ---- the attention op alone at a long context (the 64K decode/verify target) ----
    long_ctx = None
    if args.long_depth:
        ld = args.long_depth
        n_kv_l = ld + T
        n_sets_l = 8                                   # 8 x 71.8 MB = 574 MB: over twice the 256 MB Infinity Cache
        lcaches = []
        for s in range(n_sets_l):
            kc = torch.zeros((n_kv_l, ROW), dtype=torch.uint8, device=dev)
            vc = torch.zeros((n_kv_l, ROW), dtype=torch.uint8, device=dev)
            for c in (kc, vc):
                for r0 in range(0, n_kv_l, chunk):
                    n = min(chunk, n_kv_l - r0)
                    K.cpy_f32_q8_0(torch.randn((n, kv_dim), generator=gen, device=dev) * scale_vec, c, r0)
            lcaches.append((K.cache_attn_view(kc, n_kv_l, nh_kv), K.cache_attn_view(vc, n_kv_l, nh_kv), kc, vc))
        lmask_np = np.full((T, n_kv_l), 0xFC00, np.uint16)
        for i in range(T):
            lmask_np[i, :ld + i + 1] = 0
        lmask = torch.from_numpy(lmask_np.view(np.float16)).to(dev)
        lmv = K.mask_view(lmask)
        lws_bytes = K.fattn_workspace_size(qv[0], lcaches[0][0], lcaches[0][1], lmv)
        lws = torch.empty(max(lws_bytes, 256), dtype=torch.uint8, device=dev)
        for s in range(n_sets_l):
            K.flash_attn_ext(qv[0], lcaches[s][0], lcaches[s][1], lmv, scale, ov[0], ws=lws)
        torch.cuda.synchronize()
        reps = max(40, args.steps)
        e0.record(stream)
        for k in range(reps):
            s = k % n_sets_l
            K.flash_attn_ext(qv[0], lcaches[s][0], lcaches[s][1], lmv, scale, ov[0], ws=lws)
        e1.record(stream)
        torch.cuda.synchronize()
        l_us = e0.elapsed_time(e1) * 1e3 / reps
        l_bytes = n_kv_l * 2 * ROW + 2 * T * nh * hd * 4 + T * n_kv_l * 2
        long_ctx = {"depth": ld, "T": T, "us_per_launch": round(l_us, 3), "bytes_per_launch": l_bytes,
                    "GBs": round(l_bytes / (l_us * 1e-6) / 1e9, 1),
                    "frac": round(l_bytes / (l_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        log(f"[bench] attention op at depth {ld}: {l_us:.2f} us/launch, {long_ctx['GBs']} GB/s")
        del lcaches, lws
        torch.cuda.empty_cache()

    rows = None
    if not args.no_rows:
        rows = measure_rows(K, torch, np, dev, gen)
        log(f"[bench] rows: {json.dumps(rows)}")

    if args.calib_copy_mb:
        n = args.calib_copy_mb << 20
        a = torch.empty(n, dtype=torch.uint8, device=dev)
        b = torch.empty(n, dtype=torch.uint8, device=dev)
        K.state_restore([a.data_ptr()], [n], [b.data_ptr()], 1, K.SRC_DEVICE)
        torch.cuda.synchronize()
        log(f"[bench] calibration copy of {args.calib_copy_mb} MiB done")

    # ---- CPU baseline: the oracle (ggml-cpu flash_attn_ext semantics, restated in C) on
    #      one layer; 2 warm-ups, then the median of >= 10 timed reps ----
    cpu = None
    if not args.no_cpu:
        try:
            import statistics

            import kvdata as KD
            # every core the job may use: the affinity set, capped at the 16 cores that
            # are one GPU's share of the host
            affinity = len(os.sched_getaffinity(0))
            cores = min(16, affinity)
            kc, vc = caches[0][0]
            kc_h, vc_h = kc.cpu().numpy(), vc.cpu().numpy()
            q_h = q[0].cpu().numpy()[0]

            def one():
                t1 = time.perf_counter()
                KD.oracle_attn(q_h, kc_h, vc_h, n_kv, nh_kv, mask_np, scale, threads=cores, native=True)
                return time.perf_counter() - t1
            # the native build computes what the portable build does, bit for bit
            chk = KD.oracle_attn(q_h, kc_h, vc_h, n_kv, nh_kv, mask_np, scale, threads=cores)
            nat = KD.oracle_attn(q_h, kc_h, vc_h, n_kv, nh_kv, mask_np, scale, threads=cores, native=True)
            if not np.array_equal(chk, nat):
                raise RuntimeError("the -march=native oracle build differs from the portable build")
            one(), one()
            times = []
            while len(times) < 10 or (sum(times) < args.cpu_seconds and len(times) < 200):
                times.append(one())
            med = statistics.median(times)
            cpu = {"value": round(attn_bytes / med / 1e9, 3), "unit": "GB/s", "cores": cores,
                   "affinity_cores": affinity, "kind": "port", "cpu_model": cpu_model(),
                   "build": "gcc -O3 -march=native -ffp-contract=off (oracle/Makefile liboracle_native.so)",
                   "sample": f"one layer's verify attention (T={T}, {n_kv} q8_0 rows, 2 KV heads) in the scalar C "
                             f"restatement of ggml-cpu flash_attn_ext, built -O3 -march=native for this host, on "
                             f"{cores} threads: median of {len(times)} reps after 2 warm-ups, {med * 1e6:.0f} "
                             f"us/layer (min {min(times) * 1e6:.0f})",
                   "us_per_layer": round(med * 1e6, 1)}
            log(f"[bench] cpu baseline: {cpu}")
        except Exception as e:
            log(f"[bench] cpu baseline skipped: {e}")

    # HBM traffic per launch of the attention kernel, measured by the two
    # rocprofv3 --pmc passes summarised under profiles/ (FETCH_SIZE, WRITE_SIZE,
    # each scaled by what the counter reads for a plain copy of known size)
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "fa_dec.verify_16k.traffic.json")
    if os.path.exists(tpath):
        tj = json.load(open(tpath))
        w = tj.get("workload", {})
        if w.get("depth") == depth and w.get("T") == T:
            traffic = tj["traffic_bytes"]

    best_ms = min(graph_ms, eager_ms) if graph_ms is not None else eager_ms
    value = step_bytes / (best_ms * 1e-3) / 1e9
    achieved = attn_bytes / (attn_us * 1e-6) / 1e9
    res = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(best_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0 K/V (int8 + fp16 scales), f32 softmax/accumulation",
        "data": "synthetic (seeded N(0,1) K/V with 4 x8 outlier channels per KV head, N(0,1) Q)",
        "config": {"workload": f"MTP verify decode: {L} layers, depth {depth}, T={T} (1+{T - 1} drafts, causal), "
                               f"n_head {nh}, n_head_kv {nh_kv}, head 256, q8_0 KV, append {T} rows/layer",
                   "layers": L, "depth": depth, "T": T, "cache_sets": args.sets,
                   "append": "own launch" if args.separate_append else "fused into the attention launch"},
        "us_per_layer": round(best_ms * 1e3 / L, 3),
        "us_per_layer_eager": round(eager_ms * 1e3 / L, 3),
        "us_per_layer_graph": round(graph_ms * 1e3 / L, 3) if graph_ms is not None else None,
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "flash_attn_ext q8_0 verify op: k_fa_dec (the key loop) + k_fattn_merge (split merge)",
                     "us_per_launch": round(attn_us, 3), "bytes_per_launch": attn_bytes},
        "cpu_baseline": cpu,
        "long_context": long_ctx,
        "rows": rows,
        "parity_max_abs": parity[0] if parity else None,
    }
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
