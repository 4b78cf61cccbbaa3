"""Runs one op of the library at a fixed workload, for profilers (rocprofv3
--kernel-trace / --pmc): the op is launched `--reps` times on synthetic inputs
after one warm-up; nothing else runs on the GPU besides the input set-up.

  python3 qwfn-hybrid_amd/profile_ops.py verify --depth 16384 --T 3
  python3 qwfn-hybrid_amd/profile_ops.py prefill --depth 16384
  python3 qwfn-hybrid_amd/profile_ops.py cells | append | gather [--pair] | restore | produce | deltanet | pool
  python3 qwfn-hybrid_amd/profile_ops.py qsaprefill --depth 16384  (QSA-on prefill chunk over cell lists)
  python3 qwfn-hybrid_amd/profile_ops.py qsastep  (QSA-on 3-position verify step of one layer at 73700)
  python3 qwfn-hybrid_amd/profile_ops.py copy --mb 1024        (a plain device copy: counter calibration)

Cache sets are rotated (--sets) so that a repeated launch does not find its
K/V rows in the 256 MB Infinity Cache.
"""
from __future__ import annotations

import argparse
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

ROW = 544


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("op", choices=["verify", "prefill", "cells", "append", "gather", "restore", "produce", "deltanet",
                                   "pool", "select", "qsaprefill", "qsastep", "copy"])
    ap.add_argument("--depth", type=int, default=16384)
    ap.add_argument("--T", type=int, default=3)
    ap.add_argument("--reps", type=int, default=10)
    ap.add_argument("--sets", type=int, default=8)
    ap.add_argument("--mb", type=int, default=1024)
    ap.add_argument("--lib", default=None, help="library path (default: the package's build)")
    ap.add_argument("--append", action="store_true", help="verify: append the T new K/V rows in the same launch")
    ap.add_argument("--pair", action="store_true", help="gather: the K and the V cache with one index in one launch")
    ap.add_argument("--kernel", choices=["auto", "vd", "vs", "dec", "general"], default="auto",
                    help="attention ops: the kernel family to force (qwfn_fattn_force_kernel)")
    ap.add_argument("--splits", type=int, default=0, help="attention ops: a forced key-split count (0: the planner's)")
    ap.add_argument("--merge", choices=["auto", "fused", "kernel"], default="auto",
                    help="attention ops: merge the key splits inside the kernel or with a merge launch")
    a = ap.parse_args()
    import numpy as np
    import torch

    import qwfn_kv as K
    K.check((K.load(a.lib) if a.lib else K.load()).qwfn_init(0))
    K.load().qwfn_fattn_force_kernel({"auto": K.FA_KERNEL_AUTO, "vd": K.FA_KERNEL_VD, "dec": K.FA_KERNEL_DEC,
                                      "general": K.FA_KERNEL_GENERAL, "vs": K.FA_KERNEL_VS}[a.kernel])
    K.load().qwfn_fattn_force_splits(a.splits)
    K.load().qwfn_fattn_force_merge({"auto": K.FA_MERGE_AUTO, "fused": K.FA_MERGE_FUSED,
                                     "kernel": K.FA_MERGE_KERNEL}[a.merge])
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)

    def cache(n):
        c = torch.randint(-100, 100, (n, ROW), dtype=torch.int8, device=dev, generator=gen).view(torch.uint8)
        c.view(-1, 34)[:, 0] = 0x1F                 # valid fp16 scales (0x211F ~ 0.0101)
        c.view(-1, 34)[:, 1] = 0x21
        return c

    nh, hd = 16, 256
    if a.op in ("verify", "prefill"):
        T = a.T if a.op == "verify" else 512
        n_kv = a.depth + T
        sets = [(cache(n_kv), cache(n_kv)) for _ in range(a.sets)]
        m = np.full((T, n_kv), 0xFC00, np.uint16)
        for i in range(T):
            m[i, :a.depth + i + 1] = 0
        mask = torch.from_numpy(m.view(np.float16)).to(dev)
        q = torch.randn((1, T, nh, hd), generator=gen, device=dev)
        out = torch.zeros((1, T, nh, hd), dtype=torch.float32, device=dev)
        views = [(K.cache_attn_view(k, n_kv, 2), K.cache_attn_view(v, n_kv, 2)) for k, v in sets]
        ws = torch.empty(max(256, K.fattn_workspace_size(K.q_view(q), views[0][0], views[0][1], K.mask_view(mask))),
                         dtype=torch.uint8, device=dev)
        run = lambda i: K.flash_attn_ext(K.q_view(q), views[i % a.sets][0], views[i % a.sets][1], K.mask_view(mask),
                                         1 / 16, K.out_view(out), ws=ws)
        if a.append and a.op == "verify":
            newk = torch.randn((T, 512), generator=gen, device=dev)
            newv = torch.randn((T, 512), generator=gen, device=dev)
            run = lambda i: K.flash_attn_ext_append(K.q_view(q), views[i % a.sets][0], views[i % a.sets][1],
                                                    K.mask_view(mask), 1 / 16, K.out_view(out), newk, newv, a.depth, ws=ws)
    elif a.op == "cells":
        n_ctx = 65536
        sets = [(cache(n_ctx), cache(n_ctx)) for _ in range(a.sets)]
        rng = np.random.default_rng(4)
        lists = []
        for h in range(2):
            top = np.argsort(-rng.random(1024), kind="stable")[:128]
            lists.append(np.unique(np.concatenate([(top[:, None] * 64 + np.arange(64)).ravel(),
                                                   np.arange(n_ctx - 512, n_ctx)])))
        stride = (max(len(x) for x in lists) + 3) // 4 * 4
        c = np.zeros((2, stride), np.int32)
        for h, x in enumerate(lists):
            c[h, :len(x)] = x
        cells = torch.from_numpy(c).to(dev)
        n = [len(x) for x in lists]
        q = torch.randn((1, 3, nh, hd), generator=gen, device=dev)
        out = torch.zeros((1, 3, nh, hd), dtype=torch.float32, device=dev)
        views = [(K.tensor(k.data_ptr(), K.TYPE_Q8_0, (hd, n_ctx, 2, 1), (34, ROW, 272, n_ctx * ROW)),
                  K.tensor(v.data_ptr(), K.TYPE_Q8_0, (hd, n_ctx, 2, 1), (34, ROW, 272, n_ctx * ROW))) for k, v in sets]
        run = lambda i: K.flash_attn_ext_cells(K.q_view(q), views[i % a.sets][0], views[i % a.sets][1], cells, n,
                                               n_ctx - 3, 1 / 16, K.out_view(out))
    elif a.op == "append":
        T = 512
        caches = [torch.zeros((a.depth + T, ROW), dtype=torch.uint8, device=dev) for _ in range(2 * a.sets)]
        src = [torch.randn((T, 512), generator=gen, device=dev) for _ in range(2)]
        run = lambda i: K.cpy_f32_q8_0_kv(src[0], caches[(2 * i) % (2 * a.sets)], src[1],
                                          caches[(2 * i + 1) % (2 * a.sets)], a.depth)
    elif a.op == "gather":
        n_ctx = 65536
        sets = [(cache(n_ctx), cache(n_ctx)) for _ in range(a.sets)]
        rng = np.random.default_rng(4)
        lists = []
        for h in range(2):
            top = np.argsort(-rng.random(1024), kind="stable")[:128]
            lists.append(np.unique(np.concatenate([(top[:, None] * 64 + np.arange(64)).ravel(),
                                                   np.arange(n_ctx - 512, n_ctx)])))
        mlen = max(len(x) for x in lists)
        idx = torch.from_numpy(np.stack([np.concatenate([x, np.repeat(x[-1:], mlen - len(x))]) for x in lists])
                               .astype(np.int32)).to(dev)
        gk = torch.zeros((2, mlen, 272), dtype=torch.uint8, device=dev)
        gv = torch.zeros((2, mlen, 272), dtype=torch.uint8, device=dev)
        if a.pair:
            run = lambda i: K.gather_segments_kv(sets[i % a.sets][0], sets[i % a.sets][1], idx, gk, gv, 0, 272, 272)
        else:
            run = lambda i: K.gather_segments(sets[i % a.sets][i % 2], idx, gk, 0, 272, 272)
    elif a.op in ("restore", "copy"):
        if a.op == "copy":
            nbytes = [a.mb << 20]
            n_slots = 1
        else:
            nbytes = [8192 * ROW] * 24 + [32 * 128 * 128 * 4] * 36
            n_slots = 4
        src = [torch.randint(0, 256, (b,), dtype=torch.uint8, device=dev, generator=gen) for b in nbytes]
        dst = [torch.empty((n_slots, b), dtype=torch.uint8, device=dev) for b in nbytes]
        ptrs = []
        for s in range(n_slots):
            ptrs += [d[s].data_ptr() for d in dst]
        sp = [x.data_ptr() for x in src]
        run = lambda i: K.state_restore(sp, nbytes, ptrs, n_slots, K.SRC_DEVICE)
    elif a.op == "produce":
        E, kv_dim, T = 2560, 512, a.T
        wk = (torch.randn((kv_dim, E), generator=gen, device=dev) * 0.02).to(torch.float16)
        wv = (torch.randn((kv_dim, E), generator=gen, device=dev) * 0.02).to(torch.float16)
        hid = torch.randn((T, E), generator=gen, device=dev)
        pos = torch.arange(a.depth, a.depth + T, dtype=torch.int32, device=dev).repeat(4)
        kc, vc = cache(a.depth + T), cache(a.depth + T)
        knw = torch.rand(256, generator=gen, device=dev) + 0.5
        run = lambda i: K.kv_produce(hid, wk, wv, knw, pos, kc, vc, a.depth)
    elif a.op == "deltanet":
        T = a.T
        conv = torch.randn((T, 10240), generator=gen, device=dev)
        conv[:, :4096] = torch.nn.functional.normalize(conv[:, :4096].view(T, 32, 128), dim=-1).view(T, 4096)
        g = -torch.rand((T, 48), generator=gen, device=dev)
        beta = torch.rand((T, 48), generator=gen, device=dev)
        states = [torch.randn((48, 128, 128), generator=gen, device=dev) * 0.05 for _ in range(a.sets)]
        out = torch.empty((T, 48, 128), dtype=torch.float32, device=dev)
        n_snap = max(0, min(2, T - 1))
        snap = torch.empty((max(1, n_snap), 48, 128, 128), dtype=torch.float32, device=dev)
        run = lambda i: K.gated_delta_net(conv[:, :2048], conv[:, 2048:4096], conv[:, 4096:], g, beta,
                                          states[i % a.sets], out, 16, snap if n_snap else None, n_snap)
    elif a.op == "select":
        # the decode step's block selection for a 3-position verify step at 73728
        # positions: 18432 pooled f16 keys, 4 indexer heads, top 513 blocks of 4 cells
        import qwfn_state as S
        nb, kb = 73728 // 4, 513
        pool = (torch.randn((nb, 128), generator=gen, device=dev) * 0.5).to(torch.float16)
        qsel = torch.randn((3, 4, 128), generator=gen, device=dev)
        bsel = torch.zeros((3, nb), dtype=torch.float32, device=dev)
        bcells = torch.arange(nb * 4, dtype=torch.int32, device=dev)
        csel = torch.empty((3, kb * 4), dtype=torch.int32, device=dev)
        wsel = torch.empty(K.load().qwfn_qsa_select_workspace_size(nb, 3), dtype=torch.uint8, device=dev)
        run = lambda i: S.qsa_select_cells(pool, qsel, bsel, kb, bcells, 4, csel, ws=wsel)
    elif a.op == "qsaprefill":
        # the reference's default prefill (QSA on) for a 512-query chunk at `depth`:
        # chunk tables and bias, the pool rebuild, top-513 selection of blocks of 4,
        # each query's visible cells, and the attention over those lists (k_fa_qc)
        import qwfn_state as S
        T, ratio, kb = 512, 4, 513
        n_kv = a.depth + T
        nb = n_kv // ratio
        sets = [(cache(n_kv), cache(n_kv)) for _ in range(a.sets)]
        ic = torch.randn((n_kv, 128), generator=gen, device=dev).to(torch.float16)
        knw = torch.rand(128, generator=gen, device=dev) + 0.5
        q_idx = torch.randn((T, 4, 128), generator=gen, device=dev)
        bc = torch.empty(nb * ratio, dtype=torch.int32, device=dev)
        bp = torch.empty(4 * nb, dtype=torch.int32, device=dev)
        bias = torch.empty((T, nb), dtype=torch.float32, device=dev)
        pool = torch.empty((nb, 128), dtype=torch.float16, device=dev)
        cells = torch.empty((T, kb * ratio), dtype=torch.int32, device=dev)
        lists = torch.empty((T, kb * ratio), dtype=torch.int32, device=dev)
        counts = torch.empty((T,), dtype=torch.int32, device=dev)
        wsel = torch.empty(K.load().qwfn_qsa_select_workspace_size(nb, T), dtype=torch.uint8, device=dev)
        q = torch.randn((1, T, nh, hd), generator=gen, device=dev)
        out = torch.zeros((1, T, nh, hd), dtype=torch.float32, device=dev)
        views = [(K.cache_attn_view(k, n_kv, 2), K.cache_attn_view(v, n_kv, 2)) for k, v in sets]

        def run(i):
            S.qsa_chunk_inputs(a.depth, T, ratio, None, bc, bp, bias)
            K.qsa_pool_rebuild(ic, n_kv, ratio, knw, pool)
            S.qsa_select_cells(pool, q_idx, bias, kb, bc, ratio, cells, ws=wsel)
            S.qsa_visible_cells(cells, n_kv, a.depth, lists, counts)
            K.flash_attn_ext_query_cells_dev(K.q_view(q), views[i % a.sets][0], views[i % a.sets][1], lists, counts,
                                             a.depth, 1 / 16, K.out_view(out))
    elif a.op == "qsastep":
        # the reference's default verify step (QSA on) for one attention layer: the 3
        # positions' inputs and index pooling (one launch), top-513 selection of 18432
        # blocks for the 3 queries, the K/V producer, the gated per-position cells
        # attention over 3 lists of 2052 and its merge
        import qwfn_state as S
        n_ctx, ratio, nbm, T, kb, E, nh = 73728, 4, 18432, 3, 513, 2560, 24
        n_past, nc = 73700, kb * 4
        sets = [(cache(n_ctx), cache(n_ctx)) for _ in range(a.sets)]
        views = [(K.cache_attn_view(k, n_ctx, 2), K.cache_attn_view(v, n_ctx, 2)) for k, v in sets]
        ic = torch.randn((n_ctx, 128), generator=gen, device=dev).to(torch.float16)
        pool = (torch.randn((nbm, 128), generator=gen, device=dev) * 0.5).to(torch.float16)
        wk = (torch.randn((512, E), generator=gen, device=dev) * 0.02).to(torch.float16)
        wv = (torch.randn((512, E), generator=gen, device=dev) * 0.02).to(torch.float16)
        knw = torch.rand(256, generator=gen, device=dev) + 0.5
        knw_idx = torch.rand(128, generator=gen, device=dev) + 0.5
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
        aws = torch.empty(max(256, K.fattn_workspace_size_query_cells(K.q_view(q), views[0][0], views[0][1], [nc] * T, nc)),
                          dtype=torch.uint8, device=dev)

        def run(i):
            kc, vc = sets[i % a.sets]
            S.qsa_decode_prepare_pool_steps(qds, n_past, ic, k_raw, knw_idx, pool)
            S.qsa_select_cells(pool, q_idx, bias, kb, blk_cells, ratio, cells, ws=wsel)
            K.kv_produce(cur, wk, wv, knw, pos, kc, vc, n_past)
            K.flash_attn_ext_query_cells(K.q_view(q), views[i % a.sets][0], views[i % a.sets][1], cells, [nc] * T, n_past,
                                         1 / 16, K.out_view(out), gate=gate, ws=aws)
    else:  # pool: rebuild after a prefill of `depth` positions, ratio 4
        ic = torch.randn((a.depth + 64, 128), generator=gen, device=dev).to(torch.float16)
        pool = torch.zeros((a.depth // 4 + 16, 128), dtype=torch.float16, device=dev)
        knw = torch.rand(128, generator=gen, device=dev) + 0.5
        run = lambda i: K.qsa_pool_rebuild(ic, a.depth, 4, knw, pool)
    run(0)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(a.reps):
        run(i + 1)
    e1.record()
    torch.cuda.synchronize()
    kname = K.last_kernel() if a.op in ("verify", "prefill", "cells") else ""
    if kname:
        kname += {K.FA_MERGE_FUSED: " + fused merge", K.FA_MERGE_KERNEL: " + k_fattn_merge"}.get(K.last_merge(), "")
    print(f"{a.op}: {a.reps} launches done, {e0.elapsed_time(e1) * 1e3 / a.reps:.2f} us per launch (event time) {kname}",
          flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
