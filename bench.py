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
    ap.add_argument("--long-depth", type=int, default=65536,
                    help="also time the attention op alone at this depth (0: skip)")
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="also run one device copy of this many MiB (counter calibration)")
    return ap.parse_args()


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this path has no multi-GPU form to run (asked for --gpus {args.gpus}); "
              "see DESIGN.md for how it would shard.", file=sys.stderr)
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
            K.set_rows_q8_0(kc, newk[l], idx)
            K.set_rows_q8_0(vc, newv[l], idx)
            attn(s, l)

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
        K.set_rows_q8_0(kc, newk[0], idx)
        K.set_rows_q8_0(vc, newv[0], idx)
        attn(0, 0)
        torch.cuda.synchronize()
        got = out[0].cpu().numpy()[0]
        ref = KD.oracle_attn(q[0].cpu().numpy()[0], kc.cpu().numpy(), vc.cpu().numpy(), n_kv, nh_kv, mask_np,
                             scale, threads=min(16, len(os.sched_getaffinity(0))))
        parity = KD.err_stats(got, ref)
        log(f"[bench] parity vs oracle (layer 0): max abs {parity[0]:.2e} mean abs {parity[1]:.2e}")
    except Exception as e:  # the oracle is a checker; never part of the timed work
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
        n_sets_l = 4                                   # 4 x 71 MB: more than the Infinity Cache holds
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

    if args.calib_copy_mb:
        n = args.calib_copy_mb << 20
        a = torch.empty(n, dtype=torch.uint8, device=dev)
        b = torch.empty(n, dtype=torch.uint8, device=dev)
        K.state_restore([a.data_ptr()], [n], [b.data_ptr()], 1, K.SRC_DEVICE)
        torch.cuda.synchronize()
        log(f"[bench] calibration copy of {args.calib_copy_mb} MiB done")

    # ---- CPU baseline: the oracle (ggml-cpu flash_attn_ext semantics) on one layer ----
    cpu = None
    if not args.no_cpu:
        try:
            import kvdata as KD
            cores = min(16, len(os.sched_getaffinity(0)))
            kc, vc = caches[0][0]
            kc_h, vc_h = kc.cpu().numpy(), vc.cpu().numpy()
            q_h = q[0].cpu().numpy()[0]
            reps, t_cpu = 0, 0.0
            while t_cpu < args.cpu_seconds and reps < 1000:
                t1 = time.perf_counter()
                KD.oracle_attn(q_h, kc_h, vc_h, n_kv, nh_kv, mask_np, scale, threads=cores)
                t_cpu += time.perf_counter() - t1
                reps += 1
            cpu = {"value": round(attn_bytes * reps / t_cpu / 1e9, 3), "unit": "GB/s", "cores": cores,
                   "kind": "port",
                   "sample": f"{reps} x one layer's verify attention (T={T}, {n_kv} q8_0 rows, 2 KV heads) "
                             f"in the C oracle of ggml-cpu flash_attn_ext, {t_cpu:.1f}s, "
                             f"{t_cpu / reps * 1e6:.0f} us/layer"}
            log(f"[bench] cpu baseline: {cpu}")
        except Exception as e:
            log(f"[bench] cpu baseline skipped: {e}")

    # HBM traffic per launch of the attention kernel, measured by the two
    # rocprofv3 --pmc passes summarised under profiles/ (FETCH_SIZE, WRITE_SIZE,
    # each scaled by what the counter reads for a plain copy of known size)
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "fattn_q8_0.mtp_verify_16k.traffic.json")
    if os.path.exists(tpath):
        tj = json.load(open(tpath))
        w = tj.get("workload", {})
        if w.get("depth") == depth and w.get("T") == T:
            traffic = tj["traffic_bytes"]

    best_ms = graph_ms if graph_ms is not None else eager_ms
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
                   "layers": L, "depth": depth, "T": T, "cache_sets": args.sets},
        "us_per_layer": round(best_ms * 1e3 / L, 3),
        "us_per_layer_eager": round(eager_ms * 1e3 / L, 3),
        "us_per_layer_graph": round(graph_ms * 1e3 / L, 3) if graph_ms is not None else None,
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "flash_attn_ext q8_0 (k_fattn_q8_0 + k_fattn_merge)",
                     "us_per_launch": round(attn_us, 3), "bytes_per_launch": attn_bytes},
        "cpu_baseline": cpu,
        "long_context": long_ctx,
        "parity_max_abs": parity[0] if parity else None,
    }
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
