"""The reference's default verify step with QSA on, composed on the device and
checked against the oracle's position-by-position chain.

engine::attn_decode (qwfn_engine.cpp:2259-2280) runs T = 3 chained
sparse_attn_decode calls (qwfn_graph.cpp:653-705); call k
  - prepares position n_past + k (qsa_decode_prepare, then
    qsa_decode_prepare_k for k > 0: the bias window, write row, block members),
  - writes its raw index key and re-pools its block (qsa_dec_index, :529-554),
  - scores the 18432 pooled blocks of the bucket with its indexer query and
    keeps the top 513 (qsa_dec_cells, :556-581): 2052 cells,
  - writes its K/V row (qsa_dec_kv_write; the projections come from the
    step's one producer call, :441-451),
  - attends its cells masked to positions at most its own, times
    sigmoid(gate) (:662-701).
The device runs the same chain batched the way the library offers it:
prepare x3, pool decode x3 (or each in one launch for the three positions:
qwfn_qsa_decode_prepare_steps, qwfn_qsa_pool_decode_steps; or both in one
launch: qwfn_qsa_decode_prepare_pool_steps), ONE selection
over the three queries, ONE K/V producer call for the three rows, ONE
attention launch over the three lists (qwfn_flash_attn_ext_q8_0_query_cells)
with the gate. The oracle runs the
chain position by position, so the test also shows that batching the pool
writes ahead of the selection changes nothing: a later position only touches
its own block, which an earlier query either keeps by the 1e9 bias of its
incomplete block or cannot see (-inf past its position).

Checks, each against the oracle: the bias and position inputs (exact); the
index cache rows (exact F16 set_rows); the re-pooled block keys (F16 bits,
one unit in the last place allowed at 0.1% of values: libm cos/sin against
the device's); the selected blocks (the same set, best first, up to float
ties at the k-th place); the K/V rows (q8_0 bytes, quants one step off only
at rounding boundaries, as the producer test allows); the gated attention
output of each position (2e-3 max / 1e-3 mean abs, 1e-4 max as observed),
computed by the oracle over the device's cache and cell lists."""
import numpy as np
import pytest
import torch

import kvdata as KD
import qwfn_kv as KK
import qwfn_state as S
from gpu_util import dev, host, say
from oracle import oracle as O
from oracle import state_oracle as SO
from test_gpu_kv_produce import _compare_rows, _weights

pytestmark = pytest.mark.gpu
RATIO, NB_MAX, N_CTX = 4, 18432, 73728
T, NH, NH_KV, HD, IDX, IDX_H = 3, 24, 2, 256, 128, 4
K_BLOCKS = 513                      # idx_top_k / ratio + 1 (qwfn_engine.cpp:687)
E = 2560


def _ulp_ok(got_bits, ref_bits):
    d = np.abs(got_bits.astype(np.int32) - ref_bits.astype(np.int32))
    assert d.max() <= 1
    assert int((d != 0).sum()) <= max(1, d.size // 1000)


@pytest.mark.parametrize("n_past,batched", [(73700, ""), (73702, ""), (73700, "steps"), (73702, "steps"),
                                            (73700, "fused"), (73703, "fused")])
def test_qsa_verify_step_composed(gpu, oracle, n_past, batched):
    K = gpu
    rng = np.random.default_rng(n_past)
    # ---- the layer's state after a prefill to n_past
    ic = np.zeros((N_CTX, IDX), np.float16)
    ic[:n_past] = rng.standard_normal((n_past, IDX)).astype(np.float16)
    knw_idx = rng.uniform(0.6, 1.4, IDX).astype(np.float32)
    kc = KD.make_cache(KD.kv_rows(n_past, 0, KD.K_KIND, n_past, outliers=True), N_CTX)
    vc = KD.make_cache(KD.kv_rows(n_past, 0, KD.V_KIND, n_past, outliers=True), N_CTX)
    wk, wv, knw = _weights(7)
    # ---- the step's inputs: hidden rows, indexer keys and queries, attention queries, gate
    cur = KD.normal(70, 0, KD.Q_KIND, T * E).reshape(T, E)
    k_raw = rng.standard_normal((T, IDX)).astype(np.float32)
    q_idx = rng.standard_normal((T, IDX_H, IDX)).astype(np.float32)
    q = KD.q_rows(71, 0, T, NH)[0]
    gate = (rng.standard_normal((T, NH, HD)) * 3).astype(np.float32)
    pos = np.tile(np.arange(n_past, n_past + T, dtype=np.int32), 4)

    # ---- device
    ic_d, kd, vd = dev(ic), dev(kc), dev(vc)
    pool = torch.zeros((NB_MAX, IDX), dtype=torch.float16, device="cuda")
    blk_cells = torch.empty(NB_MAX * RATIO, dtype=torch.int32, device="cuda")
    S.qsa_tables(blk_cells, RATIO)
    knw_idx_d = dev(knw_idx)
    say(f"pool rebuild at n_past={n_past}")
    K.qsa_pool_rebuild(ic_d, n_past, RATIO, knw_idx_d, pool)
    bias = torch.empty((T, NB_MAX), dtype=torch.float32, device="cuda")
    qds = []
    for k in range(T):
        qd = S.QsaDecodeInputs(RATIO, NB_MAX)
        qd.bias = bias[k]
        qds.append(qd)
    qds[0].rebuild_bias(n_past)
    pool0 = host(pool).view(np.uint16).copy()     # the oracle chain starts from the device's rebuilt pool
    if batched == "fused":
        say("prepare and pool decode steps, one launch")
        S.qsa_decode_prepare_pool_steps(qds, n_past, ic_d, dev(k_raw), knw_idx_d, pool)
    elif batched:
        say("prepare steps, pool decode steps (one launch each)")
        S.qsa_decode_prepare_steps(qds, n_past)
        K.qsa_pool_decode_steps(ic_d, dev(k_raw), qds, knw_idx_d, pool)
    else:
        say("prepare / prepare_k, pool decode x3")
        for k in range(T):
            qds[k].prepare(n_past + k, prev=qds[k - 1] if k else None)
            K.qsa_pool_decode(ic_d, dev(k_raw[k]), qds[k].write_idx, qds[k].member_idx, RATIO, qds[k].blk_pos,
                              qds[k].blk_idx, knw_idx_d, pool)
    nb = qds[-1].n_bucket
    assert nb == NB_MAX
    cells = torch.full((T, K_BLOCKS * RATIO), -1, dtype=torch.int32, device="cuda")
    top = torch.full((T, K_BLOCKS), -1, dtype=torch.int32, device="cuda")
    say(f"select {K_BLOCKS} of {nb} blocks for {T} queries")
    S.qsa_select_cells(pool[:nb], dev(q_idx), bias, K_BLOCKS, blk_cells, RATIO, cells, top)
    say("K/V produce")
    K.kv_produce(dev(cur), dev(wk), dev(wv), dev(knw), dev(pos), kd, vd, n_past)
    say("attention over the three lists, gated")
    qv = dev(q[None].astype(np.float32))
    out = torch.full((1, T, NH, HD), float("nan"), dtype=torch.float32, device="cuda")
    rb = kc.shape[1]
    kv = K.tensor(kd.data_ptr(), K.TYPE_Q8_0, (HD, N_CTX, NH_KV, 1), (34, rb, 272, N_CTX * rb))
    vv = K.tensor(vd.data_ptr(), K.TYPE_Q8_0, (HD, N_CTX, NH_KV, 1), (34, rb, 272, N_CTX * rb))
    K.flash_attn_ext_query_cells(K.q_view(qv), kv, vv, cells, [K_BLOCKS * RATIO] * T, n_past, 1 / 16,
                                 K.out_view(out), gate=dev(gate[None]))
    assert K.device_status() == 0
    g_bias, g_ic, g_pool = host(bias), host(ic_d).view(np.uint16), host(pool).view(np.uint16)
    g_cells, g_top, g_k, g_v, g_out = host(cells), host(top), host(kd), host(vd), host(out)[0]

    # ---- oracle, position by position
    r_bias = SO.qsa_pool_rebuild_bias(NB_MAX, n_past, RATIO)
    r_ic = ic.view(np.uint16).copy()
    r_pool = pool0.copy()
    blk_cells_h = SO.qsa_tables(NB_MAX, RATIO, 1, 0)[0]
    k_rows, v_rows, k_f, v_f = O.kv_produce(cur, wk.view(np.uint16), wv.view(np.uint16), knw, pos, O.Q8_X86)
    for k in range(T):
        p = n_past + k
        o = SO.qsa_decode_prepare(r_bias, p, RATIO) if k == 0 else SO.qsa_decode_prepare_k(r_bias, p, RATIO)
        r_bias = o["bias"]
        for f in ("write_idx", "member_idx", "blk_pos", "blk_idx", "npast_f"):
            np.testing.assert_array_equal(host(getattr(qds[k], f)), o[f], err_msg=f"{f} at position {k}")
        np.testing.assert_array_equal(g_bias[k], r_bias, err_msg=f"bias at position {k}")
        O.set_rows_f16(r_ic, k_raw[k][None], o["write_idx"])
        b = p // RATIO
        r_pool[b] = O.qsa_pool_blocks(r_ic, o["member_idx"], RATIO, knw_idx, o["blk_pos"][None])[0]
        # this query's selection over the pool as it stands after its own write
        sc = SO.qsa_scores(r_pool[:nb].view(np.float16), q_idx[k], r_bias[:nb])
        want = SO.qsa_top_k(sc, K_BLOCKS)
        kth = sc[want[-1]]
        tol = 1e-5 * max(1.0, abs(kth))
        got = g_top[k]
        assert len(set(got.tolist())) == K_BLOCKS
        assert {int(x) for x in want if sc[x] > kth + tol} <= {int(x) for x in got}
        assert all(sc[x] >= kth - tol for x in got)
        if r_bias[b] == 1e9:
            assert got[0] == b                                 # the incomplete block of the query's own position
        np.testing.assert_array_equal(g_cells[k], SO.qsa_cells(got, blk_cells_h, RATIO))
    np.testing.assert_array_equal(g_ic, r_ic)
    touched = sorted({(n_past + k) // RATIO for k in range(T)})
    _ulp_ok(g_pool[touched], r_pool[touched])
    np.testing.assert_array_equal(np.delete(g_pool, touched, axis=0), np.delete(pool0, touched, axis=0))
    rows = np.arange(n_past, n_past + T)
    _compare_rows(g_k[rows], k_rows, k_f)
    _compare_rows(g_v[rows], v_rows, v_f)
    np.testing.assert_array_equal(np.delete(g_k, rows, axis=0), np.delete(kc, rows, axis=0))
    sig = (1.0 / (1.0 + np.exp(-gate.astype(np.float64)))).astype(np.float32)
    for k in range(T):
        ref = KD.oracle_attn_cells(q[k:k + 1], g_k, g_v, [g_cells[k], g_cells[k]], n_past + k, 1 / 16)[0] * sig[k]
        mx, mean = KD.err_stats(g_out[k], ref)
        print(f"  position {k}: max abs {mx:.3e}  mean abs {mean:.3e}", flush=True)
        assert np.isfinite(g_out[k]).all()
        assert mx <= 1e-4 and mean <= KD.MEAN_ABS_TOL
