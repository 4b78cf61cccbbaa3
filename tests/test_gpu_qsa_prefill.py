"""The reference's default prefill (QSA on) on the device, checked against the
oracle: a 512-token chunk attends, per query, only the cells of the 513 blocks
its indexer scores best (qwfn_graph.cpp:313-414, :466).

Pieces: the chunk's block tables and per-query bias (engine::fill_chunk_qsa,
qwfn_engine.cpp:1276-1320: qwfn_qsa_chunk_inputs), the pooled block keys
(whole blocks by the pool rebuild, the partial tail block -- its last cell
repeated -- by the pool decode), the top-k selection (qwfn_qsa_select_cells),
the selection mask (-inf, 0 at the selected cells, plus the causal mask:
qwfn_qsa_mask_f16) and flash attention over that mask (k_fa_pre). Tables,
bias and mask are compared bit for bit; pooled keys to one F16 unit in the
last place on at most 0.1% of the values (libm cos/sin against the
device's); each query's selection as a set, best first, up to float ties at
the k-th place; the attention output against the oracle over the device's
mask (2e-3 max / 1e-3 mean abs, 1e-4 max as observed)."""
import numpy as np
import pytest
import torch

import kvdata as KD
import qwfn_state as S
from gpu_util import dev, host, say
from oracle import oracle as O
from oracle import state_oracle as SO

pytestmark = pytest.mark.gpu
IDX, IDX_H, TOP_K = 128, 4, 2048


@pytest.mark.parametrize("n_past_c,Tc,ratio", [(16384, 512, 4), (16385, 510, 4), (0, 512, 4), (0, 7, 4), (300, 37, 32),
                                               (5, 9, 1)])
def test_chunk_inputs_match_oracle(gpu, n_past_c, Tc, ratio):
    n_kv = n_past_c + Tc
    nb = -(-n_kv // ratio)
    cb = torch.full((n_kv,), -7, dtype=torch.int32, device="cuda")
    bc = torch.full((nb * ratio,), -7, dtype=torch.int32, device="cuda")
    bp = torch.full((4 * nb,), -7, dtype=torch.int32, device="cuda")
    bias = torch.full((Tc, nb + 5), 7.0, dtype=torch.float32, device="cuda")   # padded rows: untouched past n_blocks
    say(f"chunk inputs n_past_c={n_past_c} Tc={Tc} ratio={ratio}")
    assert S.qsa_chunk_inputs(n_past_c, Tc, ratio, cb, bc, bp, bias) == nb
    o = SO.fill_chunk_qsa(n_past_c, Tc, ratio)
    np.testing.assert_array_equal(host(cb), o["cell_blk"])
    np.testing.assert_array_equal(host(bc), o["blk_cells"])
    np.testing.assert_array_equal(host(bp), o["blk_pos"])
    b = host(bias)
    np.testing.assert_array_equal(b[:, :nb], o["bias"])
    assert (b[:, nb:] == 7.0).all()


def test_visible_cells_match_oracle(gpu):
    """The keys each query sees, as sorted lists: the distinct selected cells at or before
    the query's position (the zeros of the selection mask over the causal mask), bit for
    bit; a cell outside the keys is skipped and flagged."""
    K = gpu
    rng = np.random.default_rng(6)
    for T, n_past, width in ((64, 5000, 300), (7, 0, 40), (33, 100000, 2052)):
        n_kv = n_past + T
        cells = rng.integers(0, n_kv, (T, width)).astype(np.int32)
        cells[:, width // 2:width // 2 + 10] = cells[:, :10]     # repeats
        lists = torch.full((T, width + 4), -7, dtype=torch.int32, device="cuda")
        counts = torch.full((T,), -7, dtype=torch.int32, device="cuda")
        say(f"visible cells T={T} n_past={n_past} width={width}")
        S.qsa_visible_cells(dev(cells), n_kv, n_past, lists, counts)
        assert K.device_status() == 0
        g_l, g_n = host(lists), host(counts)
        for t in range(T):
            want = SO.visible_cells(cells[t], n_kv, n_past + t)
            assert g_n[t] == len(want), f"row {t}"
            np.testing.assert_array_equal(g_l[t, :len(want)], want)
            assert (g_l[t, len(want):] == -7).all()
    say("visible cells with a cell outside the keys")
    cells[5, 7] = n_kv + 3
    cells[6, 1] = -1
    S.qsa_visible_cells(dev(cells), n_kv, n_past, lists, counts)
    assert K.device_status() & 1
    for t in (5, 6):
        want = SO.visible_cells(cells[t][(cells[t] >= 0) & (cells[t] < n_kv)], n_kv, n_past + t)
        np.testing.assert_array_equal(host(lists)[t, :len(want)], want)
        assert host(counts)[t] == len(want)


def test_qsa_mask_matches_oracle(gpu):
    K = gpu
    rng = np.random.default_rng(5)
    T, n_past, width, row = 64, 5000, 300, 5072
    n_kv = n_past + T
    causal = np.full((T, row), SO.F16_NEG_INF, np.uint16)
    for t in range(T):
        causal[t, :n_past + t + 1] = SO.F16_ZERO
    causal[:, 17] = 0x3C00                                       # a finite causal value passes through where selected
    cells = rng.integers(0, n_kv, (T, width)).astype(np.int32)
    cells[:, 100:110] = cells[:, :10]                            # repeats
    cells[3, 0] = 17
    mask = torch.full((T, row), 0x1234, dtype=torch.int16, device="cuda")
    say("qsa mask 64 x 5064")
    S.qsa_mask_f16(dev(cells), dev(causal.view(np.float16)), n_kv, mask.view(torch.float16))
    np.testing.assert_array_equal(host(mask).view(np.uint16), SO.qsa_mask(cells, causal, n_kv, row))
    assert K.device_status() == 0
    say("qsa mask with a cell outside the keys")
    cells[5, 7] = n_kv + 3
    S.qsa_mask_f16(dev(cells), dev(causal.view(np.float16)), n_kv, mask.view(torch.float16))
    assert K.device_status() & 1
    want = SO.qsa_mask(np.delete(cells[5:6], 7, axis=1), causal[5:6], n_kv, row)
    np.testing.assert_array_equal(host(mask).view(np.uint16)[5:6], want)


def _ulp_ok(got_bits, ref_bits):
    d = np.abs(got_bits.astype(np.int32) - ref_bits.astype(np.int32))
    assert d.max() <= 1
    assert int((d != 0).sum()) <= max(1, d.size // 1000)


@pytest.mark.parametrize("n_past_c,Tc", [(16384, 512), (16385, 510)])
def test_qsa_prefill_chunk_chain(gpu, oracle, n_past_c, Tc):
    """qsa_top_k -> qsa_mask -> flash attention for a chunk at depth 16384: 16 query
    heads over 2 KV heads, the indexer's 4 heads of 128, ratio 4 (4224 blocks, the
    second case with a partial tail block), 513 blocks kept per query."""
    K = gpu
    ratio, nh = 4, 16
    n_kv = n_past_c + Tc
    nb = -(-n_kv // ratio)
    n_bid = n_kv // ratio
    width = min(n_kv, TOP_K + ratio - 1)
    kb = min(nb, -(-width // ratio))
    rng = np.random.default_rng(n_past_c)
    ic = rng.standard_normal((n_kv, IDX)).astype(np.float16)
    knw = rng.uniform(0.6, 1.4, IDX).astype(np.float32)
    q_idx = rng.standard_normal((Tc, IDX_H, IDX)).astype(np.float32)
    kc, vc = (KD.make_cache(KD.kv_rows(n_past_c, 0, kind, n_kv, outliers=True), n_kv) for kind in (KD.K_KIND, KD.V_KIND))
    q = KD.q_rows(n_past_c, 1, Tc, nh)[0]
    row = (n_kv + 63) // 64 * 64

    # ---- device chain
    ic_d, knw_d = dev(ic), dev(knw)
    bc = torch.empty(nb * ratio, dtype=torch.int32, device="cuda")
    bp = torch.empty(4 * nb, dtype=torch.int32, device="cuda")
    bias = torch.empty((Tc, nb), dtype=torch.float32, device="cuda")
    say(f"chunk inputs n_past_c={n_past_c} Tc={Tc}")
    S.qsa_chunk_inputs(n_past_c, Tc, ratio, None, bc, bp, bias)
    pool = torch.zeros((nb, IDX), dtype=torch.float16, device="cuda")
    say("pool: whole blocks, then the tail block")
    K.qsa_pool_rebuild(ic_d, n_kv, ratio, knw_d, pool)
    if n_bid < nb:
        K.qsa_pool_decode(ic_d, None, dev(np.array([0], np.int32)), bc[n_bid * ratio:(n_bid + 1) * ratio], ratio,
                          dev(np.full(4, n_bid * ratio, np.int32)), dev(np.array([n_bid], np.int32)), knw_d, pool)
    cells = torch.full((Tc, kb * ratio), -1, dtype=torch.int32, device="cuda")
    top = torch.full((Tc, kb), -1, dtype=torch.int32, device="cuda")
    say(f"select {kb} of {nb} blocks for {Tc} queries")
    S.qsa_select_cells(pool, dev(q_idx), bias, kb, bc, ratio, cells, top)
    causal = torch.empty((Tc, row), dtype=torch.float16, device="cuda")
    S.causal_mask_f16(causal, n_kv, Tc, n_past_c)
    qmask = torch.empty((Tc, row), dtype=torch.float16, device="cuda")
    say("selection mask")
    S.qsa_mask_f16(cells, causal, n_kv, qmask)
    say("attention over the selection mask")
    qd = dev(q[None].astype(np.float32))
    out = torch.full((1, Tc, nh, 256), float("nan"), dtype=torch.float32, device="cuda")
    kd, vd = dev(kc), dev(vc)
    K.flash_attn_ext(K.q_view(qd), K.cache_attn_view(kd, n_kv, 2), K.cache_attn_view(vd, n_kv, 2),
                     K.mask_view(qmask), 1 / 16, K.out_view(out))
    assert K.last_kernel().startswith("k_fa_pre<")
    assert K.device_status() == 0
    g_bc, g_bias, g_pool = host(bc), host(bias), host(pool).view(np.uint16)
    g_cells, g_top, g_causal, g_mask = host(cells), host(top), host(causal).view(np.uint16), host(qmask).view(np.uint16)
    g_out = host(out)[0]

    # ---- oracle
    o = SO.fill_chunk_qsa(n_past_c, Tc, ratio)
    np.testing.assert_array_equal(g_bc, o["blk_cells"])
    np.testing.assert_array_equal(g_bias, o["bias"])
    r_pool = O.qsa_pool_blocks(ic.view(np.uint16), o["blk_cells"], ratio, knw,
                               np.repeat((np.arange(nb) * ratio)[:, None], 4, axis=1).astype(np.int32))
    _ulp_ok(g_pool, r_pool)
    for t in range(Tc):
        sc = SO.qsa_scores(g_pool.view(np.float16), q_idx[t], o["bias"][t])
        want = SO.qsa_top_k(sc, kb)
        kth = sc[want[-1]]
        tol = 1e-5 * max(1.0, abs(kth))
        got = g_top[t]
        assert len(set(got.tolist())) == kb
        assert {int(x) for x in want if sc[x] > kth + tol} <= {int(x) for x in got}, f"query {t}"
        assert all(sc[x] >= kth - tol for x in got), f"query {t}"
        np.testing.assert_array_equal(g_cells[t], SO.qsa_cells(got, o["blk_cells"], ratio))
    ref_causal = np.full((Tc, row), SO.F16_NEG_INF, np.uint16)
    for t in range(Tc):
        ref_causal[t, :n_past_c + t + 1] = SO.F16_ZERO
    np.testing.assert_array_equal(g_causal, ref_causal)
    np.testing.assert_array_equal(g_mask, SO.qsa_mask(g_cells, g_causal, n_kv, row))
    live = (g_mask[:, :n_kv] == SO.F16_ZERO).sum(axis=1)
    print(f"  visible cells per query: min {live.min()} max {live.max()} of {n_kv}", flush=True)
    ref = KD.oracle_attn(q, kc, vc, n_kv, 2, np.ascontiguousarray(g_mask[:, :n_kv]), 1 / 16)
    mx, mean = KD.err_stats(g_out, ref)
    print(f"  max abs {mx:.3e}  mean abs {mean:.3e}", flush=True)
    assert np.isfinite(g_out).all()
    assert mx <= 1e-4 and mean <= KD.MEAN_ABS_TOL

    # ---- the same keys as lists: visible cells, then attention over them (no mask)
    say("visible cells and attention over the lists")
    lists = torch.full((Tc, cells.shape[1]), -7, dtype=torch.int32, device="cuda")
    counts = torch.empty((Tc,), dtype=torch.int32, device="cuda")
    S.qsa_visible_cells(cells, n_kv, n_past_c, lists, counts)
    out2 = torch.full((1, Tc, nh, 256), float("nan"), dtype=torch.float32, device="cuda")
    K.flash_attn_ext_query_cells_dev(K.q_view(qd), K.cache_attn_view(kd, n_kv, 2), K.cache_attn_view(vd, n_kv, 2),
                                     lists, counts, n_past_c, 1 / 16, K.out_view(out2))
    assert K.device_status() == 0
    g_lists, g_counts = host(lists), host(counts)
    for t in range(Tc):
        want = np.flatnonzero(g_mask[t, :n_kv] == SO.F16_ZERO).astype(np.int32)
        assert g_counts[t] == len(want), f"query {t}"
        np.testing.assert_array_equal(g_lists[t, :len(want)], want)
    g_out2 = host(out2)[0]
    mx, mean = KD.err_stats(g_out2, ref)
    print(f"  lists: max abs {mx:.3e}  mean abs {mean:.3e}", flush=True)
    assert np.isfinite(g_out2).all()
    assert mx <= 1e-4 and mean <= KD.MEAN_ABS_TOL
    # each within 1e-4 of the oracle, so within 2e-4 of each other (9.2e-5 observed)
    np.testing.assert_allclose(g_out2, g_out, rtol=0, atol=2e-4)
