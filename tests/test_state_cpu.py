"""CPU tests of the state rows: the oracle restatement pinned against the
reference's logged numbers and its own independent code paths, and the
library's layout-only state, bookkeeping and host-side validation (no GPU)."""
import ctypes

import numpy as np
import pytest

import qwfn_kv as K
import qwfn_state as S
from oracle import state_oracle as SO

# The summary line every run in the reference's benchmark logs prints at 73728
# positions (bench/evidence/raw/llamabench/*.log, engine::memory_summary).
GOLDEN_SUMMARY_73728 = ("state @ 73728 ctx: KV 0.962593 GB (q8_0), indexer 0.226492 GB, deltanet 113.246 MB "
                        "(constant), conv 4.79232 MB  =>  total 1.30712 GB on the device")


def layout_state(n_ctx, **kw):
    st = S.State()
    ok, err = st.init(S.config(n_ctx, **kw), S.LAYOUT_ONLY)
    assert ok, err
    return st


def small_cfg(**kw):
    d = dict(n_layer=8, ssm_d_state=16, ssm_n_group=2, ssm_dt_rank=4, hc_count=2, n_embd=64, n_rollback=2)
    d.update(kw)
    return d


# ------------------------------------------------------------------ oracle pins

def test_oracle_summary_matches_reference_log():
    cfg = SO.config_default(73728)
    total = sum(t["nbytes"] for t in SO.declare_tensors(cfg))
    assert SO.summary(cfg, total) == GOLDEN_SUMMARY_73728


def test_oracle_sizes_match_reference_comments():
    # qwfn_state.h:4-8: KV @128K q8_0 1.71 GB (f16 3.22 GB), indexer @128K f16
    # 0.40 GB, 113 MB f32 of DeltaNet state for all 36 layers
    for typ, gb in ((SO.TYPE_Q8_0, 1.71), (SO.TYPE_F16, 3.22)):
        cfg = SO.config_default(131072)
        cfg["type_k"] = cfg["type_v"] = typ
        ts = SO.declare_tensors(cfg)
        kv = sum(t["nbytes"] for t in ts if t["kind"] in (SO.K, SO.V))
        assert round(kv / 1e9, 2) == gb
        assert round(sum(t["nbytes"] for t in ts if t["kind"] == SO.IDX) / 1e9, 2) == 0.40
        assert round(sum(t["nbytes"] for t in ts if t["kind"] == SO.RS) / 1e6) == 113
    # 12 attention layers, 36 DeltaNet layers (qwfn_hparams.h:30)
    ts = SO.declare_tensors(SO.config_default(1024))
    assert sum(t["kind"] == SO.K for t in ts) == 12 and sum(t["kind"] == SO.RS for t in ts) == 36


def test_oracle_snapshot_parts_closed_form():
    cfg = SO.config_default(73728)
    parts = SO.snapshot_parts([cfg], 8192)
    assert len(parts) == 12 * 3 + 36 * 2 + 1
    kv = sum(b for _, k, _, b in parts if k in (SO.K, SO.V))
    assert kv == 12 * 8192 * 1088                            # 106.95 MB per slot
    assert sum(b for _, k, _, b in parts if k == SO.IDX) == 12 * 8192 * 256   # 25.2 MB
    # positional parts are capped at the tensor, recurrent parts are whole
    full = SO.snapshot_parts([cfg], 10 ** 6)
    assert sum(b for _, k, _, b in full if k == SO.K) == 12 * 73728 * 544
    assert all(b == 0 for _, k, _, b in SO.snapshot_parts([cfg], 0) if k in (SO.K, SO.V, SO.IDX))
    # order: layer by layer, K V idx or rs conv, the PLE history last; a second state follows
    kinds = [k for _, k, _, _ in parts]
    assert kinds[:6] == [SO.RS, SO.CONV] * 3 and kinds[6:9] == [SO.K, SO.V, SO.IDX] and kinds[-1] == SO.PLE_CONV
    two = SO.snapshot_parts([cfg, cfg], 5)
    assert two[:len(two) // 2] == [(0,) + p[1:] for p in SO.snapshot_parts([cfg], 5)]
    assert {p[0] for p in two[len(two) // 2:]} == {1}


def test_oracle_causal_mask_builders_agree():
    from oracle import oracle as O
    for n_past in (0, 1, 7, 64):
        for T in (1, 2, 3, 9):
            a = SO.attn_inputs_mask(n_past, T)
            assert np.array_equal(a, SO.step_inputs_mask(n_past, T))
            assert np.array_equal(a, SO.mtp_mask(n_past, T))
            assert np.array_equal(a, O.causal_mask(T, n_past))
            # the last row sees every key, the first n_past + 1
            assert (a[-1] == SO.F16_ZERO).all() and (a[0] == SO.F16_ZERO).sum() == n_past + 1


def test_oracle_cell_mask_op_chain_is_an_integer_compare():
    rng = np.random.default_rng(5)
    for n_past in (0, 3, 1000, 73727):
        cells = np.concatenate([rng.integers(0, 73728, 200), [n_past, n_past + 1, max(n_past - 1, 0)]]).astype(np.int32)
        mask, g = SO.cell_mask(cells, n_past, 256)
        ref = np.where(cells <= n_past, SO.F16_ZERO, SO.F16_NEG_INF)
        assert np.array_equal(mask[:cells.size], ref)
        assert (mask[cells.size:] == SO.F16_NEG_INF).all()
        assert np.array_equal(g[:cells.size], cells) and np.array_equal(g[cells.size:], cells[:256 - cells.size])


def test_oracle_bias_window_equals_full_rebuild():
    # Applying the per-token window from a reset bias for positions 0..n gives
    # qsa_pool_rebuild's full bias at n: two separate reference functions.
    for ratio in (1, 4, 5):
        nb_max = 40
        bias = SO.qsa_reset_bias(nb_max)
        for n in range(ratio * nb_max + 3):
            SO.qsa_decode_prepare(bias, n, ratio)
            assert np.array_equal(bias, SO.qsa_pool_rebuild_bias(nb_max, n, ratio)), (ratio, n)
            prev = bias.copy()
            k = SO.qsa_decode_prepare_k(prev, n + 1, ratio)["bias"]
            assert np.array_equal(k, SO.qsa_pool_rebuild_bias(nb_max, n + 1, ratio)), (ratio, n)


def test_oracle_decode_inputs_and_bucket():
    o = SO.qsa_decode_prepare(SO.qsa_reset_bias(16), 13, 4)
    assert o["write_idx"][0] == 13 and o["blk_idx"][0] == 3
    assert list(o["member_idx"]) == [12, 13, 14, 15] and list(o["blk_pos"]) == [12] * 4
    assert o["npast_f"][0] == 13.0
    assert list(o["bias"][:5]) == [-np.inf, -np.inf, 0.0, 1e9, -np.inf]   # only the window is written
    assert SO.qsa_bucket(0, 4, 18432) == 768
    assert SO.qsa_bucket(4 * 767, 4, 18432) == 768 and SO.qsa_bucket(4 * 768, 4, 18432) == 1024
    assert SO.qsa_bucket(73727, 4, 18432) == 18432 and SO.qsa_bucket(10 ** 6, 4, 1000) == 1000


def test_oracle_rollback_bookkeeping():
    assert SO.rollback_depth_after_step(3, True, 2) == 2
    assert SO.rollback_depth_after_step(3, True, 1) == 1
    assert SO.rollback_depth_after_step(1, True, 2) == 0
    assert SO.rollback_depth_after_step(3, False, 2) == 0
    assert SO.rollback_depth_after_step(3, True, 0) == 0
    assert not SO.rollback_ok(0, 2) and SO.rollback_ok(2, 2) and not SO.rollback_ok(3, 2)


# ------------------------------------------------------- library, layout only

def test_library_summary_matches_reference_log():
    st = layout_state(73728)
    assert st.summary() == GOLDEN_SUMMARY_73728
    assert st.bytes() == 1307123712 and st.n_ctx() == 73728 and st.host_bytes() == 0


@pytest.mark.parametrize("n_ctx,kw", [(73728, {}), (1000, small_cfg()), (4096, small_cfg(type_k=1, type_v=1)),
                                      (512, small_cfg(ple_n_head=0, full_attention_interval=2, type_idx=0)),
                                      (300, small_cfg(kv_host=1, idx_host=1))])
def test_library_layout_matches_oracle(n_ctx, kw):
    st = layout_state(n_ctx, **kw)
    cfg = SO.config_default(n_ctx)
    cfg.update(kw)
    ts = SO.declare_tensors(cfg)
    seen = []
    for t in ts:
        d = st.tensor(t["kind"], t["il"])
        assert d is not None and d.type == t["type"] and list(d.ne) == t["ne"]
        assert d.nb[3] * d.ne[3] == t["nbytes"] and (d.data or 0) % 256 == 0
        seen.append((bool(kw.get("kv_host") if t["kind"] in (0, 1) else kw.get("idx_host") if t["kind"] == 2 else 0),
                     d.data or 0, t["nbytes"]))
    for arena in (False, True):                 # no overlaps within an arena
        spans = sorted((a, a + n) for h, a, n in seen if h == arena)
        assert all(e0 <= a1 for (_, e0), (a1, _) in zip(spans, spans[1:]))
    # the wrong layer kind gives null, like k_cache() on a DeltaNet layer
    assert st.k_cache(0) is None and st.rs_state(cfg["full_attention_interval"] - 1) is None
    assert st.tensor(S.STATE_K, 10 ** 6) is None
    dev_total = sum(n for h, _, n in seen if not h)
    host_total = sum(n for h, _, n in seen if h)
    assert dev_total <= st.bytes() <= dev_total + 256 * len(ts)
    assert host_total <= st.host_bytes() <= host_total + 256 * len(ts)
    assert st.summary() == SO.summary(cfg, st.bytes(), st.host_bytes())
    # snapshot parts: the oracle's order and sizes
    for n_past in (0, 1, 77, n_ctx, n_ctx + 5):
        got = S.snapshot_parts([st, st], n_past)
        want = SO.snapshot_parts([cfg, cfg], n_past)
        assert [b for _, b in got] == [p[3] for p in want]


def test_library_rollback_slots_layout():
    # each rollback slot is an image of the live recurrent region, same layout
    st = layout_state(256, **small_cfg(n_rollback=3))
    rec = [(k, il) for il in range(8) for k in (S.STATE_RS, S.STATE_CONV) if st.tensor(k, il) is not None]
    rec.append((S.STATE_PLE_CONV, 0))
    live = {r: st.tensor(*r) for r in rec}
    base = min(t.data or 0 for t in live.values())
    span = st.rollback_bytes() // 3
    assert span * 3 == st.rollback_bytes() and span >= sum(t.nb[3] * t.ne[3] for t in live.values())
    for r, t in live.items():
        for s in range(3):
            d = st.rollback_slot(r[0], r[1], s)
            assert (d.data or 0) == s * span + (t.data or 0) - base and list(d.ne) == list(t.ne)
    with pytest.raises(K.QwfnError):
        st.rollback_slot(S.STATE_RS, 0, 3)
    with pytest.raises(K.QwfnError):
        st.rollback_slot(S.STATE_K, 3, 0)


def test_library_bookkeeping_and_rollback_guard():
    st = layout_state(64, **small_cfg(n_rollback=2))
    st.step_done(10)
    assert st.n_past() == 10 and st.rollback_depth() == 0
    st.step_done(3, verified=True)
    assert st.n_past() == 13 and st.rollback_depth() == 2
    ok, err = st.rollback_n(3, stream=0)
    assert not ok and err == "rollback: no snapshot of the state 3 tokens back"
    ok, err = st.rollback_n(0, stream=0)
    assert not ok and "0 tokens back" in err
    ok, err = st.rollback_n(1, stream=0)         # guard passes; no memory without a device
    assert not ok and "no rollback memory" in err
    with pytest.raises(K.QwfnError, match="context exhausted"):
        st.step_done(64 - 13 + 1)
    st.step_done(64 - 13)
    assert st.n_past() == 64
    st.reset(stream=0)                           # bookkeeping only without memory
    assert st.n_past() == 0 and st.rollback_depth() == 0


def test_library_config_validation():
    for kw, needle in ((dict(n_ctx=0), "n_ctx"), (dict(type_k=26), "type_k"), (dict(type_idx=8), "type_idx"),
                       (dict(n_head_kv=3, n_embd_head_k=8, n_embd_head_v=8), "32-value"),
                       (dict(ssm_d_conv=1), "d_conv"), (dict(n_rollback=65), "rollback")):
        cfg = S.config(kw.pop("n_ctx", 128), **kw)
        ok, err = S.State().init(cfg, S.LAYOUT_ONLY)
        assert not ok and needle in err, (kw, err)


def test_library_bucket():
    L = K.load()
    for n_past, ratio, nb in ((0, 4, 18432), (3067, 4, 18432), (3072, 4, 18432), (73727, 4, 18432), (10 ** 6, 4, 1000),
                              (5, 1, 700)):
        assert L.qwfn_qsa_bucket(n_past, ratio, nb) == SO.qsa_bucket(n_past, ratio, nb)


def test_step_input_validation():
    L = K.load()
    FAKE = 0x7F0000000000

    def err(rc, code, needle):
        assert rc == code, (rc, L.qwfn_last_error())
        assert needle in L.qwfn_last_error().decode()

    err(L.qwfn_causal_mask_f16(None, 4, 1, 0, 8, None), K.EINVAL, "NULL")
    err(L.qwfn_causal_mask_f16(FAKE, 4, 1, 0, 6, None), K.EALIGN, "row_stride")
    err(L.qwfn_causal_mask_f16(FAKE, 4, 1, 0, 9, None), K.EALIGN, "row_stride")
    err(L.qwfn_cell_mask_f16(FAKE, 10, 21, 0, FAKE, None, None), K.EINVAL, "n_pad")
    err(L.qwfn_cell_mask_f16(FAKE, 10, 9, 0, FAKE, None, None), K.EINVAL, "n_pad")
    err(L.qwfn_cell_mask_f16(FAKE, 10, 16, -1, FAKE, None, None), K.EINVAL, "n_past")
    q = K.QsaInputs()
    err(L.qwfn_qsa_decode_prepare(ctypes.byref(q), None, 0, None), K.EINVAL, "NULL")
    for f in ("bias", "write_idx", "member_idx", "blk_pos", "blk_idx", "npast_f"):
        setattr(q, f, FAKE)
    q.ratio, q.n_blocks_max = 0, 16
    err(L.qwfn_qsa_decode_prepare(ctypes.byref(q), None, 0, None), K.EINVAL, "ratio")
    # the step forms: 1 to 16 positions, one ratio, bias rows apart, k_raw rows of idx_dim floats
    arr = (K.QsaInputs * 2)()
    for qq in arr:
        for f in ("bias", "write_idx", "member_idx", "blk_pos", "blk_idx", "npast_f"):
            setattr(qq, f, FAKE)
        qq.ratio, qq.n_blocks_max = 4, 16
    err(L.qwfn_qsa_decode_prepare_steps(arr, 0, 5, None), K.ENOTSUP, "1 to 16")
    err(L.qwfn_qsa_decode_prepare_steps(arr, 17, 5, None), K.ENOTSUP, "1 to 16")
    err(L.qwfn_qsa_decode_prepare_steps(arr, 2, -1, None), K.EINVAL, "positions")
    err(L.qwfn_qsa_decode_prepare_steps(arr, 2, 5, None), K.EINVAL, "overlap")
    arr[1].bias, arr[1].ratio = FAKE + 4096, 8
    err(L.qwfn_qsa_decode_prepare_steps(arr, 2, 5, None), K.EINVAL, "same ratio")
    arr[1].ratio = 4
    cfg = K.QsaPoolCfg()
    L.qwfn_qsa_pool_cfg_default(ctypes.byref(cfg))
    err(L.qwfn_qsa_pool_decode_steps(FAKE, 100, FAKE, 512, arr, 17, FAKE, FAKE, 10, ctypes.byref(cfg), None),
        K.ENOTSUP, "1 to 16")
    err(L.qwfn_qsa_pool_decode_steps(FAKE, 100, FAKE, 256, arr, 2, FAKE, FAKE, 10, ctypes.byref(cfg), None),
        K.EALIGN, "shorter")
    # the fused form checks both sets of arguments, the preparation's first
    PP = L.qwfn_qsa_decode_prepare_pool_steps
    err(PP(None, 2, 5, FAKE, 100, FAKE, 512, FAKE, FAKE, 10, ctypes.byref(cfg), None), K.EINVAL, "NULL inputs")
    err(PP(arr, 17, 5, FAKE, 100, FAKE, 512, FAKE, FAKE, 10, ctypes.byref(cfg), None), K.ENOTSUP, "1 to 16")
    err(PP(arr, 2, -1, FAKE, 100, FAKE, 512, FAKE, FAKE, 10, ctypes.byref(cfg), None), K.EINVAL, "positions")
    err(PP(arr, 2, 5, FAKE, 100, FAKE, 256, FAKE, FAKE, 10, ctypes.byref(cfg), None), K.EALIGN, "shorter")
    err(PP(arr, 2, 5, None, 100, FAKE, 512, FAKE, FAKE, 10, ctypes.byref(cfg), None), K.EINVAL, "NULL pointer")
    err(PP(arr, 2, 5, FAKE, 100, FAKE, 512, None, FAKE, 10, ctypes.byref(cfg), None), K.EINVAL, "k_norm")
    assert L.qwfn_last_error().decode().startswith("qsa_pool"), L.qwfn_last_error()
    arr[1].ratio = 8
    err(L.qwfn_qsa_pool_decode_steps(FAKE, 100, FAKE, 512, arr, 2, FAKE, FAKE, 10, ctypes.byref(cfg), None),
        K.EINVAL, "ratios")
    err(PP(arr, 2, 5, FAKE, 100, FAKE, 512, FAKE, FAKE, 10, ctypes.byref(cfg), None), K.EINVAL, "same ratio")
    err(L.qwfn_qsa_bias_rebuild(FAKE, 16, -2, 4, None), K.EINVAL, "sizes")
    err(L.qwfn_qsa_tables(FAKE, 1 << 30, 4, None, 0, None, 0, None), K.ERANGE, "int32")
    # snapshot calls need states with memory
    st = layout_state(64, **small_cfg())
    H = (ctypes.c_void_p * 1)(st.handle)
    err(L.qwfn_snapshot_save(H, 1, None, None, 0, 0, None, None), K.EINVAL, "no memory")
    err(L.qwfn_snapshot_load(H, 1, 0, None, None, 0, 0, None), K.EINVAL, "no memory")
    n = ctypes.c_int32(0)
    err(L.qwfn_snapshot_parts(H, 1, -1, None, 0, ctypes.byref(n)), K.EINVAL, "position")


# ------------------------------------------------------- saved-sequence pool

def _toks(n, seed=0, prefix=()):
    rng = np.random.default_rng(seed)
    return list(prefix) + [int(x) for x in rng.integers(0, 248000, n - len(prefix))]


def test_oracle_pool_scripted():
    P = SO.SnapPool(cap=100, max_entries=4)
    for i in range(5):
        assert P.save_seq([i] * 3, 3, 10)
    assert [e[0] for e in P.saved] == [(1,) * 3, (2,) * 3, (3,) * 3, (4,) * 3]   # at most four, oldest gone
    assert not P.save_seq([9], 1, 101) and len(P.saved) == 4                      # larger than the cap: not kept
    assert P.save_seq([2] * 3, 3, 10) and P.saved[-1][0] == (2,) * 3 and len(P.saved) == 4   # replaced, now newest
    assert P.save_seq([7], 1, 75)                                                 # the byte cap evicts the oldest
    assert [e[0] for e in P.saved] == [(4,) * 3, (2,) * 3, (7,)] and sum(e[2] for e in P.saved) <= 100
    # best_saved: the longest sequence the prompt strictly extends
    Q = SO.SnapPool(cap=10 ** 9)
    Q.save_seq([1, 2], 2, 1)
    Q.save_seq([1, 2, 3], 3, 1)
    Q.save_seq([1, 2, 3, 4], 4, 1)
    assert Q.best_saved([1, 2, 3, 4, 5]) == 2 and Q.best_saved([1, 2, 3, 4]) == 1   # equal length is not an extension
    assert Q.best_saved([1, 2, 3, 9, 9]) == 1 and Q.best_saved([2, 2, 3]) == -1
    assert Q.best_saved([1, 2, 3, 4, 5], has_images=True) == -1
    Q.load(0)
    assert Q.saved[-1][0] == (1, 2)                                               # most recently used last


def test_oracle_pool_restore_and_split():
    P = SO.SnapPool(cap=10 ** 9)
    a = _toks(3000, 1)
    assert P.restore_or_reset(a, 10, False, _toks(10, 2)) == 0 and len(P.saved) == 1   # set aside, reset
    assert P.restore_or_reset(_toks(2047, 3), 10, False, a + [5]) == 3000    # short one not saved; a restored
    assert len(P.saved) == 1
    assert P.restore_or_reset(_toks(2500, 4), 10, True, a + [5]) == 3000     # images: not set aside
    assert len(P.saved) == 1
    # the split: a shared prefix of >= 2048 tokens past what the engine holds, the prompt going on
    sys_prompt = _toks(2500, 5)
    P2 = SO.SnapPool(cap=10 ** 9)
    P2.save_seq(sys_prompt + _toks(600, 6), 3100, 1)
    prompt = sys_prompt + _toks(400, 7)
    assert P2.shared_prefix_split(prompt, 0) == 2500
    assert P2.shared_prefix_split(prompt, 2499) == 0                    # not 2 past what the engine holds
    assert P2.shared_prefix_split(prompt, 2048) == 0                    # the engine holds >= 2048: no split
    assert P2.shared_prefix_split(prompt[:2510], 0) == 0                # fewer than 16 tokens after it
    assert P2.shared_prefix_split(prompt, 0, has_images=True) == 0
    P2.save_seq(sys_prompt, 2500, 1)
    assert P2.shared_prefix_split(prompt, 0) == 0                       # already saved at that point
    assert P2.shared_prefix_split(_toks(3000, 8), 0) == 0               # nothing shared


def _pool_states(n_ctx=4096):
    return [layout_state(n_ctx, **small_cfg(n_rollback=0)),
            layout_state(n_ctx, **small_cfg(n_layer=4, ple_n_head=0, n_rollback=0))]


def _set_past(states, n):
    for s in states:
        if s.n_past() > n:
            s.reset(stream=0)
        s.step_done(n - s.n_past()) if n > s.n_past() else None


def test_library_pool_matches_oracle_dry():
    states = _pool_states()
    size = lambda n: sum(b for _, b in S.snapshot_parts(states, n))
    rng = np.random.default_rng(11)
    for cap_n, max_e in ((4096 * 3, 4), (2500, 2), (10 ** 6, 3)):
        cap = size(cap_n) if cap_n < 10 ** 6 else 1 << 40
        pool = S.SnapPool(cap, max_e, S.LAYOUT_ONLY)
        ref = SO.SnapPool(cap, max_e)
        seqs = [_toks(int(n), int(i)) for i, n in enumerate(rng.integers(1, 4000, 8))]
        seqs += [seqs[0][:2100] + _toks(50, 99), seqs[1] + [7, 7]]
        for step in range(60):
            op = rng.integers(0, 4)
            t = seqs[int(rng.integers(0, len(seqs)))]
            if op == 0:
                _set_past(states, len(t))
                assert pool.save_seq(states, t, stream=0) == ref.save_seq(t, len(t), size(len(t)))
            elif op == 1:
                assert pool.best_saved(t) == ref.best_saved(t)
                nc = int(rng.integers(0, 3000))
                assert pool.shared_prefix_split(t, nc) == ref.shared_prefix_split(t, nc)
            elif op == 2 and ref.saved:
                k = int(rng.integers(0, len(ref.saved)))
                ok, err = pool.load(k, states, stream=0)
                assert ok, err
                e = ref.load(k)
                assert states[0].n_past() == e[1] and states[1].n_past() == e[1]
            else:
                _set_past(states, len(t))
                prompt = seqs[int(rng.integers(0, len(seqs)))]
                prompt = prompt + [1, 2, 3] if rng.integers(0, 2) else prompt
                got = pool.restore_or_reset(states, t, prompt, stream=0)
                want = ref.restore_or_reset(t, size(len(t)), False, prompt)
                assert got == want and states[0].n_past() == want
            assert pool.count() == len(ref.saved)
            assert [pool.entry(k)[0] for k in range(pool.count())] == [list(e[0]) for e in ref.saved]
            assert pool.bytes() == sum(e[2] for e in ref.saved)


def test_library_pool_split_matches_oracle():
    pool = S.SnapPool(1 << 40, 4, S.LAYOUT_ONLY)
    ref = SO.SnapPool(1 << 40, 4)
    states = _pool_states()
    sys_prompt = _toks(2500, 5)
    for t in (sys_prompt + _toks(600, 6), _toks(3000, 8)):
        _set_past(states, len(t))
        assert pool.save_seq(states, t, stream=0) and ref.save_seq(t, len(t), 1)
    prompt = sys_prompt + _toks(400, 7)
    for n_consumed in (0, 100, 2497, 2498, 2499, 2048, 3000):
        for p in (prompt, prompt[:2516], prompt[:2517], _toks(3000, 8) + [1] * 20):
            for img in (False, True):
                assert pool.shared_prefix_split(p, n_consumed, img) == ref.shared_prefix_split(p, n_consumed, img)


def test_library_pool_validation():
    L = K.load()
    h = ctypes.c_void_p(None)
    assert L.qwfn_snap_pool_create(1 << 20, 0, S.LAYOUT_ONLY, ctypes.byref(h)) == K.EINVAL
    assert L.qwfn_snap_pool_create(1 << 20, 65, S.LAYOUT_ONLY, ctypes.byref(h)) == K.EINVAL
    pool = S.SnapPool(1 << 20, 4, S.LAYOUT_ONLY)
    with pytest.raises(K.QwfnError, match="no such entry"):
        pool.entry(0)
    states = _pool_states()
    states[0].step_done(10)
    with pytest.raises(K.QwfnError, match="disagree"):
        pool.save_seq(states, [1] * 10, stream=0)
    with pytest.raises(K.QwfnError, match="positions"):
        pool.restore_or_reset(states[:1], [1] * 9, [1] * 20, stream=0)


def test_qsa_select_validation():
    L = K.load()
    FAKE = 0x7F0000000000

    def err(rc, code, needle):
        assert rc == code, (rc, L.qwfn_last_error())
        assert needle in L.qwfn_last_error().decode()

    ws = L.qwfn_qsa_select_workspace_size(768, 1)
    assert ws == 768 * 4
    call = lambda **kw: L.qwfn_qsa_select_cells(
        kw.get("pool", FAKE), kw.get("pool_nb1", 256), kw.get("nb", 768), kw.get("q", FAKE), kw.get("nh", 4), 2048,
        FAKE, 3072, kw.get("T", 1), kw.get("k", 513), FAKE, kw.get("ratio", 4), FAKE, None, FAKE, kw.get("ws", ws), None)
    err(call(pool=None), K.EINVAL, "NULL")
    err(call(k=769), K.EINVAL, "k_blocks")
    err(call(k=1025, nb=2000, ws=8000), K.EINVAL, "k_blocks")
    err(call(nh=9), K.ENOTSUP, "heads")
    err(call(pool_nb1=200), K.EALIGN, "16-byte")
    err(call(ws=100), K.ENOMEM, "workspace")
    err(call(ratio=17), K.ENOTSUP, "16 cells")
    err(call(nb=49153, ws=L.qwfn_qsa_select_workspace_size(49153, 1)), K.ENOTSUP, "49152")
    err(call(q=FAKE + 4), K.EALIGN, "q [128")
    # scores of query t sit at rows of n_blocks rounded up to 64 floats
    assert L.qwfn_qsa_select_workspace_size(1000, 3) == 1024 * 3 * 4
    # the oracle's tie rule on a closed form: equal scores keep the lower block first
    sc = np.array([1.0, 3.0, 3.0, 2.0, 3.0])
    assert list(SO.qsa_top_k(sc, 3)) == [1, 2, 4] and list(SO.qsa_top_k(sc, 4)) == [1, 2, 4, 3]


def test_oracle_qsa_selection_pins():
    """The selection oracle against closed forms and a brute force over tiny inputs."""
    rng = np.random.default_rng(11)
    nb, H = 40, 3
    pool = rng.standard_normal((nb, 128)).astype(np.float16)
    bias = rng.standard_normal(nb).astype(np.float32)
    # a zero query: every head's dot product is 0, relu keeps 0: the score is the bias
    np.testing.assert_array_equal(SO.qsa_scores(pool, np.zeros((H, 128), np.float32), bias), bias.astype(np.float64))
    # planted keys: block j holds j/8 in dim 5; a query 1 in dim 5 of head 0 and -1 in
    # head 1 scores j/8 (head 1 is clipped by relu)
    planted = np.zeros((nb, 128), np.float16)
    planted[:, 5] = np.arange(nb) / 8.0
    q = np.zeros((H, 128), np.float32)
    q[0, 5], q[1, 5] = 1.0, -1.0
    np.testing.assert_array_equal(SO.qsa_scores(planted, q, np.zeros(nb, np.float32)), np.arange(nb) / 8.0)
    # the query is rounded to f16 before the products: 1 + 2^-12 is 1.0 in f16
    q[0, 5] = 1.0 + 2.0 ** -12
    np.testing.assert_array_equal(SO.qsa_scores(planted, q, np.zeros(nb, np.float32)), np.arange(nb) / 8.0)
    # brute force: explicit loops over blocks, heads and dims
    qr = rng.standard_normal((H, 128)).astype(np.float32)
    got = SO.qsa_scores(pool, qr, bias)
    for b in range(0, nb, 7):
        tot = 0.0
        for h in range(H):
            d = 0.0
            for i in range(128):
                d += float(pool[b, i]) * float(np.float16(qr[h, i]))
            tot += d if d > 0.0 else 0.0
        assert abs(got[b] - (tot + float(bias[b]))) <= 1e-9 * max(1.0, abs(tot))
    # top-k: a brute-force selection by (score descending, block ascending)
    sc = np.round(rng.standard_normal(64) * 2.0) / 2.0            # many ties
    for k in (1, 7, 33, 64):
        want = sorted(range(64), key=lambda b: (-sc[b], b))[:k]
        assert list(SO.qsa_top_k(sc, k)) == want
    # cells: the table of a 1-sequence layout maps block b to cells b*ratio .. b*ratio+ratio-1
    blk_cells, _, _ = SO.qsa_tables(16, 4, 1, 0)
    top = np.array([5, 0, 15], np.int32)
    assert list(SO.qsa_cells(top, blk_cells, 4)) == [20, 21, 22, 23, 0, 1, 2, 3, 60, 61, 62, 63]


def test_qsa_select_wrapper_checks_shapes():
    """The Python wrapper refuses tensors whose sizes the C ABI cannot see (CPU tensors: no call is made)."""
    import torch
    nb, k, T, ratio = 64, 8, 2, 4
    pool = torch.zeros((nb, 128), dtype=torch.float16)
    q = torch.zeros((T, 4, 128), dtype=torch.float32)
    bias = torch.zeros((T, nb), dtype=torch.float32)
    blk = torch.zeros(nb * ratio, dtype=torch.int32)
    cells = torch.zeros((T, k * ratio), dtype=torch.int32)
    bad = [dict(blk_cells=blk[: nb * ratio - 1]), dict(cells=cells[:, :-1].contiguous()),
           dict(q=q.transpose(1, 2).contiguous().transpose(1, 2)), dict(bias=bias.double()),
           dict(pool=pool[:, :64]), dict(top=torch.zeros((T, k - 1), dtype=torch.int32))]
    bad.append(dict(pool=pool.to(torch.bfloat16)))
    for kw in bad:
        args = dict(pool=pool, q=q, bias=bias, k_blocks=k, blk_cells=blk, ratio=ratio, cells=cells, stream=0)
        args.update(kw)
        with pytest.raises(ValueError, match="must be"):
            S.qsa_select_cells(**args)
    # well-shaped host tensors: the kernels would read host addresses, so the wrapper refuses them
    with pytest.raises(ValueError, match="GPU tensor"):
        S.qsa_select_cells(pool=pool, q=q, bias=bias, k_blocks=k, blk_cells=blk, ratio=ratio, cells=cells, stream=0)


# ---- the prefill chunk's sparse-attention inputs (fill_chunk_qsa, qsa_mask)

@pytest.mark.parametrize("n_past_c,Tc,ratio", [(0, 512, 4), (16384, 512, 4), (16385, 510, 4), (7, 1, 4), (0, 3, 4),
                                               (100, 37, 32), (5, 9, 1), (4093, 512, 4), (0, 1, 4), (31, 64, 32)])
def test_fill_chunk_qsa_closed_form(n_past_c, Tc, ratio):
    """The reference's procedural fills against the per-block closed form: a whole
    block that ends at or before the query scores on its merit (0), the block that
    holds the query mid-block and the partial tail block at or before it are forced
    (1e9), a block wholly after the query is pushed out (-1e9); no block is -inf
    since n_blocks = ceil(n_kv / ratio). The tables: every cell's block, each
    block's cells (the tail block's last real cell repeated), each block's first
    position in all four rope sections."""
    o = SO.fill_chunk_qsa(n_past_c, Tc, ratio)
    n_kv = n_past_c + Tc
    nb = -(-n_kv // ratio)
    assert o["n_blocks"] == nb
    np.testing.assert_array_equal(o["cell_blk"], np.arange(n_kv) // ratio)
    np.testing.assert_array_equal(o["blk_cells"], np.minimum(np.arange(nb * ratio), n_kv - 1))
    np.testing.assert_array_equal(o["blk_pos"], np.tile(np.arange(nb) * ratio, 4))
    b = np.arange(nb)
    start, last = b * ratio, np.minimum((b + 1) * ratio, n_kv) - 1
    whole = (b + 1) * ratio <= n_kv
    for i in range(Tc):
        q = n_past_c + i
        want = np.where(start > q, -1e9, np.where(whole & (last <= q), 0.0, 1e9)).astype(np.float32)
        np.testing.assert_array_equal(o["bias"][i], want, err_msg=f"row {i}")
        assert (o["bias"][i] == 1e9).sum() == (0 if (q + 1) % ratio == 0 and q + 1 <= (n_kv // ratio) * ratio else 1)


def _causal_bits(T, n_past, row_len):
    m = np.full((T, row_len), SO.F16_NEG_INF, np.uint16)
    for t in range(T):
        m[t, :n_past + t + 1] = SO.F16_ZERO
    return m


def test_qsa_mask_limits_and_zeros():
    """Every cell selected gives the causal mask; none gives -inf; otherwise the
    zeros are exactly the selected cells the query may see, repeats changing
    nothing; the padding past n_kv is -inf; a selected -0 becomes +0 (f16 add)."""
    rng = np.random.default_rng(3)
    T, n_past, row_len = 6, 290, 304
    n_kv = n_past + T
    causal = _causal_bits(T, n_past, row_len)
    every = np.tile(np.arange(n_kv, dtype=np.int32), (T, 1))
    got = SO.qsa_mask(every, causal, n_kv, row_len)
    np.testing.assert_array_equal(got[:, :n_kv], causal[:, :n_kv])
    assert (got[:, n_kv:] == SO.F16_NEG_INF).all()
    none = np.zeros((T, 0), np.int32)
    assert (SO.qsa_mask(none, causal, n_kv, row_len) == SO.F16_NEG_INF).all()
    cells = rng.integers(0, n_kv, (T, 120)).astype(np.int32)
    cells[:, 60:70] = cells[:, :10]                                  # repeats
    got = SO.qsa_mask(cells, causal, n_kv, row_len)
    for t in range(T):
        want = {int(c) for c in cells[t] if c <= n_past + t}
        assert set(np.flatnonzero(got[t] == SO.F16_ZERO).tolist()) == want
        assert (got[t][got[t] != SO.F16_ZERO] == SO.F16_NEG_INF).all()
    negz = causal.copy()
    negz[:, 5] = 0x8000
    got = SO.qsa_mask(every, negz, n_kv, row_len)
    assert (got[:, 5] == SO.F16_ZERO).all()


def test_visible_cells_closed_forms():
    """The keys a query sees: its distinct selected cells at or before its position,
    ascending (the position itself included, the one after it not); none for an empty
    selection; every key up to the position when every cell is selected."""
    np.testing.assert_array_equal(SO.visible_cells(np.array([5, 3, 3, 9, 8, 100]), 200, 8), [3, 5, 8])
    np.testing.assert_array_equal(SO.visible_cells(np.array([9]), 200, 8), np.zeros(0, np.int32))
    assert len(SO.visible_cells(np.zeros(0, np.int32), 50, 49)) == 0
    np.testing.assert_array_equal(SO.visible_cells(np.arange(40)[::-1], 40, 17), np.arange(18))
    rng = np.random.default_rng(9)
    for pos in (0, 77, 299):
        c = rng.integers(0, 300, 150)
        np.testing.assert_array_equal(SO.visible_cells(c, 300, pos), sorted({int(x) for x in c if x <= pos}))


def test_visible_cells_and_query_cells_dev_validation():
    """Host checks of the prefill-list entry points (nothing reaches a device)."""
    import ctypes
    L = K.load()
    buf = (ctypes.c_int32 * 64)()
    p = ctypes.addressof(buf)
    # NULL pointers, negative sizes, short rows, overlapping outputs
    assert L.qwfn_qsa_visible_cells(None, 4, 16, 10, 1, 0, p, 16, p + 128, None) == K.EINVAL
    assert L.qwfn_qsa_visible_cells(p, -1, 16, 10, 1, 0, p + 64, 16, p + 128, None) == K.EINVAL
    assert L.qwfn_qsa_visible_cells(p, 4, 12, 10, 1, 0, p + 64, 16, p + 128, None) == K.EINVAL
    assert L.qwfn_qsa_visible_cells(p, 4, 16, 10, 1, 0, p + 8, 16, p + 128, None) == K.EINVAL
    assert L.qwfn_qsa_visible_cells(p, 4, 16, 600000, 1, 0, p + 64, 16, p + 128, None) == K.ENOTSUP
    assert L.qwfn_flash_attn_ext_q8_0_query_cells_dev(None, None, None, None, None, 4, 0, 1.0, None, None, 1,
                                                      None) == K.EINVAL
