"""GPU tests of the state rows through the C ABI: the state owner (layout,
initial zero, reset), MTP-verify rollback, session snapshots (device and host
blobs, part checks), and the device-built step inputs (causal and cell masks,
decode sparse-attention inputs) against the oracle restatement, bit-exact.
Mirrors the reference's snapshot check (tools/qwfn_snaptest.cpp:67-82): save,
run an unrelated sequence, load, and the state must be what was saved."""
import numpy as np
import pytest

import qwfn_kv as K
import qwfn_state as S
from gpu_util import dev, host, say
from oracle import state_oracle as SO

pytestmark = pytest.mark.gpu

GOLDEN_SUMMARY_73728 = ("state @ 73728 ctx: KV 0.962593 GB (q8_0), indexer 0.226492 GB, deltanet 113.246 MB "
                        "(constant), conv 4.79232 MB  =>  total 1.30712 GB on the device")


def small_cfg(n_ctx=1024, **kw):
    d = dict(n_layer=8, ssm_d_state=16, ssm_n_group=2, ssm_dt_rank=4, hc_count=2, n_embd=64, n_rollback=2)
    d.update(kw)
    return S.config(n_ctx, **d)


def new_state(cfg):
    st = S.State()
    ok, err = st.init(cfg, 0)
    assert ok, err
    return st


def read(addr, n):
    import torch
    buf = torch.empty(max(n, 1), dtype=torch.uint8, device="cuda")
    if n:
        K.state_restore([addr], [n], [buf.data_ptr()], 1)
    return host(buf)[:n]


def write(addr, data):
    t = dev(np.ascontiguousarray(data).view(np.uint8).ravel())
    K.state_restore([t.data_ptr()], [t.numel()], [addr], 1)
    host(t)   # synchronise before t is freed


def nbytes(t):
    return t.nb[3] * t.ne[3]


def all_tensors(st, cfg):
    out = []
    for il in range(cfg.n_layer):
        for k in (S.STATE_K, S.STATE_V, S.STATE_IDX, S.STATE_RS, S.STATE_CONV):
            t = st.tensor(k, il)
            if t is not None:
                out.append(((k, il), t))
    t = st.ple_conv()
    if t is not None:
        out.append(((S.STATE_PLE_CONV, 0), t))
    return out


def recurrent(key):
    return key[0] in (S.STATE_RS, S.STATE_CONV, S.STATE_PLE_CONV)


def scribble(st, cfg, rng):
    """Random bytes into every tensor; returns {key: bytes}."""
    data = {}
    for key, t in all_tensors(st, cfg):
        data[key] = rng.integers(0, 256, nbytes(t), dtype=np.uint8)
        write(t.data, data[key])
    return data


def test_full_model_state_layout_and_initial_zero(gpu):
    say("state: full model at 73728 positions, 2 rollback slots")
    cfg = S.config(73728, n_rollback=2)
    st = new_state(cfg)
    assert st.summary() == GOLDEN_SUMMARY_73728
    assert st.bytes() == 1307123712
    rec = [t for key, t in all_tensors(st, cfg) if recurrent(key)]
    lo = min(t.data for t in rec)
    hi = max(t.data + nbytes(t) for t in rec)
    assert hi - lo == sum(nbytes(t) for t in rec)          # one contiguous region
    assert st.rollback_bytes() == 2 * (hi - lo)
    assert not read(lo, hi - lo).any()                      # state::init zeroes it
    st.close()


def test_reset_zeroes_recurrent_only(gpu):
    rng = np.random.default_rng(1)
    cfg = small_cfg()
    st = new_state(cfg)
    data = scribble(st, cfg, rng)
    st.step_done(100)
    say("state: reset")
    st.reset()
    for key, t in all_tensors(st, cfg):
        got = read(t.data, nbytes(t))
        if recurrent(key):
            assert not got.any(), key
        else:
            np.testing.assert_array_equal(got, data[key])   # the caches are not cleared
    assert st.n_past() == 0 and st.rollback_depth() == 0


def test_rollback_restores_the_slot(gpu):
    rng = np.random.default_rng(2)
    cfg = small_cfg()
    st = new_state(cfg)
    scribble(st, cfg, rng)
    rec = [(key, t) for key, t in all_tensors(st, cfg) if recurrent(key)]
    slots = []
    for s in range(2):
        img = {}
        for key, t in rec:
            img[key] = rng.integers(0, 256, nbytes(t), dtype=np.uint8)
            write(st.rollback_slot(key[0], key[1], s).data, img[key])
        slots.append(img)
    st.step_done(40)
    st.step_done(3, verified=True)
    assert st.rollback_depth() == 2 and st.n_past() == 43
    say("state: rollback 2")
    ok, err = st.rollback_n(2)
    assert ok, err
    for key, t in rec:
        np.testing.assert_array_equal(read(t.data, nbytes(t)), slots[1][key])
    assert st.n_past() == 41 and st.rollback_depth() == 0
    ok, err = st.rollback_n(1)
    assert not ok and err == "rollback: no snapshot of the state 1 tokens back"
    st.step_done(3, verified=True)
    say("state: rollback 1")
    assert st.rollback_n(1)[0]
    for key, t in rec:
        np.testing.assert_array_equal(read(t.data, nbytes(t)), slots[0][key])
    assert st.n_past() == 43


@pytest.mark.parametrize("where", ["device", "pinned", "pageable"])
def test_snapshot_save_unrelated_load(gpu, where):
    import torch
    rng = np.random.default_rng(3)
    cfg = small_cfg()
    head_cfg = small_cfg(n_layer=4, full_attention_interval=4, ple_n_head=0, n_rollback=0)
    trunk, head = new_state(cfg), new_state(head_cfg)
    states = [trunk, head]
    saved = [scribble(trunk, cfg, rng), scribble(head, head_cfg, rng)]
    n_past = 777
    for s in states:
        s.step_done(n_past)
    say(f"snapshot: save ({where})")
    snap = S.snapshot_save(states, S.MEM_DEVICE if where == "device" else S.MEM_HOST)
    if where == "pageable":
        snap = S.Snapshot(snap.n_past, [b.cpu().clone() for b in snap.blobs])
        assert not snap.blobs[0].is_pinned()
    want = SO.snapshot_parts([{**SO.config_default(1024), **_cfg_dict(cfg)},
                              {**SO.config_default(1024), **_cfg_dict(head_cfg)}], n_past)
    assert snap.n_past == n_past and [b.numel() for b in snap.blobs] == [p[3] for p in want]
    # an unrelated sequence in between
    scribble(trunk, cfg, rng)
    scribble(head, head_cfg, rng)
    for s in states:
        s.step_done(5)
    say(f"snapshot: load ({where})")
    ok, err = S.snapshot_load(states, snap)
    assert ok, err
    torch.cuda.synchronize()
    for s, c, sv in ((trunk, cfg, saved[0]), (head, head_cfg, saved[1])):
        assert s.n_past() == n_past
        for key, t in all_tensors(s, c):
            n = nbytes(t) if recurrent(key) else min(nbytes(t), n_past * (t.nb[1] // cfg.n_ctx))
            np.testing.assert_array_equal(read(t.data, n), sv[key][:n], err_msg=str(key))


def _cfg_dict(c):
    return {f: getattr(c, f) for f, _ in K.StateConfig._fields_}


def test_snapshot_mismatch_is_rejected_after_reset(gpu):
    rng = np.random.default_rng(4)
    cfg = small_cfg()
    st = new_state(cfg)
    scribble(st, cfg, rng)
    st.step_done(64)
    snap = S.snapshot_save([st], S.MEM_DEVICE)
    short = S.Snapshot(snap.n_past, snap.blobs[:-1])
    say("snapshot: part count mismatch")
    ok, err = S.snapshot_load([st], short)
    assert not ok and "parts given" in err
    assert st.n_past() == 0
    for key, t in all_tensors(st, cfg):
        if recurrent(key):
            assert not read(t.data, nbytes(t)).any()        # reset before the check, as the reference
    bad = S.Snapshot(snap.n_past + 1, snap.blobs)            # positional parts one row short
    ok, err = S.snapshot_load([st], bad)
    assert not ok and "expected" in err
    ok, err = S.snapshot_load([st], snap)
    assert ok and st.n_past() == 64


def test_host_resident_caches_snapshot(gpu):
    rng = np.random.default_rng(5)
    cfg = small_cfg(n_ctx=512, kv_host=1, idx_host=1)
    st = new_state(cfg)
    assert st.host_bytes() > 0 and "pinned host memory" in st.summary()
    data = scribble(st, cfg, rng)
    st.step_done(300)
    say("snapshot: host-resident caches")
    snap = S.snapshot_save([st], S.MEM_DEVICE)
    scribble(st, cfg, rng)
    assert S.snapshot_load([st], snap)[0]
    for key, t in all_tensors(st, cfg):
        n = nbytes(t) if recurrent(key) else min(nbytes(t), 300 * (t.nb[1] // 512))
        np.testing.assert_array_equal(read(t.data, n), data[key][:n], err_msg=str(key))


def test_state_caches_feed_attention(gpu):
    """The state's K/V caches are the reference's views: appending into them and
    attending over them gives the bytes and outputs of a separately held cache."""
    import torch
    import kvdata as KD
    from gpu_util import gpu_attn
    cfg = S.config(2048)
    st = new_state(cfg)
    il = 3
    kt, vt = st.k_cache(il), st.v_cache(il)
    n = 700
    krows = KD.kv_rows(7, il, KD.K_KIND, n)
    vrows = KD.kv_rows(7, il, KD.V_KIND, n)
    idx = dev(np.arange(n, dtype=np.int32))
    rb = 544
    say("state: set_rows into the state's caches, then attention")
    import ctypes
    iv = K.tensor(idx.data_ptr(), K.TYPE_I32, (n,), (4,))
    for t, rows in ((kt, krows), (vt, vrows)):
        dst = K.tensor(t.data, K.TYPE_Q8_0, (512, 2048), (34, rb))
        src = dev(rows)
        K.check(K.load().qwfn_set_rows_q8_0(ctypes.byref(dst), ctypes.byref(K.f32_view(src)), ctypes.byref(iv),
                                            K.Q8_X86, K._stream(None)))
        host(src)
    kc = read(kt.data, n * rb).reshape(n, rb)
    vc = read(vt.data, n * rb).reshape(n, rb)
    from oracle import oracle as O
    ref_k = np.zeros((n, rb), np.uint8)
    ref_v = np.zeros((n, rb), np.uint8)
    O.set_rows(ref_k, krows, np.arange(n, dtype=np.int32))
    O.set_rows(ref_v, vrows, np.arange(n, dtype=np.int32))
    np.testing.assert_array_equal(kc, ref_k)
    np.testing.assert_array_equal(vc, ref_v)
    q = KD.q_rows(7, il, 3, 16)[0]
    mask = SO.attn_inputs_mask(n - 3, 3)
    out = torch.empty((1, 3, 16, 256), dtype=torch.float32, device="cuda")
    qd = dev(q[None].astype(np.float32))
    md = dev(mask.view(np.float16))
    kv = K.tensor(kt.data, K.TYPE_Q8_0, (256, n, 2, 1), (34, rb, 272, n * rb))
    vv = K.tensor(vt.data, K.TYPE_Q8_0, (256, n, 2, 1), (34, rb, 272, n * rb))
    K.flash_attn_ext(K.q_view(qd), kv, vv, K.mask_view(md), 1 / 16, K.out_view(out), K.Q8_X86)
    got = host(out)[0]
    np.testing.assert_array_equal(got, gpu_attn(K, q, kc, vc, n, 2, mask, 1 / 16))
    del torch


@pytest.mark.parametrize("n_kv,T,n_past,row", [(19, 3, 16, 19), (1027, 5, 1022, 1088), (4608, 512, 4096, 4608),
                                               (16387, 3, 16384, 16387), (8, 1, 7, 8), (40, 2, 0, 64),
                                               (8, 65540, 0, 8)])
def test_causal_mask_matches_oracle(gpu, n_kv, T, n_past, row):
    import torch
    m = torch.full((T, row), 0x1234, dtype=torch.int16, device="cuda")
    say(f"causal mask n_kv={n_kv} T={T} n_past={n_past} row={row}")
    K.check(K.load().qwfn_causal_mask_f16(m.data_ptr(), n_kv, T, n_past, row * 2, K._stream(None)))
    got = host(m).view(np.uint16)
    want = np.full((T, row), SO.F16_NEG_INF, np.uint16)
    vis = np.arange(row)[None, :] <= (n_past + np.arange(T))[:, None]
    want[(vis) & (np.arange(row)[None, :] < n_kv)] = SO.F16_ZERO
    if n_kv == n_past + T:
        np.testing.assert_array_equal(want[:, :n_kv], SO.attn_inputs_mask(n_past, T))
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("n_cells,n_pad,n_past", [(2052, 2304, 65535), (2052, 2304, 100), (256, 256, 0), (5, 9, 3)])
def test_cell_mask_matches_oracle(gpu, n_cells, n_pad, n_past):
    import torch
    rng = np.random.default_rng(n_cells + n_past)
    cells = np.sort(rng.choice(max(n_past + 50, n_cells + 10), n_cells, replace=False)).astype(np.int32)
    cd = dev(cells)
    m = torch.full((n_pad,), 0x1234, dtype=torch.int16, device="cuda")
    g = torch.full((n_pad,), -7, dtype=torch.int32, device="cuda")
    say(f"cell mask n_cells={n_cells} n_pad={n_pad} n_past={n_past}")
    S.cell_mask_f16(cd, n_past, n_pad, m, g)
    want_m, want_g = SO.cell_mask(cells, n_past, n_pad)
    np.testing.assert_array_equal(host(m).view(np.uint16), want_m)
    np.testing.assert_array_equal(host(g), want_g)


def test_qsa_decode_inputs_match_oracle(gpu):
    ratio, nb_max = 4, 64
    qd = S.QsaDecodeInputs(ratio, nb_max)
    qk = S.QsaDecodeInputs(ratio, nb_max)
    bias = SO.qsa_reset_bias(nb_max)
    say("qsa decode inputs: positions 0..259")
    for n in range(0, 260):
        qd.prepare(n)
        o = SO.qsa_decode_prepare(bias, n, ratio)
        for f in ("write_idx", "member_idx", "blk_pos", "blk_idx", "npast_f", "bias"):
            np.testing.assert_array_equal(host(getattr(qd, f)), o[f], err_msg=f"{f} at {n}")
        qk.prepare(n + 1, prev=qd)
        ok_ = SO.qsa_decode_prepare_k(bias, n + 1, ratio)
        for f in ("write_idx", "member_idx", "blk_pos", "blk_idx", "npast_f", "bias"):
            np.testing.assert_array_equal(host(getattr(qk, f)), ok_[f], err_msg=f"k {f} at {n}")
        assert qk.n_bucket == qd.n_bucket == max(SO.qsa_bucket(n, ratio, nb_max), SO.qsa_bucket(n + 1, ratio, nb_max))
    for n in (-1, 0, 3, 4, 100, 255, 256, 10 ** 5):
        qd.rebuild_bias(n)
        want = SO.qsa_reset_bias(nb_max) if n < 0 else SO.qsa_pool_rebuild_bias(nb_max, n, ratio)
        np.testing.assert_array_equal(host(qd.bias), want, err_msg=str(n))


def test_qsa_tables_match_oracle(gpu):
    import torch
    ratio, nb_max, n_ctx, n_whole = 4, 300, 1200, 77
    bc = torch.full((nb_max * ratio,), -1, dtype=torch.int32, device="cuda")
    cp = torch.full((n_ctx,), -1.0, dtype=torch.float32, device="cuda")
    bp = torch.full((4 * n_whole,), -1, dtype=torch.int32, device="cuda")
    say("qsa tables")
    S.qsa_tables(bc, ratio, cp, bp, n_whole)
    w_bc, w_cp, w_bp = SO.qsa_tables(nb_max, ratio, n_ctx, n_whole)
    np.testing.assert_array_equal(host(bc), w_bc)
    np.testing.assert_array_equal(host(cp), w_cp)
    np.testing.assert_array_equal(host(bp), w_bp)


# ------------------------------------------------------- saved-sequence pool

def _pool_pair(n_ctx=4096):
    cfg = small_cfg(n_ctx=n_ctx, n_rollback=0)
    head_cfg = small_cfg(n_ctx=n_ctx, n_layer=4, ple_n_head=0, n_rollback=0)
    return [new_state(cfg), new_state(head_cfg)], [cfg, head_cfg]


def _fill(states, cfgs, n_past, rng):
    for s in states:
        s.reset()
        s.step_done(n_past)
    return [scribble(s, c, rng) for s, c in zip(states, cfgs)]


def _check(states, cfgs, data, n_past, what):
    for s, c, sv in zip(states, cfgs, data):
        assert s.n_past() == n_past
        for key, t in all_tensors(s, c):
            n = nbytes(t) if recurrent(key) else min(nbytes(t), n_past * (t.nb[1] // c.n_ctx))
            np.testing.assert_array_equal(read(t.data, n), sv[key][:n], err_msg=f"{what} {key}")


def test_pool_keeps_snapshots_across_compaction(gpu):
    """Four saved sequences; replacing one by a longer snapshot leaves no gap
    large enough, so the pool compacts into its other half. Every saved
    sequence then restores byte for byte."""
    rng = np.random.default_rng(21)
    states, cfgs = _pool_pair()
    size = lambda n: sum(b for _, b in S.snapshot_parts(states, n))
    # 4 x size(1000) fit; after replacing one by size(1500) the free tail is too small
    cap = 3 * size(1000) + size(1500) + 4096
    pool = S.SnapPool(cap, 4, 0)
    seqs = {name: [i] * 1000 for i, name in enumerate("abcd")}
    saved = {}
    for name, tok in seqs.items():
        saved[name] = (_fill(states, cfgs, 1000, rng), 1000)
        say(f"pool: save {name}")
        assert pool.save_seq(states, tok)
    b2 = [1] * 1000                                           # b's tokens, a longer state
    saved["b"] = (_fill(states, cfgs, 1500, rng), 1500)
    say("pool: replace b (compaction)")
    assert pool.save_seq(states, b2)
    assert [pool.entry(k)[0][0] for k in range(4)] == [0, 2, 3, 1]
    scribble(states[0], cfgs[0], rng)
    for k in range(4):
        name = "abcd"[pool.entry(0)[0][0]]
        say(f"pool: load {name}")
        ok, err = pool.load(0, states)
        assert ok, err
        _check(states, cfgs, saved[name][0], saved[name][1], name)


def test_pool_restore_or_reset_round_trip(gpu):
    """The server's flow: a long conversation is set aside when a side request
    arrives, and restored when the conversation continues."""
    rng = np.random.default_rng(22)
    states, cfgs = _pool_pair()
    pool = S.SnapPool(64 << 20, 4, 0)
    conv = [int(x) for x in rng.integers(0, 1000, 3000)]
    data = _fill(states, cfgs, 3000, rng)
    say("pool: set aside, reset for a side request")
    assert pool.restore_or_reset(states, conv, [5, 6, 7]) == 0
    assert states[0].n_past() == 0 and pool.count() == 1
    for key, t in all_tensors(states[0], cfgs[0]):
        if recurrent(key):
            assert not read(t.data, nbytes(t)).any()
    side = [int(x) for x in rng.integers(0, 1000, 100)]
    _fill(states, cfgs, 100, rng)
    say("pool: restore the conversation")
    assert pool.restore_or_reset(states, side, conv + [1, 2]) == 3000
    _check(states, cfgs, data, 3000, "restored")


# ------------------------------------------------- sparse block selection

def _select(pool, q, bias, k, blk_cells, ratio):
    import torch
    T = q.shape[0]
    pd = dev(pool.view(np.uint16))
    qd, bd, cd = dev(q.astype(np.float32)), dev(bias.astype(np.float32)), dev(blk_cells.astype(np.int32))
    cells = torch.full((T, k * ratio), -1, dtype=torch.int32, device="cuda")
    top = torch.full((T, k), -1, dtype=torch.int32, device="cuda")
    S.qsa_select_cells(pd, qd, bd, k, cd, ratio, cells, top)
    return host(cells), host(top)


def _bias(nb, n_past, ratio):
    return SO.qsa_pool_rebuild_bias(nb, n_past, ratio)


def _exact_top(scores, k):
    """The k best blocks of one query's f32 scores: score descending, ties to
    the lower block (stable sort of the negated scores)."""
    return np.argsort(-scores.astype(np.float64), kind="stable")[:k].astype(np.int32)


@pytest.mark.parametrize("case", ["random", "all_equal", "few_values", "mostly_masked", "k1024", "just_above_2048",
                                  "two_tied_bins", "ties_in_candidates", "small", "kpt12", "kpt32", "kpt40", "rising",
                                  "t1", "t16", "t17"])
def test_qsa_topk_exact_on_device_scores(gpu, case):
    """The selection alone, bit for bit: the kernel's own scores are read back
    from the workspace and the expected blocks are an exact sort of them. The
    cases reach both the fast path (a threshold from a sample of the scores,
    or none at 1024 blocks or fewer, then one sort of the keys above it) and
    the full select it falls back to: all scores tied, a few distinct values,
    most blocks masked, k above 768, ties around the k-th place, every kept
    block in the last part of the pool ("rising"), and 1, 16 and 17 queries
    in one call."""
    import torch
    rng = np.random.default_rng(sum(map(ord, case)))
    nb, k, T, ratio = 18432, 513, 3, 4
    pool = (rng.standard_normal((nb, 128)) * 0.5).astype(np.float16)
    q = rng.standard_normal((T, 4, 128)).astype(np.float32)
    bias = np.zeros((T, nb), np.float32)
    if case == "all_equal":
        pool[:] = 0
    elif case == "few_values":
        pool[:] = 0
        pool[:, 0] = rng.integers(0, 6, nb) / 4.0
        q[:] = 0
        q[:, 0, 0] = 1.0
    elif case == "mostly_masked":
        bias[:, 3000:] = -np.inf
    elif case == "k1024":
        k = 1024
    elif case == "just_above_2048":
        nb = 2049
        pool, bias = pool[:nb], bias[:, :nb]
    elif case == "ties_in_candidates":
        # about 9 blocks per distinct score: ties at the k-th place among the candidates
        pool[:] = 0
        pool[:, 0] = rng.integers(0, 2048, nb) / 64.0
        q[:] = 0
        q[:, 0, 0] = 1.0
    elif case == "small":
        nb, k = 1000, 100
        pool, bias = pool[:nb], bias[:, :nb]
    elif case in ("kpt12", "kpt32", "kpt40"):
        # 12 and 32 scores a thread take the sampled path, 40 the full select
        nb = {"kpt12": 10000, "kpt32": 30000, "kpt40": 36000}[case]
        pool = (rng.standard_normal((nb, 128)) * 0.5).astype(np.float16)
        bias = np.zeros((T, nb), np.float32)
    elif case == "rising":
        pool[:] = 0
        pool[:, 0] = (np.arange(nb) / nb).astype(np.float16)
        q[:] = 0
        q[:, 0, 0] = 1.0
    elif case in ("t1", "t16", "t17"):
        T = int(case[1:])
        q = rng.standard_normal((T, 4, 128)).astype(np.float32)
        bias = np.zeros((T, nb), np.float32)
    elif case == "two_tied_bins":
        # every score one of two values, the better one held by exactly k - 1 blocks
        pool[:] = 0
        pool[:, 0] = 0.25
        pool[rng.choice(nb, k - 1, replace=False), 0] = 0.5
        q[:] = 0
        q[:, 0, 0] = 1.0
    blk_cells, _, _ = SO.qsa_tables(nb, ratio, 1, 0)
    pd = dev(pool.view(np.uint16))
    qd, bd, cd = dev(q), dev(bias), dev(blk_cells.astype(np.int32))
    cells = torch.full((T, k * ratio), -1, dtype=torch.int32, device="cuda")
    top = torch.full((T, k), -1, dtype=torch.int32, device="cuda")
    ws = torch.zeros(K.load().qwfn_qsa_select_workspace_size(nb, T), dtype=torch.uint8, device="cuda")
    say(f"qsa top-k exact: {case} nb={nb} k={k}")
    S.qsa_select_cells(pd, qd, bd, k, cd, ratio, cells, top, ws=ws)
    ld = (nb + 63) // 64 * 64
    # the workspace holds the scores, the bias added there for up to 8 queries
    # (one pass over the pool) and by the top-k for more (one f32 addition)
    sc = host(ws).view(np.float32)[:T * ld].reshape(T, ld)[:, :nb]
    if T > 8:
        sc = sc + bias
    got = host(top)
    for t in range(T):
        np.testing.assert_array_equal(got[t], _exact_top(sc[t], k))
    np.testing.assert_array_equal(host(cells), np.stack([SO.qsa_cells(got[t], blk_cells, ratio) for t in range(T)]))


def test_qsa_select_closed_forms(gpu):
    rng = np.random.default_rng(70)
    nb, ratio, k = 768, 4, 513
    blk_cells, _, _ = SO.qsa_tables(nb, ratio, 1, 0)
    pool = rng.standard_normal((nb, 128)).astype(np.float16)
    # a zero query: every relu term is 0, the score is the bias: the incomplete
    # block of n_past (1e9) first, then the whole blocks lowest first
    n_past = 4 * 600 + 1
    b = _bias(nb, n_past, ratio)
    say("qsa select: zero query")
    cells, top = _select(pool, np.zeros((1, 4, 128), np.float32), b[None], k, blk_cells, ratio)
    assert top[0][0] == 600 and list(top[0][1:]) == list(range(512))
    assert list(cells[0][:4]) == [2400, 2401, 2402, 2403]
    # planted scores: block j's key is j * e0 and the query e0: score j, best first
    pool2 = np.zeros((nb, 128), np.float16)
    pool2[:, 0] = np.arange(nb) / 64.0
    q2 = np.zeros((2, 4, 128), np.float32)
    q2[:, 0, 0] = 1.0
    say("qsa select: planted scores, two queries")
    _, top2 = _select(pool2, q2, np.zeros((2, nb), np.float32), k, blk_cells, ratio)
    assert list(top2[0]) == list(range(nb - 1, nb - 1 - k, -1)) and list(top2[1]) == list(top2[0])
    # relu: a query opposite to every key scores 0 everywhere, blocks in order
    say("qsa select: relu")
    _, top3 = _select(pool2, -q2[:1], np.zeros((1, nb), np.float32), 5, blk_cells, ratio)
    assert list(top3[0]) == [0, 1, 2, 3, 4]


@pytest.mark.parametrize("nb,k,T,n_past,H", [(768, 513, 1, 3000, 4), (18432, 513, 3, 73000, 4), (4096, 1, 2, 9000, 4),
                                             (1024, 1024, 1, 4095, 4), (777, 776, 1, 3100, 1), (1000, 100, 9, 3000, 3),
                                             (5000, 300, 2, 19000, 8), (4100, 64, 12, 16000, 2),
                                             # scores per thread 12, 16, 24, 32, 40, 48
                                             (10000, 200, 1, 40000, 4), (16000, 513, 2, 64000, 4),
                                             (24000, 513, 1, 96000, 4), (30000, 513, 1, 120000, 4),
                                             (36000, 700, 1, 144000, 4), (45000, 1000, 1, 180000, 4)])
def test_qsa_select_matches_oracle(gpu, nb, k, T, n_past, H):
    rng = np.random.default_rng(nb + k)
    ratio = 4
    blk_cells, _, _ = SO.qsa_tables(nb, ratio, 1, 0)
    pool = (rng.standard_normal((nb, 128)) * 0.5).astype(np.float16)
    q = rng.standard_normal((T, H, 128)).astype(np.float32)
    bias = np.stack([_bias(nb, n_past + t, ratio) for t in range(T)])
    say(f"qsa select nb={nb} k={k} T={T} heads={H}")
    cells, top = _select(pool, q, bias, k, blk_cells, ratio)
    for t in range(T):
        sc = SO.qsa_scores(pool, q[t], bias[t])
        want = SO.qsa_top_k(sc, k)
        got = top[t]
        # the same blocks, best first, except where scores tie within float
        # rounding at the k-th place (a sum of 512 f32 products)
        kth = sc[want[-1]]
        tol = 1e-5 * max(1.0, abs(kth)) if np.isfinite(kth) else 0.0
        sure = set(int(b) for b in want if sc[b] > kth + tol)
        assert sure <= set(int(b) for b in got)
        assert all(sc[b] >= kth - tol for b in got)
        assert len(set(got.tolist())) == k
        assert np.all(np.diff(sc[got]) <= tol + 1e-12 * np.abs(sc[got][1:]))   # best first
        np.testing.assert_array_equal(cells[t], SO.qsa_cells(got, blk_cells, ratio))
