"""GPU parity of sparse decode attention with the gather fused in
(qwfn_flash_attn_ext_q8_0_cells) against the oracle's attention over the
gathered copy with its cell mask (qwfn_graph.cpp:632-699): the full-size
selection (per-KV-head lists of 8576 and 8640 cells of a 65536-row cache, 3
queries), the reference's one shared list, multi-split lists of different
lengths per head, and the edge cases: an empty list, repeated and unsorted
cells, cells outside the cache (masked and flagged), a query that sees no
cell. Tolerance: 2e-3 max / 1e-3 mean abs of ggml-cpu semantics, 1e-4 max
as observed."""
import numpy as np
import pytest
import torch

import kvdata as KD
from gpu_util import dev, host, say
from oracle import oracle as O

pytestmark = pytest.mark.gpu
TIGHT = 1e-4


def check(got, ref, tight=TIGHT):
    mx, mean = KD.err_stats(got, ref)
    print(f"  max abs {mx:.3e}  mean abs {mean:.3e}", flush=True)
    assert np.isfinite(got).all()
    assert mx <= KD.MAX_ABS_TOL and mean <= KD.MEAN_ABS_TOL
    assert mx <= tight


def cells_attn(K, q, kd, vd, n_rows, lists, pos0, stride=None, variant=1, ws=False, shared=False):
    """q [T, nh, 256] numpy; kd/vd device caches uint8 [n_ctx, 544]; returns (out, device flags)."""
    T, nh, hd = q.shape
    nh_kv = len(lists)
    n = [len(x) for x in lists]
    if shared:
        stride = 0
        cells = dev(np.asarray(lists[0], np.int32)[None])
    else:
        stride = stride or max(4, (max(n) + 3) // 4 * 4)
        c = np.full((nh_kv, stride), -7, np.int32)
        for h, x in enumerate(lists):
            c[h, :len(x)] = x
        cells = dev(c)
    rb = kd.shape[1]
    kv = K.tensor(kd.data_ptr(), K.TYPE_Q8_0, (hd, n_rows, nh_kv, 1), (34, rb, hd // 32 * 34, n_rows * rb))
    vv = K.tensor(vd.data_ptr(), K.TYPE_Q8_0, (hd, n_rows, nh_kv, 1), (34, rb, hd // 32 * 34, n_rows * rb))
    qd = dev(q[None].astype(np.float32))
    out = torch.full((1, T, nh, hd), float("nan"), dtype=torch.float32, device="cuda")
    wst = None
    if ws:
        nb = K.fattn_workspace_size_cells(K.q_view(qd), kv, vv, n, stride)
        assert nb >= 256
        wst = torch.empty(nb, dtype=torch.uint8, device="cuda")
    K.flash_attn_ext_cells(K.q_view(qd), kv, vv, cells, n, pos0, 1 / 16, K.out_view(out), variant, ws=wst,
                           shared=shared)
    flags = K.device_status()
    return host(out)[0], flags


def test_cells_full_size_selection(gpu, oracle):
    """64K cache, the per-head top-128 blocks of 64 plus the last 512 positions, 3 queries at 65533-65535."""
    K = gpu
    n_ctx, T, nh = 65536, 3, 16
    lists = KD.selection_lists(4, n_ctx)
    assert [len(x) for x in lists] == [8576, 8640]
    kc = KD.make_cache(KD.kv_rows(4, 0, KD.K_KIND, n_ctx), n_ctx)
    vc = KD.make_cache(KD.kv_rows(4, 0, KD.V_KIND, n_ctx), n_ctx)
    q = KD.q_rows(4, 1, T, nh)[0]
    kd, vd = dev(kc), dev(vc)
    say("cells attention: 8576 / 8640 cells of 65536, T=3")
    got, flags = cells_attn(K, q, kd, vd, n_ctx, lists, n_ctx - T, ws=True)
    assert flags == 0
    check(got, KD.oracle_attn_cells(q, kc, vc, lists, n_ctx - T, 1 / 16))
    say("cells attention: library workspace, same bits")
    got2, _ = cells_attn(K, q, kd, vd, n_ctx, lists, n_ctx - T)
    np.testing.assert_array_equal(got2, got)


def test_cells_shared_list(gpu, oracle):
    """The reference's form: one list of 2052 cells for both KV heads (2 of them past the query), T = 1."""
    K = gpu
    n_ctx, T, nh = 8192, 1, 16
    u = O.uniform(O.stream_key(9, 0, KD.SCORE_KIND, 0), n_ctx)
    sel = np.sort(np.argsort(u, kind="stable")[:2050]).astype(np.int32)
    pos0 = 6000
    lst = np.concatenate([sel[sel <= pos0], [pos0 + 5, pos0 + 9], sel[sel > pos0]])[:2052].astype(np.int32)
    kc = KD.make_cache(KD.kv_rows(9, 0, KD.K_KIND, n_ctx, outliers=True), n_ctx)
    vc = KD.make_cache(KD.kv_rows(9, 0, KD.V_KIND, n_ctx, outliers=True), n_ctx)
    q = KD.q_rows(9, 1, T, nh)[0]
    kd, vd = dev(kc), dev(vc)
    say("cells attention: one shared list of 2052 cells, T=1")
    got, flags = cells_attn(K, q, kd, vd, n_ctx, [lst, lst], pos0, shared=True)
    assert flags == 0
    check(got, KD.oracle_attn_cells(q, kc, vc, [lst, lst], pos0, 1 / 16))


@pytest.mark.parametrize("variant", [0, 1])
def test_cells_multi_split_ragged_heads(gpu, oracle, variant):
    """1500 and 37 cells (several 512-cell splits for one head, one partial tile for the other), T = 2."""
    K = gpu
    n_ctx, T, nh = 4096, 2, 16
    l0 = np.sort(np.argsort(O.uniform(O.stream_key(11, 0, KD.SCORE_KIND, 0), n_ctx), kind="stable")[:1500])
    l1 = np.sort(np.argsort(O.uniform(O.stream_key(11, 0, KD.SCORE_KIND, 1), n_ctx), kind="stable")[:37])
    lists = [l0.astype(np.int32), l1.astype(np.int32)]
    kc = KD.make_cache(KD.kv_rows(11, 0, KD.K_KIND, n_ctx), n_ctx, variant)
    vc = KD.make_cache(KD.kv_rows(11, 0, KD.V_KIND, n_ctx), n_ctx, variant)
    q = KD.q_rows(11, 1, T, nh)[0]
    kd, vd = dev(kc), dev(vc)
    say(f"cells attention: 1500 / 37 cells, T=2, variant {variant}")
    got, flags = cells_attn(K, q, kd, vd, n_ctx, lists, n_ctx - T, variant=variant)
    assert flags == 0
    check(got, KD.oracle_attn_cells(q, kc, vc, lists, n_ctx - T, 1 / 16, variant))


def test_cells_edge_cases(gpu, oracle):
    """Head 0: no cells. Head 1: unsorted, repeated cells, two outside the cache
    (masked, flag raised) and cells that only the second query sees."""
    K = gpu
    n_ctx, T, nh = 1024, 2, 16
    pos0 = 700
    rng = np.random.default_rng(5)
    base = rng.permutation(pos0 + 1)[:300].astype(np.int32)
    l1 = np.concatenate([base, base[:20], [n_ctx + 3, -1], [pos0 + 1] * 3]).astype(np.int32)
    rng.shuffle(l1)
    lists = [np.zeros(0, np.int32), l1]
    kc = KD.make_cache(KD.kv_rows(12, 0, KD.K_KIND, n_ctx), n_ctx)
    vc = KD.make_cache(KD.kv_rows(12, 0, KD.V_KIND, n_ctx), n_ctx)
    q = KD.q_rows(12, 1, T, nh)[0]
    kd, vd = dev(kc), dev(vc)
    say("cells attention: empty list, repeats, cells outside the cache")
    got, flags = cells_attn(K, q, kd, vd, n_ctx, lists, pos0)
    assert flags & 2, flags
    assert (got[:, :8] == 0).all()
    check(got, KD.oracle_attn_cells(q, kc, vc, lists, pos0, 1 / 16))
    say("cells attention: a query that sees no cell")
    late = [np.array([pos0 + 1, pos0 + 1], np.int32), np.array([pos0 + 1], np.int32)]
    got, flags = cells_attn(K, q, kd, vd, n_ctx, late, pos0)
    assert flags == 0
    assert (got[0] == 0).all()
    check(got, KD.oracle_attn_cells(q, kc, vc, late, pos0, 1 / 16))


def test_cells_matches_gather_then_attention(gpu, oracle):
    """The fused call against the separate path it replaces: gather the cells'
    halves, then masked attention over the gathered copy (within float rounding)."""
    K = gpu
    n_ctx, T, nh, seg = 16384, 3, 16, KD.SEG
    lists = KD.selection_lists(6, n_ctx, blocks=256, bsz=64, top=32, tail=512)
    kc = KD.make_cache(KD.kv_rows(6, 0, KD.K_KIND, n_ctx), n_ctx)
    vc = KD.make_cache(KD.kv_rows(6, 0, KD.V_KIND, n_ctx), n_ctx)
    q = KD.q_rows(6, 1, T, nh)[0]
    kd, vd = dev(kc), dev(vc)
    say("cells attention vs gather + masked attention at 16384")
    fused, _ = cells_attn(K, q, kd, vd, n_ctx, lists, n_ctx - T)
    m = ((max(len(x) for x in lists) + 255) // 256) * 256
    idx = np.stack([np.concatenate([x, np.repeat(x[-1:], m - len(x))]) for x in lists]).astype(np.int32)
    gk = torch.zeros((2, m, seg), dtype=torch.uint8, device="cuda")
    gv = torch.zeros((2, m, seg), dtype=torch.uint8, device="cuda")
    idd = dev(idx)
    K.gather_segments(kd, idd, gk, 0, seg, seg)
    K.gather_segments(vd, idd, gv, 0, seg, seg)
    qpos = np.arange(n_ctx - T, n_ctx)
    mask = np.full((1, nh, T, m), O.F16_NEG_INF, np.uint16)
    for h in range(nh):
        lst = lists[h // 8]
        for t in range(T):
            mask[0, h, t, :len(lst)][lst <= qpos[t]] = 0
    kview = K.tensor(gk.data_ptr(), K.TYPE_Q8_0, (256, m, 2, 1), (34, seg, m * seg, 2 * m * seg))
    vview = K.tensor(gv.data_ptr(), K.TYPE_Q8_0, (256, m, 2, 1), (34, seg, m * seg, 2 * m * seg))
    qd, md = dev(q[None].astype(np.float32)), dev(mask.view(np.float16))
    out = torch.full((1, T, nh, 256), float("nan"), dtype=torch.float32, device="cuda")
    K.flash_attn_ext(K.q_view(qd), kview, vview, K.mask_view(md), 1 / 16, K.out_view(out))
    sep = host(out)[0]
    check(fused, sep, tight=2e-5)


def query_cells_attn(K, q, kd, vd, n_rows, lists, pos0, gate=None, ws=False):
    """One list per query position (qwfn_flash_attn_ext_q8_0_query_cells); lists: T arrays,
    or one array that every position reads."""
    T, nh, hd = q.shape
    n = [len(x) for x in lists]
    stride = max(4, (max(n) + 3) // 4 * 4)
    c = np.full((len(lists), stride), -7, np.int32)
    for t, x in enumerate(lists):
        c[t, :len(x)] = x
    rb = kd.shape[1]
    kv = K.tensor(kd.data_ptr(), K.TYPE_Q8_0, (hd, n_rows, 2, 1), (34, rb, hd // 32 * 34, n_rows * rb))
    vv = K.tensor(vd.data_ptr(), K.TYPE_Q8_0, (hd, n_rows, 2, 1), (34, rb, hd // 32 * 34, n_rows * rb))
    qd = dev(q[None].astype(np.float32))
    out = torch.full((1, T, nh, hd), float("nan"), dtype=torch.float32, device="cuda")
    wst = None
    if ws:
        nb = K.fattn_workspace_size_query_cells(K.q_view(qd), kv, vv, n if len(lists) == T else n * T,
                                                0 if len(lists) == 1 else stride)
        assert nb >= 256
        wst = torch.empty(nb, dtype=torch.uint8, device="cuda")
    cnt = n if len(lists) == T else n * T
    K.flash_attn_ext_query_cells(K.q_view(qd), kv, vv, dev(c), cnt, pos0, 1 / 16, K.out_view(out),
                                 gate=dev(gate[None]) if gate is not None else None, ws=wst)
    flags = K.device_status()
    return host(out)[0], flags


def _query_lists(seed, n_rows, pos0, T, n_cells):
    """T lists in the reference's shape: the top blocks of 4 cells of position pos0 + t (a
    random ranking that changes a little from one position to the next), the block of
    pos0 + t among them."""
    rng = np.random.default_rng(seed)
    nb = (pos0 + T + 3) // 4
    base = rng.permutation(nb)
    lists = []
    for t in range(T):
        order = base.copy()
        swap = rng.choice(nb, 40, replace=False)
        order[swap] = order[rng.permutation(swap)]
        own = (pos0 + t) // 4
        top = [own] + [b for b in order if b != own][:n_cells // 4 - 1]
        lists.append((np.asarray(top, np.int64)[:, None] * 4 + np.arange(4)).reshape(-1).astype(np.int32))
    return lists


@pytest.mark.parametrize("gated", [False, True])
def test_query_cells_reference_shape(gpu, oracle, gated):
    """The reference's verify step: T = 3 positions, each with its own 2052 cells (513
    blocks of 4, its own block among them, cells past it masked), in one launch."""
    K = gpu
    n_rows, T, nh = 20000, 3, 16
    pos0 = n_rows - 8
    lists = _query_lists(11, n_rows, pos0, T, 2052)
    kc = KD.make_cache(KD.kv_rows(11, 0, KD.K_KIND, n_rows, outliers=True), n_rows)
    vc = KD.make_cache(KD.kv_rows(11, 0, KD.V_KIND, n_rows, outliers=True), n_rows)
    q = KD.q_rows(11, 1, T, nh)[0]
    gate = (np.random.default_rng(12).standard_normal((T, nh, 256)) * 3).astype(np.float32) if gated else None
    kd, vd = dev(kc), dev(vc)
    say(f"query cells T=3 x 2052 gated={gated}")
    got, flags = query_cells_attn(K, q, kd, vd, n_rows, lists, pos0, gate=gate, ws=True)
    assert flags == 0
    ref = np.stack([KD.oracle_attn_cells(q[t:t + 1], kc, vc, [lists[t], lists[t]], pos0 + t, 1 / 16)[0]
                    for t in range(T)])
    if gated:
        ref = ref * (1.0 / (1.0 + np.exp(-gate.astype(np.float64)))).astype(np.float32)
    check(got, ref)


def test_query_cells_agree_with_the_shared_list_forms(gpu, oracle):
    """One position: identical bits to the shared-list cells call. Three positions reading
    one list (cell_stride 0): the shared-list cells call to float rounding."""
    K = gpu
    n_rows, nh = 9000, 16
    pos0 = 8990
    lst = _query_lists(13, n_rows, pos0, 1, 2052)[0]
    kc = KD.make_cache(KD.kv_rows(13, 0, KD.K_KIND, n_rows, outliers=True), n_rows)
    vc = KD.make_cache(KD.kv_rows(13, 0, KD.V_KIND, n_rows, outliers=True), n_rows)
    kd, vd = dev(kc), dev(vc)
    q1 = KD.q_rows(13, 1, 1, nh)[0]
    say("query cells T=1 against the cells call")
    a, _ = query_cells_attn(K, q1, kd, vd, n_rows, [lst], pos0)
    b, _ = cells_attn(K, q1, kd, vd, n_rows, [lst, lst], pos0, shared=True)
    np.testing.assert_array_equal(a, b)
    q3 = KD.q_rows(13, 2, 3, nh)[0]
    say("query cells T=3, one list for every position")
    a3, _ = query_cells_attn(K, q3, kd, vd, n_rows, [lst], pos0)
    b3, _ = cells_attn(K, q3, kd, vd, n_rows, [lst, lst], pos0, shared=True)
    np.testing.assert_allclose(a3, b3, rtol=1e-5, atol=1e-6)
    check(a3, KD.oracle_attn_cells(q3, kc, vc, [lst, lst], pos0, 1 / 16))


def test_query_cells_edges(gpu, oracle):
    """Lists of different lengths (one empty: its query gets 0), repeats, unsorted cells,
    a cell outside the cache (masked, flagged), and a split count that differs per list."""
    K = gpu
    n_rows, T, nh = 5000, 4, 16
    pos0 = 4000
    rng = np.random.default_rng(14)
    lists = [rng.choice(pos0, 1500, replace=False).astype(np.int32),
             np.array([], np.int32),
             np.concatenate([rng.choice(n_rows, 37), [3, 3, 3]]).astype(np.int32),
             np.concatenate([rng.choice(pos0, 700, replace=False), [n_rows + 5]]).astype(np.int32)]
    kc = KD.make_cache(KD.kv_rows(14, 0, KD.K_KIND, n_rows), n_rows)
    vc = KD.make_cache(KD.kv_rows(14, 0, KD.V_KIND, n_rows), n_rows)
    q = KD.q_rows(14, 1, T, nh)[0]
    kd, vd = dev(kc), dev(vc)
    say("query cells edges")
    got, flags = query_cells_attn(K, q, kd, vd, n_rows, lists, pos0)
    assert flags & 2
    ref = np.stack([KD.oracle_attn_cells(q[t:t + 1], kc, vc, [lists[t], lists[t]], pos0 + t, 1 / 16)[0]
                    for t in range(T)])
    assert not got[1].any()
    check(got, ref)


def query_cells_dev_attn(K, q, kd, vd, n_rows, lists, pos0, gate=None, counts=None, stride=None):
    """qwfn_flash_attn_ext_q8_0_query_cells_dev: list t for position t, the counts on the
    device (default: the list lengths); returns (out, device flags)."""
    T, nh, hd = q.shape
    n = [len(x) for x in lists]
    stride = stride or max(4, (max(n) + 3) // 4 * 4)
    c = np.full((T, stride), -7, np.int32)
    for t, x in enumerate(lists):
        c[t, :len(x)] = x[:stride]
    cnt = np.asarray(n if counts is None else counts, np.int32)
    rb = kd.shape[1]
    kv = K.tensor(kd.data_ptr(), K.TYPE_Q8_0, (hd, n_rows, 2, 1), (34, rb, hd // 32 * 34, n_rows * rb))
    vv = K.tensor(vd.data_ptr(), K.TYPE_Q8_0, (hd, n_rows, 2, 1), (34, rb, hd // 32 * 34, n_rows * rb))
    qd = dev(q[None].astype(np.float32))
    out = torch.full((1, T, nh, hd), float("nan"), dtype=torch.float32, device="cuda")
    K.flash_attn_ext_query_cells_dev(K.q_view(qd), kv, vv, dev(c), dev(cnt), pos0, 1 / 16, K.out_view(out),
                                     gate=dev(gate[None]) if gate is not None else None)
    flags = K.device_status()
    return host(out)[0], flags


def _oracle_per_position(q, kc, vc, lists, pos0):
    return np.stack([KD.oracle_attn_cells(q[t:t + 1], kc, vc, [lists[t], lists[t]], pos0 + t, 1 / 16)[0]
                     for t in range(q.shape[0])])


@pytest.mark.parametrize("T,n_cells", [(37, 2052), (256, 516), (512, 260)])
def test_query_cells_dev_many_positions(gpu, oracle, T, n_cells):
    """Many positions, each over its own list in the reference's shape (blocks of 4, the
    position's own block among them, cells past it masked), the counts on the device: 2, 4
    and 8 waves a list (512, 256 and 37 positions over 2 KV heads)."""
    K = gpu
    n_rows, nh = 6000, 16
    pos0 = n_rows - T - 3
    lists = _query_lists(20 + T, n_rows, pos0, T, n_cells)
    kc = KD.make_cache(KD.kv_rows(20 + T, 0, KD.K_KIND, n_rows, outliers=True), n_rows)
    vc = KD.make_cache(KD.kv_rows(20 + T, 0, KD.V_KIND, n_rows, outliers=True), n_rows)
    q = KD.q_rows(20 + T, 1, T, nh)[0]
    kd, vd = dev(kc), dev(vc)
    say(f"query cells (device counts) T={T} x {n_cells}")
    got, flags = query_cells_dev_attn(K, q, kd, vd, n_rows, lists, pos0)
    assert flags == 0
    check(got, _oracle_per_position(q, kc, vc, lists, pos0))


@pytest.mark.parametrize("nh", [8, 16, 32])
def test_query_cells_dev_edges(gpu, oracle, nh):
    """Head groups of 4, 8 and 16 rows; lists of different lengths (one empty: its query
    gets 0; one whose length is not a multiple of 16), repeats, unsorted cells, cells past
    the position, a cell outside the cache (masked, flagged), a count above the row stride
    (clipped, flagged), and the gate."""
    K = gpu
    n_rows, T = 3000, 9
    pos0 = 2500
    rng = np.random.default_rng(30 + nh)
    lists = [rng.choice(pos0, 700, replace=False).astype(np.int32),
             np.array([], np.int32),
             np.concatenate([rng.choice(n_rows, 37), [3, 3, 3]]).astype(np.int32),
             np.concatenate([rng.choice(pos0, 300, replace=False), [n_rows + 5]]).astype(np.int32),
             rng.choice(n_rows, 17).astype(np.int32),
             np.arange(pos0, pos0 + 9, dtype=np.int32),
             rng.choice(pos0, 1, replace=False).astype(np.int32),
             rng.choice(pos0 + 8, 64, replace=False).astype(np.int32),
             rng.choice(pos0, 650, replace=False).astype(np.int32)]
    stride = 704
    counts = [len(x) for x in lists]
    counts[8] = stride + 40                                       # past the row: clipped to the stride
    kc = KD.make_cache(KD.kv_rows(30 + nh, 0, KD.K_KIND, n_rows), n_rows)
    vc = KD.make_cache(KD.kv_rows(30 + nh, 0, KD.V_KIND, n_rows), n_rows)
    q = KD.q_rows(30 + nh, 1, T, nh)[0]
    gate = (rng.standard_normal((T, nh, 256)) * 3).astype(np.float32)
    kd, vd = dev(kc), dev(vc)
    say(f"query cells (device counts) edges nh={nh}")
    got, flags = query_cells_dev_attn(K, q, kd, vd, n_rows, lists, pos0, gate=gate, counts=counts, stride=stride)
    assert flags & 2
    ref_lists = [x[:stride] for x in lists]
    ref = _oracle_per_position(q, kc, vc, ref_lists, pos0)
    ref = ref * (1.0 / (1.0 + np.exp(-gate.astype(np.float64)))).astype(np.float32)
    assert not got[1].any()
    check(got, ref)
    say("the same without the out-of-range cell and count: no flag")
    lists[3] = lists[3][:-1]
    counts = [min(len(x), stride) for x in lists]
    got2, flags2 = query_cells_dev_attn(K, q, kd, vd, n_rows, lists, pos0, counts=counts, stride=stride)
    assert flags2 == 0
    check(got2, _oracle_per_position(q, kc, vc, [x[:stride] for x in lists], pos0))


def test_query_cells_dev_agrees_with_query_cells(gpu, oracle):
    """Three positions of the reference's verify shape: the device-count call and the
    host-count call (k_fa_dec with key splits) agree to float rounding."""
    K = gpu
    n_rows, T, nh = 20000, 3, 16
    pos0 = n_rows - 8
    lists = _query_lists(41, n_rows, pos0, T, 2052)
    kc = KD.make_cache(KD.kv_rows(41, 0, KD.K_KIND, n_rows, outliers=True), n_rows)
    vc = KD.make_cache(KD.kv_rows(41, 0, KD.V_KIND, n_rows, outliers=True), n_rows)
    q = KD.q_rows(41, 1, T, nh)[0]
    kd, vd = dev(kc), dev(vc)
    say("query cells: device counts against host counts")
    a, _ = query_cells_dev_attn(K, q, kd, vd, n_rows, lists, pos0)
    b, _ = query_cells_attn(K, q, kd, vd, n_rows, lists, pos0)
    np.testing.assert_allclose(a, b, rtol=1e-5, atol=2e-6)
