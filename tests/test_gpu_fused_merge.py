"""The key-split merge inside k_fa_dec, k_fa_vd and k_fa_vs, through the C ABI.

A call with several key splits either merges them in the attention kernel
itself (the last blocks of each (batch, KV head) group to finish claim its
rows) or launches k_fattn_merge; qwfn_fattn_force_merge picks the path and
qwfn_fattn_last_merge reports it. Each case runs both paths on the same
inputs: both are held to the oracle's ggml-cpu flash_attn_ext (2e-3 max /
1e-3 mean abs, 1e-4 max in practice) and to each other (they differ only in
the order of the float sums). The planner's default is the merge launch
(faster on this GPU); the in-kernel merge runs when forced. Further cases:
repeated calls give identical
bits (every call takes new counter slots and a new epoch), grids several
times larger than the GPU's 256 CUs (blocks of a group that are not yet
resident when its first mergers arrive), batches of several sequences (one
counter group per sequence and KV head), and gathered cells."""
import numpy as np
import pytest
import torch

import kvdata as KD
import qwfn_kv as KK
from gpu_util import dev, host, say
from oracle import oracle as O

pytestmark = pytest.mark.gpu
HD = 256
TIGHT = 1e-4


def check(got, ref):
    mx, mean = KD.err_stats(got, ref)
    print(f"  max abs {mx:.3e}  mean abs {mean:.3e}", flush=True)
    assert np.isfinite(got).all()
    assert mx <= KD.MAX_ABS_TOL and mean <= KD.MEAN_ABS_TOL
    assert mx <= TIGHT


def layer(seed, n_kv):
    kc = KD.make_cache(KD.kv_rows(seed, 0, KD.K_KIND, n_kv, outliers=True), n_kv)
    vc = KD.make_cache(KD.kv_rows(seed, 0, KD.V_KIND, n_kv, outliers=True), n_kv)
    return kc, vc


class forced:
    """Kernel family, split count and merge path for the calls inside the block."""
    def __init__(self, kind=KK.FA_KERNEL_AUTO, splits=0, merge=KK.FA_MERGE_AUTO):
        self.kind, self.splits, self.merge = kind, splits, merge

    def __enter__(self):
        L = KK.load()
        L.qwfn_fattn_force_kernel(self.kind)
        L.qwfn_fattn_force_splits(self.splits)
        L.qwfn_fattn_force_merge(self.merge)

    def __exit__(self, *e):
        L = KK.load()
        L.qwfn_fattn_force_kernel(KK.FA_KERNEL_AUTO)
        L.qwfn_fattn_force_splits(0)
        L.qwfn_fattn_force_merge(KK.FA_MERGE_AUTO)
        return False


def run(K, q, kd, vd, n_kv, md):
    """q [B, T, nh, HD] numpy; kd/vd device caches shared by the batch; md device mask or None."""
    qd = dev(q.astype(np.float32))
    out = torch.full(q.shape, float("nan"), dtype=torch.float32, device="cuda")
    K.flash_attn_ext(K.q_view(qd), K.cache_attn_view(kd, n_kv, 2), K.cache_attn_view(vd, n_kv, 2),
                     K.mask_view(md) if md is not None else None, 1 / 16, K.out_view(out))
    return host(out), K.last_kernel(), K.last_merge()


FAMILIES = {"vd": KK.FA_KERNEL_VD, "vs": KK.FA_KERNEL_VS, "dec": KK.FA_KERNEL_DEC}


@pytest.mark.parametrize("fam,n_past,T,causal", [
    ("dec", 16384, 3, True), ("vd", 16384, 3, True),
    ("dec", 4096, 1, False), ("vd", 4096, 1, False),
    ("dec", 3000, 2, True), ("vd", 3000, 2, True),
    ("vs", 16384, 3, True), ("vs", 4096, 1, False), ("vs", 3000, 2, True),
])
def test_fused_merge_matches_kernel_merge(gpu, oracle, fam, n_past, T, causal):
    K = gpu
    nh, n_kv = 16, n_past + T
    kc, vc = layer(201, n_kv)
    q = KD.q_rows(201, 0, T, nh)[0]
    mask = O.causal_mask(T, n_past) if causal else None
    kd, vd = dev(kc), dev(vc)
    md = dev(mask.view(np.float16)) if mask is not None else None
    ref = KD.oracle_attn(q, kc, vc, n_kv, 2, mask, 1 / 16)
    outs = {}
    for mode in (KK.FA_MERGE_FUSED, KK.FA_MERGE_KERNEL):
        say(f"merge {mode} {fam} n_past={n_past} T={T}")
        with forced(FAMILIES[fam], merge=mode):
            got, name, how = run(K, q[None], kd, vd, n_kv, md)
        assert name.startswith(f"k_fa_{fam}<")
        assert how == mode
        check(got[0], ref)
        outs[mode] = got
    np.testing.assert_allclose(outs[KK.FA_MERGE_FUSED], outs[KK.FA_MERGE_KERNEL], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("fam", ["dec", "vd", "vs"])
def test_fused_merge_repeats_bit_identical(gpu, oracle, fam):
    K = gpu
    nh, T, n_past = 16, 3, 8192
    n_kv = n_past + T
    kc, vc = layer(202, n_kv)
    q = KD.q_rows(202, 0, T, nh)[0]
    mask = O.causal_mask(T, n_past)
    kd, vd = dev(kc), dev(vc)
    md = dev(mask.view(np.float16))
    runs = []
    for i in range(4):
        say(f"repeat {i} {fam}")
        with forced(FAMILIES[fam], merge=KK.FA_MERGE_FUSED):
            got, _, how = run(K, q[None], kd, vd, n_kv, md)
        assert how == KK.FA_MERGE_FUSED
        runs.append(got)
    check(runs[0][0], KD.oracle_attn(q, kc, vc, n_kv, 2, mask, 1 / 16))
    for r in runs[1:]:
        np.testing.assert_array_equal(r, runs[0])


def test_fused_merge_grid_beyond_the_gpu(gpu, oracle):
    """k_fa_dec with a forced 512 splits at depth 16384 (48-key splits, 342 per KV
    head): a grid of 688 blocks, more than twice the CUs, so many of a group's
    splits start only after its first mergers have arrived."""
    K = gpu
    nh, T, n_past = 16, 3, 16384
    n_kv = n_past + T
    kc, vc = layer(203, n_kv)
    q = KD.q_rows(203, 0, T, nh)[0]
    mask = O.causal_mask(T, n_past)
    kd, vd = dev(kc), dev(vc)
    md = dev(mask.view(np.float16))
    ref = KD.oracle_attn(q, kc, vc, n_kv, 2, mask, 1 / 16)
    for mode in (KK.FA_MERGE_FUSED, KK.FA_MERGE_KERNEL):
        say(f"big grid merge {mode}")
        with forced(KK.FA_KERNEL_DEC, splits=512, merge=mode):
            got, name, how = run(K, q[None], kd, vd, n_kv, md)
        assert how == mode
        check(got[0], ref)


@pytest.mark.parametrize("fam", ["dec", "vd", "vs"])
def test_fused_merge_batch_of_sequences(gpu, oracle, fam):
    """Four query sequences over one cache (B = 4, the cache broadcast): eight merge
    groups in one launch."""
    K = gpu
    nh, T, n_past, B = 16, 1, 6000, 4
    n_kv = n_past + T
    kc, vc = layer(204, n_kv)
    q = np.stack([KD.q_rows(204, b, T, nh)[0] for b in range(B)])
    kd, vd = dev(kc), dev(vc)
    for mode in (KK.FA_MERGE_FUSED, KK.FA_MERGE_KERNEL):
        say(f"batch {B} {fam} merge {mode}")
        with forced(FAMILIES[fam], merge=mode):
            got, _, how = run(K, q, kd, vd, n_kv, None)
        assert how == mode
        for b in range(B):
            check(got[b], KD.oracle_attn(q[b], kc, vc, n_kv, 2, None, 1 / 16))


def test_fused_merge_cells(gpu, oracle):
    """Gathered cells (k_fa_dec<.., GATHER>): 2052 cells shared by both KV heads, the
    reference's decode shape, and per-head lists of different lengths."""
    K = gpu
    nh, T, n_rows = 16, 3, 20000
    kc, vc = layer(205, n_rows)
    rng = np.random.default_rng(205)
    pos0 = n_rows - T
    shared = np.sort(rng.choice(pos0, 2052 - T, replace=False)).astype(np.int32)
    shared = np.concatenate([shared, np.arange(pos0, n_rows, dtype=np.int32)])
    lists = [shared, np.sort(rng.choice(n_rows, 900, replace=False)).astype(np.int32)]
    q = KD.q_rows(205, 0, T, nh)[0]
    kd, vd = dev(kc), dev(vc)
    for lst in (lists, [shared, shared]):
        n = [len(x) for x in lst]
        stride = (max(n) + 3) // 4 * 4
        c = np.zeros((2, stride), np.int32)
        for h, x in enumerate(lst):
            c[h, :len(x)] = x
        ref = KD.oracle_attn_cells(q, kc, vc, lst, pos0, 1 / 16)
        outs = {}
        for mode in (KK.FA_MERGE_FUSED, KK.FA_MERGE_KERNEL):
            say(f"cells {n} merge {mode}")
            kv = K.tensor(kd.data_ptr(), K.TYPE_Q8_0, (HD, n_rows, 2, 1), (34, 544, 272, n_rows * 544))
            vv = K.tensor(vd.data_ptr(), K.TYPE_Q8_0, (HD, n_rows, 2, 1), (34, 544, 272, n_rows * 544))
            qd = dev(q[None].astype(np.float32))
            out = torch.full((1, T, nh, HD), float("nan"), dtype=torch.float32, device="cuda")
            with forced(merge=mode):
                K.flash_attn_ext_cells(K.q_view(qd), kv, vv, dev(c), n, pos0, 1 / 16, K.out_view(out))
                assert K.last_merge() == mode
            assert K.device_status() == 0
            outs[mode] = host(out)[0]
            check(outs[mode], ref)
        np.testing.assert_allclose(outs[KK.FA_MERGE_FUSED], outs[KK.FA_MERGE_KERNEL], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("fam", ["dec", "vd", "vs"])
def test_fused_merge_alternating_calls(gpu, oracle, fam):
    """Calls on the library's workspace that alternate between two layers (other
    queries, other caches): each call's mergers must read that call's partials,
    never a copy of the previous call's at the same addresses."""
    K = gpu
    nh, T, n_past = 16, 3, 8192
    n_kv = n_past + T
    mask = O.causal_mask(T, n_past)
    md = dev(mask.view(np.float16))
    cases = []
    for seed in (206, 207):
        kc, vc = layer(seed, n_kv)
        q = KD.q_rows(seed, 0, T, nh)[0]
        cases.append((q, dev(kc), dev(vc), KD.oracle_attn(q, kc, vc, n_kv, 2, mask, 1 / 16)))
    first = [None, None]
    for i in range(6):
        q, kd, vd, ref = cases[i % 2]
        say(f"alternating call {i} {fam}")
        with forced(FAMILIES[fam], merge=KK.FA_MERGE_FUSED):
            got, _, how = run(K, q[None], kd, vd, n_kv, md)
        assert how == KK.FA_MERGE_FUSED
        if first[i % 2] is None:
            check(got[0], ref)
            first[i % 2] = got
        else:
            np.testing.assert_array_equal(got, first[i % 2])


def test_merge_launch_is_the_default(gpu):
    K = gpu
    nh, T, n_past = 16, 3, 4096
    n_kv = n_past + T
    kc, vc = layer(208, n_kv)
    q = KD.q_rows(208, 0, T, nh)[0]
    _, _, how = run(K, q[None], dev(kc), dev(vc), n_kv, None)
    assert how == KK.FA_MERGE_KERNEL
