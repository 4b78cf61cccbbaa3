"""GPU parity of the long-query-block attention kernel (k_fa_pre: more than 32
query rows per KV head with a mask shared by the heads or none, GQA >= 4)
against the oracle's ggml-cpu flash_attn_ext: the reference model's 24 heads
over a 512-token chunk, GQA 4 (a block's mask rows at their most), batches
without a mask, general masks (finite values, -inf holes, a fully masked
token) and split-count invariance. Tolerance: 2e-3 max / 1e-3 mean abs of
ggml-cpu semantics, 1e-4 max as observed."""
import numpy as np
import pytest

import kvdata as KD
from gpu_util import gpu_attn, say
from oracle import oracle as O

pytestmark = pytest.mark.gpu
TIGHT = 1e-4


def layer(seed, n_kv, nh_kv=2, outliers=False):
    kc = KD.make_cache(KD.kv_rows(seed, 0, KD.K_KIND, n_kv, n_head_kv=nh_kv, outliers=outliers), n_kv)
    vc = KD.make_cache(KD.kv_rows(seed, 0, KD.V_KIND, n_kv, n_head_kv=nh_kv, outliers=outliers), n_kv)
    return kc, vc


def check(got, ref, tight=TIGHT):
    mx, mean = KD.err_stats(got, ref)
    print(f"  max abs {mx:.3e}  mean abs {mean:.3e}", flush=True)
    assert np.isfinite(got).all()
    assert mx <= KD.MAX_ABS_TOL and mean <= KD.MEAN_ABS_TOL
    assert mx <= tight


def test_prefill_gqa12_chunk(gpu, oracle):
    """The reference model's shape: 24 heads over 2 KV heads, a 512-token chunk at depth 1000, causal."""
    K = gpu
    T, d0, nh = 512, 1000, 24
    kc, vc = layer(41, d0 + T, outliers=True)
    q = KD.q_rows(41, 0, T, nh)[0]
    mask = O.causal_mask(T, d0)
    say("k_fa_pre gqa 12 T=512 depth 1000")
    got = gpu_attn(K, q, kc, vc, d0 + T, 2, mask, 1 / 16)
    check(got, KD.oracle_attn(q, kc, vc, d0 + T, 2, mask, 1 / 16))


@pytest.mark.parametrize("variant", [O.Q8_REF, O.Q8_X86])
def test_prefill_gqa4_mask_rows(gpu, oracle, variant):
    """GQA 4 (8 heads over 2 KV heads): a block's 128 rows span 32 query positions."""
    K = gpu
    T, d0, nh = 100, 300, 8
    kc, vc = layer(42, d0 + T)
    q = KD.q_rows(42, 0, T, nh)[0]
    mask = O.causal_mask(T, d0)
    say(f"k_fa_pre gqa 4 T=100 variant {variant}")
    got = gpu_attn(K, q, kc, vc, d0 + T, 2, mask, 1 / 16, variant=variant)
    check(got, KD.oracle_attn(q, kc, vc, d0 + T, 2, mask, 1 / 16, variant=variant))


def test_prefill_batch_without_mask(gpu, oracle):
    """Two sequences of 40 queries over their own caches, no mask (every key visible)."""
    K = gpu
    T, n_kv, nh = 40, 2500, 16
    kcs, vcs = zip(*[layer(43 + s, n_kv) for s in range(2)])
    kc, vc = np.stack(kcs), np.stack(vcs)
    q = KD.q_rows(43, 0, T, nh, batch=2)
    say("k_fa_pre batch 2 T=40 no mask")
    got = gpu_attn(K, q, kc, vc, n_kv, 2, None, 1 / 16)
    for s in range(2):
        check(got[s], KD.oracle_attn(q[s], kcs[s], vcs[s], n_kv, 2, None, 1 / 16))


def test_prefill_general_mask(gpu, oracle):
    """A shared mask with finite values, -inf holes and a fully masked query position."""
    K = gpu
    T, n_kv, nh = 48, 1500, 16
    kc, vc = layer(45, n_kv)
    q = KD.q_rows(45, 0, T, nh)[0]
    rng = np.random.default_rng(45)
    m = rng.uniform(-6, 2, (T, n_kv)).astype(np.float16).view(np.uint16)
    m[:, ::7] = O.F16_NEG_INF
    m[:, 1000:1100] = O.F16_NEG_INF
    m[17, :] = O.F16_NEG_INF
    say("k_fa_pre general mask")
    got = gpu_attn(K, q, kc, vc, n_kv, 2, m, 1 / 16)
    check(got, KD.oracle_attn(q, kc, vc, n_kv, 2, m, 1 / 16))
    assert not got[17].any()


def test_prefill_odd_mask_rows(gpu, oracle):
    """An odd key count: the unpadded mask's rows start 2 bytes into a word on
    every other row (the kernel reads them as f16 pairs), and the split's last
    chunk holds a single key."""
    K = gpu
    T, n_kv, nh = 40, 1473, 16
    kc, vc = layer(47, n_kv)
    q = KD.q_rows(47, 0, T, nh)[0]
    rng = np.random.default_rng(47)
    m = rng.uniform(-5, 1, (T, n_kv)).astype(np.float16).view(np.uint16)
    m[:, 3::5] = O.F16_NEG_INF
    m[5, :] = O.F16_NEG_INF
    say("k_fa_pre odd mask rows n_kv=1473")
    got = gpu_attn(K, q, kc, vc, n_kv, 2, m, 1 / 16)
    check(got, KD.oracle_attn(q, kc, vc, n_kv, 2, m, 1 / 16))
    assert not got[5].any()


def test_prefill_split_invariance(gpu, oracle):
    """The same call with 1, 2, 5 and 13 key splits agrees with the oracle and across splits."""
    K = gpu
    T, d0, nh = 64, 3000, 16
    kc, vc = layer(46, d0 + T)
    q = KD.q_rows(46, 0, T, nh)[0]
    mask = O.causal_mask(T, d0)
    ref = KD.oracle_attn(q, kc, vc, d0 + T, 2, mask, 1 / 16)
    outs = []
    for ns in (1, 2, 5, 13):
        K.load().qwfn_fattn_force_splits(ns)
        try:
            say(f"k_fa_pre splits={ns}")
            outs.append(gpu_attn(K, q, kc, vc, d0 + T, 2, mask, 1 / 16, ws=(ns == 5)))
        finally:
            K.load().qwfn_fattn_force_splits(0)
        check(outs[-1], ref)
    for o in outs[1:]:
        assert KD.err_stats(o, outs[0])[0] < 2e-5
