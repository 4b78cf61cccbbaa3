"""The verify step's per-position QSA inputs and index updates in one launch
each, bit for bit against the per-position calls they replace (engine::
attn_decode's T chained positions, qwfn_engine.cpp:2259-2280):

  qwfn_qsa_decode_prepare_steps(qd, T, n_past) ==
      qwfn_qsa_decode_prepare(qd[0], NULL, n_past); then qwfn_qsa_decode_prepare(qd[t], qd[t-1].bias, n_past + t)
  qwfn_qsa_pool_decode_steps(ic, k_raw, qd, T, ...) ==
      qwfn_qsa_pool_decode(ic, k_raw[t], qd[t] ...) for t = 0 .. T-1 in order

The per-position calls are pinned against the oracle elsewhere (test_gpu_state.py,
test_gpu_qsa_pool.py); the cases here cross block edges at several ratios, start
at a block's first and last cell, and run 1, 3 and 16 positions (several
positions of one block, each block pooled once, by its last position)."""
import numpy as np
import pytest
import torch

import qwfn_state as S
from gpu_util import dev, host, say

pytestmark = pytest.mark.gpu
DIM = 128


def _running_bias(nb, n_past, ratio, rng):
    """A running bias as the previous step left it, with a few arbitrary values so that
    rows copied from it are told apart from rows rebuilt."""
    qd = S.QsaDecodeInputs(ratio, nb)
    qd.rebuild_bias(n_past - 1)
    b = host(qd.bias).copy()
    pick = rng.choice(nb, 5, replace=False)
    b[pick] = rng.standard_normal(5).astype(np.float32)
    return b


@pytest.mark.parametrize("ratio,n_past,T", [(4, 73700, 3), (4, 73703, 3), (4, 73701, 16), (1, 500, 3), (16, 4095, 16),
                                            (32, 8190, 3), (4, 8, 1)])
def test_prepare_steps_matches_chained_prepares(gpu, ratio, n_past, T):
    rng = np.random.default_rng(n_past + T)
    nb = (n_past + T) // ratio + 40
    base = _running_bias(nb, n_past, ratio, rng)
    seq = [S.QsaDecodeInputs(ratio, nb) for _ in range(T)]
    bat = [S.QsaDecodeInputs(ratio, nb) for _ in range(T)]
    seq[0].bias.copy_(dev(base))
    bat[0].bias.copy_(dev(base))
    for t in range(1, T):                                        # later rows start as garbage
        seq[t].bias.fill_(7.0)
        bat[t].bias.fill_(-3.0)
    say(f"prepare x{T} at {n_past}, ratio {ratio}")
    for t in range(T):
        seq[t].prepare(n_past + t, prev=seq[t - 1] if t else None)
    S.qsa_decode_prepare_steps(bat, n_past)
    for t in range(T):
        for f in ("bias", "write_idx", "member_idx", "blk_pos", "blk_idx", "npast_f"):
            np.testing.assert_array_equal(host(getattr(bat[t], f)), host(getattr(seq[t], f)), err_msg=f"{f} at {t}")
        assert bat[t].n_bucket == seq[-1].n_bucket


@pytest.mark.parametrize("ratio,n_past,T", [(4, 73700, 3), (4, 73702, 3), (4, 73701, 16), (1, 500, 3), (16, 4095, 16),
                                            (32, 8190, 3)])
def test_pool_decode_steps_matches_chained_calls(gpu, ratio, n_past, T):
    K = gpu
    rng = np.random.default_rng(n_past * 3 + T)
    n_ctx = n_past + T + 64
    nb = n_ctx // ratio + 8
    ic = rng.standard_normal((n_ctx, DIM)).astype(np.float16)
    pool0 = (rng.standard_normal((nb, DIM)) * 0.3).astype(np.float16)
    w = rng.uniform(0.6, 1.4, DIM).astype(np.float32)
    k_raw = rng.standard_normal((T, DIM)).astype(np.float32)
    qds = [S.QsaDecodeInputs(ratio, nb) for _ in range(T)]
    S.qsa_decode_prepare_steps(qds, n_past)
    w_d, kr_d = dev(w), dev(k_raw)
    ic_s, pool_s = dev(ic), dev(pool0)
    say(f"pool decode x{T} one at a time at {n_past}, ratio {ratio}")
    for t in range(T):
        K.qsa_pool_decode(ic_s, kr_d[t], qds[t].write_idx, qds[t].member_idx, ratio, qds[t].blk_pos, qds[t].blk_idx,
                          w_d, pool_s)
    ic_b, pool_b = dev(ic), dev(pool0)
    say("pool decode, one launch")
    K.qsa_pool_decode_steps(ic_b, kr_d, qds, w_d, pool_b)
    assert K.device_status() == 0
    np.testing.assert_array_equal(host(ic_b).view(np.uint16), host(ic_s).view(np.uint16))
    np.testing.assert_array_equal(host(pool_b).view(np.uint16), host(pool_s).view(np.uint16))
    # strided key rows, and the pool-only form (no keys written) re-pools the same blocks
    wide = torch.zeros((T, 2 * DIM), dtype=torch.float32, device="cuda")
    wide[:, :DIM] = kr_d
    ic_w, pool_w = dev(ic), dev(pool0)
    K.qsa_pool_decode_steps(ic_w, wide[:, :DIM], qds, w_d, pool_w)
    np.testing.assert_array_equal(host(pool_w).view(np.uint16), host(pool_s).view(np.uint16))
    pool_n = dev(pool0)
    K.qsa_pool_decode_steps(ic_b, None, qds, w_d, pool_n)
    np.testing.assert_array_equal(host(pool_n).view(np.uint16), host(pool_s).view(np.uint16))


@pytest.mark.parametrize("ratio,n_past,T,dim,keys", [(4, 73700, 3, 128, True), (4, 73703, 3, 128, True),
                                                     (4, 73701, 16, 128, True), (1, 500, 3, 128, True),
                                                     (16, 4095, 16, 128, True), (32, 8190, 3, 128, False),
                                                     (128, 1000, 5, 128, True), (4, 4097, 3, 256, True),
                                                     (4, 0, 1, 128, True)])
def test_prepare_pool_steps_matches_separate_calls(gpu, ratio, n_past, T, dim, keys):
    """qwfn_qsa_decode_prepare_pool_steps == qwfn_qsa_decode_prepare_steps then
    qwfn_qsa_pool_decode_steps: bias rows, small inputs, index cache and pool, bit for bit
    (ratio 128: members past one wave's lanes; idx_dim 256; no keys)."""
    K = gpu
    rng = np.random.default_rng(n_past * 7 + T + dim)
    cfg = K.qsa_pool_cfg(idx_dim=dim)
    n_ctx = (n_past + T) // ratio * ratio + 2 * ratio + 64        # every member row of the step's blocks
    nb = n_ctx // ratio + 8
    base = _running_bias(nb, max(n_past, 1), ratio, rng)
    ic = rng.standard_normal((n_ctx, dim)).astype(np.float16)
    pool0 = (rng.standard_normal((nb, dim)) * 0.3).astype(np.float16)
    w = rng.uniform(0.6, 1.4, dim).astype(np.float32)
    kr_d = dev(rng.standard_normal((T, dim)).astype(np.float32)) if keys else None
    w_d = dev(w)
    sets = []
    for _ in range(2):
        qds = [S.QsaDecodeInputs(ratio, nb) for _ in range(T)]
        qds[0].bias.copy_(dev(base))
        for t in range(1, T):
            qds[t].bias.fill_(5.0)
        sets.append(qds)
    seq, fused = sets
    ic_s, pool_s = dev(ic), dev(pool0)
    say(f"prepare + pool x{T} at {n_past}, ratio {ratio}, dim {dim}: two launches")
    S.qsa_decode_prepare_steps(seq, n_past)
    K.qsa_pool_decode_steps(ic_s, kr_d, seq, w_d, pool_s, cfg=cfg)
    ic_f, pool_f = dev(ic), dev(pool0)
    say("one launch")
    S.qsa_decode_prepare_pool_steps(fused, n_past, ic_f, kr_d, w_d, pool_f, cfg=cfg)
    assert K.device_status() == 0
    for t in range(T):
        for f in ("bias", "write_idx", "member_idx", "blk_pos", "blk_idx", "npast_f"):
            np.testing.assert_array_equal(host(getattr(fused[t], f)), host(getattr(seq[t], f)), err_msg=f"{f} at {t}")
        assert fused[t].n_bucket == seq[t].n_bucket
    np.testing.assert_array_equal(host(ic_f).view(np.uint16), host(ic_s).view(np.uint16))
    np.testing.assert_array_equal(host(pool_f).view(np.uint16), host(pool_s).view(np.uint16))
    assert not np.array_equal(host(pool_f).view(np.uint16), pool0.view(np.uint16))
