"""GPU parity of the QSA index producer against the oracle: the F16 set_rows
(bit-exact IEEE conversion), the pool rebuild after a prefill (every whole
block's mean-pooled, RMS-normed, IMROPE-roped key; qwfn_graph.cpp:478-495 and
:282-301) and the decode step's raw key plus its block's pooled key
(:529-554), chained over a verify window that crosses a block edge. Pooled
keys are compared as F16 bits; the device's cos / sin (fp64 rounded to f32)
and the oracle's libm cosf / sinf may differ in the last float bit, so a key
value may differ by one F16 unit in the last place at a rounding boundary --
the tests allow that on at most 0.1% of the values and require the rest to
be identical."""
import numpy as np
import pytest
import torch

from gpu_util import dev, host, say
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DIM = 128


def _ulp_check(got_bits, ref_bits):
    g = got_bits.astype(np.int32)
    r = ref_bits.astype(np.int32)
    diff = np.abs(g - r)
    n_diff = int((diff != 0).sum())
    print(f"  differing f16 values: {n_diff} of {diff.size}, max {int(diff.max())} ulp", flush=True)
    assert diff.max() <= 1
    assert n_diff <= max(1, diff.size // 1000)


def test_set_rows_f16_bit_exact(gpu, oracle):
    K = gpu
    rng = np.random.default_rng(1)
    src = (rng.standard_normal((9, 192)) * np.exp(rng.uniform(-22, 12, (9, 192)))).astype(np.float32)
    src[0, :5] = [65520.0, -65519.0, 5.9604645e-08, 2.9802322e-08, -0.0]
    idx = np.array([4, 0, 31, 7, 8, 15, 16, 2, 30], np.int32)
    dst = torch.zeros((32, 192), dtype=torch.float16, device="cuda")
    say("set_rows_f16 9 rows of 192")
    K.set_rows_f16(dst, dev(src), dev(idx))
    ref = np.zeros((32, 192), np.uint16)
    O.set_rows_f16(ref, src, idx)
    np.testing.assert_array_equal(host(dst).view(np.uint16), ref)
    assert K.device_status() == 0
    say("set_rows_f16 out-of-range index")
    K.set_rows_f16(dst, dev(src[:2]), dev(np.array([3, 32], np.int32)))
    assert K.device_status() & 1


def _weights(seed):
    return np.random.default_rng(seed).uniform(0.6, 1.4, DIM).astype(np.float32)


@pytest.mark.parametrize("n_past,ratio", [(16424, 32), (5000, 4), (31, 32), (97, 1)])
def test_pool_rebuild_matches_oracle(gpu, oracle, n_past, ratio):
    K = gpu
    rng = np.random.default_rng(n_past)
    rows = n_past + 50
    ic = (rng.standard_normal((rows, DIM)) * 2).astype(np.float16)
    w = _weights(ratio)
    n_whole = n_past // ratio
    nb_max = n_whole + 17
    pool = torch.zeros((nb_max, DIM), dtype=torch.float16, device="cuda")
    say(f"pool rebuild n_past={n_past} ratio={ratio}")
    K.qsa_pool_rebuild(dev(ic), n_past, ratio, dev(w), pool)
    got = host(pool).view(np.uint16)
    assert K.device_status() == 0
    assert not got[n_whole:].any()
    if n_whole == 0:
        return
    members = np.arange(n_whole * ratio, dtype=np.int32)
    pos4 = np.repeat((np.arange(n_whole) * ratio)[:, None], 4, axis=1).astype(np.int32)
    ref = O.qsa_pool_blocks(ic.view(np.uint16), members, ratio, w, pos4)
    _ulp_check(got[:n_whole], ref)


@pytest.mark.parametrize("dim,n_dims", [(96, 64), (256, 128), (64, 48)])
def test_pool_rebuild_other_dims(gpu, oracle, dim, n_dims):
    """Index keys of other lengths: 96 takes the one-block-per-wave kernel (96 / 8
    is not a power of two), 256 and 64 the 16-byte-lane kernel with 2 and 8
    blocks a wave (64 with a rotated part that is not a whole lane's 8 dims)."""
    K = gpu
    rng = np.random.default_rng(dim)
    n_past, ratio = 4099, 4
    ic = (rng.standard_normal((n_past + 5, dim)) * 2).astype(np.float16)
    w = rng.uniform(0.6, 1.4, dim).astype(np.float32)
    n_whole = n_past // ratio
    pool = torch.zeros((n_whole + 3, dim), dtype=torch.float16, device="cuda")
    cfg = K.qsa_pool_cfg(idx_dim=dim, n_dims=n_dims)
    say(f"pool rebuild dim={dim} n_dims={n_dims}")
    K.qsa_pool_rebuild(dev(ic), n_past, ratio, dev(w), pool, cfg=cfg)
    got = host(pool).view(np.uint16)
    assert K.device_status() == 0
    assert not got[n_whole:].any()
    members = np.arange(n_whole * ratio, dtype=np.int32)
    pos4 = np.repeat((np.arange(n_whole) * ratio)[:, None], 4, axis=1).astype(np.int32)
    ref = O.qsa_pool_blocks(ic.view(np.uint16), members, ratio, w, pos4, n_dims=n_dims)
    _ulp_check(got[:n_whole], ref)


def test_pool_decode_chain_across_a_block_edge(gpu, oracle):
    """Three chained positions 8190, 8191, 8192 (ratio 32): the raw key of each
    goes to its row, its block's key is re-pooled (the first two block 255,
    the third block 256); a final rebuild agrees with the chain's blocks."""
    K = gpu
    from qwfn_state import QsaDecodeInputs
    rng = np.random.default_rng(7)
    ratio, n_ctx, nb_max = 32, 8192 + 64, 512
    ic = (rng.standard_normal((n_ctx, DIM))).astype(np.float16)
    ic_d = dev(ic)
    pool = torch.zeros((nb_max, DIM), dtype=torch.float16, device="cuda")
    w = _weights(3)
    w_d = dev(w)
    ref_ic = ic.view(np.uint16).copy()
    ref_pool = np.zeros((nb_max, DIM), np.uint16)
    qd = QsaDecodeInputs(ratio, nb_max)
    for n_past in (8190, 8191, 8192):
        k_raw = rng.standard_normal(DIM).astype(np.float32)
        qd.prepare(n_past)
        say(f"pool decode n_past={n_past}")
        K.qsa_pool_decode(ic_d, dev(k_raw), qd.write_idx, qd.member_idx, ratio, qd.blk_pos, qd.blk_idx, w_d, pool)
        O.set_rows_f16(ref_ic, k_raw[None], np.array([n_past], np.int32))
        b = n_past // ratio
        members = np.arange(b * ratio, b * ratio + ratio, dtype=np.int32)
        ref_pool[b] = O.qsa_pool_blocks(ref_ic, members, ratio, w, np.full((1, 4), b * ratio, np.int32))[0]
        assert K.device_status() == 0
    np.testing.assert_array_equal(host(ic_d).view(np.uint16), ref_ic)
    got = host(pool).view(np.uint16)
    _ulp_check(got[[255, 256]], ref_pool[[255, 256]])
    assert not np.delete(got, [255, 256], axis=0).any()
    # the pool-only form (no key) re-pools block 256 with the same result
    say("pool decode without a key")
    pool2 = torch.zeros_like(pool)
    K.qsa_pool_decode(ic_d, None, qd.write_idx, qd.member_idx, ratio, qd.blk_pos, qd.blk_idx, w_d, pool2)
    np.testing.assert_array_equal(host(pool2).view(np.uint16)[256], got[256])
    # a rebuild of the whole blocks at n_past = 8192 (256 blocks) gives block 255 as the chain did
    say("pool rebuild after the chain")
    pool3 = torch.zeros_like(pool)
    K.qsa_pool_rebuild(ic_d, 8192, ratio, w_d, pool3)
    np.testing.assert_array_equal(host(pool3).view(np.uint16)[255], got[255])


def test_pool_decode_out_of_range_rows_flagged(gpu, oracle):
    K = gpu
    ratio = 4
    ic = torch.zeros((64, DIM), dtype=torch.float16, device="cuda")
    pool = torch.zeros((8, DIM), dtype=torch.float16, device="cuda")
    w = dev(_weights(5))
    wi = dev(np.array([64], np.int32))                    # one past the cache
    mi = dev(np.arange(60, 64, dtype=np.int32))
    bp = dev(np.full(4, 60, np.int32))
    bi = dev(np.array([15], np.int32))                    # past the pool
    say("pool decode out-of-range rows")
    K.qsa_pool_decode(ic, dev(np.ones(DIM, np.float32)), wi, mi, ratio, bp, bi, w, pool)
    assert K.device_status() & 1
    assert not host(pool).view(np.uint16).any() and not host(ic).view(np.uint16).any()
