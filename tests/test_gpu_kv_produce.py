"""GPU parity of the K/V producer (projection -> K RMS norm -> IMROPE -> q8_0
append, qwfn_graph.cpp:441-451, :129-132, :370-384) and of the attention
output gate (qwfn_graph.cpp:474, :701) against the oracle, with seeded
synthetic weights of the model's shapes (n_embd 2560, 2 KV heads of 256).

The projection's float rows differ from the oracle's (summed in double) by
float rounding only, so a q8_0 value may sit on the other side of a rounding
boundary: the K/V bytes must be identical except for such quants (at most 1 in
1000, each one step off where the oracle's scaled value lies within 1e-3 of a
half-integer) and the block scales identical except at most 1 in 200 (one
f16 step). The gated output equals the ungated one times sigmoid(gate) to
float rounding and the oracle within the attention tolerance."""
import numpy as np
import pytest
import torch

import kvdata as KD
from gpu_util import dev, host, say
from oracle import oracle as O

pytestmark = pytest.mark.gpu
E, KV_DIM, SEG = 2560, 512, 272


def _weights(seed):
    rng = np.random.default_rng(seed)
    wk = (rng.standard_normal((KV_DIM, E)) * 0.02).astype(np.float16)
    wv = (rng.standard_normal((KV_DIM, E)) * 0.02).astype(np.float16)
    knw = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    return wk, wv, knw


def _compare_rows(got: np.ndarray, ref: np.ndarray, ref_f32: np.ndarray):
    """got/ref uint8 [T, 544] q8_0 rows; ref_f32 the oracle's float rows [T, 512]."""
    g = got.reshape(-1, 34)
    r = ref.reshape(-1, 34)
    d_g, d_r = g[:, :2].copy().view(np.uint16)[:, 0], r[:, :2].copy().view(np.uint16)[:, 0]
    n_d = int((d_g != d_r).sum())
    assert n_d <= max(1, len(d_r) // 200), n_d
    assert np.abs(d_g.astype(np.int32) - d_r.astype(np.int32)).max() <= 1
    q_g = g[:, 2:].view(np.int8).astype(np.int32)
    q_r = r[:, 2:].view(np.int8).astype(np.int32)
    same_d = d_g == d_r
    diff = q_g[same_d] != q_r[same_d]
    n_q = int(diff.sum())
    print(f"  scales differing: {n_d} of {len(d_r)}; quants differing: {n_q} of {q_r[same_d].size}", flush=True)
    assert n_q <= max(1, q_r.size // 1000)
    if n_q:
        assert np.abs(q_g[same_d] - q_r[same_d]).max() <= 1
        # only at rounding boundaries: the oracle's x / d lies within 1e-3 of k + 1/2
        d = O.fp16_bits_to_fp32(d_r).astype(np.float64)[same_d]
        x = ref_f32.reshape(-1, 32).astype(np.float64)[same_d]
        frac = np.abs(np.abs(x / np.where(d == 0, 1, d)[:, None]) % 1.0 - 0.5)
        assert (frac[diff] < 1e-3).all()


@pytest.mark.parametrize("T,n_past,variant", [(1, 5000, O.Q8_X86), (3, 16384, O.Q8_X86), (16, 700, O.Q8_REF)])
def test_kv_produce_matches_oracle(gpu, oracle, T, n_past, variant):
    K = gpu
    wk, wv, knw = _weights(T)
    cur = KD.normal(60 + T, 0, KD.Q_KIND, T * E).reshape(T, E)
    pos = np.tile(np.arange(n_past, n_past + T, dtype=np.int32), 4)
    n_rows = n_past + T + 8
    rng = np.random.default_rng(T)
    kc0 = rng.integers(0, 256, (n_rows, 544), dtype=np.uint8)
    vc0 = rng.integers(0, 256, (n_rows, 544), dtype=np.uint8)
    kd, vd = dev(kc0), dev(vc0)
    say(f"kv_produce T={T} first_row={n_past}")
    K.kv_produce(dev(cur), dev(wk), dev(wv), dev(knw), dev(pos), kd, vd, n_past, variant=variant)
    kg, vg = host(kd), host(vd)
    k_rows, v_rows, k_f, v_f = O.kv_produce(cur, wk.view(np.uint16), wv.view(np.uint16), knw, pos, variant)
    others = np.r_[0:n_past, n_past + T:n_rows]
    np.testing.assert_array_equal(kg[others], kc0[others])
    np.testing.assert_array_equal(vg[others], vc0[others])
    _compare_rows(kg[n_past:n_past + T], k_rows, k_f)
    _compare_rows(vg[n_past:n_past + T], v_rows, v_f)


@pytest.mark.parametrize("T,n_past", [(1, 5000), (3, 16384), (16, 700)])
def test_kv_produce_bf16_weights(gpu, oracle, T, n_past):
    """BF16 attn_k / attn_v weights: the hidden rows rounded to BF16 on the device,
    the same tolerance on the q8_0 bytes as for F16 weights."""
    K = gpu
    rng = np.random.default_rng(100 + T)
    wk = torch.from_numpy((rng.standard_normal((KV_DIM, E)) * 0.02).astype(np.float32)).to(torch.bfloat16)
    wv = torch.from_numpy((rng.standard_normal((KV_DIM, E)) * 0.02).astype(np.float32)).to(torch.bfloat16)
    knw = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    cur = KD.normal(80 + T, 0, KD.Q_KIND, T * E).reshape(T, E)
    pos = np.tile(np.arange(n_past, n_past + T, dtype=np.int32), 4)
    n_rows = n_past + T + 8
    kd = torch.zeros((n_rows, 544), dtype=torch.uint8, device="cuda")
    vd = torch.zeros((n_rows, 544), dtype=torch.uint8, device="cuda")
    say(f"kv_produce bf16 T={T} first_row={n_past}")
    K.kv_produce(dev(cur), wk.cuda(), wv.cuda(), dev(knw), dev(pos), kd, vd, n_past)
    wk_bits = wk.view(torch.int16).numpy().view(np.uint16)
    wv_bits = wv.view(torch.int16).numpy().view(np.uint16)
    k_rows, v_rows, k_f, v_f = O.kv_produce(cur, wk_bits, wv_bits, knw, pos, O.Q8_X86, w_bf16=True)
    _compare_rows(host(kd)[n_past:n_past + T], k_rows, k_f)
    _compare_rows(host(vd)[n_past:n_past + T], v_rows, v_f)
    assert not host(kd)[:n_past].any() and not host(kd)[n_past + T:].any()


def test_kv_produce_then_attention(gpu, oracle):
    """The produced rows feed the verify attention like appended ones: decode over
    the cache after a 3-token producer step matches the oracle on the same cache."""
    K = gpu
    T, n_past, nh = 3, 2000, 16
    wk, wv, knw = _weights(9)
    kc = KD.make_cache(KD.kv_rows(61, 0, KD.K_KIND, n_past), n_past + T)
    vc = KD.make_cache(KD.kv_rows(61, 0, KD.V_KIND, n_past), n_past + T)
    cur = KD.normal(61, 0, KD.Q_KIND, T * E).reshape(T, E)
    pos = np.tile(np.arange(n_past, n_past + T, dtype=np.int32), 4)
    kd, vd = dev(kc), dev(vc)
    say("kv_produce then verify attention")
    K.kv_produce(dev(cur), dev(wk), dev(wv), dev(knw), dev(pos), kd, vd, n_past)
    kh, vh = host(kd), host(vd)
    q = KD.q_rows(61, 1, T, nh)[0]
    mask = O.causal_mask(T, n_past)
    from gpu_util import gpu_attn
    got = gpu_attn(K, q, kh, vh, n_past + T, 2, mask, 1 / 16)
    ref = KD.oracle_attn(q, kh, vh, n_past + T, 2, mask, 1 / 16)
    mx, mean = KD.err_stats(got, ref)
    assert mx <= 1e-4 and mean <= KD.MEAN_ABS_TOL


@pytest.mark.parametrize("T,n_kv,splits", [(3, 16387, 0), (3, 4099, 1), (64, 3064, 0), (64, 3064, 1), (2, 40000, 300)])
def test_gated_attention(gpu, oracle, T, n_kv, splits):
    """Gate on every kernel path: decode / verify (split merge, one split, the
    long merge) and the prefill kernel (row merge, one split)."""
    K = gpu
    nh = 16
    kc = KD.make_cache(KD.kv_rows(62, 0, KD.K_KIND, n_kv), n_kv)
    vc = KD.make_cache(KD.kv_rows(62, 0, KD.V_KIND, n_kv), n_kv)
    q = KD.q_rows(62, 1, T, nh)[0]
    mask = O.causal_mask(T, n_kv - T)
    gate = (np.random.default_rng(T).standard_normal((1, T, nh, 256)) * 3).astype(np.float32)
    kd, vd = dev(kc), dev(vc)
    qd, md, gd = dev(q[None].astype(np.float32)), dev(mask.view(np.float16)), dev(gate)
    kv, vv = K.cache_attn_view(kd, n_kv, 2), K.cache_attn_view(vd, n_kv, 2)
    outs = []
    if splits:
        K.load().qwfn_fattn_force_splits(splits)
    try:
        for gated in (False, True):
            out = torch.full((1, T, nh, 256), float("nan"), dtype=torch.float32, device="cuda")
            say(f"gated={gated} T={T} n_kv={n_kv} splits={splits}")
            if gated:
                K.flash_attn_ext_gated(K.q_view(qd), kv, vv, K.mask_view(md), 1 / 16, K.out_view(out), gd)
            else:
                K.flash_attn_ext(K.q_view(qd), kv, vv, K.mask_view(md), 1 / 16, K.out_view(out))
            outs.append(host(out)[0])
    finally:
        K.load().qwfn_fattn_force_splits(0)
    sig = (1.0 / (1.0 + np.exp(-gate[0].astype(np.float64)))).astype(np.float32)
    np.testing.assert_allclose(outs[1], outs[0] * sig, rtol=2e-6, atol=1e-7)
    ref = KD.oracle_attn(q, kc, vc, n_kv, 2, mask, 1 / 16) * sig
    mx, mean = KD.err_stats(outs[1], ref)
    assert mx <= 1e-4 and mean <= KD.MEAN_ABS_TOL
