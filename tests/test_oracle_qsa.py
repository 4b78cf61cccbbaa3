"""Pins of the oracle's QSA index producer (qsa_pool_blocks, qwfn_graph.cpp:282-301;
the raw-key set_rows, :536-543; the pool rebuild, :478-495): ggml_rms_norm by its
closed form, ggml_rope_multi (IMROPE) by what the mathematics fixes -- the
reduction to standard neox rotary embedding at equal section positions, norm
preservation, relative-position invariance, the interleaved section pattern of
Qwen3-VL and an fp64 restatement --, the F16 set_rows by numpy's IEEE
conversion, and the pooled row by an fp64 composition of the same steps."""
import numpy as np
import pytest

from oracle import oracle as O

N_DIMS = O.ROPE_DIM
BASE = O.ROPE_FREQ_BASE


def test_rms_norm_closed_form():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((50, 128)) * rng.uniform(0.01, 30, (50, 1))).astype(np.float32)
    y = O.rms_norm(x, 1e-6)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-6)
    np.testing.assert_allclose(y, ref, rtol=3e-7, atol=0)
    # the output's mean square is ms / (ms + eps)
    ms = (x64 ** 2).mean(axis=1)
    np.testing.assert_allclose((y.astype(np.float64) ** 2).mean(axis=1), ms / (ms + 1e-6), rtol=2e-6)
    # a zero row stays zero; a constant row becomes its sign (up to eps)
    z = O.rms_norm(np.zeros((1, 128), np.float32))
    assert not z.any()
    c = O.rms_norm(np.full((1, 128), -3.0, np.float32))
    np.testing.assert_allclose(c, -1.0, rtol=1e-6)


def _angles_f32(pos: float, n_pairs: int) -> np.ndarray:
    """The running float32 product theta_k = pos * ts^k, ts = base^(-2/n_dims) in float32."""
    ts = np.float32(np.power(np.float32(BASE), np.float32(-2.0 / N_DIMS)))
    th = np.float32(pos)
    out = np.empty(n_pairs, np.float32)
    for k in range(n_pairs):
        out[k] = th
        th = np.float32(th * ts)
    return out


def _neox(x: np.ndarray, ang: np.ndarray) -> np.ndarray:
    x = x.astype(np.float64)
    h = len(ang)
    y = x.copy()
    c, s = np.cos(ang.astype(np.float64)), np.sin(ang.astype(np.float64))
    y[:h] = x[:h] * c - x[h:2 * h] * s
    y[h:2 * h] = x[:h] * s + x[h:2 * h] * c
    return y


@pytest.mark.parametrize("pos", [0, 1, 77, 4095, 65536, 262143])
def test_rope_equal_positions_is_neox_rope(pos):
    """t = h = w = e: every pair uses the same position, so IMROPE is neox rope
    over the first 64 dims (fp64 restatement of the float32 angle recurrence)."""
    rng = np.random.default_rng(pos)
    x = rng.standard_normal(128).astype(np.float32)
    y = O.rope_multi(x, pos)
    ref = _neox(x, _angles_f32(pos, N_DIMS // 2))
    np.testing.assert_allclose(y, ref, atol=2e-6 * max(1.0, np.abs(x).max()))
    np.testing.assert_array_equal(y[N_DIMS:], x[N_DIMS:])       # the other dims pass through


def test_rope_small_positions_match_textbook_frequencies():
    """At small positions the float32 recurrence equals theta_k = p * base^(-2k/64) in fp64."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal(128).astype(np.float32)
    for pos in (1, 5, 31):
        ang = pos * np.power(BASE, -2.0 * np.arange(N_DIMS // 2) / N_DIMS)
        np.testing.assert_allclose(O.rope_multi(x, pos), _neox(x, ang), atol=2e-5)


def test_rope_preserves_norm_and_relative_position():
    rng = np.random.default_rng(4)
    q = rng.standard_normal(128).astype(np.float32)
    k = rng.standard_normal(128).astype(np.float32)
    for pos in (0, 9, 1000, 100000):
        y = O.rope_multi(q, pos)
        assert abs(np.linalg.norm(y[:N_DIMS]) - np.linalg.norm(q[:N_DIMS])) < 1e-5 * np.linalg.norm(q)
    # <rope(q, a), rope(k, b)> depends on a - b only (small positions: float32 angles are exact enough)
    d0 = float(np.dot(O.rope_multi(q, 7).astype(np.float64), O.rope_multi(k, 3)))
    for s in (1, 10, 40):
        d = float(np.dot(O.rope_multi(q, 7 + s).astype(np.float64), O.rope_multi(k, 3 + s)))
        assert abs(d - d0) < 2e-4
    # and changes with the offset
    assert abs(float(np.dot(O.rope_multi(q, 8).astype(np.float64), O.rope_multi(k, 3))) - d0) > 1e-3


def test_imrope_interleaves_sections():
    """Qwen3-VL's interleaved layout for sections (11, 11, 10): pairs 0..31 take
    t, h, w, t, h, w, ... (10 full rounds, then t, h); a pair turns by the angle
    of its own section's position."""
    expect = (["t", "h", "w"] * 11)[:32]
    assert expect.count("t") == 11 and expect.count("h") == 11 and expect.count("w") == 10
    pos = {"t": 3, "h": 50, "w": 700}
    ang = {s: _angles_f32(p, N_DIMS // 2) for s, p in pos.items()}
    for k in range(N_DIMS // 2):
        x = np.zeros(128, np.float32)
        x[k] = 1.0
        y = O.rope_multi(x, [pos["t"], pos["h"], pos["w"], 9])
        a = ang[expect[k]][k].astype(np.float64)
        assert abs(y[k] - np.cos(a)) < 1e-6 and abs(y[k + N_DIMS // 2] - np.sin(a)) < 1e-6, k


def test_set_rows_f16_is_ieee_rne():
    rng = np.random.default_rng(5)
    src = (rng.standard_normal((7, 128)) * np.exp(rng.uniform(-20, 12, (7, 128)))).astype(np.float32)
    src[0, :4] = [65520.0, 65519.0, 5.9604645e-08, 2.9802322e-08]   # overflow, max, min subnormal, tie to 0
    dst = np.zeros((20, 128), np.uint16)
    idx = np.array([3, 19, 0, 7, 8, 11, 12], np.int32)
    O.set_rows_f16(dst, src, idx)
    with np.errstate(over="ignore"):
        np.testing.assert_array_equal(dst[idx], src.astype(np.float16).view(np.uint16))
    assert not dst[[1, 2, 4, 5, 6, 9, 10, 13]].any()
    with pytest.raises(IndexError):
        O.set_rows_f16(dst, src[:1], np.array([20], np.int32))


@pytest.mark.parametrize("r", [1, 4, 32])
def test_pool_blocks_composition(r):
    """Mean of r F16 rows, RMS norm, k_norm weight, IMROPE at the block position,
    fp16: against the same steps in fp64 (angles from the float32 recurrence)."""
    rng = np.random.default_rng(r)
    n_blk, idx_dim = 9, 128
    ic = rng.standard_normal((n_blk * r + 5, idx_dim)).astype(np.float16)
    w = rng.uniform(0.5, 1.5, idx_dim).astype(np.float32)
    members = np.arange(n_blk * r, dtype=np.int32)
    pos4 = np.repeat((np.arange(n_blk) * r)[:, None], 4, axis=1).astype(np.int32)
    got = O.qsa_pool_blocks(ic.view(np.uint16), members, r, w, pos4).view(np.float16).astype(np.float64)
    for b in range(n_blk):
        m = ic[b * r:(b + 1) * r].astype(np.float64).mean(axis=0)
        n = m / np.sqrt((m ** 2).mean() + O.RMS_EPS) * w
        ref = _neox(n, _angles_f32(b * r, N_DIMS // 2))
        np.testing.assert_allclose(got[b], ref, rtol=2e-3, atol=1e-4)


@pytest.mark.parametrize("T,variant", [(1, O.Q8_X86), (3, O.Q8_REF)])
def test_kv_produce_composition(T, variant):
    """The oracle's K/V producer (qwfn_graph.cpp:441-451, then the q8_0 append)
    against the same steps done independently: the projection in fp64 numpy of
    the F16 weights and the F16-rounded hidden rows (ggml_mul_mat's conversion
    of src1), the K heads through the pinned rms_norm x weight and rope_multi,
    both tensors through the pinned quantiser."""
    rng = np.random.default_rng(40 + T)
    E, kv_dim = 96, 512
    cur = rng.standard_normal((T, E)).astype(np.float32)
    wk = (rng.standard_normal((kv_dim, E)) * 0.1).astype(np.float16)
    wv = (rng.standard_normal((kv_dim, E)) * 0.1).astype(np.float16)
    knw = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    pos = np.tile(np.arange(700, 700 + T, dtype=np.int32), 4)
    k_rows, v_rows, k_f, v_f = O.kv_produce(cur, wk.view(np.uint16), wv.view(np.uint16), knw, pos, variant)
    c16 = cur.astype(np.float16).astype(np.float64)
    kp = c16 @ wk.astype(np.float64).T
    vp = c16 @ wv.astype(np.float64).T
    np.testing.assert_allclose(v_f, vp, rtol=1e-6, atol=1e-6)
    for t in range(T):
        heads = kp[t].astype(np.float32).reshape(2, 256)
        kn = O.rms_norm(heads) * knw
        ref_k = O.rope_multi(kn, int(pos[t])).reshape(-1)
        np.testing.assert_allclose(k_f[t], ref_k, rtol=1e-5, atol=1e-5)
        np.testing.assert_array_equal(k_rows[t], O.quantize(k_f[t], variant).reshape(-1))
        np.testing.assert_array_equal(v_rows[t], O.quantize(v_f[t], variant).reshape(-1))


def test_fp32_to_bf16_is_rne():
    """The oracle's F32 -> BF16 (src1 of a BF16 mul_mat) against torch's round to
    nearest even: ties both ways, values just off a tie, overflow to inf, signed
    zero, subnormals, inf; a NaN stays a NaN."""
    import torch
    rng = np.random.default_rng(9)
    x = (rng.standard_normal(4000) * np.exp(rng.uniform(-90, 88, 4000))).astype(np.float32)
    u = x.view(np.uint32)
    u[:16] = (u[:16] & 0xFFFF0000) | 0x8000                       # exact ties
    u[16:32] = (u[16:32] & 0xFFFF0000) | 0x7FFF                   # just below a tie
    u[32:48] = (u[32:48] & 0xFFFF0000) | 0x8001                   # just above
    x[48:53] = [3.4028235e38, -0.0, 1e-45, -1e-41, np.inf]
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(O.fp32_to_bf16_bits(x), want)
    nan = O.fp32_to_bf16_bits(np.array([np.nan], np.float32))[0]
    assert (nan & 0x7F80) == 0x7F80 and (nan & 0x007F) != 0


@pytest.mark.parametrize("T", [1, 3])
def test_kv_produce_composition_bf16(T):
    """The producer with BF16 weights: the hidden rows rounded to BF16 (pinned above),
    the projection in fp64 of the BF16 values, then the same norm / rope / quantiser."""
    import torch
    rng = np.random.default_rng(60 + T)
    E, kv_dim = 96, 512
    cur = rng.standard_normal((T, E)).astype(np.float32)
    wk = torch.from_numpy((rng.standard_normal((kv_dim, E)) * 0.1).astype(np.float32)).to(torch.bfloat16)
    wv = torch.from_numpy((rng.standard_normal((kv_dim, E)) * 0.1).astype(np.float32)).to(torch.bfloat16)
    wk_bits = wk.view(torch.int16).numpy().view(np.uint16)
    wv_bits = wv.view(torch.int16).numpy().view(np.uint16)
    knw = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    pos = np.tile(np.arange(900, 900 + T, dtype=np.int32), 4)
    k_rows, v_rows, k_f, v_f = O.kv_produce(cur, wk_bits, wv_bits, knw, pos, O.Q8_X86, w_bf16=True)
    cb = torch.from_numpy(cur).to(torch.bfloat16).to(torch.float64).numpy()
    kp = cb @ wk.to(torch.float64).numpy().T
    vp = cb @ wv.to(torch.float64).numpy().T
    np.testing.assert_allclose(v_f, vp, rtol=1e-6, atol=1e-6)
    for t in range(T):
        kn = O.rms_norm(kp[t].astype(np.float32).reshape(2, 256)) * knw
        np.testing.assert_allclose(k_f[t], O.rope_multi(kn, int(pos[t])).reshape(-1), rtol=1e-5, atol=1e-5)
        np.testing.assert_array_equal(k_rows[t], O.quantize(k_f[t], O.Q8_X86).reshape(-1))
        np.testing.assert_array_equal(v_rows[t], O.quantize(v_f[t], O.Q8_X86).reshape(-1))
