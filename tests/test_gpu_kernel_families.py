"""Every attention kernel instantiation the library can launch, reached through
the C ABI and checked against the oracle's ggml-cpu flash_attn_ext on the same
inputs.

The planner picks one kernel family per call (k_fa_dec for up to 32 query
rows per KV head, k_fa_pre for prefill blocks, k_fattn_q8_0 for the rest;
k_fa_vd and k_fa_vs, up to 24 rows, when forced); qwfn_fattn_force_kernel makes a family take a call it can serve, so
the same shapes run through each of them, and qwfn_fattn_last_kernel names
the instantiation that ran. Forms: dense (qwfn_flash_attn_ext_q8_0),
per-sequence key counts (_seq), gathered cells (_cells), the fused append and
the output gate. Masks: none, causal over the new positions (shared by the
heads), finite values with -inf holes, per-head. The last test checks that
the cases reached every instantiation the library refuses to run when it
spills (its scratch check). Bar: 2e-3 max / 1e-3 mean abs, held to 1e-4 max."""
import numpy as np
import pytest
import torch

import kvdata as KD
import qwfn_kv as KK
from gpu_util import dev, host, say
from oracle import oracle as O

pytestmark = pytest.mark.gpu
TIGHT = 1e-4
HD = 256

# every attention kernel instantiation of the library (its scratch check list)
ALL_KERNELS = (
    [f"k_fa_{f}<{nf}, {pk}, {m}, {rg}, {g}>" for f in ("vd", "vs") for nf, pk in ((0, 1), (1, 0), (1, 1))
     for m, rg, g in (("false", "false", "false"), ("true", "false", "false"), ("false", "true", "false"),
                      ("true", "true", "false"), ("false", "false", "true"))]
    + [f"k_fa_dec<{rt}, {m}, {rg}, false>" for rt in (1, 2) for m in ("false", "true") for rg in ("false", "true")]
    + ["k_fa_dec<1, false, false, true>", "k_fa_dec<2, false, false, true>"]
    + ["k_fa_pre<false>", "k_fa_pre<true>"]
    + [f"k_fattn_q8_0<{k}, {rg}>" for rg in ("false", "true")
       for k in ("1, false, WAVES_PAIR, 16", "1, true, WAVES_PAIR, 16", "2, false, WAVES_PAIR, 32",
                 "2, true, WAVES_PAIR, 32", "2, true, WAVES, 16")])
REACHED = set()


def check(got, ref, tight=TIGHT):
    mx, mean = KD.err_stats(got, ref)
    print(f"  max abs {mx:.3e}  mean abs {mean:.3e}", flush=True)
    assert np.isfinite(got).all()
    assert mx <= KD.MAX_ABS_TOL and mean <= KD.MEAN_ABS_TOL
    assert mx <= tight


def layer(seed, n_kv, n_ctx=None, outliers=True):
    n_ctx = n_ctx or n_kv
    kc = KD.make_cache(KD.kv_rows(seed, 0, KD.K_KIND, n_kv, outliers=outliers), n_ctx)
    vc = KD.make_cache(KD.kv_rows(seed, 0, KD.V_KIND, n_kv, outliers=outliers), n_ctx)
    return kc, vc


def make_mask(kind, T, n_kv, nh, seed):
    """F16 bits: [T, n_kv] shared by the heads, or [1, nh, T, n_kv] per head."""
    if kind is None:
        return None
    if kind == "causal":
        return O.causal_mask(T, n_kv - T)
    rng = np.random.default_rng(seed)
    if kind == "finite":
        m = rng.uniform(-4, 1, (T, n_kv)).astype(np.float16).view(np.uint16)
        m[:, ::7] = O.F16_NEG_INF
        return m
    assert kind == "perhead"
    m = rng.uniform(-2, 0, (1, nh, T, n_kv)).astype(np.float16).view(np.uint16)
    m[0, 3, :, n_kv // 3:] = O.F16_NEG_INF
    m[0, :, :, -T:] = np.where(np.tri(T, dtype=bool)[None], m[0, :, :, -T:], O.F16_NEG_INF)
    return m


def ref_dense(q, kc, vc, n_kv, mask, nh):
    """Oracle of one sequence: q [T, nh, HD]; mask shared [T, n_kv] or per head [1, nh, T, n_kv]."""
    if mask is None or mask.ndim == 2:
        return KD.oracle_attn(q, kc, vc, n_kv, 2, mask, 1 / 16)
    T = q.shape[0]
    qv, kv, vv = O.cache_views(np.ascontiguousarray(q, np.float32), kc, vc, n_kv, 2, HD)
    mh = np.ascontiguousarray(mask[0, :, :, :n_kv])
    mview = O.view(mh, (n_kv, T, nh, 1), (2, n_kv * 2, T * n_kv * 2, nh * T * n_kv * 2))
    return O.flash_attn_ext(qv, kv, vv, mview, 1 / 16, (T, nh, HD), O.Q8_X86, O.Q8_X86, 8)


def run_dense(K, q, kc, vc, n_kv, mask):
    qd = dev(q[None].astype(np.float32))
    kd, vd = dev(kc), dev(vc)
    md = dev(mask.view(np.float16)) if mask is not None else None
    out = torch.full((1,) + q.shape, float("nan"), dtype=torch.float32, device="cuda")
    K.flash_attn_ext(K.q_view(qd), K.cache_attn_view(kd, n_kv, 2), K.cache_attn_view(vd, n_kv, 2),
                     K.mask_view(md) if md is not None else None, 1 / 16, K.out_view(out))
    name = K.last_kernel()
    return host(out)[0], name


def run_seq(K, q, kc, vc, n_ctx, depths, mask):
    """q [B, T, nh, HD]; kc/vc [B, n_ctx, 544]; mask [B, 1, T, n_ctx] (shared by heads) or None."""
    B, T, nh, _ = q.shape
    qd = dev(q.astype(np.float32))
    kd, vd = dev(kc), dev(vc)
    rb = kc.shape[-1]
    kv = K.tensor(kd.data_ptr(), K.TYPE_Q8_0, (HD, n_ctx, 2, B), (34, rb, 272, n_ctx * rb))
    vv = K.tensor(vd.data_ptr(), K.TYPE_Q8_0, (HD, n_ctx, 2, B), (34, rb, 272, n_ctx * rb))
    md = dev(mask.view(np.float16)) if mask is not None else None
    mv = K.mask_view(md) if md is not None else None
    out = torch.full((B, T, nh, HD), float("nan"), dtype=torch.float32, device="cuda")
    ws = torch.empty(max(256, K.fattn_workspace_size_seq(K.q_view(qd), kv, vv, mv, depths)), dtype=torch.uint8,
                     device="cuda")
    K.flash_attn_ext_seq(K.q_view(qd), kv, vv, mv, 1 / 16, K.out_view(out), depths, ws=ws)
    name = K.last_kernel()
    return host(out), name


def run_cells(K, q, kc, vc, lists, pos0):
    T, nh, _ = q.shape
    n = [len(x) for x in lists]
    stride = max(4, (max(n) + 3) // 4 * 4)
    c = np.zeros((2, stride), np.int32)
    for h, x in enumerate(lists):
        c[h, :len(x)] = x
    kd, vd = dev(kc), dev(vc)
    n_rows, rb = kc.shape
    kv = K.tensor(kd.data_ptr(), K.TYPE_Q8_0, (HD, n_rows, 2, 1), (34, rb, 272, n_rows * rb))
    vv = K.tensor(vd.data_ptr(), K.TYPE_Q8_0, (HD, n_rows, 2, 1), (34, rb, 272, n_rows * rb))
    qd = dev(q[None].astype(np.float32))
    out = torch.full((1, T, nh, HD), float("nan"), dtype=torch.float32, device="cuda")
    K.flash_attn_ext_cells(K.q_view(qd), kv, vv, dev(c), n, pos0, 1 / 16, K.out_view(out))
    name = K.last_kernel()
    assert K.device_status() == 0
    return host(out)[0], name


def forced(kind, splits=0):
    class _F:
        def __enter__(self):
            KK.load().qwfn_fattn_force_kernel(kind)
            KK.load().qwfn_fattn_force_splits(splits)

        def __exit__(self, *e):
            KK.load().qwfn_fattn_force_kernel(KK.FA_KERNEL_AUTO)
            KK.load().qwfn_fattn_force_splits(0)
            return False
    return _F()


FAMILY = {"vd": KK.FA_KERNEL_VD, "vs": KK.FA_KERNEL_VS, "dec": KK.FA_KERNEL_DEC, "general": KK.FA_KERNEL_GENERAL,
          "auto": KK.FA_KERNEL_AUTO}

# (family, T, mask, forced splits, expected instantiation) over a dense layer of 3000 keys
DENSE = [
    ("vd", 1, None, 0, "k_fa_vd<0, 1, false, false, false>"),
    ("vd", 1, "finite", 0, "k_fa_vd<0, 1, true, false, false>"),
    ("vd", 2, None, 0, "k_fa_vd<1, 0, false, false, false>"),
    ("vd", 2, "causal", 0, "k_fa_vd<1, 0, true, false, false>"),
    ("vd", 3, None, 0, "k_fa_vd<1, 1, false, false, false>"),
    ("vd", 3, "causal", 0, "k_fa_vd<1, 1, true, false, false>"),
    ("vd", 3, "finite", 3, "k_fa_vd<1, 1, true, false, false>"),
    ("vs", 1, None, 0, "k_fa_vs<0, 1, false, false, false>"),
    ("vs", 1, "finite", 0, "k_fa_vs<0, 1, true, false, false>"),
    ("vs", 1, None, 1, "k_fa_vs<0, 1, false, false, false>"),
    ("vs", 2, None, 0, "k_fa_vs<1, 0, false, false, false>"),
    ("vs", 2, "causal", 0, "k_fa_vs<1, 0, true, false, false>"),
    ("vs", 3, None, 0, "k_fa_vs<1, 1, false, false, false>"),
    ("vs", 3, "causal", 0, "k_fa_vs<1, 1, true, false, false>"),
    ("vs", 3, "finite", 3, "k_fa_vs<1, 1, true, false, false>"),
    ("auto", 3, "causal", 0, "k_fa_dec<2, true, false, false>"),
    ("auto", 1, "finite", 0, "k_fa_vs<0, 1, true, false, false>"),
    ("dec", 2, None, 0, "k_fa_dec<1, false, false, false>"),
    ("dec", 2, "causal", 0, "k_fa_dec<1, true, false, false>"),
    ("dec", 3, None, 0, "k_fa_dec<2, false, false, false>"),
    ("dec", 3, "causal", 0, "k_fa_dec<2, true, false, false>"),
    ("auto", 3, "perhead", 0, "k_fa_dec<2, true, false, false>"),
    ("general", 2, None, 0, "k_fattn_q8_0<1, false, WAVES_PAIR, 16, false>"),
    ("general", 2, "causal", 1, "k_fattn_q8_0<1, true, WAVES_PAIR, 16, false>"),
    ("general", 3, None, 0, "k_fattn_q8_0<2, false, WAVES_PAIR, 32, false>"),
    ("general", 3, "causal", 1, "k_fattn_q8_0<2, true, WAVES_PAIR, 32, false>"),
    ("general", 3, "perhead", 1, "k_fattn_q8_0<2, true, WAVES, 16, false>"),
]


@pytest.mark.parametrize("fam,T,mask_kind,splits,expect", DENSE)
def test_dense_family(gpu, oracle, fam, T, mask_kind, splits, expect):
    K = gpu
    nh, n_kv = 16, 3000
    kc, vc = layer(70 + T, n_kv)
    q = KD.q_rows(70 + T, 1, T, nh)[0]
    mask = make_mask(mask_kind, T, n_kv, nh, 70 + T)
    say(f"dense {fam} T={T} mask={mask_kind} splits={splits} (expect {expect})")
    with forced(FAMILY[fam], splits):
        got, name = run_dense(K, q, kc, vc, n_kv, mask)
    REACHED.add(name)
    assert name == expect
    check(got, ref_dense(q, kc, vc, n_kv, mask, nh))


# per-sequence key counts: two sequences of a 3000-row batch, depths 700 and 2900
SEQ = [
    ("vd", 1, False, 0, "k_fa_vd<0, 1, false, true, false>"),
    ("vd", 1, True, 0, "k_fa_vd<0, 1, true, true, false>"),
    ("vd", 2, False, 0, "k_fa_vd<1, 0, false, true, false>"),
    ("vd", 2, True, 0, "k_fa_vd<1, 0, true, true, false>"),
    ("vd", 3, False, 0, "k_fa_vd<1, 1, false, true, false>"),
    ("vd", 3, True, 0, "k_fa_vd<1, 1, true, true, false>"),
    ("vs", 1, False, 0, "k_fa_vs<0, 1, false, true, false>"),
    ("vs", 1, True, 0, "k_fa_vs<0, 1, true, true, false>"),
    ("vs", 2, False, 0, "k_fa_vs<1, 0, false, true, false>"),
    ("vs", 2, True, 0, "k_fa_vs<1, 0, true, true, false>"),
    ("vs", 3, False, 0, "k_fa_vs<1, 1, false, true, false>"),
    ("vs", 3, True, 0, "k_fa_vs<1, 1, true, true, false>"),
    ("dec", 2, False, 0, "k_fa_dec<1, false, true, false>"),
    ("dec", 2, True, 0, "k_fa_dec<1, true, true, false>"),
    ("dec", 3, False, 0, "k_fa_dec<2, false, true, false>"),
    ("dec", 3, True, 0, "k_fa_dec<2, true, true, false>"),
    ("general", 2, False, 0, "k_fattn_q8_0<1, false, WAVES_PAIR, 16, true>"),
    ("general", 2, True, 1, "k_fattn_q8_0<1, true, WAVES_PAIR, 16, true>"),
    ("general", 3, False, 0, "k_fattn_q8_0<2, false, WAVES_PAIR, 32, true>"),
    ("general", 3, True, 1, "k_fattn_q8_0<2, true, WAVES_PAIR, 32, true>"),
]


@pytest.mark.parametrize("fam,T,masked,splits,expect", SEQ)
def test_seq_family(gpu, oracle, fam, T, masked, splits, expect):
    K = gpu
    nh, n_ctx, depths = 16, 3000, [700, 2900]
    kcs, vcs = zip(*[layer(80 + s, n_ctx) for s in range(2)])
    kc, vc = np.stack(kcs), np.stack(vcs)
    q = KD.q_rows(80 + T, 1, T, nh, batch=2)
    mask = None
    if masked:
        mask = np.stack([make_mask("finite", T, n_ctx, nh, 80 + s)[None] for s in range(2)])   # [2, 1, T, n_ctx]
    say(f"seq {fam} T={T} masked={masked} splits={splits} (expect {expect})")
    with forced(FAMILY[fam], splits):
        got, name = run_seq(K, q, kc, vc, n_ctx, depths, mask)
    REACHED.add(name)
    assert name == expect
    for s, dpt in enumerate(depths):
        m = mask[s, 0][:, :dpt].copy() if masked else None
        check(got[s], KD.oracle_attn(q[s], kcs[s], vcs[s], dpt, 2, m, 1 / 16))


def test_seq_perhead_mask_general(gpu, oracle):
    """Per-sequence counts with a per-head mask: the general kernel's 8-wave mask-tile form."""
    K = gpu
    nh, n_ctx, depths, T = 16, 2000, [2000, 1500], 3
    kcs, vcs = zip(*[layer(90 + s, n_ctx) for s in range(2)])
    kc, vc = np.stack(kcs), np.stack(vcs)
    q = KD.q_rows(90, 1, T, nh, batch=2)
    mask = np.concatenate([make_mask("perhead", T, n_ctx, nh, 90 + s) for s in range(2)])   # [2, nh, T, n_ctx]
    say("seq general, per-head mask")
    with forced(KK.FA_KERNEL_GENERAL, 1):
        qd = dev(q.astype(np.float32))
        kd, vd = dev(kc), dev(vc)
        kv = K.tensor(kd.data_ptr(), K.TYPE_Q8_0, (HD, n_ctx, 2, 2), (34, 544, 272, n_ctx * 544))
        vv = K.tensor(vd.data_ptr(), K.TYPE_Q8_0, (HD, n_ctx, 2, 2), (34, 544, 272, n_ctx * 544))
        md = dev(mask.view(np.float16))
        mv = K.mask_view(md)
        out = torch.full((2, T, nh, HD), float("nan"), dtype=torch.float32, device="cuda")
        ws = torch.empty(max(256, K.fattn_workspace_size_seq(K.q_view(qd), kv, vv, mv, depths)), dtype=torch.uint8,
                         device="cuda")
        K.flash_attn_ext_seq(K.q_view(qd), kv, vv, mv, 1 / 16, K.out_view(out), depths, ws=ws)
        name = K.last_kernel()
        got = host(out)
    REACHED.add(name)
    assert name == "k_fattn_q8_0<2, true, WAVES, 16, true>"
    for s, dpt in enumerate(depths):
        check(got[s], ref_dense(q[s], kcs[s], vcs[s], dpt, mask[s:s + 1, :, :, :dpt], nh))


CELLS = [
    ("vd", 1, "k_fa_vd<0, 1, false, false, true>"),
    ("vd", 2, "k_fa_vd<1, 0, false, false, true>"),
    ("vd", 3, "k_fa_vd<1, 1, false, false, true>"),
    ("vs", 1, "k_fa_vs<0, 1, false, false, true>"),
    ("vs", 2, "k_fa_vs<1, 0, false, false, true>"),
    ("vs", 3, "k_fa_vs<1, 1, false, false, true>"),
    ("dec", 2, "k_fa_dec<1, false, false, true>"),
    ("dec", 3, "k_fa_dec<2, false, false, true>"),
]


@pytest.mark.parametrize("fam,T,expect", CELLS)
def test_cells_family(gpu, oracle, fam, T, expect):
    K = gpu
    nh, n_rows = 16, 4096
    kc, vc = layer(95, n_rows)
    rng = np.random.default_rng(95 + T)
    lists = [np.union1d(rng.choice(n_rows - 64, 600 + 37 * h, replace=False), np.arange(n_rows - 64, n_rows))
             .astype(np.int32) for h in range(2)]
    q = KD.q_rows(95, T, T, nh)[0]
    say(f"cells {fam} T={T} (expect {expect})")
    with forced(FAMILY[fam]):
        got, name = run_cells(K, q, kc, vc, lists, n_rows - T)
    REACHED.add(name)
    assert name == expect
    check(got, KD.oracle_attn_cells(q, kc, vc, lists, n_rows - T, 1 / 16))


@pytest.mark.parametrize("masked", [False, True])
def test_prefill_family(gpu, oracle, masked):
    K = gpu
    T, nh, n_past = 64, 16, 1000
    kc, vc = layer(97, n_past + T)
    q = KD.q_rows(97, 1, T, nh)[0]
    mask = O.causal_mask(T, n_past) if masked else None
    say(f"prefill T=64 masked={masked}")
    got, name = run_dense(K, q, kc, vc, n_past + T, mask)
    REACHED.add(name)
    assert name == f"k_fa_pre<{'true' if masked else 'false'}>"
    check(got, ref_dense(q, kc, vc, n_past + T, mask, nh))


def test_perhead_mask_long_block(gpu, oracle):
    """8 positions x 8 heads per KV head (64 rows) with a per-head mask: the planner's general kernel."""
    K = gpu
    T, nh, n_kv = 8, 16, 2500
    kc, vc = layer(98, n_kv)
    q = KD.q_rows(98, 1, T, nh)[0]
    mask = make_mask("perhead", T, n_kv, nh, 98)
    say("per-head mask, T=8, GQA 8")
    got, name = run_dense(K, q, kc, vc, n_kv, mask)
    REACHED.add(name)
    assert name.startswith("k_fattn_q8_0<")
    check(got, ref_dense(q, kc, vc, n_kv, mask, nh))


def test_gqa2_causal_block_gated(gpu, oracle):
    """4 query heads over 2 KV heads, 40 causal positions (80 rows per KV head): the
    general kernel, plain and with the output gate."""
    K = gpu
    T, nh, n_kv = 40, 4, 2040
    kc, vc = layer(99, n_kv)
    q = KD.q_rows(99, 1, T, nh)[0]
    mask = O.causal_mask(T, n_kv - T)
    say("gqa 2, T=40, causal")
    got, name = run_dense(K, q, kc, vc, n_kv, mask)
    REACHED.add(name)
    assert name.startswith("k_fattn_q8_0<")
    ref = ref_dense(q, kc, vc, n_kv, mask, nh)
    check(got, ref)
    gate = (np.random.default_rng(99).standard_normal((1, T, nh, HD)) * 2).astype(np.float32)
    qd, kd, vd, md, gd = dev(q[None].astype(np.float32)), dev(kc), dev(vc), dev(mask.view(np.float16)), dev(gate)
    out = torch.full((1, T, nh, HD), float("nan"), dtype=torch.float32, device="cuda")
    say("gqa 2, T=40, causal, gated")
    K.flash_attn_ext_gated(K.q_view(qd), K.cache_attn_view(kd, n_kv, 2), K.cache_attn_view(vd, n_kv, 2),
                           K.mask_view(md), 1 / 16, K.out_view(out), gd)
    assert K.last_kernel() == name
    sig = (1.0 / (1.0 + np.exp(-gate[0].astype(np.float64)))).astype(np.float32)
    check(host(out)[0], ref * sig)


@pytest.mark.parametrize("fam,splits", [("vs", 1), ("vs", 0), ("vd", 1)])
def test_gated_verify_family(gpu, oracle, fam, splits):
    """The output gate on the verify kernels: with one split the kernel writes the gated
    rows itself, with several the merge launch does."""
    K = gpu
    T, nh, n_kv = 3, 16, 2500
    kc, vc = layer(103, n_kv)
    q = KD.q_rows(103, 1, T, nh)[0]
    mask = O.causal_mask(T, n_kv - T)
    gate = (np.random.default_rng(103).standard_normal((1, T, nh, HD)) * 2).astype(np.float32)
    qd, kd, vd, md, gd = dev(q[None].astype(np.float32)), dev(kc), dev(vc), dev(mask.view(np.float16)), dev(gate)
    out = torch.full((1, T, nh, HD), float("nan"), dtype=torch.float32, device="cuda")
    say(f"gated {fam} splits={splits}")
    with forced(FAMILY[fam], splits):
        K.flash_attn_ext_gated(K.q_view(qd), K.cache_attn_view(kd, n_kv, 2), K.cache_attn_view(vd, n_kv, 2),
                               K.mask_view(md), 1 / 16, K.out_view(out), gd)
        name = K.last_kernel()
    assert name == f"k_fa_{fam}<1, 1, true, false, false>"
    sig = (1.0 / (1.0 + np.exp(-gate[0].astype(np.float64)))).astype(np.float32)
    check(host(out)[0], ref_dense(q, kc, vc, n_kv, mask, nh) * sig)


def test_seq_long_block(gpu, oracle):
    """Per-sequence counts with 8 positions per sequence (64 rows per KV head)."""
    K = gpu
    nh, n_ctx, depths, T = 16, 2000, [1200, 2000], 8
    kcs, vcs = zip(*[layer(100 + s, n_ctx) for s in range(2)])
    kc, vc = np.stack(kcs), np.stack(vcs)
    q = KD.q_rows(100, 1, T, nh, batch=2)
    say("seq T=8")
    got, name = run_seq(K, q, kc, vc, n_ctx, depths, None)
    REACHED.add(name)
    assert name.startswith("k_fattn_q8_0<")
    for s, dpt in enumerate(depths):
        check(got[s], KD.oracle_attn(q[s], kcs[s], vcs[s], dpt, 2, None, 1 / 16))


@pytest.mark.parametrize("fam,T", [("vd", 3), ("vs", 3), ("dec", 3), ("general", 3), ("auto", 8)])
def test_append_family(gpu, oracle, fam, T):
    """The fused K/V append on each family: cache bytes are the oracle's quantisation of
    the new rows, and the output is the oracle's attention over the appended cache."""
    K = gpu
    nh, n_past = 16, 2000
    n_kv = n_past + T
    kc, vc = layer(101, n_kv, n_kv)
    newk = KD.kv_rows(101, 1, KD.K_KIND, T, first_row=n_past, outliers=True)
    newv = KD.kv_rows(101, 1, KD.V_KIND, T, first_row=n_past, outliers=True)
    q = KD.q_rows(101, 2, T, nh)[0]
    mask = O.causal_mask(T, n_past)
    kd, vd = dev(kc), dev(vc)
    qd, md = dev(q[None].astype(np.float32)), dev(mask.view(np.float16))
    out = torch.full((1, T, nh, HD), float("nan"), dtype=torch.float32, device="cuda")
    say(f"append {fam} T={T}")
    with forced(FAMILY[fam]):
        K.flash_attn_ext_append(K.q_view(qd), K.cache_attn_view(kd, n_kv, 2), K.cache_attn_view(vd, n_kv, 2),
                                K.mask_view(md), 1 / 16, K.out_view(out), dev(newk.astype(np.float32)),
                                dev(newv.astype(np.float32)), n_past)
        name = K.last_kernel()
    REACHED.add(name)
    O.cpy(kc, newk, n_past, O.Q8_X86)
    O.cpy(vc, newv, n_past, O.Q8_X86)
    np.testing.assert_array_equal(host(kd), kc)
    np.testing.assert_array_equal(host(vd), vc)
    check(host(out)[0], KD.oracle_attn(q, kc, vc, n_kv, 2, mask, 1 / 16))


def test_forced_family_refuses_shapes_it_cannot_take(gpu):
    K = gpu
    T, nh, n_kv = 8, 16, 600
    kc, vc = layer(102, n_kv)
    q = KD.q_rows(102, 1, T, nh)[0]
    for fam in ("vd", "vs", "dec"):
        with forced(FAMILY[fam]):
            with pytest.raises(K.QwfnError) as e:
                run_dense(K, q, kc, vc, n_kv, None)
        assert e.value.code == K.ENOTSUP


def test_zz_every_kernel_reached():
    """Run after the cases above in this module: each instantiation was launched by one of them."""
    missing = sorted(set(ALL_KERNELS) - REACHED)
    assert not missing, missing
