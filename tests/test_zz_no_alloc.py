"""The allocation-free attention entry point (qwfn_flash_attn_ext_q8_0_noalloc)
against qwfn_flash_attn_ext_q8_0 with a caller workspace, through the C ABI,
on consecutive calls of decreasing size: the first (a 512-query prefill
chunk) needs more split partials than its 16 MiB scratch holds, so it runs
with fewer key splits and may differ by float rounding; the later ones (verify
at 16384, decode) use the same plan as the workspace call and must give
identical bits. Each result is also held to the oracle's tolerance."""
import ctypes

import numpy as np
import pytest
import torch

import kvdata as KD
from gpu_util import dev, host, say
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _case(K, seed, n_past, T, outliers):
    n_kv = n_past + T
    kc = KD.make_cache(KD.kv_rows(seed, 0, KD.K_KIND, n_kv, outliers=outliers), n_kv)
    vc = KD.make_cache(KD.kv_rows(seed, 0, KD.V_KIND, n_kv, outliers=outliers), n_kv)
    q = KD.q_rows(seed, 0, T, 16)[0]
    mask = O.causal_mask(T, n_past) if T > 1 else None
    kd, vd, qd = dev(kc), dev(vc), dev(q[None].astype(np.float32))
    kv, vv = K.cache_attn_view(kd, n_kv, 2), K.cache_attn_view(vd, n_kv, 2)
    md = dev(mask.view(np.float16)) if mask is not None else None
    mv = K.mask_view(md) if md is not None else None
    qv = K.q_view(qd)
    r = ctypes.byref
    L = K.load()
    out_ws = torch.full((1, T, 16, 256), float("nan"), dtype=torch.float32, device="cuda")
    n = K.fattn_workspace_size(qv, kv, vv, mv)
    ws = torch.empty(max(n, 256), dtype=torch.uint8, device="cuda")
    K.check(L.qwfn_flash_attn_ext_q8_0(r(qv), r(kv), r(vv), r(mv) if mv is not None else None, 1 / 16, 0.0, 0.0,
                                       r(K.out_view(out_ws)), K.Q8_X86, ws.data_ptr(), ws.numel(), None))
    out_na = torch.full((1, T, 16, 256), float("nan"), dtype=torch.float32, device="cuda")
    K.check(L.qwfn_flash_attn_ext_q8_0_noalloc(r(qv), r(kv), r(vv), r(mv) if mv is not None else None, 1 / 16, 0.0,
                                               0.0, r(K.out_view(out_na)), K.Q8_X86, None))
    a, b = host(out_ws)[0], host(out_na)[0]
    if T <= 4:
        ref = KD.oracle_attn(q, kc, vc, n_kv, 2, mask, 1 / 16)
    else:   # long query blocks: a subset of tokens, each over the keys its causal row shows
        toks = (0, 1, T // 2, T - 1)
        a, b = a[list(toks)], b[list(toks)]
        ref = np.concatenate([KD.oracle_attn(q[t:t + 1], kc, vc, n_past + t + 1, 2, None, 1 / 16) for t in toks])
    return a, b, ref, n


def test_noalloc_matches_workspace_entry_point(gpu, oracle):
    K = gpu
    # 1: a 512-query prefill chunk at depth 4096: the workspace plan's partials exceed 16 MiB
    say("noalloc: T=512 depth 4096 (capped splits)")
    a, b, ref, n = _case(K, 31, 4096, 512, True)
    assert n > 16 << 20
    assert np.isfinite(b).all()
    assert KD.err_stats(b, a)[0] <= 2e-5
    mx, mean = KD.err_stats(b, ref)
    assert mx <= KD.MAX_ABS_TOL and mean <= KD.MEAN_ABS_TOL
    # 2: a smaller call right after (verify at 16384): same plan, same bits
    say("noalloc: T=3 depth 16384")
    a, b, ref, n = _case(K, 32, 16384, 3, True)
    assert n <= 16 << 20
    assert np.array_equal(a, b)
    mx, mean = KD.err_stats(b, ref)
    assert mx <= KD.MAX_ABS_TOL and mean <= KD.MEAN_ABS_TOL
    # 3: smaller again (decode at 3000, no mask)
    say("noalloc: T=1 depth 3000")
    a, b, ref, _ = _case(K, 33, 3000, 1, False)
    assert np.array_equal(a, b)
    mx, mean = KD.err_stats(b, ref)
    assert mx <= KD.MAX_ABS_TOL and mean <= KD.MEAN_ABS_TOL


def test_noalloc_rejects_bad_calls(gpu):
    K = gpu
    L = K.load()
    q = K.tensor(0x7F0000000000, K.TYPE_F32, (256, 1, 16, 1), (4, 1024, 1024, 16384))
    kv = K.tensor(0x7F0000000000, K.TYPE_Q8_0, (128, 10, 2, 1), (34, 544, 272, 5440))
    r = ctypes.byref
    assert L.qwfn_flash_attn_ext_q8_0_noalloc(r(q), r(kv), r(kv), None, 1.0, 0.0, 0.0, r(q), 1, None) == K.ENOTSUP
