"""GPU parity of the byte paths: q8_0 append (set_rows / cpy), raw gather and
snapshot restore. All results must be bit-exact against the oracle."""
import numpy as np
import pytest

import kvdata as KD
from gpu_util import dev, host, say
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def crafted_rows(rng) -> np.ndarray:
    """Rows that exercise rounding ties, 1-ulp inverse scales, zeros and fp16-subnormal scales."""
    rows = []
    r = np.zeros(512, np.float32)
    r[:8] = [127.0, 63.5, 62.5, 0.5, -0.5, -62.5, 1.5, -2.5]
    r[32:40] = [254.0, 1.0, -1.0, 3.0, -3.0, 5.0, 127.0, -127.0]
    rows.append(r)
    rows.append(np.zeros(512, np.float32))
    rows.append((rng.standard_normal(512) * 1e-4).astype(np.float32))       # d is an fp16 subnormal
    rows.append((rng.standard_normal(512) * 1e-7).astype(np.float32))       # d rounds to 0 in fp16
    rows.append((rng.standard_normal(512) * 3e4).astype(np.float32))
    # values placed at k + 0.5 steps of the x86 inverse scale
    amax = np.float32(2.7)
    idv = np.float32(np.float32(127) / amax)
    r = ((np.arange(512) % 120 + 0.5) / idv).astype(np.float32)
    r[::32] = amax
    rows.append(r)
    return np.stack(rows)


@pytest.mark.parametrize("variant", [O.Q8_REF, O.Q8_X86])
def test_set_rows_bit_exact(gpu, oracle, variant):
    K = gpu
    rng = np.random.default_rng(100 + variant)
    n_ctx = 1024
    cache = rng.integers(0, 256, (n_ctx, 544), dtype=np.uint8)
    src = np.concatenate([crafted_rows(rng), rng.standard_normal((250, 512)).astype(np.float32) *
                          (10.0 ** rng.uniform(-3, 3, (250, 1))).astype(np.float32)])
    idx = rng.permutation(n_ctx)[:src.shape[0]].astype(np.int32)
    say(f"set_rows variant={variant} n={src.shape[0]}")
    cd = dev(cache)
    K.set_rows_q8_0(cd, dev(src), dev(idx), variant)
    got = host(cd)
    exp = cache.copy()
    O.set_rows(exp, src, idx, variant)
    np.testing.assert_array_equal(got, exp)
    assert K.device_status() == 0


@pytest.mark.parametrize("variant", [O.Q8_REF, O.Q8_X86])
def test_cpy_prefill_chunk_bit_exact(gpu, oracle, variant):
    # config 3 shape: 512 rows appended at depth 4096 of one layer
    K = gpu
    rows = KD.kv_rows(3, 0, KD.K_KIND, 512, first_row=4096)
    cache = np.full((4096 + 600, 544), 0xA5, np.uint8)
    say(f"cpy 512 rows at 4096 variant={variant}")
    cd = dev(cache)
    K.cpy_f32_q8_0(dev(rows), cd, 4096, variant)
    got = host(cd)
    exp = cache.copy()
    O.cpy(exp, rows, 4096, variant)
    np.testing.assert_array_equal(got, exp)


def test_set_rows_strided_source(gpu, oracle):
    # src rows with a padded stride (not 16-byte multiple): scalar-load path
    K = gpu
    rng = np.random.default_rng(7)
    big = rng.standard_normal((5, 513)).astype(np.float32)
    src = big[:, :512]
    import torch
    sd = dev(big)[:, :512]
    idx = np.array([3, 1, 4, 0, 2], np.int32)
    cache = np.zeros((8, 544), np.uint8)
    say("set_rows strided source")
    cd = dev(cache)
    K.set_rows_q8_0(cd, sd, dev(idx), O.Q8_X86)
    exp = cache.copy()
    O.set_rows(exp, np.ascontiguousarray(src), idx)
    np.testing.assert_array_equal(host(cd), exp)
    del torch


def test_set_rows_out_of_range_index_is_flagged(gpu, oracle):
    K = gpu
    rng = np.random.default_rng(8)
    cache = rng.integers(0, 256, (16, 544), dtype=np.uint8)
    src = rng.standard_normal((3, 512)).astype(np.float32)
    idx = np.array([2, 16, 5], np.int32)                    # 16 is out of range
    say("set_rows with an out-of-range index")
    cd = dev(cache)
    K.set_rows_q8_0(cd, dev(src), dev(idx), O.Q8_X86)
    flags = K.device_status()
    got = host(cd)
    assert flags & K.DEVERR_SET_ROWS_INDEX
    exp = cache.copy()
    O.set_rows(exp, src[[0, 2]], idx[[0, 2]])
    np.testing.assert_array_equal(got, exp)
    assert K.device_status() == 0                           # flags clear on read


@pytest.mark.parametrize("variant", [O.Q8_REF, O.Q8_X86])
def test_fused_kv_append_bit_exact(gpu, oracle, variant):
    """The K and V appends of one layer in one launch equal two single appends, and the oracle:
    set_rows with crafted rows and one out-of-range index, and a 3-row cpy at a depth."""
    K = gpu
    rng = np.random.default_rng(300 + variant)
    n_ctx = 512
    kc = rng.integers(0, 256, (n_ctx, 544), dtype=np.uint8)
    vc = rng.integers(0, 256, (n_ctx, 544), dtype=np.uint8)
    ks = np.concatenate([crafted_rows(rng), rng.standard_normal((40, 512)).astype(np.float32)])
    vs = (rng.standard_normal(ks.shape) * 7).astype(np.float32)
    idx = rng.permutation(n_ctx)[:ks.shape[0]].astype(np.int32)
    idx[5] = n_ctx + 3                                       # flagged, row skipped
    say(f"set_rows_kv variant={variant} n={ks.shape[0]}")
    kd, vd = dev(kc), dev(vc)
    K.set_rows_q8_0_kv(kd, dev(ks), vd, dev(vs), dev(idx), variant)
    assert K.device_status() & K.DEVERR_SET_ROWS_INDEX
    keep = np.arange(ks.shape[0]) != 5
    for got, cache, src in ((host(kd), kc, ks), (host(vd), vc, vs)):
        exp = cache.copy()
        O.set_rows(exp, src[keep], idx[keep], variant)
        np.testing.assert_array_equal(got, exp)
    # the same through two single calls
    k2, v2 = dev(kc), dev(vc)
    K.set_rows_q8_0(k2, dev(ks), dev(idx), variant)
    K.set_rows_q8_0(v2, dev(vs), dev(idx), variant)
    K.device_status()
    np.testing.assert_array_equal(host(kd), host(k2))
    np.testing.assert_array_equal(host(vd), host(v2))
    # cpy of 3 rows at depth 300
    say(f"cpy_kv 3 rows at 300 variant={variant}")
    kd, vd = dev(kc), dev(vc)
    K.cpy_f32_q8_0_kv(dev(ks[:3]), kd, dev(vs[:3]), vd, 300, variant)
    for got, cache, src in ((host(kd), kc, ks[:3]), (host(vd), vc, vs[:3])):
        exp = cache.copy()
        O.cpy(exp, src, 300, variant)
        np.testing.assert_array_equal(got, exp)
    assert K.device_status() == 0


def test_get_rows_raw_cells(gpu, oracle):
    # qsa_gather raw: 2052 cells padded to 2304 with duplicates (qwfn_graph.cpp:681-693)
    K = gpu
    import torch
    rng = np.random.default_rng(9)
    cache = rng.integers(0, 256, (20000, 544), dtype=np.uint8)
    cells = np.sort(rng.choice(20000, 2052, replace=False)).astype(np.int32)
    gcells = np.concatenate([cells, cells[:2304 - 2052]])
    say("get_rows 2304 raw cells")
    out = torch.zeros((2304, 544), dtype=torch.uint8, device="cuda")
    K.get_rows_i32(dev(cache), dev(gcells), out)
    np.testing.assert_array_equal(host(out), O.get_rows(cache, gcells))


def test_gather_segments_per_head(gpu, oracle):
    # config 4: per-KV-head lists of top-128 blocks of 64 positions + the last 512
    K = gpu
    import torch
    n_ctx = 65536
    rng = np.random.default_rng(10)
    cache = rng.integers(0, 256, (n_ctx, 544), dtype=np.uint8)
    lists = []
    for h in range(2):
        scores = O.uniform(O.stream_key(4, 0, KD.SCORE_KIND, h), 1024)
        top = np.argsort(-scores, kind="stable")[:128]
        pos = (top[:, None] * 64 + np.arange(64)[None, :]).ravel()
        pos = np.union1d(pos, np.arange(n_ctx - 512, n_ctx))
        lists.append(pos.astype(np.int32))
    m = max(len(x) for x in lists)
    idx = np.stack([np.concatenate([x, np.repeat(x[-1:], m - len(x))]) for x in lists])
    say(f"gather_segments 2 x {m}")
    out = torch.zeros((2, m, 272), dtype=torch.uint8, device="cuda")
    K.gather_segments(dev(cache), dev(idx), out, 0, 272, 272)
    got = host(out)
    for h in range(2):
        np.testing.assert_array_equal(got[h], O.get_rows(cache, idx[h], 272, 272 * h))


@pytest.mark.parametrize("seg,m", [(272, 8704), (136, 100), (4, 1)])
def test_gather_segments_kv_pair(gpu, oracle, seg, m):
    """K and V gathered in one launch: the same bytes as the oracle's get_rows of each
    (16-byte units at 272 / 136, 4-byte units at 4); the outputs keep no stale bytes."""
    K = gpu
    import torch
    n_ctx = 65536
    rng = np.random.default_rng(seg + m)
    kc = rng.integers(0, 256, (n_ctx, 544), dtype=np.uint8)
    vc = rng.integers(0, 256, (n_ctx, 544), dtype=np.uint8)
    idx = np.stack([np.sort(rng.choice(n_ctx, m, replace=False)) for _ in range(2)]).astype(np.int32)
    say(f"gather_segments_kv 2 x {m} x {seg} B")
    gk = torch.full((2, m, seg), 7, dtype=torch.uint8, device="cuda")
    gv = torch.full((2, m, seg), 9, dtype=torch.uint8, device="cuda")
    K.gather_segments_kv(dev(kc), dev(vc), dev(idx), gk, gv, 0, 272, seg)
    assert K.device_status() == 0
    for h in range(2):
        np.testing.assert_array_equal(host(gk)[h], O.get_rows(kc, idx[h], seg, 272 * h))
        np.testing.assert_array_equal(host(gv)[h], O.get_rows(vc, idx[h], seg, 272 * h))


def test_gather_out_of_range_flagged(gpu, oracle):
    K = gpu
    import torch
    cache = np.arange(10 * 544, dtype=np.uint32).astype(np.uint8).reshape(10, 544)
    idx = np.array([1, 10, 3, -1], np.int32)
    say("get_rows with out-of-range indices")
    out = torch.zeros((4, 544), dtype=torch.uint8, device="cuda")
    K.get_rows_i32(dev(cache), dev(idx), out)
    assert K.device_status() & K.DEVERR_GET_ROWS_INDEX
    got = host(out)
    np.testing.assert_array_equal(got[0], cache[1])
    np.testing.assert_array_equal(got[2], cache[3])
    assert not got[1].any() and not got[3].any()


@pytest.mark.parametrize("src_kind", [0, 1])
def test_restore_into_slots(gpu, src_kind):
    # config 5 in miniature: KV parts (rows * 544) and recurrent-state parts into 4 slots
    K = gpu
    import torch
    rng = np.random.default_rng(11)
    sizes = [1000 * 544, 1000 * 544, 32 * 128 * 128 * 4, 3 * 10240 * 4, 37]
    parts = [rng.integers(0, 256, s, dtype=np.uint8) for s in sizes]
    if src_kind == 0:
        src_t = [dev(p) for p in parts]
    else:
        src_t = [torch.from_numpy(p).pin_memory() for p in parts]
    n_slots = 4
    dst_t = [[torch.zeros(s + 64, dtype=torch.uint8, device="cuda") for s in sizes] for _ in range(n_slots)]
    say(f"state_restore kind={src_kind}")
    K.state_restore([t.data_ptr() for t in src_t], sizes,
                    [dst_t[s][p].data_ptr() for s in range(n_slots) for p in range(len(sizes))], n_slots, src_kind)
    torch.cuda.synchronize()
    for s in range(n_slots):
        for p in range(len(sizes)):
            got = dst_t[s][p].cpu().numpy()
            np.testing.assert_array_equal(got[:sizes[p]], parts[p])
            assert not got[sizes[p]:].any()
