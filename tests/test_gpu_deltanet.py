"""GPU parity of the Gated DeltaNet recurrent update with in-kernel rollback
snapshots (qwfn_graph.cpp:240-278, :208-238) against the oracle's gated delta
rule, at the model's shapes (16 key heads, 48 value heads of 128; q, k, v read
as the views of one [T, 10240] conv output, as the reference's
deltanet_conv_qkv takes them). Tolerance: the kernel's column sums run in 8
partial sums where the oracle sums in order, so outputs and states agree to
float rounding (2e-5 relative, 1e-6 absolute). Also: T tokens in one launch
equal T launches of one token, and snapshot s equals the final state of a
launch over T - s tokens."""
import numpy as np
import pytest
import torch

from gpu_util import dev, host, say
from oracle import oracle as O

pytestmark = pytest.mark.gpu
NK, NV, D, CONV = 16, 48, 128, 10240


def _inputs(seed, T):
    rng = np.random.default_rng(seed)
    conv = rng.standard_normal((T, CONV)).astype(np.float32)
    qk = conv[:, :2 * NK * D].reshape(T, 2, NK, D)
    qk /= np.linalg.norm(qk, axis=-1, keepdims=True)             # the l2 norm of deltanet_conv_qkv
    conv[:, :2 * NK * D] = qk.reshape(T, -1)
    g = -rng.uniform(0.0, 1.5, (T, NV)).astype(np.float32)
    beta = rng.uniform(0.0, 1.0, (T, NV)).astype(np.float32)
    s0 = (rng.standard_normal((NV, D, D)) * 0.05).astype(np.float32)
    return conv, g, beta, s0


def _views(conv):
    T = conv.shape[0]
    q = conv[:, :NK * D].reshape(T, NK, D)
    k = conv[:, NK * D:2 * NK * D].reshape(T, NK, D)
    v = conv[:, 2 * NK * D:].reshape(T, NV, D)
    return q, k, v


def _run(K, conv_d, g_d, beta_d, state_d, T, n_snap):
    out = torch.zeros((T, NV, D), dtype=torch.float32, device="cuda")
    snap = torch.zeros((max(n_snap, 1), NV, D, D), dtype=torch.float32, device="cuda")
    K.gated_delta_net(conv_d[:, :NK * D], conv_d[:, NK * D:2 * NK * D], conv_d[:, 2 * NK * D:], g_d, beta_d, state_d,
                      out, NK, snap if n_snap else None, n_snap)
    return out, snap


# the kernel loads the inputs of 4 tokens at a time: 5 and 9 tokens end in a
# partial group, and 8 snapshots of 9 tokens are taken inside earlier groups
@pytest.mark.parametrize("T,n_snap", [(1, 0), (3, 2), (4, 3), (5, 4), (9, 8), (16, 3)])
def test_gated_delta_net_matches_oracle(gpu, oracle, T, n_snap):
    K = gpu
    conv, g, beta, s0 = _inputs(T, T)
    conv_d, g_d, beta_d, state_d = dev(conv), dev(g), dev(beta), dev(s0)
    say(f"gated_delta_net T={T} n_snap={n_snap}")
    out, snap = _run(K, conv_d, g_d, beta_d, state_d, T, n_snap)
    q, k, v = _views(conv)
    r_out, r_st, r_snap = O.gated_delta_net(q, k, v, g, beta, s0, n_snap=n_snap)
    np.testing.assert_allclose(host(out), r_out, rtol=2e-5, atol=1e-6)
    np.testing.assert_allclose(host(state_d), r_st, rtol=2e-5, atol=1e-6)
    if n_snap:
        np.testing.assert_allclose(host(snap)[:n_snap], r_snap, rtol=2e-5, atol=1e-6)


def test_gated_delta_net_chaining_and_snapshots(gpu, oracle):
    K = gpu
    T = 4
    conv, g, beta, s0 = _inputs(99, T)
    conv_d, g_d, beta_d = dev(conv), dev(g), dev(beta)
    say("gated_delta_net: one launch of 4 tokens")
    st_all = dev(s0)
    out_all, snap = _run(K, conv_d, g_d, beta_d, st_all, T, T - 1)
    say("gated_delta_net: four launches of one token")
    st_one = dev(s0)
    outs = []
    states = []
    for t in range(T):
        o, _ = _run(K, conv_d[t:t + 1], g_d[t:t + 1], beta_d[t:t + 1], st_one, 1, 0)
        outs.append(host(o)[0])
        states.append(host(st_one).copy())
    np.testing.assert_array_equal(host(out_all), np.stack(outs))
    np.testing.assert_array_equal(host(st_all), states[-1])
    for s in range(1, T):
        np.testing.assert_array_equal(host(snap)[s - 1], states[T - 1 - s])
