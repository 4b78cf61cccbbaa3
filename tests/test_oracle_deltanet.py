"""Pins of the oracle's gated delta rule (the recurrence ggml_gated_delta_net
computes, qwfn_graph.cpp:240-278): an fp64 brute force in the matrix form
S_t = (I - beta k k^T) e^g S_{t-1} + beta k v^T, out_t = S_t^T q scale; the
closed forms at beta = 0 (pure decay) and of one write into a zero state; the
rollback snapshots equal the recurrence stopped early; key heads shared by
consecutive value heads."""
import numpy as np
import pytest

from oracle import oracle as O


def _inputs(seed, T, n_k, n_v, d):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((T, n_k, d)).astype(np.float32)
    k = rng.standard_normal((T, n_k, d)).astype(np.float32)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((T, n_v, d)).astype(np.float32)
    g = -rng.uniform(0.01, 2.0, (T, n_v)).astype(np.float32)
    beta = rng.uniform(0.05, 0.95, (T, n_v)).astype(np.float32)
    s0 = (rng.standard_normal((n_v, d, d)) * 0.1).astype(np.float32)
    return q, k, v, g, beta, s0


def _brute(q, k, v, g, beta, s0, scale):
    T, n_k, d = q.shape
    n_v = v.shape[1]
    rep = n_v // n_k
    S = s0.astype(np.float64).copy()
    out = np.zeros((T, n_v, d))
    states = []
    for t in range(T):
        for h in range(n_v):
            kk = k[t, h // rep].astype(np.float64)
            qq = q[t, h // rep].astype(np.float64)
            b = float(beta[t, h])
            A = np.eye(d) - b * np.outer(kk, kk)
            S[h] = A @ (np.exp(float(g[t, h])) * S[h]) + b * np.outer(kk, v[t, h].astype(np.float64))
            out[t, h] = S[h].T @ qq * scale
        states.append(S.copy())
    return out, states


@pytest.mark.parametrize("T,n_k,n_v,d", [(5, 1, 3, 4), (7, 2, 6, 8), (3, 16, 48, 16)])
def test_gated_delta_net_fp64_brute_force(T, n_k, n_v, d):
    q, k, v, g, beta, s0 = _inputs(T * d, T, n_k, n_v, d)
    scale = 1.0 / np.sqrt(d)
    out, st, snap = O.gated_delta_net(q, k, v, g, beta, s0, n_snap=T - 1)
    ref_out, states = _brute(q, k, v, g, beta, s0, scale)
    np.testing.assert_allclose(out, ref_out, rtol=1e-4, atol=2e-5)
    np.testing.assert_allclose(st, states[-1], rtol=1e-4, atol=2e-5)
    for s in range(1, T):
        np.testing.assert_allclose(snap[s - 1], states[T - 1 - s], rtol=1e-4, atol=2e-5)


def test_gated_delta_net_closed_forms():
    T, n_k, n_v, d = 4, 1, 2, 8
    q, k, v, g, beta, s0 = _inputs(11, T, n_k, n_v, d)
    # beta = 0: the state only decays, by exp of the summed gates
    out, st, _ = O.gated_delta_net(q, k, v, g, np.zeros_like(beta), s0)
    decay = np.exp(g.astype(np.float64).sum(axis=0))
    np.testing.assert_allclose(st, s0 * decay[:, None, None], rtol=2e-5, atol=1e-7)
    # one token, zero state, no decay: S = beta k v^T, out = beta (k . q) v / sqrt(d)
    out, st, _ = O.gated_delta_net(q[:1], k[:1], v[:1], np.zeros((1, n_v), np.float32), beta[:1],
                                   np.zeros_like(s0))
    for h in range(n_v):
        np.testing.assert_allclose(st[h], beta[0, h] * np.outer(k[0, 0], v[0, h]), rtol=1e-5, atol=1e-7)
        np.testing.assert_allclose(out[0, h], beta[0, h] * float(k[0, 0] @ q[0, 0]) * v[0, h] / np.sqrt(d),
                                   rtol=1e-4, atol=1e-6)
    # a written key is recalled exactly with beta = 1 (delta rule): S^T k = v
    out, st, _ = O.gated_delta_net(q[:1], k[:1], v[:1], np.zeros((1, n_v), np.float32), np.ones((1, n_v), np.float32),
                                   s0)
    for h in range(n_v):
        np.testing.assert_allclose(st[h].T @ k[0, 0], v[0, h], rtol=1e-4, atol=1e-5)
