"""Pins the oracle's gated delta rule (math.rs:492-546) and the token-serial scan
against the delta-rule invariants and a float64 brute-force recurrence (CPU only)."""
from __future__ import annotations

import numpy as np


def _unit(rng, d):
    x = rng.standard_normal(d)
    return (x / np.linalg.norm(x)).astype(np.float32)


def test_delta_rule_retrieval_invariant(orc):
    """g = 1, beta = 1, |k| = 1: after the update S^T k == v, so o(q = k) == v."""
    rng = np.random.default_rng(1)
    d = 128
    S = rng.standard_normal((d, d)).astype(np.float32) * 0.1
    k = _unit(rng, d)
    v = rng.standard_normal(d).astype(np.float32)
    S2, o = orc.deltanet_head_step(S.reshape(-1), k, k, v, 1.0, 1.0)
    assert np.allclose(o, v, atol=2e-5)
    assert np.allclose(S2.reshape(d, d).astype(np.float64).T @ k, v, atol=2e-5)


def test_beta_zero_is_pure_decay(orc):
    """beta = 0: delta = 0, so S' = g S and o = (g S)^T q."""
    rng = np.random.default_rng(2)
    d = 64
    S = rng.standard_normal((d, d)).astype(np.float32)
    q = rng.standard_normal(d).astype(np.float32)
    k = rng.standard_normal(d).astype(np.float32)
    v = rng.standard_normal(d).astype(np.float32)
    g = np.float32(0.93)
    S2, o = orc.deltanet_head_step(S.reshape(-1), q, k, v, float(g), 0.0)
    assert np.array_equal(S2.reshape(d, d), (S * g).astype(np.float32))
    assert np.allclose(o, (S * g).astype(np.float64).T @ q, rtol=1e-5, atol=1e-5)


def test_zero_k_and_q_rows_are_skipped_exactly(orc):
    """math.rs:520-523, 540-543: k_j == 0 / q_j == 0 rows are exact no-ops; o(q=0) == 0."""
    rng = np.random.default_rng(3)
    d = 32
    S = rng.standard_normal((d, d)).astype(np.float32)
    z = np.zeros(d, np.float32)
    v = rng.standard_normal(d).astype(np.float32)
    S2, o = orc.deltanet_head_step(S.reshape(-1), z, z, v, 1.0, 0.7)
    assert np.array_equal(S2.reshape(d, d), S)
    assert not o.any()


def _brute(q, k, v, gate, beta, S0, eps, d):
    """float64 gated delta rule with the projected_state normalisation (math.rs:833-846)."""
    T, H, _ = q.shape
    S = S0.astype(np.float64).copy()
    out = np.zeros((T, H, d))
    for t in range(T):
        for h in range(H):
            qq = q[t, h].astype(np.float64)
            kk = k[t, h].astype(np.float64)
            qq = qq / np.sqrt((qq ** 2).sum() + eps) / np.sqrt(d)
            kk = kk / np.sqrt((kk ** 2).sum() + eps)
            g = np.exp(np.float64(gate[t, h]))
            Sh = S[h] * g
            delta = beta[t, h] * (v[t, h] - Sh.T @ kk)
            Sh = Sh + np.outer(kk, delta)
            S[h] = Sh
            out[t, h] = Sh.T @ qq
    return out, S


def test_scan_matches_float64_bruteforce(orc):
    rng = np.random.default_rng(5)
    T, H, d, eps = 48, 3, 32, 1e-6
    q = rng.standard_normal((T, H, d)).astype(np.float32)
    k = rng.standard_normal((T, H, d)).astype(np.float32)
    v = rng.standard_normal((T, H, d)).astype(np.float32)
    gate = rng.uniform(-0.1, 0.0, (T, H)).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((T, H))))).astype(np.float32)
    S0 = (rng.standard_normal((H, d, d)) * 0.1).astype(np.float32)
    out, S = orc.deltanet_scan(q, k, v, gate, beta, S0, eps=eps, n_threads=2)
    exp, Sexp = _brute(q, k, v, gate, beta, S0, eps, d)
    assert np.allclose(out, exp, atol=2e-5)
    assert np.allclose(S, Sexp, atol=5e-5)


def test_scan_thread_invariant(orc):
    rng = np.random.default_rng(6)
    T, H, d = 8, 16, 128
    args = [rng.standard_normal((T, H, d)).astype(np.float32) for _ in range(3)]
    gate = rng.uniform(-0.1, 0.0, (T, H)).astype(np.float32)
    beta = rng.uniform(0, 1, (T, H)).astype(np.float32)
    S0 = np.zeros((H, d, d), np.float32)
    a = orc.deltanet_scan(*args, gate, beta, S0, n_threads=1)
    b = orc.deltanet_scan(*args, gate, beta, S0, n_threads=8)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
