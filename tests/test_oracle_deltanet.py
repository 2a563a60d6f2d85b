"""Pins the oracle's gated delta rule (math.rs:492-546) and the token-serial scan
against the delta-rule invariants and a float64 brute-force recurrence (CPU only)."""
from __future__ import annotations

import numpy as np
import pytest


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


# ---- the SSM layer around the recurrence (math.rs:766-953) ---------------------

@pytest.mark.parametrize("fused", [True, False])
def test_qwen3next_ssm_token_loop_closed_form(orc, fused):
    rng = np.random.default_rng(60 + int(fused))
    nk, nv, d, K, T, eps = 2, 4, 16, 4, 7, 1e-6
    conv_dim = nv * d + 2 * nk * d
    qkv = rng.standard_normal((T, conv_dim)).astype(np.float32)
    z = rng.standard_normal((T, nv * d)).astype(np.float32)
    ga = rng.standard_normal((T, 2 * nv if fused else nv)).astype(np.float32)
    gb = None if fused else rng.standard_normal((T, nv)).astype(np.float32)
    ga[2, 0] = 25.0                                       # softplus branches x > 20 / x < -20
    ga[3, 1] = -30.0
    cw = (0.3 * rng.standard_normal(conv_dim * K)).astype(np.float32)
    db = (0.1 * rng.standard_normal(nv)).astype(np.float32)
    sa = -rng.uniform(0.2, 1.0, nv).astype(np.float32)
    sn = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    out, hist, st = orc.qwen3next_ssm_tokens(qkv, z, ga, gb, n_k_heads=nk, n_v_heads=nv, head_dim=d,
                                            conv_kernel=K, conv_w=cw, dt_bias=db, ssm_a=sa, ssm_norm=sn,
                                            eps=eps)
    e_out, e_hist, e_st = orc.qwen3next_ssm_tokens_f64(
        qkv, z, ga, gb, n_k_heads=nk, n_v_heads=nv, head_dim=d, conv_kernel=K, conv_w=cw,
        dt_bias=db, ssm_a=sa, ssm_norm=sn, eps=eps)
    assert np.allclose(out, e_out, rtol=2e-5, atol=2e-5)
    assert np.array_equal(hist, qkv[T - (K - 1):])        # history = the last K-1 raw inputs
    assert np.array_equal(e_hist, hist)
    assert np.allclose(st, e_st, rtol=2e-5, atol=2e-5)


def test_qwen3next_ssm_tiling_is_periodic(orc):
    """K -> V head tiling repeats the key heads periodically ([h0..h(nk-1), h0..],
    math.rs:824-826): with distinct key heads and identical gates / values, value
    heads h and h + nk see the same q and k, so their outputs coincide."""
    rng = np.random.default_rng(70)
    nk, nv, d, K = 2, 4, 8, 2
    conv_dim = nv * d + 2 * nk * d
    qkv = rng.standard_normal((3, conv_dim)).astype(np.float32)
    v_part = qkv[:, 2 * nk * d:].reshape(3, nv, d)
    v_part[:, 2:] = v_part[:, :2]                         # v of heads 2,3 = heads 0,1
    qkv[:, 2 * nk * d:] = v_part.reshape(3, -1)
    z = np.ones((3, nv * d), np.float32)
    ga = np.zeros((3, nv), np.float32)
    gb = np.zeros((3, nv), np.float32)
    cw = np.tile(np.array([0.2, 0.9], np.float32), conv_dim)
    out, _, _ = orc.qwen3next_ssm_tokens(qkv, z, ga, gb, n_k_heads=nk, n_v_heads=nv, head_dim=d,
                                        conv_kernel=K, conv_w=cw, dt_bias=np.zeros(nv, np.float32),
                                        ssm_a=-np.ones(nv, np.float32), ssm_norm=np.ones(d, np.float32),
                                        eps=1e-6)
    o = out.reshape(3, nv, d)
    assert np.array_equal(o[:, 2:], o[:, :2]) and not np.allclose(o[:, 0], o[:, 1])


def _ssm_case(rng, nk, nv, d, K, T, fused):
    conv_dim = nv * d + 2 * nk * d
    return dict(
        qkv=rng.standard_normal((T, conv_dim)).astype(np.float32),
        z=rng.standard_normal((T, nv * d)).astype(np.float32),
        gate_a=rng.standard_normal((T, 2 * nv if fused else nv)).astype(np.float32),
        gate_b=None if fused else rng.standard_normal((T, nv)).astype(np.float32))


@pytest.mark.parametrize("nk,fused", [(8, True), (16, False)])
def test_qwen3next_ssm_f64_statement_at_config5_shape(orc, nk, fused):
    """The float64 statement (the reference point of the GPU SSM test) against the
    oracle's fp32 token loop at the config-5 shape, over two consecutive calls that
    carry the conv history and the state: they agree to fp32 rounding, and splitting
    the tokens over two calls changes neither."""
    rng = np.random.default_rng(90 + nk)
    nv, d, K, eps = 16, 128, 4, 1e-6
    conv_dim = nv * d + 2 * nk * d
    w = dict(conv_w=(0.3 * rng.standard_normal((conv_dim, K))).astype(np.float32),
             dt_bias=(0.1 * rng.standard_normal(nv)).astype(np.float32),
             ssm_a=-rng.uniform(0.2, 1.2, nv).astype(np.float32),
             ssm_norm=(1 + 0.1 * rng.standard_normal(d)).astype(np.float32))
    shape = dict(n_k_heads=nk, n_v_heads=nv, head_dim=d, conv_kernel=K, eps=eps)
    a = _ssm_case(rng, nk, nv, d, K, 9, fused)
    b = _ssm_case(rng, nk, nv, d, K, 6, fused)
    o1, h1, s1 = orc.qwen3next_ssm_tokens(**a, **shape, **w)
    o2, h2, s2 = orc.qwen3next_ssm_tokens(**b, **shape, **w, conv_hist=h1, state=s1)
    e1, eh1, es1 = orc.qwen3next_ssm_tokens_f64(**a, **shape, **w)
    e2, eh2, es2 = orc.qwen3next_ssm_tokens_f64(**b, **shape, **w, conv_hist=eh1, state=es1)
    for o, e in ((o1, e1), (o2, e2)):
        assert np.abs(o - e).max() <= 2e-5 * max(1.0, np.abs(e).max())
    assert np.array_equal(h2, eh2)
    assert np.abs(s2 - es2).max() <= 1e-5
    cat = {key: (None if a[key] is None else np.concatenate([a[key], b[key]])) for key in a}
    ec, ehc, esc = orc.qwen3next_ssm_tokens_f64(**cat, **shape, **w)
    assert np.allclose(ec, np.concatenate([e1, e2]), rtol=1e-12, atol=1e-12)
    assert np.array_equal(ehc, eh2) and np.allclose(esc, es2, rtol=1e-12, atol=1e-12)


def test_scan_sanitises_nonfinite_v_elements(orc):
    """v_dst = finite_or_zero(v_src) (math.rs:845): a NaN or inf value element acts as 0."""
    rng = np.random.default_rng(7)
    T, H, d = 6, 2, 16
    q, k, v = (rng.standard_normal((T, H, d)).astype(np.float32) for _ in range(3))
    gate = rng.uniform(-0.2, 0.0, (T, H)).astype(np.float32)
    beta = rng.uniform(0.2, 1.0, (T, H)).astype(np.float32)
    S0 = np.zeros((H, d, d), np.float32)
    vz = v.copy()
    vz[2, 1, 3] = 0.0
    vz[4, 0, 0] = 0.0
    vn = v.copy()
    vn[2, 1, 3] = np.nan
    vn[4, 0, 0] = -np.inf
    a = orc.deltanet_scan(q, k, vz, gate, beta, S0)
    b = orc.deltanet_scan(q, k, vn, gate, beta, S0)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    assert not np.array_equal(a[0], orc.deltanet_scan(q, k, v, gate, beta, S0)[0])
