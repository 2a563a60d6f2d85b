"""Pins the oracle's Turbo KV codec (KvCacheFormat::Turbo, reference
inference.rs:346-1334) on the CPU:

  * SplitMix64 against its published known answers (seed 0; seed 1234567);
  * the reference's own self-inverse transform tests for power-of-two and other
    head sizes (4546-4566);
  * the transform against the closed form S2 (H / sqrt(n)) S1 with a Sylvester
    Hadamard matrix from scipy;
  * the head quantiser against its definition evaluated in float64
    (sigma, codes by threshold, residual norm, residual sign sketch);
  * attention over a Turbo cache against the float64 closed form
    score = sigma (q_rot . C[code]) + gamma sqrt(pi/2/d) (q_proj . sgn),
    out = R^-1 (sum p sigma C + Rres^-1 sum p r sgn),
    at the reference's attention-oracle tolerance 2e-5 * max(|x|, 1)
    (src/engine/multimodal/mod.rs:724-728).
"""
from __future__ import annotations

import numpy as np
import pytest
from scipy.linalg import hadamard

C = np.array([-1.510417, -0.45278, 0.45278, 1.510417], np.float64)
TH = 0.9815985


def test_splitmix64_known_answers(orc):
    assert orc.splitmix64(0) == 0xE220A8397B1DCDAF
    g = 0x9E3779B97F4A7C15
    seq = [orc.splitmix64((1234567 + k * g) % 2**64) for k in range(5)]
    assert seq == [6457827717110365317, 3203168211198807973, 9817491932198370423,
                   4593380528125082431, 16408922859458223821]


def _py_sign_bits(orc, layer, kv_head, salt, n):
    """The sign rule of turboquant_build_sign_table (inference.rs:370-395) with the
    oracle's SplitMix64 (pinned above)."""
    seed = orc.splitmix64(((layer << 32) ^ kv_head ^ salt) % 2**64)
    return np.array([orc.splitmix64(seed ^ i) & 1 for i in range(n)], np.uint8)


SALTS = [0x9E3779B97F4A7C15, 0xC2B2AE3D27D4EB4F, 0x165667B19E3779F9, 0xD6E8FEB86659FD93]


def test_sign_table_layout(orc):
    L, G, d = 3, 5, 40
    t = orc.turbo_sign_table(L, G, d)
    assert t.shape == (4, L, G, 5)
    for slot in range(4):
        for layer in range(L):
            for g in range(G):
                bits = np.unpackbits(t[slot, layer, g], bitorder="little")[:d]
                assert np.array_equal(bits, _py_sign_bits(orc, layer, g, SALTS[slot], d))


def _signs(t, slot, layer, g, n):
    return 1.0 - 2.0 * np.unpackbits(t[slot, layer, g], bitorder="little")[:n].astype(np.float64)


def test_transform_self_inverse_reference_cases(orc):
    """inference.rs:4546-4566: rotation salts at (layer 2, kv head 3), n = 8 (1e-5);
    residual salts at (layer 1, kv head 7), n = 6 (no FWHT, 1e-6)."""
    t8 = orc.turbo_sign_table(3, 8, 8)
    v = np.array([0.25, -0.5, 1.0, -1.5, 0.75, 0.125, -0.25, 0.5], np.float32)
    fwd = orc.turbo_transform(v, t8[0, 2, 3], t8[1, 2, 3])
    back = orc.turbo_transform(fwd, t8[1, 2, 3], t8[0, 2, 3])
    assert np.all(np.abs(back - v) < 1e-5)
    assert not np.allclose(fwd, v)
    t6 = orc.turbo_sign_table(2, 8, 6)
    w = np.array([0.25, -0.5, 1.0, -1.5, 0.75, 0.125], np.float32)
    fwd6 = orc.turbo_transform(w, t6[2, 1, 7], t6[3, 1, 7])
    assert np.all(np.abs(orc.turbo_transform(fwd6, t6[3, 1, 7], t6[2, 1, 7]) - w) < 1e-6)
    # non-power-of-two: only the two sign flips apply
    s = _signs(t6, 2, 1, 7, 6) * _signs(t6, 3, 1, 7, 6)
    assert np.array_equal(fwd6, (w * s).astype(np.float32))


@pytest.mark.parametrize("n", [8, 64, 128, 256])
def test_transform_hadamard_closed_form(orc, n):
    t = orc.turbo_sign_table(1, 2, n)
    x = np.random.default_rng(n).standard_normal(n).astype(np.float32)
    got = orc.turbo_transform(x, t[0, 0, 1], t[1, 0, 1])
    H = hadamard(n).astype(np.float64) / np.sqrt(n)
    exp = _signs(t, 1, 0, 1, n) * (H @ (_signs(t, 0, 0, 1, n) * x.astype(np.float64)))
    assert np.allclose(got, exp, rtol=0, atol=2e-6 * np.abs(x).max() * np.sqrt(np.log2(n)))


def _rot(t, slot_a, slot_b, layer, g, x):
    n = x.size
    H = hadamard(n).astype(np.float64) / np.sqrt(n)
    return _signs(t, slot_b, layer, g, n) * (H @ (_signs(t, slot_a, layer, g, n) * x))


@pytest.mark.parametrize("n", [64, 128])
def test_quantize_head_definition(orc, n):
    t = orc.turbo_sign_table(2, 3, n)
    rng = np.random.default_rng(3 + n)
    for trial in range(20):
        x = (rng.standard_normal(n) * rng.uniform(0.1, 10)).astype(np.float32)
        base, sign, sigma, gamma = orc.turbo_quantize_head(x, t, 1, 2)
        rot = _rot(t, 0, 1, 1, 2, x.astype(np.float64))
        assert abs(sigma - np.linalg.norm(rot) / np.sqrt(n)) <= 1e-5 * sigma
        codes = np.array([(base[i // 4] >> (2 * (i % 4))) & 3 for i in range(n)])
        z = rot / sigma
        exp = np.where(z < -TH, 0, np.where(z < 0, 1, np.where(z < TH, 2, 3)))
        clear = (np.abs(np.abs(z) - TH) > 1e-4) & (np.abs(z) > 1e-4)
        assert np.array_equal(codes[clear], exp[clear])
        res = rot - C[codes] * sigma
        assert abs(gamma - np.linalg.norm(res)) <= 1e-4 * max(gamma, 1e-3)
        sk = _rot(t, 2, 3, 1, 2, res / np.linalg.norm(res))
        bits = np.unpackbits(sign, bitorder="little")[:n]
        ok = np.abs(sk) > 1e-5
        assert np.array_equal(bits[ok], (sk[ok] >= 0).astype(np.uint8))
    base, sign, sigma, gamma = orc.turbo_quantize_head(np.zeros(n, np.float32), t, 0, 0)
    assert sigma == 0.0 and gamma == 0.0 and not base.any() and np.all(sign == 0xFF)


def _decode_turbo_head(c: "object", row, g, d):
    """(codes [d], signs +-1 [d], sigma, gamma) of (row, kv head g) from a TurboCache."""
    kv_dim = c.n_kv_heads * d
    off = row * kv_dim + g * d
    aux = row * c.n_kv_heads + g
    out = []
    for base, sign, sc, rs in ((c.kbase, c.ksign, c.kscale, c.kres), (c.vbase, c.vsign, c.vscale, c.vres)):
        idx = off + np.arange(d)
        codes = (base[idx // 4] >> (2 * (idx % 4))) & 3
        sg = np.where((sign[idx // 8] >> (idx % 8)) & 1, 1.0, -1.0)
        out.append((codes, sg, float(sc[aux]), float(rs[aux])))
    return out


@pytest.mark.parametrize("online", [False, True])
def test_attention_turbo_closed_form(orc, online):
    H, G, d, L, layer, n_layers = 8, 2, 128, 150, 1, 2
    t = orc.turbo_sign_table(n_layers, G, d)
    rng = np.random.default_rng(17)
    cache = orc.TurboCache(L, G, d)
    K = rng.standard_normal((L, G * d)).astype(np.float32)
    V = rng.standard_normal((L, G * d)).astype(np.float32)
    for r in range(L):
        orc.kv_write_turbo(cache, r, K[r], V[r], t, layer)
    q = rng.standard_normal(H * d).astype(np.float32)
    s0, s1 = 7, 149
    out = orc.attention_token_turbo(q, cache, t, layer, H, s0, s1, online=online, n_threads=4)
    rfac = np.sqrt(np.float64(np.float32(1.5707964)) / d)
    for h in range(H):
        g = h // (H // G)
        qr = _rot(t, 0, 1, layer, g, q[h * d:(h + 1) * d].astype(np.float64))
        qp = _rot(t, 2, 3, layer, g, qr)
        sc = np.zeros(s1 - s0)
        vb = []
        for j, r in enumerate(range(s0, s1)):
            (kc, ks, ksig, kgam), (vc, vsg, vsig, vgam) = _decode_turbo_head(cache, r, g, d)
            sc[j] = ksig * (qr @ C[kc]) + kgam * rfac * (qp @ ks)
            vb.append((vc, vsg, vsig, vgam))
        sc /= np.sqrt(d)
        p = np.exp(sc - sc.max())
        p /= p.sum()
        base = sum(p[j] * vb[j][2] * C[vb[j][0]] for j in range(len(vb)))
        resid = sum(p[j] * vb[j][3] * rfac * vb[j][1] for j in range(len(vb)))
        # inverse rotations swap the pre / post sign slots
        o = _rot(t, 1, 0, layer, g, base + _rot(t, 3, 2, layer, g, resid))
        got = out[h * d:(h + 1) * d]
        assert np.all(np.abs(got - o) <= 2e-5 * np.maximum(np.abs(o), 1.0)), np.abs(got - o).max()
