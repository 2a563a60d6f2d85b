"""Pins the oracle's attention_token / prefill loop against the float64 closed form
softmax(q K^T s) V and the special cases the mathematics fixes (CPU only).

Tolerance 2e-5 * max(|x|, 1): the reference's own attention-oracle tolerance
(src/engine/multimodal/mod.rs:724-728)."""
from __future__ import annotations

import numpy as np
import pytest


def _np_attention(q, K, V, scale):
    s = (K.astype(np.float64) @ q.astype(np.float64)) * scale
    p = np.exp(s - s.max())
    return (p / p.sum()) @ V.astype(np.float64)


def _tol(x):
    return 2e-5 * np.maximum(np.abs(x), 1.0)


@pytest.mark.parametrize("online", [False, True])
@pytest.mark.parametrize("fmt", [0, 1, 2])
def test_attention_token_closed_form_gqa(orc, online, fmt):
    rng = np.random.default_rng(21 + fmt)
    H, Hk, d, L = 8, 2, 64, 300
    q = rng.standard_normal(H * d).astype(np.float32)
    kf = rng.standard_normal((L, Hk * d)).astype(np.float32)
    vf = rng.standard_normal((L, Hk * d)).astype(np.float32)
    if fmt == orc.F32:
        kc, vc = kf, vf
    else:
        conv = orc.f16_bits if fmt == orc.F16 else orc.bf16_bits
        kc, vc = conv(kf), conv(vf)
    K = orc.upcast(kc, fmt).reshape(L, Hk, d)
    V = orc.upcast(vc, fmt).reshape(L, Hk, d)
    s0, s1 = 17, 250
    out = orc.attention_token(q, kc, vc, fmt, H, Hk, d, s0, s1, online=online, n_threads=4)
    scale = 1.0 / np.sqrt(d)
    for h in range(H):
        g = h // (H // Hk)  # GQA: kv_head = h / kv_mul (inference.rs:2019)
        exp = _np_attention(q[h * d:(h + 1) * d], K[s0:s1, g], V[s0:s1, g], scale)
        assert np.all(np.abs(out[h * d:(h + 1) * d] - exp) <= _tol(exp))


def test_attention_token_special_cases(orc):
    rng = np.random.default_rng(4)
    H, d, L = 2, 32, 40
    kc = rng.standard_normal((L, H * d)).astype(np.float32)
    vc = rng.standard_normal((L, H * d)).astype(np.float32)
    q = rng.standard_normal(H * d).astype(np.float32)
    # one visible key: xb == v of that key
    out = orc.attention_token(q, kc, vc, orc.F32, H, H, d, 9, 10)
    assert np.array_equal(out, vc[9])
    # q == 0: uniform weights -> mean of V over the visible range
    out0 = orc.attention_token(np.zeros_like(q), kc, vc, orc.F32, H, H, d, 0, L)
    assert np.allclose(out0, vc.astype(np.float64).mean(axis=0), atol=2e-6)
    # identical keys: uniform weights too
    kc_eq = np.repeat(kc[:1], L, axis=0)
    out_eq = orc.attention_token(q, kc_eq, vc, orc.F32, H, H, d, 0, L)
    assert np.allclose(out_eq, vc.astype(np.float64).mean(axis=0), atol=2e-6)
    # apply_attn_scale off (Gemma3) equals scale 1
    a = orc.attention_token(q, kc, vc, orc.F32, H, H, d, 0, L, apply_attn_scale=False)
    b = orc.attention_token(q, kc, vc, orc.F32, H, H, d, 0, L, attn_scale=1.0)
    assert np.array_equal(a, b)


def test_attention_thread_count_invariant(orc):
    """The rayon-style parallel branch equals the serial one bit for bit."""
    rng = np.random.default_rng(8)
    H, Hk, d, L = 16, 8, 128, 513
    q = rng.standard_normal(H * d).astype(np.float32)
    kc = rng.standard_normal((L, Hk * d)).astype(np.float32)
    vc = rng.standard_normal((L, Hk * d)).astype(np.float32)
    a = orc.attention_token(q, kc, vc, orc.F32, H, Hk, d, 0, L, n_threads=1)
    b = orc.attention_token(q, kc, vc, orc.F32, H, Hk, d, 0, L, n_threads=8)
    assert np.array_equal(a, b)


def test_prefill_layer_closed_form_window_norm_rope(orc):
    """The token-serial prefill (norm -> RoPE -> write -> attend) against a float64
    restatement built from numpy primitives, local window 5, NeoX, Gemma scaling."""
    rng = np.random.default_rng(12)
    m, H, Hk, d, W, eps = 23, 4, 2, 32, 5, 1e-6
    q = rng.standard_normal((m, H * d)).astype(np.float32)
    k = rng.standard_normal((m, Hk * d)).astype(np.float32)
    v = rng.standard_normal((m, Hk * d)).astype(np.float32)
    qn = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    fr = orc.rope_freqs(1e4, d)
    out, kc, vc = orc.prefill_layer(q, k, v, n_heads=H, n_kv_heads=Hk, head_size=d, seq_len=m,
                                    fmt=orc.F32, rope_dim=d, neox=True, rope_freqs_tab=fr,
                                    rope_scale=1.0, is_gemma3=True, window=W, q_norm=qn,
                                    k_norm=kn, eps=eps)

    def norm(x, w, nh):
        x = x.astype(np.float64).reshape(nh, d)
        return (w * x / np.sqrt((x ** 2).mean(axis=1, keepdims=True) + eps))

    def rope(x, pos):
        ang = pos * fr.astype(np.float64)
        a, b = x[:, : d // 2], x[:, d // 2:]
        return np.concatenate([a * np.cos(ang) - b * np.sin(ang),
                               a * np.sin(ang) + b * np.cos(ang)], axis=1)

    Ks = np.stack([rope(norm(k[t], kn, Hk), t) for t in range(m)])
    Vs = v.astype(np.float64).reshape(m, Hk, d)
    assert np.allclose(kc.reshape(m, Hk, d), Ks, atol=2e-5)
    for t in range(m):
        qq = rope(norm(q[t], qn, H), t) / np.sqrt(d)
        s0 = max(0, t + 1 - W)
        for h in range(H):
            g = h // (H // Hk)
            exp = _np_attention(qq[h], Ks[s0:t + 1, g], Vs[s0:t + 1, g], 1.0)
            got = out[t, h * d:(h + 1) * d]
            assert np.all(np.abs(got - exp) <= 5e-5 * np.maximum(np.abs(exp), 1.0))


@pytest.mark.parametrize("online", [False, True])
@pytest.mark.parametrize("block", [False, True])
def test_attention_token_q8_closed_form(orc, online, block):
    """Q8 KV (inference.rs:1337-1483): scores and values use c * scale with the row's
    scale (row mode) or the 32-element block's scale (GGUF_Q8_BLOCK_SCALES).  Blocks
    and rows get very different magnitudes, so a wrong scale index fails."""
    rng = np.random.default_rng(31 + int(block))
    H, Hk, d, L = 8, 2, 128, 200
    kv_dim = Hk * d
    q = rng.standard_normal(H * d).astype(np.float32) * 0.2
    kf = rng.standard_normal((L, kv_dim)).astype(np.float32)
    vf = rng.standard_normal((L, kv_dim)).astype(np.float32)
    mag = np.exp(rng.uniform(-2, 2, size=(L, kv_dim // 32))).astype(np.float32)
    kf *= np.repeat(mag, 32, axis=1)
    vf *= np.repeat(mag[:, ::-1], 32, axis=1)
    rows = [orc.kv_quantize_row(kf[t], block) for t in range(L)]
    kq = np.stack([r[0] for r in rows])
    ks = np.concatenate([r[1] for r in rows])
    rows = [orc.kv_quantize_row(vf[t], block) for t in range(L)]
    vq = np.stack([r[0] for r in rows])
    vs = np.concatenate([r[1] for r in rows])
    per = kv_dim // 32 if block else 1
    Kd = (kq.astype(np.float64) * np.repeat(ks.reshape(L, per), kv_dim // per, axis=1))
    Vd = (vq.astype(np.float64) * np.repeat(vs.reshape(L, per), kv_dim // per, axis=1))
    fmt = orc.Q8B if block else orc.Q8
    s0, s1 = 5, 190
    out = orc.attention_token(q, kq, vq, fmt, H, Hk, d, s0, s1, key_scale=ks, value_scale=vs,
                              online=online, n_threads=4)
    for h in range(H):
        g = h // (H // Hk)
        exp = _np_attention(q[h * d:(h + 1) * d], Kd[s0:s1, g * d:(g + 1) * d],
                            Vd[s0:s1, g * d:(g + 1) * d], 1.0 / np.sqrt(d))
        assert np.all(np.abs(out[h * d:(h + 1) * d] - exp) <= _tol(exp))


@pytest.mark.parametrize("block", [False, True])
def test_prefill_layer_q8_writes_quantised_rows(orc, block):
    """Q8 prefill: every written row dequantises to within half a step of the post-RoPE
    K (resp. V) row, and each token's output is the closed form over the dequantised
    rows it can see."""
    rng = np.random.default_rng(41)
    H, Hk, d, m = 4, 2, 64, 24
    kv_dim = Hk * d
    q = rng.standard_normal((m, H * d)).astype(np.float32)
    k = rng.standard_normal((m, kv_dim)).astype(np.float32)
    v = rng.standard_normal((m, kv_dim)).astype(np.float32)
    fr = orc.rope_freqs(10000.0, d)
    fmt = orc.Q8B if block else orc.Q8
    xb, (kq, ks), (vq, vs) = orc.prefill_layer(q, k, v, n_heads=H, n_kv_heads=Hk, head_size=d,
                                               seq_len=m, fmt=fmt, rope_dim=d, neox=True,
                                               rope_freqs_tab=fr, rope_scale=1.0)
    per = kv_dim // 32 if block else 1
    Ks = np.repeat(ks.reshape(m, per), kv_dim // per, axis=1)
    Vs = np.repeat(vs.reshape(m, per), kv_dim // per, axis=1)
    Kd = kq.astype(np.float64) * Ks
    Vd = vq.astype(np.float64) * Vs
    assert np.all(np.abs(Vd - v) <= 0.5001 * Vs)
    for i in range(m):
        c, s = orc.rope_cache(fr, i, 1.0)
        qi, ki = orc.apply_rope_qk(q[i], k[i], H, Hk, d, c, s, neox=True)
        assert np.all(np.abs(Kd[i] - ki) <= 0.5001 * Ks[i])
        for h in range(H):
            g = h // (H // Hk)
            exp = _np_attention(qi[h * d:(h + 1) * d], Kd[:i + 1, g * d:(g + 1) * d],
                                Vd[:i + 1, g * d:(g + 1) * d], 1.0 / np.sqrt(d))
            assert np.all(np.abs(xb[i, h * d:(h + 1) * d] - exp) <= _tol(exp))


def test_prefill_attend_rows_matches_full_run(orc):
    """attend_rows only skips the attention of the other rows: the sampled rows and the
    caches are bit-identical to the full token-serial run, the rest of xb stays 0."""
    rng = np.random.default_rng(7)
    m, h, kvh, d = 40, 4, 2, 16
    q = rng.standard_normal((m, h * d)).astype(np.float32)
    k = rng.standard_normal((m, kvh * d)).astype(np.float32)
    v = rng.standard_normal((m, kvh * d)).astype(np.float32)
    kw = dict(n_heads=h, n_kv_heads=kvh, head_size=d, seq_len=m, fmt=orc.BF16, rope_dim=d,
              neox=True, rope_freqs_tab=orc.rope_freqs(1e4, d), rope_scale=1.0, window=9,
              q_norm=np.full(d, 1.1, np.float32), k_norm=np.full(d, 0.9, np.float32))
    full, kc, vc = orc.prefill_layer(q, k, v, **kw)
    rows = [0, 5, 8, 9, 39]
    part, kc2, vc2 = orc.prefill_layer(q, k, v, attend_rows=rows, **kw)
    assert np.array_equal(part[rows], full[rows])
    assert np.array_equal(kc2, kc) and np.array_equal(vc2, vc)
    others = np.setdiff1d(np.arange(m), rows)
    assert not part[others].any()


@pytest.mark.parametrize("window", [0, 8, 3])
def test_image_block_visibility_closed_form(orc, window):
    """Bidirectional image block (attention.rs:87-94, media_prefill.rs:84-121): 6 causal
    history rows, then a 5-row block at base_pos 6.  Row pos of the block attends to
    [min(start(pos), 6), 11) with start(pos) = pos + 1 - W (saturating) or 0: window 8
    reaches the history (row 6 sees 0..11, row 10 sees 3..11), window 3 does not (row 10
    sees the block only, row 6 sees 4..11), and every row sees the later block rows.
    Checked against float64 softmax(q K^T / sqrt(d)) V over exactly those keys."""
    rng = np.random.default_rng(11 + window)
    h, kvh, d, hist, blk = 4, 2, 16, 6, 5
    n = hist + blk
    q = rng.standard_normal((n, h * d)).astype(np.float32)
    k = rng.standard_normal((n, kvh * d)).astype(np.float32)
    v = rng.standard_normal((n, kvh * d)).astype(np.float32)
    kw = dict(n_heads=h, n_kv_heads=kvh, head_size=d, seq_len=n, fmt=orc.F32, rope_dim=0,
              neox=False, rope_freqs_tab=None, rope_scale=1.0, window=window)
    _, kc, vc = orc.prefill_layer(q[:hist], k[:hist], v[:hist], **kw)
    out, kc, vc = orc.prefill_layer(q[hist:], k[hist:], v[hist:], base_pos=hist, key_cache=kc,
                                    value_cache=vc, image_block=True, **kw)
    K = kc.astype(np.float64).reshape(n, kvh, d)
    V = vc.astype(np.float64).reshape(n, kvh, d)
    for i in range(blk):
        pos = hist + i
        start = max(0, pos + 1 - window) if window > 0 else 0
        lo, hi = min(start, hist), n
        for hh in range(h):
            g = hh // (h // kvh)
            s = K[lo:hi, g] @ q[pos, hh * d:(hh + 1) * d].astype(np.float64) / np.sqrt(d)
            p = np.exp(s - s.max())
            ref = (p / p.sum()) @ V[lo:hi, g]
            np.testing.assert_allclose(out[i, hh * d:(hh + 1) * d], ref, rtol=0, atol=2e-5)


def _encoder_fixture():
    """The inputs of encoder_attention_matches_reference_and_isolates_sequences
    (multimodal/mod.rs:656-676): 2 sequences x 3 tokens, 2 heads of dim 2."""
    ns, tps, hc, hd = 2, 3, 2, 2
    dim = hc * hd
    total = ns * tps
    idx = np.arange(total * dim)
    q = (((idx * 7) % 19).astype(np.float32) - 9.0) * np.float32(0.125)
    k = (((idx * 11) % 23).astype(np.float32) - 11.0) * np.float32(0.1)
    seq = idx // (tps * dim)
    v = seq.astype(np.float32) * 100.0 + (idx % (tps * dim)).astype(np.float32) * np.float32(0.25)
    return ns, tps, hc, hd, q.reshape(total, dim), k.reshape(total, dim), v.reshape(total, dim)


def test_encoder_attention_reference_fixture(orc):
    """The reference's own test (multimodal/mod.rs:656-738): the scalar two-pass softmax of
    each (sequence, token, head) within 2e-5 * max(|x|, 1); sequence 0's outputs stay below
    10 and sequence 1's above 90 (no attention across sequences)."""
    ns, tps, hc, hd, q, k, v = _encoder_fixture()
    got = orc.encoder_self_attention(q, k, v, n_seq=ns, tokens=tps, heads=hc, head_dim=hd)
    inv = np.float32(1.0) / np.sqrt(np.float32(hd))
    want = np.zeros_like(got)
    for s in range(ns):
        for t in range(tps):
            for h in range(hc):
                qt = q[s * tps + t, h * hd:(h + 1) * hd]
                sc = np.array([np.float32(sum(qt[i] * k[s * tps + j, h * hd + i] for i in range(hd)))
                               * inv for j in range(tps)], np.float32)
                w = np.exp(sc - sc.max())
                for j in range(tps):
                    want[s * tps + t, h * hd:(h + 1) * hd] += w[j] / w.sum() * v[s * tps + j, h * hd:(h + 1) * hd]
    assert np.all(np.abs(got - want) <= 2e-5 * np.maximum(np.abs(want), 1.0))
    assert np.all(got[:tps] < 10.0) and np.all(got[tps:] > 90.0)


@pytest.mark.parametrize("hd", [64, 72, 80])
def test_encoder_attention_float64_closed_form(orc, hd):
    """softmax(q K^T / sqrt(d)) V per sequence in float64, with head dims that exercise the
    16-wide FMA blocks and the scalar tail of the reference's dot (72, 80 are not
    multiples of 16)."""
    rng = np.random.default_rng(hd)
    ns, tps, hc = 3, 17, 2
    q, k, v = (rng.standard_normal((ns * tps, hc * hd)).astype(np.float32) for _ in range(3))
    got = orc.encoder_self_attention(q, k, v, n_seq=ns, tokens=tps, heads=hc, head_dim=hd)
    for s in range(ns):
        rows = slice(s * tps, (s + 1) * tps)
        for h in range(hc):
            cols = slice(h * hd, (h + 1) * hd)
            sc = q[rows, cols].astype(np.float64) @ k[rows, cols].astype(np.float64).T / np.sqrt(hd)
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            ref = (p / p.sum(axis=1, keepdims=True)) @ v[rows, cols].astype(np.float64)
            np.testing.assert_allclose(got[rows, cols], ref, rtol=0, atol=2e-5)


def test_sigmoid_mul_matches_float64_and_special_cases(orc):
    """orc_sigmoid_mul (the Qwen3.5 output gate, math.rs:396-403): x / (1 + exp(-g))
    against float64 to fp32 rounding over the exp range; g = +inf gives x, g = -inf
    gives 0 (exp(inf) = inf), a NaN gate or a product that overflows gives 0."""
    rng = np.random.default_rng(11)
    x = rng.standard_normal(50_000).astype(np.float32) * 10
    g = rng.uniform(-90, 90, 50_000).astype(np.float32)
    got = orc.sigmoid_mul(x, g)
    exp = x.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64)))
    assert np.all(np.abs(got - exp) <= 4e-7 * np.maximum(np.abs(exp), 1e-30) + 1e-37)
    xs = np.array([3.0, 3.0, 3.0, 3.0, np.inf, 3.4e38, -2.0], np.float32)
    gs = np.array([np.inf, -np.inf, np.nan, 0.0, 1.0, 100.0, 0.0], np.float32)
    assert orc.sigmoid_mul(xs, gs).tolist() == [3.0, 0.0, 0.0, 1.5, 0.0, np.float32(3.4e38), -1.0]
