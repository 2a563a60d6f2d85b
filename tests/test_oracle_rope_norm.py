"""Pins the oracle's RoPE, QK-norm, softmax, Q8 and window functions against the
reference's own unit-test constants and against closed forms (CPU only)."""
from __future__ import annotations

import math

import numpy as np
import pytest


# ---- RoPE ------------------------------------------------------------------

def test_rope_local_global_scaling_reference_constants(orc):
    """inference.rs:4098-4118: 1 head, head_dim 4, theta 1e4, adjacent pairs (Llama path),
    q[0] = k[0] = 1 at pos 8; local layer (scale 1) -> angle 8, global layer
    (rope_scaling.global = 0.125) -> angle 1; (q0, q1) == (cos, sin) within 1e-7."""
    freqs = orc.rope_freqs(10_000.0, 4)
    for scale, angle in [(1.0, 8.0), (0.125, 1.0), (1.0, 8.0)]:
        c, s = orc.rope_cache(freqs, 8, scale)
        q = np.array([1, 0, 0, 0], np.float32)
        k = q.copy()
        q2, k2 = orc.apply_rope_qk(q, k, 1, 1, 4, c, s, neox=False)
        for vals in (q2, k2):
            assert abs(vals[0] - np.float32(math.cos(angle))) < 1e-7
            assert abs(vals[1] - np.float32(math.sin(angle))) < 1e-7


@pytest.mark.parametrize("head_dim,rope_dim", [(128, 128), (256, 64)])
def test_rope_neox_pairing_partial_tail_reference_constants(orc, head_dim, rope_dim):
    """inference.rs:4133-4182 with text positions: unit frequencies isolate the angle;
    NeoX pairs (i, i + rope_dim/2); the partial-RoPE tail is untouched; cos/sin of
    2, 3, 4, 5 match the reference constants within 1e-7."""
    half = rope_dim // 2
    ones = np.ones(half, np.float32)
    for pos, cos_ref, sin_ref in [(2, -0.416_146_84, 0.909_297_4), (3, -0.989_992_5, 0.141_12),
                                  (4, -0.653_643_6, -0.756_802_5), (5, 0.283_662_2, -0.958_924_3)]:
        c, s = orc.rope_cache(ones, pos, 1.0)
        assert np.all(np.abs(c - np.float32(cos_ref)) < 1e-7)
        assert np.all(np.abs(s - np.float32(sin_ref)) < 1e-7)
        q = np.zeros(head_dim, np.float32)
        q[:half] = 1.0
        q[rope_dim:] = 0.75
        q2, k2 = orc.apply_rope_qk(q, q.copy(), 1, 1, head_dim, c, s, neox=True)
        assert np.all(np.abs(q2[:half] - np.float32(cos_ref)) < 1e-7)
        assert np.all(np.abs(q2[half:rope_dim] - np.float32(sin_ref)) < 1e-7)
        assert np.array_equal(q2, k2)
        assert np.all(q2[rope_dim:] == 0.75)


@pytest.mark.parametrize("theta,dim", [(5e5, 128), (1e4, 256), (1e6, 256)])
def test_rope_freqs_closed_form(orc, theta, dim):
    f = orc.rope_freqs(theta, dim)
    exp = 1.0 / np.power(np.float64(theta), np.arange(0, dim, 2) / dim)
    assert np.allclose(f, exp, rtol=2e-7, atol=0)
    assert f[0] == 1.0


@pytest.mark.parametrize("neox", [False, True])
def test_rope_rotation_invariants(orc, neox):
    """Each rotated pair keeps its norm; position 0 is the identity; the rotation of
    the correct pair partner (a transposed index fails this against float64)."""
    rng = np.random.default_rng(3)
    H, Hk, d = 4, 2, 128
    q = rng.standard_normal(H * d).astype(np.float32)
    k = rng.standard_normal(Hk * d).astype(np.float32)
    f = orc.rope_freqs(1e4, d)
    c0, s0 = orc.rope_cache(f, 0, 1.0)
    q0, k0 = orc.apply_rope_qk(q, k, H, Hk, d, c0, s0, neox=neox)
    assert np.array_equal(q0, q) and np.array_equal(k0, k)
    pos = 1234
    c, s = orc.rope_cache(f, pos, 1.0)
    q2, _ = orc.apply_rope_qk(q, k, H, Hk, d, c, s, neox=neox)
    ang = pos * f.astype(np.float64)
    qq = q.astype(np.float64).reshape(H, d)
    if neox:
        a, b = qq[:, : d // 2], qq[:, d // 2:]
        ra = a * np.cos(ang) - b * np.sin(ang)
        rb = a * np.sin(ang) + b * np.cos(ang)
        exp = np.concatenate([ra, rb], axis=1)
    else:
        a, b = qq[:, 0::2], qq[:, 1::2]
        exp = np.empty_like(qq)
        exp[:, 0::2] = a * np.cos(ang) - b * np.sin(ang)
        exp[:, 1::2] = a * np.sin(ang) + b * np.cos(ang)
    # f32 angle rounding (pos*freq in f32) dominates the error at pos 1234
    assert np.allclose(q2.reshape(H, d), exp, atol=5e-4)
    n_before = np.hypot(a, b)
    q2r = q2.reshape(H, d).astype(np.float64)
    n_after = (np.hypot(q2r[:, : d // 2], q2r[:, d // 2:]) if neox
               else np.hypot(q2r[:, 0::2], q2r[:, 1::2]))
    assert np.allclose(n_before, n_after, rtol=1e-6)


def test_gemma_q_scale_after_rope(orc):
    """inference.rs:1871-1873: Gemma3 multiplies q (not k) by 1/sqrt(head_dim) after RoPE."""
    q = np.ones(256, np.float32)
    k = np.ones(256, np.float32)
    c, s = orc.rope_cache(orc.rope_freqs(1e4, 256), 0, 1.0)
    q2, k2 = orc.apply_rope_qk(q, k, 1, 1, 256, c, s, neox=True, gemma_q_scale=True)
    assert np.all(q2 == np.float32(1.0 / 16.0))
    assert np.all(k2 == 1.0)


# ---- QK RMSNorm ------------------------------------------------------------

def test_rmsnorm_per_head_closed_form(orc):
    rng = np.random.default_rng(5)
    H, d, eps = 3, 256, 1e-6
    x = rng.standard_normal(H * d).astype(np.float32) * 3
    w = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    y = orc.rmsnorm_per_head(x, w, H, d, eps)
    xx = x.astype(np.float64).reshape(H, d)
    exp = w * xx / np.sqrt((xx ** 2).mean(axis=1, keepdims=True) + eps)
    assert np.allclose(y.reshape(H, d), exp, rtol=2e-6, atol=1e-6)
    y1 = orc.rmsnorm_per_head(x, np.ones(d, np.float32), H, d, 0.0).reshape(H, d)
    assert np.allclose(np.sqrt((y1.astype(np.float64) ** 2).mean(axis=1)), 1.0, atol=1e-6)


# ---- softmax / Q8 ----------------------------------------------------------

def test_softmax_closed_form(orc):
    rng = np.random.default_rng(11)
    x = rng.standard_normal(1000).astype(np.float32) * 4
    y = orc.softmax(x)
    e = np.exp(x.astype(np.float64) - x.max())
    assert np.allclose(y, e / e.sum(), rtol=1e-5, atol=1e-9)
    assert abs(float(y.astype(np.float64).sum()) - 1.0) < 1e-5


def test_quantize_row_q8_closed_form_and_ties(orc):
    """inference.rs:249-268: scale = amax/127, q = round_half_away(x*127/amax) in [-127, 127];
    amax == 0 -> scale 1, zeros."""
    x = np.array([1.27, -1.27, 0.005, -0.005, 0.015, 0.0, 0.635, -0.635], np.float32)
    q, s = orc.quantize_row_q8(x)
    assert s == np.float32(np.float32(1.27) / np.float32(127.0))
    inv = np.float32(127.0) / np.float32(1.27)
    prod = (x * inv).astype(np.float32)
    exp = np.where(prod >= 0, np.floor(prod + 0.5), -np.floor(-prod + 0.5)).clip(-127, 127)
    assert np.array_equal(q, exp.astype(np.int8))
    assert q[0] == 127 and q[1] == -127
    q0, s0 = orc.quantize_row_q8(np.zeros(32, np.float32))
    assert s0 == 1.0 and not q0.any()
    # exact half: 0.5 rounds away from zero (Rust f32::round), not to even
    y = np.array([127.0, 0.5, -0.5, 1.5, 2.5], np.float32)
    qy, _ = orc.quantize_row_q8(y)
    assert list(qy[1:]) == [1, -1, 2, 3]


# ---- windows ---------------------------------------------------------------

def test_visible_keys_reference_cases(orc):
    """attention.rs:171-172 (causal 0..q+1) and the window rule of types.rs:614-616:
    W keys including the current one, saturating at 0."""
    assert orc.visible_keys(0, 3) == (0, 4)
    assert orc.visible_keys(1024, 0) == (0, 1)
    assert orc.visible_keys(1024, 1023) == (0, 1024)
    assert orc.visible_keys(1024, 1024) == (1, 1025)
    assert orc.visible_keys(1, 77) == (77, 78)


def test_kv_quantize_row_block_and_row_modes(orc):
    """kv_write_token's Q8 branch (inference.rs:1886-1917): block mode quantises each
    32-element block on its own (scale_b = amax_b/127), row mode uses one scale."""
    rng = np.random.default_rng(12)
    kv_dim = 256
    x = rng.standard_normal(kv_dim).astype(np.float32)
    x[32:64] *= 40.0   # one loud block
    x[96:128] = 0.0    # one silent block: scale 1, zeros
    qb, sb = orc.kv_quantize_row(x, True)
    assert sb.shape == (kv_dim // 32,)
    for b in range(kv_dim // 32):
        blk = x[32 * b:32 * (b + 1)]
        amax = np.float32(np.abs(blk).max())
        if amax == 0:
            assert sb[b] == 1.0 and not qb[32 * b:32 * (b + 1)].any()
            continue
        assert sb[b] == np.float32(amax / np.float32(127.0))
        prod = (blk * (np.float32(127.0) / amax)).astype(np.float32)
        exp = np.where(prod >= 0, np.floor(prod + 0.5), -np.floor(-prod + 0.5)).clip(-127, 127)
        assert np.array_equal(qb[32 * b:32 * (b + 1)], exp.astype(np.int8))
        # dequantised values sit within half a step of the input
        assert np.all(np.abs(qb[32 * b:32 * (b + 1)] * sb[b] - blk) <= 0.5001 * sb[b])
    qr, sr = orc.kv_quantize_row(x, False)
    assert sr.shape == (1,) and sr[0] == np.float32(np.float32(np.abs(x).max()) / np.float32(127.0))
    assert np.array_equal(qr, orc.quantize_row_q8(x)[0])
