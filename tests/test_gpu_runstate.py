"""The run-state entry points (the drop-ins for the reference's Rust call sites)
against the CPU oracle and against the reference's own unit-test constants."""
from __future__ import annotations

import math

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-5
ATOL_16, RTOL_16 = 2e-3, 1e-2


def test_rope_scaling_switches_local_and_global_layers_at_the_same_position(dev):
    """inference.rs:4098-4118 through gr_apply_rope_qk: adjacent pairs, layer 0 local
    (window 1024, scale 1) -> angle 8, layer 1 global (scale 0.125) -> angle 1."""
    from gguf_runner_amd import ffi, runtime as rt
    p = rt.Config(n_layers=2, n_heads=1, n_kv_heads=1, head_dim=64, seq_len=16,
                  rope_mode=ffi.ROPE_ADJACENT, rope_theta=10_000.0, layer_windows=[1024, None],
                  rope_scale_global=0.125)
    s = rt.malloc_run_state(p)
    for layer, angle in [(0, 8.0), (1, 1.0), (0, 8.0)]:
        s.q.fill(0.0)
        s.k.fill(0.0)
        s.q[0] = 1.0
        s.k[0] = 1.0
        rt.apply_rope_qk(p, s, layer, 8)
        for values in (s.q, s.k):
            assert abs(values[0] - math.cos(angle)) < 1e-7
            assert abs(values[1] - math.sin(angle)) < 1e-7


def test_swa_pattern_selects_local_rope_without_layer_windows(dev, orc):
    """is_swa_layer's swa_pattern branch (inference.rs:1820-1825; Gemma period 6, no
    layer_windows): layers l % 6 < 5 rotate with the local theta and scale, every sixth
    layer with the global ones (rebuild_rope_cache, 1485-1510), through gr_apply_rope_qk
    against the oracle's apply_rope_qk for the branch the pattern names."""
    from gguf_runner_amd import ffi, runtime as rt
    n_layers, d, pos = 13, 128, 37
    p = rt.Config(n_layers=n_layers, n_heads=2, n_kv_heads=1, head_dim=d, seq_len=64,
                  rope_mode=ffi.ROPE_NEOX, rope_theta=1e6, rope_theta_swa=1e4, swa_pattern=6,
                  is_gemma3=True, rope_scale_global=0.125, rope_scale_local=1.0)
    s = rt.malloc_run_state(p)
    rng = np.random.default_rng(6)
    q0 = rng.standard_normal(p.q_dim).astype(np.float32)
    k0 = rng.standard_normal(p.kv_dim).astype(np.float32)
    want = {}
    for swa in (False, True):
        c, sn = orc.rope_cache(orc.rope_freqs(1e4 if swa else 1e6, d), pos, 1.0 if swa else 0.125)
        want[swa] = orc.apply_rope_qk(q0, k0, 2, 1, d, c, sn, neox=True, gemma_q_scale=True)
    # the two branches differ well beyond the tolerance, so the check names the branch
    assert np.abs(want[True][1] - want[False][1]).max() > 0.1
    for layer in list(range(n_layers)) + [5, 0]:
        swa = layer % 6 < 5
        s.q[:] = q0
        s.k[:] = k0
        rt.apply_rope_qk(p, s, layer, pos)
        qr, kr = want[swa]
        assert np.abs(s.q - qr).max() <= TOL_F32, (layer, swa)
        assert np.abs(s.k - kr).max() <= TOL_F32, (layer, swa)


def test_neox_rope_partial_tail_through_device(dev, orc):
    """NeoX pairing with rope_dim < head_dim leaves the tail untouched (4133-4182) and
    matches the oracle's apply_rope_qk to 1 ulp-level."""
    from gguf_runner_amd import ffi, runtime as rt
    p = rt.Config(n_layers=1, n_heads=2, n_kv_heads=1, head_dim=256, rope_dim=64, seq_len=8,
                  rope_mode=ffi.ROPE_NEOX, rope_theta=1e6)
    s = rt.malloc_run_state(p)
    rng = np.random.default_rng(0)
    q0 = rng.standard_normal(p.q_dim).astype(np.float32)
    k0 = rng.standard_normal(p.kv_dim).astype(np.float32)
    s.q[:] = q0
    s.k[:] = k0
    rt.apply_rope_qk(p, s, 0, 5)
    c, sn = orc.rope_cache(orc.rope_freqs(1e6, 64), 5, 1.0)
    qr, kr = orc.apply_rope_qk(q0, k0, 2, 1, 256, c, sn, neox=True)
    assert np.allclose(s.q, qr, atol=1e-6) and np.allclose(s.k, kr, atol=1e-6)
    assert np.array_equal(s.q.reshape(2, 256)[:, 64:], q0.reshape(2, 256)[:, 64:])


def _qwen3_config(rt, ffi, kv_dtype, n_seq=1, seq_len=256):
    rng = np.random.default_rng(42)
    return rt.Config(n_layers=2, n_heads=16, n_kv_heads=8, head_dim=128, seq_len=seq_len,
                     n_seq=n_seq, kv_dtype=kv_dtype, rope_mode=ffi.ROPE_NEOX, rope_theta=1e6,
                     rms_norm_eps=1e-6,
                     q_norm=(1 + 0.1 * rng.standard_normal((2, 128))).astype(np.float32),
                     k_norm=(1 + 0.1 * rng.standard_normal((2, 128))).astype(np.float32))


def test_layer_token_loop_matches_oracle_f32(dev, orc):
    """Qwen3-0.6B-shaped layer (16 Q / 8 KV heads, d128, QK-norm, NeoX theta 1e6, f32
    KV): gr_attention_layer_token per token == the oracle's token-serial prefill loop
    (inference.rs:2981-3017) within 1e-5."""
    from gguf_runner_amd import ffi, runtime as rt
    p = _qwen3_config(rt, ffi, ffi.DTYPE_F32)
    s = rt.malloc_run_state(p)
    rng = np.random.default_rng(1)
    m, layer = 97, 1
    q = rng.standard_normal((m, p.q_dim)).astype(np.float32)
    k = rng.standard_normal((m, p.kv_dim)).astype(np.float32)
    v = rng.standard_normal((m, p.kv_dim)).astype(np.float32)
    got = np.zeros((m, p.q_dim), np.float32)
    for t in range(m):
        s.q[:], s.k[:], s.v[:] = q[t], k[t], v[t]
        rt.attention_layer_token(p, s, layer, t)
        got[t] = s.xb
    ref, kc, vc = orc.prefill_layer(q, k, v, n_heads=16, n_kv_heads=8, head_size=128,
                                    seq_len=m, fmt=orc.F32, rope_dim=128, neox=True,
                                    rope_freqs_tab=orc.rope_freqs(1e6, 128), rope_scale=1.0,
                                    q_norm=p.q_norm[layer], k_norm=p.k_norm[layer], eps=1e-6,
                                    n_threads=orc.env_threads())
    assert float(np.abs(got - ref).max()) <= TOL_F32
    kd, vd = rt.read_kv_rows(p, s, layer, 0, m)
    assert np.allclose(kd, kc, atol=1e-6) and np.array_equal(vd, vc)


@pytest.mark.parametrize("kv_dtype", [0, 1, 2])
def test_chunked_prefill_equals_sequential(dev, orc, kv_dtype):
    """Analogue of image_positions_preserve_chunked_prefill_kv_rows_and_decode_results
    (inference.rs:4184-4284): 64-token chunked prefill writes the same KV rows as the
    token-by-token path, and the attention outputs agree."""
    from gguf_runner_amd import ffi, runtime as rt
    p = _qwen3_config(rt, ffi, kv_dtype)
    s_seq = rt.malloc_run_state(p)
    s_chk = rt.malloc_run_state(p)
    rng = np.random.default_rng(2)
    m, layer = 150, 0
    q = rng.standard_normal((m, p.q_dim)).astype(np.float32)
    k = rng.standard_normal((m, p.kv_dim)).astype(np.float32)
    v = rng.standard_normal((m, p.kv_dim)).astype(np.float32)
    seq_out = np.zeros((m, p.q_dim), np.float32)
    for t in range(m):
        s_seq.q[:], s_seq.k[:], s_seq.v[:] = q[t], k[t], v[t]
        rt.attention_layer_token(p, s_seq, layer, t)
        seq_out[t] = s_seq.xb
    chk = []
    for b in range(0, m, 64):
        chk.append(rt.prefill_attention_chunk(p, s_chk, layer, b, q[b:b + 64], k[b:b + 64],
                                              v[b:b + 64]))
    chk = np.concatenate(chk)
    k1, v1 = rt.read_kv_rows(p, s_seq, layer, 0, m)
    k2, v2 = rt.read_kv_rows(p, s_chk, layer, 0, m)
    assert np.array_equal(k1, k2) and np.array_equal(v1, v2)
    err = np.abs(chk - seq_out)
    if kv_dtype == ffi.DTYPE_F32:
        assert float(err.max()) <= TOL_F32
    else:
        assert (err <= ATOL_16 + RTOL_16 * np.abs(seq_out)).all(), err.max()


def test_decode_layer_batch_equals_per_sequence(dev):
    """One batched decode launch over 3 sequence slots == per-slot layer tokens, to the
    f16 path's bar: the two launches split the keys differently, and the f16 kernel
    rounds P = 2^(s - m) relative to a running maximum m that depends on the split."""
    from gguf_runner_amd import ffi, runtime as rt
    p = _qwen3_config(rt, ffi, ffi.DTYPE_F16, n_seq=3, seq_len=300)
    s_a = rt.malloc_run_state(p)
    s_b = rt.malloc_run_state(p)
    rng = np.random.default_rng(3)
    lens = [40, 250, 7]
    layer = 1
    for seq, L in enumerate(lens):
        q = rng.standard_normal((L, p.q_dim)).astype(np.float32)
        k = rng.standard_normal((L, p.kv_dim)).astype(np.float32)
        v = rng.standard_normal((L, p.kv_dim)).astype(np.float32)
        for st in (s_a, s_b):
            rt.prefill_attention_chunk(p, st, layer, 0, q, k, v, seq=seq)
    qn = rng.standard_normal((3, p.q_dim)).astype(np.float32)
    kn = rng.standard_normal((3, p.kv_dim)).astype(np.float32)
    vn = rng.standard_normal((3, p.kv_dim)).astype(np.float32)
    batch = rt.decode_layer_batch(p, s_a, layer, [0, 1, 2], lens, qn, kn, vn)
    for seq, L in enumerate(lens):
        s_b.q[:], s_b.k[:], s_b.v[:] = qn[seq], kn[seq], vn[seq]
        rt.attention_layer_token(p, s_b, layer, L, seq=seq)
        err = np.abs(batch[seq] - s_b.xb)
        assert (err <= ATOL_16 + RTOL_16 * np.abs(s_b.xb)).all(), float(err.max())


def test_errors_follow_reference_messages(dev):
    from gguf_runner_amd import ffi, runtime as rt
    p = _qwen3_config(rt, ffi, ffi.DTYPE_F16, seq_len=64)
    s = rt.malloc_run_state(p)
    z = np.zeros((10, p.q_dim), np.float32)
    zk = np.zeros((10, p.kv_dim), np.float32)
    with pytest.raises(ffi.GrError, match="exceeds context"):
        rt.prefill_attention_chunk(p, s, 0, 60, z, zk, zk)
    with pytest.raises(ffi.GrError, match="layer"):
        rt.attention_token(p, s, 5, 0)


def test_qwen3next_state_step_matches_oracle(dev, orc):
    """gr_qwen3next_state_step over 16 heads x 20 tokens == qwen3next_state_head_step
    (math.rs:492-546) on the oracle, g given as the decay factor."""
    from gguf_runner_amd import runtime as rt
    H, d = 16, 128
    p = rt.Config(n_layers=1, n_heads=1, n_kv_heads=1, head_dim=128, seq_len=8,
                  ssm_n_heads=H, ssm_head_dim=d)
    s = rt.malloc_run_state(p)
    rng = np.random.default_rng(4)
    S = (0.1 * rng.standard_normal((H, d, d))).astype(np.float32)
    rt.write_ssm_state(p, s, 0, S)
    for t in range(20):
        q = rng.standard_normal((H, d)).astype(np.float32)
        k = rng.standard_normal((H, d)).astype(np.float32)
        q /= np.linalg.norm(q, axis=1, keepdims=True) * np.sqrt(d)
        k /= np.linalg.norm(k, axis=1, keepdims=True)
        v = rng.standard_normal((H, d)).astype(np.float32)
        g = np.exp(rng.uniform(-0.1, 0, H)).astype(np.float32)
        beta = rng.uniform(0, 1, H).astype(np.float32)
        out = rt.qwen3next_state_step(p, s, 0, q, k, v, g, beta).reshape(H, d)
        for h in range(H):
            s_new, o = orc.deltanet_head_step(S[h].reshape(-1), q[h], k[h], v[h], float(g[h]),
                                              float(beta[h]))
            S[h] = s_new.reshape(d, d)
            assert float(np.abs(out[h] - o).max()) <= TOL_F32
    assert float(np.abs(rt.read_ssm_state(p, s, 0) - S).max()) <= TOL_F32


def test_qwen3next_prefill_matches_oracle_scan(dev, orc):
    from gguf_runner_amd import runtime as rt
    H, d, T = 8, 128, 300
    p = rt.Config(n_layers=2, n_heads=1, n_kv_heads=1, head_dim=128, seq_len=8,
                  ssm_n_heads=H, ssm_head_dim=d, rms_norm_eps=1e-6)
    s = rt.malloc_run_state(p)
    rng = np.random.default_rng(5)
    q = rng.standard_normal((T, H, d)).astype(np.float32)
    k = rng.standard_normal((T, H, d)).astype(np.float32)
    v = rng.standard_normal((T, H, d)).astype(np.float32)
    gate = rng.uniform(-0.1, 0, (T, H)).astype(np.float32)
    beta = rng.uniform(0, 1, (T, H)).astype(np.float32)
    out = rt.qwen3next_prefill(p, s, 1, q.reshape(T, -1), k.reshape(T, -1), v.reshape(T, -1),
                               gate, beta).reshape(T, H, d)
    ref, Sref = orc.deltanet_scan(q, k, v, gate, beta, np.zeros((H, d, d), np.float32),
                                  eps=1e-6, n_threads=orc.env_threads())
    assert float(np.abs(out - ref).max()) <= TOL_F32
    assert float(np.abs(rt.read_ssm_state(p, s, 1) - Sref).max()) <= TOL_F32


def test_qwen3next_prefill_in_overlapped_pieces(dev, orc):
    """2000 tokens of 16 heads (65 MB of host rows): the call runs as overlapped pieces
    of 256, 448, 512, 512 and 272 tokens (cut at multiples of the chunked scan's 64), the
    state carried from piece to piece on the device; outputs and the final state ==
    the oracle's token scan (1e-5)."""
    from gguf_runner_amd import runtime as rt
    H, d, T = 16, 128, 2000
    p = rt.Config(n_layers=1, n_heads=1, n_kv_heads=1, head_dim=128, seq_len=8,
                  ssm_n_heads=H, ssm_head_dim=d, rms_norm_eps=1e-6)
    s = rt.malloc_run_state(p)
    rng = np.random.default_rng(2000)
    q = rng.standard_normal((T, H, d)).astype(np.float32)
    k = rng.standard_normal((T, H, d)).astype(np.float32)
    v = rng.standard_normal((T, H, d)).astype(np.float32)
    gate = rng.uniform(-0.1, 0, (T, H)).astype(np.float32)
    beta = rng.uniform(0, 1, (T, H)).astype(np.float32)
    out = rt.qwen3next_prefill(p, s, 0, q.reshape(T, -1), k.reshape(T, -1), v.reshape(T, -1),
                               gate, beta).reshape(T, H, d)
    ref, Sref = orc.deltanet_scan(q, k, v, gate, beta, np.zeros((H, d, d), np.float32),
                                  eps=1e-6, n_threads=orc.env_threads())
    assert float(np.abs(out - ref).max()) <= TOL_F32
    assert float(np.abs(rt.read_ssm_state(p, s, 0) - Sref).max()) <= TOL_F32


@pytest.mark.parametrize("kv_dtype", [1, 3])
def test_prefill_image_block_runstate(dev, orc, kv_dtype):
    """gr_prefill_image_block (transformer_prefill_image_block's attention) after 40 causal
    rows: f16 cache (MFMA prefill kernel, bidirectional) and Q8 cache (codec write, then the
    batched decode kernels over the block ranges) against the oracle."""
    from gguf_runner_amd import ffi, runtime as rt
    p = _qwen3_config(rt, ffi, kv_dtype)
    s = rt.malloc_run_state(p)
    rng = np.random.default_rng(5)
    hist, blk, layer = 40, 70, 1
    n = hist + blk
    q = rng.standard_normal((n, p.q_dim)).astype(np.float32)
    k = rng.standard_normal((n, p.kv_dim)).astype(np.float32)
    v = rng.standard_normal((n, p.kv_dim)).astype(np.float32)
    rt.prefill_attention_chunk(p, s, layer, 0, q[:hist], k[:hist], v[:hist])
    got = rt.prefill_image_block(p, s, layer, hist, q[hist:], k[hist:], v[hist:])
    fmt = orc.F16 if kv_dtype == ffi.DTYPE_F16 else orc.Q8
    kw = dict(n_heads=16, n_kv_heads=8, head_size=128, seq_len=n, fmt=fmt, rope_dim=128,
              neox=True, rope_freqs_tab=orc.rope_freqs(1e6, 128), rope_scale=1.0,
              q_norm=p.q_norm[layer], k_norm=p.k_norm[layer], eps=1e-6, n_threads=orc.env_threads())
    _, kc, vc = orc.prefill_layer(q[:hist], k[:hist], v[:hist], **kw)
    ref, _, _ = orc.prefill_layer(q[hist:], k[hist:], v[hist:], base_pos=hist, key_cache=kc,
                                  value_cache=vc, image_block=True, **kw)
    err = np.abs(got - ref)
    assert (err <= ATOL_16 + RTOL_16 * np.abs(ref)).all(), err.max()


def test_prefill_image_block_outside_context_is_rejected(dev):
    """media_prefill.rs:31-39: a block that does not fit the context is an error."""
    from gguf_runner_amd import ffi, runtime as rt
    p = _qwen3_config(rt, ffi, ffi.DTYPE_F16, seq_len=64)
    s = rt.malloc_run_state(p)
    z = np.zeros((10, p.q_dim), np.float32)
    zk = np.zeros((10, p.kv_dim), np.float32)
    with pytest.raises(ffi.GrError, match="image-block prefill must evaluate one complete"):
        rt.prefill_image_block(p, s, 0, 60, z, zk, zk)


def test_large_host_rows_through_the_pinned_ring(dev):
    """Host rows above the staging threshold travel through the run state's pinned
    rings: one 2600-row chunk over an f32 cache runs as six overlapped pieces (256,
    four of ~522, 256 rows; uploads, kernels and downloads of neighbouring pieces at
    once), twice with new rows into the same output buffer; the K / V rows read back
    bit-exact (single 16 MB slot reads after the pipelined call) and sampled output
    rows, piece edges included, against a float64 restatement of the causal softmax
    within 1e-5."""
    from gguf_runner_amd import ffi, runtime as rt
    m, H, G, d = 2600, 16, 8, 128
    p = rt.Config(n_layers=1, n_heads=H, n_kv_heads=G, head_dim=d, seq_len=m,
                  kv_dtype=ffi.DTYPE_F32, rope_mode=ffi.ROPE_NONE)
    s = rt.malloc_run_state(p)
    rng = np.random.default_rng(77)
    xb = np.zeros((m, p.q_dim), np.float32)
    for rep in range(2):
        q = rng.standard_normal((m, p.q_dim)).astype(np.float32)
        k = rng.standard_normal((m, p.kv_dim)).astype(np.float32)
        v = rng.standard_normal((m, p.kv_dim)).astype(np.float32)
        got = rt.prefill_attention_chunk(p, s, 0, 0, q, k, v, out=xb)
        assert got is xb
        kd, vd = rt.read_kv_rows(p, s, 0, 0, m)
        assert np.array_equal(kd, k) and np.array_equal(vd, v), rep
        for t in (0, 1, 255, 256, 777, 778, 1000, 2047, 2048, 2343, 2344, m - 1):
            for h in range(H):
                g = h // (H // G)
                kk = k[:t + 1, g * d:(g + 1) * d].astype(np.float64)
                vv = v[:t + 1, g * d:(g + 1) * d].astype(np.float64)
                sc = kk @ q[t, h * d:(h + 1) * d].astype(np.float64) / math.sqrt(d)
                w = np.exp(sc - sc.max())
                ref = (w / w.sum()) @ vv
                err = np.abs(xb[t, h * d:(h + 1) * d] - ref).max()
                assert err <= TOL_F32, (rep, t, h, err)


@pytest.mark.parametrize("kv_dtype,window", [(1, None), (2, 300)])
def test_large_f16_chunk_runs_in_overlapped_pieces(dev, orc, kv_dtype, window):
    """A 2048-row chunk over an f16 / bf16 cache (32 / 8 heads, d128, global or
    window-300 layer) is cut into overlapped pieces of 256, 512, 512, 512 and 256
    rows; the MFMA prefill of each piece sees the rows the pieces before it wrote.  The cache rows
    == the host rows rounded to the cache type (bit-exact) and sampled output rows
    (piece edges included) == the oracle's attention_token over the device's rows,
    to the 16-bit MFMA bar."""
    from gguf_runner_amd import ffi, runtime as rt
    n_heads, n_kv, d, m = 32, 8, 128, 2048
    p = rt.Config(n_layers=1, n_heads=n_heads, n_kv_heads=n_kv, head_dim=d, seq_len=m,
                  kv_dtype=kv_dtype, rope_mode=ffi.ROPE_NONE, layer_windows=[window])
    s = rt.malloc_run_state(p)
    rng = np.random.default_rng(512 + kv_dtype)
    q = rng.standard_normal((m, p.q_dim)).astype(np.float32)
    k = rng.standard_normal((m, p.kv_dim)).astype(np.float32)
    v = rng.standard_normal((m, p.kv_dim)).astype(np.float32)
    got = rt.prefill_attention_chunk(p, s, 0, 0, q, k, v)
    kd, vd = rt.read_kv_rows(p, s, 0, 0, m)
    cast = orc.c_f32_to_f16 if kv_dtype == ffi.DTYPE_F16 else orc.c_f32_to_bf16
    assert np.array_equal(kd.reshape(-1), cast(k)) and np.array_equal(vd.reshape(-1), cast(v))
    fmt = orc.F16 if kv_dtype == ffi.DTYPE_F16 else orc.BF16
    rows = sorted({0, 1, 255, 256, 767, 768, 1279, 1280, 1791, 1792, m - 1} | set(rng.integers(0, m, 8).tolist()))
    for t in rows:
        start = max(0, t + 1 - window) if window else 0
        ref = orc.attention_token(q[t], kd, vd, fmt, n_heads, n_kv, d, start, t + 1)
        assert (np.abs(got[t] - ref) <= ATOL_16 + RTOL_16 * np.abs(ref)).all(), (t, float(np.abs(got[t] - ref).max()))
