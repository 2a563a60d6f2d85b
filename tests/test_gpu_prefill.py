"""Prefill parity: gr_prefill_attention (Q/K/V prep + MFMA flash kernel) vs the
CPU oracle's token-serial prefill (reference inference.rs:2981-3017: QK-norm ->
apply_rope_qk -> kv_write_token -> attention_token per token) on identical
seeded f16/bf16 inputs.

Tolerance for the f16/bf16 MFMA path (written here, fixed before measuring):
  |gpu - ref| <= 2e-3 + 1e-2 * |ref| elementwise.
Cache rows: V is copied bit-exactly; post-RoPE K may differ from the oracle's
by the rounding of the 16-bit store (1 ulp), checked at 2 ulp.
"""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def _t16(bits: np.ndarray, fmt, orc, dev):
    dt = torch.float16 if fmt == orc.F16 else torch.bfloat16
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(dt).to(dev)


def _bits(x, fmt, orc):
    return orc.f16_bits(x) if fmt == orc.F16 else orc.bf16_bits(x)


def _case(orc, dev, *, m, n_heads, n_kv, d, fmt, seed, rope_mode, theta, rope_scale=1.0,
          window=0, norm=False, is_gemma3=False, base_chunks=None, eps=1e-6, rope_dim=None,
          attend_rows=None, patch=None, bias=None):
    from gguf_runner_amd import ffi, ops
    rng = np.random.default_rng(seed)
    qf = rng.standard_normal((m, n_heads, d), dtype=np.float32)
    kf = rng.standard_normal((m, n_kv, d), dtype=np.float32)
    vf = rng.standard_normal((m, n_kv, d), dtype=np.float32)
    if patch:
        patch(qf, kf, vf)
    qb, kb, vb = (_bits(x, fmt, orc) for x in (qf, kf, vf))
    qn = kn = None
    if norm:
        qn = (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)
        kn = (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    rope_dim = d if rope_dim is None else rope_dim
    freqs = orc.rope_freqs(theta, rope_dim)
    # oracle (token-serial, raw cache of the same 16-bit format); Qwen2 biases are
    # f32 additions to the rows before everything else (inference.rs:2545-2559)
    qo, ko, vo = (orc.upcast(x, fmt).reshape(m, -1) for x in (qb, kb, vb))
    if bias is not None:
        qo, ko, vo = qo + bias[0][None, :], ko + bias[1][None, :], vo + bias[2][None, :]
    ref, kc_ref, vc_ref = orc.prefill_layer(
        qo, ko, vo, n_heads=n_heads, n_kv_heads=n_kv, head_size=d,
        seq_len=m, fmt=fmt, rope_dim=(0 if rope_mode == ffi.ROPE_NONE else rope_dim), neox=(rope_mode == ffi.ROPE_NEOX), rope_freqs_tab=freqs,
        rope_scale=rope_scale, is_gemma3=is_gemma3, window=window, q_norm=qn, k_norm=kn, eps=eps,
        n_threads=orc.env_threads(), attend_rows=attend_rows)
    # GPU
    q, k, v = (_t16(x, fmt, orc, dev) for x in (qb, kb, vb))
    kc = torch.zeros((m, n_kv, d), dtype=q.dtype, device=dev)
    vc = torch.zeros_like(kc)
    fr = torch.tensor(ops.rope_freqs(theta, rope_dim), dtype=torch.float32, device=dev)
    qnt = torch.from_numpy(qn).to(dev) if norm else None
    knt = torch.from_numpy(kn).to(dev) if norm else None
    chunks = base_chunks or [m]
    out = torch.empty((m, n_heads, d), dtype=torch.float32, device=dev)
    bt = [torch.from_numpy(x).to(dev) for x in bias] if bias is not None else [None] * 3
    b = 0
    for c in chunks:
        ops.PrefillCall(q[b:b + c].contiguous(), k[b:b + c].contiguous(), v[b:b + c].contiguous(),
                        kc, vc, out_view := torch.empty((c, n_heads, d), dtype=torch.float32,
                                                        device=dev),
                        base_pos=b, window=window, rope_mode=rope_mode, rope_dim=rope_dim,
                        rope_scale=rope_scale, rope_freqs=fr, q_norm=qnt, k_norm=knt,
                        norm_eps=eps, is_gemma3=is_gemma3, q_bias=bt[0], k_bias=bt[1], v_bias=bt[2])()
        out[b:b + c] = out_view
        b += c
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(m, -1)
    kc_got = kc.cpu().view(torch.int16).numpy().view(np.uint16).reshape(m, -1)
    vc_got = vc.cpu().view(torch.int16).numpy().view(np.uint16).reshape(m, -1)
    return got, ref, (kc_got, kc_ref), (vc_got, vc_ref)


def _assert_close(got, ref):
    err = np.abs(got - ref)
    bad = ~(err <= ATOL + RTOL * np.abs(ref))  # NaN counts as out of tolerance
    assert not bad.any(), f"{bad.sum()} / {bad.size} out of tolerance; max abs {err.max():.3e}"


def _assert_cache(kc, vc, fmt, orc):
    kg, kr = kc
    vg, vr = vc
    assert np.array_equal(vg, vr), "V cache rows must be copied exactly"
    a = orc.upcast(kg, fmt)
    b = orc.upcast(kr, fmt)
    ulp = 2.0 ** (-10 if fmt == orc.F16 else -7)
    assert np.all(np.abs(a - b) <= 2 * ulp * np.maximum(np.abs(b), 2.0 ** -14)), \
        f"K cache max diff {np.abs(a - b).max():.3e}"


@pytest.mark.parametrize("rope_dim", [32, 64, 96, 40])
@pytest.mark.parametrize("fmt_name", ["F16", "BF16"])
def test_prefill_partial_neox_rope_with_qk_norm(orc, dev, rope_dim, fmt_name):
    """Partial NeoX RoPE (apply_rope_qk's rope_dim < head_dim tail, inference.rs:1817-1874)
    with QK-norm on d128: widths whose rotation pairs (i, i + rope_dim/2) stay inside a
    lane's Q fragments (32 / 64 / 96, prepared inside the attention kernel) and one whose
    pairs do not (40, prepared by the staging pass)."""
    from gguf_runner_amd import ffi
    fmt = getattr(orc, fmt_name)
    got, ref, kc, vc = _case(orc, dev, m=300, n_heads=8, n_kv=2, d=128, fmt=fmt, seed=rope_dim,
                             rope_mode=ffi.ROPE_NEOX, theta=1e6, norm=True, rope_dim=rope_dim,
                             base_chunks=[100, 200])
    _assert_close(got, ref)
    _assert_cache(kc, vc, fmt, orc)


def test_config2_llama3_8b_prefill_f16(orc, dev):
    """Config 2: 32 Q / 8 KV heads, d128, 2048 tokens, f16, adjacent-pair RoPE theta 5e5
    fused on load, causal, fp32 accumulate, output [2048, 32, 128]."""
    from gguf_runner_amd import ffi
    got, ref, kc, vc = _case(orc, dev, m=2048, n_heads=32, n_kv=8, d=128, fmt=orc.F16, seed=1002,
                             rope_mode=ffi.ROPE_ADJACENT, theta=5e5)
    _assert_close(got, ref)
    _assert_cache(kc, vc, orc.F16, orc)


def test_config2_shape_prefill_8192_sampled_rows(orc, dev):
    """The 8k prefill the benchmark times, at full size: 8192 tokens, 32 Q / 8 KV
    heads, d128, f16, adjacent-pair RoPE theta 5e5, one call (the eight-wave
    kernel).  The oracle prepares and caches every row and attends a sample of
    rows: the edges of the 256-row query blocks, the last rows, and random ones;
    every cache row is checked."""
    from gguf_runner_amd import ffi
    m = 8192
    rows = np.unique(np.concatenate([[0, 1, 31, 32, 255, 256, 257, 511, 4095, 4096, 8063, 8190, 8191],
                                     np.random.default_rng(88).integers(0, m, 20)]))
    got, ref, kc, vc = _case(orc, dev, m=m, n_heads=32, n_kv=8, d=128, fmt=orc.F16, seed=8192,
                             rope_mode=ffi.ROPE_ADJACENT, theta=5e5, attend_rows=rows)
    _assert_close(got[rows], ref[rows])
    _assert_cache(kc, vc, orc.F16, orc)


@pytest.mark.parametrize("layer", ["local", "global"])
def test_config4_gemma3_prefill_bf16(orc, dev, layer):
    """Config 4 (reduced length): 8 Q / 4 KV heads, d256, bf16, QK RMSNorm eps 1e-6 with
    weights ~N(1, 0.1), NeoX RoPE; local layer theta 1e4 window 1024, global layer theta 1e6
    x 0.125; q pre-scaled by 1/16 and scores unscaled."""
    from gguf_runner_amd import ffi
    local = layer == "local"
    got, ref, kc, vc = _case(orc, dev, m=2048 if local else 1280, n_heads=8, n_kv=4, d=256,
                             fmt=orc.BF16, seed=1004, rope_mode=ffi.ROPE_NEOX,
                             theta=1e4 if local else 1e6, rope_scale=1.0 if local else 0.125,
                             window=1024 if local else 0, norm=True, is_gemma3=True)
    _assert_close(got, ref)
    _assert_cache(kc, vc, orc.BF16, orc)


@pytest.mark.parametrize("chunks", [[64, 64, 72], [1, 127, 129, 3], [200]])
def test_prefill_chunked_continuation(orc, dev, chunks):
    """Chunks continue from base_pos over the rows earlier chunks wrote (the 64-token
    prefill chunking of generation.rs:4869-4923), ragged m, f16 NeoX RoPE."""
    from gguf_runner_amd import ffi
    m = sum(chunks)
    got, ref, kc, vc = _case(orc, dev, m=m, n_heads=8, n_kv=2, d=128, fmt=orc.F16, seed=m,
                             rope_mode=ffi.ROPE_NEOX, theta=1e6, base_chunks=chunks)
    _assert_close(got, ref)
    _assert_cache(kc, vc, orc.F16, orc)


@pytest.mark.parametrize("window", [1, 7, 64, 100])
def test_prefill_small_windows(orc, dev, window):
    """Window edge cases: W=1 attends only to itself (out == v row), W not a tile multiple."""
    from gguf_runner_amd import ffi
    got, ref, kc, vc = _case(orc, dev, m=300, n_heads=4, n_kv=4, d=128, fmt=orc.BF16,
                             seed=window, rope_mode=ffi.ROPE_NEOX, theta=1e4, window=window)
    _assert_close(got, ref)


def test_prefill_window_one_returns_v(orc, dev):
    """W = 1: softmax over one key is exactly 1, so the output is the V row itself."""
    from gguf_runner_amd import ffi
    got, ref, kc, vc = _case(orc, dev, m=130, n_heads=4, n_kv=2, d=128, fmt=orc.F16, seed=5,
                             rope_mode=ffi.ROPE_NONE, theta=1e4, window=1)
    v = orc.upcast(vc[0], orc.F16).reshape(130, 2, 128)
    exp = np.repeat(v, 2, axis=1).reshape(130, -1)
    assert np.array_equal(got, exp)


def test_prefill_eight_wave_blocks_f16(orc, dev):
    """Launches with >= 256 (query head, block pair) items take 256-row workgroups of
    8 waves: 64 Q / 8 KV heads over 2048 tokens (64 x 4 pairs) selects them."""
    from gguf_runner_amd import ffi
    got, ref, kc, vc = _case(orc, dev, m=2048, n_heads=64, n_kv=8, d=128, fmt=orc.F16,
                             seed=2048, rope_mode=ffi.ROPE_ADJACENT, theta=5e5)
    _assert_close(got, ref)
    _assert_cache(kc, vc, orc.F16, orc)


@pytest.mark.parametrize("fmt_name", ["BF16", "F16"])
def test_prefill_eight_wave_blocks_window_chunked(orc, dev, fmt_name):
    """8-wave workgroups with a sliding window and a continuation chunk (base_pos 700,
    1348 tokens, 96 heads: 96 x 3 pairs), ragged last block: bf16 (f16 copy of the
    rows), f16 (the split-role kernel: score and value waves)."""
    from gguf_runner_amd import ffi
    fmt = getattr(orc, fmt_name)
    got, ref, kc, vc = _case(orc, dev, m=2048, n_heads=96, n_kv=8, d=128, fmt=fmt,
                             seed=96, rope_mode=ffi.ROPE_NEOX, theta=1e4, window=300,
                             base_chunks=[700, 1348])
    _assert_close(got, ref)
    _assert_cache(kc, vc, fmt, orc)


def _image_block_case(orc, dev, *, hist, blk, n_heads, n_kv, d, fmt, seed, window, rope_mode,
                      theta, sample=None):
    """`hist` causal rows, then one bidirectional image block of `blk` rows (the
    attention of transformer_prefill_image_block, media_prefill.rs:84-121)."""
    from gguf_runner_amd import ffi, ops
    rng = np.random.default_rng(seed)
    n = hist + blk
    qb = _bits(rng.standard_normal((n, n_heads, d), dtype=np.float32), fmt, orc)
    kb = _bits(rng.standard_normal((n, n_kv, d), dtype=np.float32), fmt, orc)
    vb = _bits(rng.standard_normal((n, n_kv, d), dtype=np.float32), fmt, orc)
    freqs = orc.rope_freqs(theta, d)
    rope_dim = 0 if rope_mode == ffi.ROPE_NONE else d
    kw = dict(n_heads=n_heads, n_kv_heads=n_kv, head_size=d, seq_len=n, fmt=fmt, rope_dim=rope_dim,
              neox=(rope_mode == ffi.ROPE_NEOX), rope_freqs_tab=freqs, rope_scale=1.0, window=window,
              n_threads=orc.env_threads())
    up = lambda x: orc.upcast(x, fmt).reshape(x.shape[0], -1)
    _, kc_ref, vc_ref = orc.prefill_layer(up(qb[:hist]), up(kb[:hist]), up(vb[:hist]), **kw)
    rows = None if sample is None else sample
    ref, kc_ref, vc_ref = orc.prefill_layer(up(qb[hist:]), up(kb[hist:]), up(vb[hist:]),
                                            base_pos=hist, key_cache=kc_ref, value_cache=vc_ref,
                                            image_block=True, attend_rows=rows, **kw)
    q, k, v = (_t16(x, fmt, orc, dev) for x in (qb, kb, vb))
    kc = torch.zeros((n, n_kv, d), dtype=q.dtype, device=dev)
    vc = torch.zeros_like(kc)
    fr = torch.tensor(ops.rope_freqs(theta, d), dtype=torch.float32, device=dev)
    common = dict(window=window, rope_mode=rope_mode, rope_dim=rope_dim, rope_freqs=fr)
    h_out = torch.empty((hist, n_heads, d), dtype=torch.float32, device=dev)
    ops.PrefillCall(q[:hist].contiguous(), k[:hist].contiguous(), v[:hist].contiguous(), kc, vc,
                    h_out, base_pos=0, **common)()
    out = torch.empty((blk, n_heads, d), dtype=torch.float32, device=dev)
    ops.PrefillCall(q[hist:].contiguous(), k[hist:].contiguous(), v[hist:].contiguous(), kc, vc,
                    out, base_pos=hist, bidirectional=True, **common)()
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(blk, -1)
    if sample is not None:
        return got[sample], ref[sample]
    return got, ref


@pytest.mark.parametrize("d,fmt_name,window", [(128, "F16", 0), (128, "BF16", 64),
                                               (256, "BF16", 96), (256, "F16", 0),
                                               (64, "F16", 0), (64, "BF16", 64)])
def test_prefill_image_block_bidirectional(orc, dev, d, fmt_name, window):
    """bidirectional = 1: 150 causal history rows, then a 200-row image block whose rows see
    every block key (later ones included) plus their causal / window history
    [min(start(pos), base_pos), base_pos + m) (attention.rs:87-94).  Window 64 / 96 < block
    length: late rows see the whole block but no history."""
    from gguf_runner_amd import ffi
    fmt = getattr(orc, fmt_name)
    got, ref = _image_block_case(orc, dev, hist=150, blk=200, n_heads=8, n_kv=2, d=d, fmt=fmt,
                                 seed=d + window, window=window, rope_mode=ffi.ROPE_NEOX, theta=1e4)
    _assert_close(got, ref)


def test_prefill_image_block_eight_wave_sampled(orc, dev):
    """A 2048-row block with 64 Q heads takes the 8-wave workgroups (64 x 4 pairs);
    checked on 40 sampled rows of the oracle's block attention."""
    from gguf_runner_amd import ffi
    rng = np.random.default_rng(99)
    sample = np.unique(np.concatenate([[0, 1, 255, 256, 1023, 1024, 2046, 2047],
                                       rng.integers(0, 2048, 32)]))
    got, ref = _image_block_case(orc, dev, hist=100, blk=2048, n_heads=64, n_kv=8, d=128,
                                 fmt=orc.F16, seed=7, window=0, rope_mode=ffi.ROPE_ADJACENT,
                                 theta=5e5, sample=sample)
    _assert_close(got, ref)


@pytest.mark.parametrize("where", ["chunk", "history"])
@pytest.mark.parametrize("which", ["k", "v"])
@pytest.mark.parametrize("d", [128, 256])
def test_bf16_prefill_values_outside_f16_take_the_exact_path(orc, dev, d, which, where):
    """bf16 caches run the single-pass f16 MFMA path on an exact f16 copy of their rows;
    a bf16 value f16 cannot hold (V: 70144 and -98304; K: 1e6 and -3e6 before RoPE, of
    which a rotated pair keeps at least 1/sqrt(2) in one element; in the chunk's own rows
    or in the history rows an earlier call wrote) sends the launch to the bf16 hi + lo
    path instead.  On the f16 path these values would become inf and the outputs inf or
    NaN; here they match the oracle's token-serial prefill."""
    from gguf_runner_amd import ffi
    rows = [30, 31] if where == "history" else [150, 260]

    def patch(q, k, v):
        x, big = (k, (1e6, -3e6)) if which == "k" else (v, (70144.0, -98304.0))
        x[rows[0], 0, 5] = big[0]
        x[rows[1], 1, d - 3] = big[1]

    got, ref, kc, vc = _case(orc, dev, m=300, n_heads=8, n_kv=2, d=d, fmt=orc.BF16, seed=77 + d,
                             rope_mode=ffi.ROPE_NEOX, theta=1e6, base_chunks=[100, 200], patch=patch)
    assert np.isfinite(ref).all()
    _assert_close(got, ref)
    _assert_cache(kc, vc, orc.BF16, orc)


@pytest.mark.parametrize("fmt_name,window,chunks", [("F16", 0, [100, 200]), ("BF16", 37, [64, 236]),
                                                   ("F16", 1, [300]), ("BF16", 0, [1, 127, 172])])
def test_prefill_head_dim_64(orc, dev, fmt_name, window, chunks):
    """head_dim 64 (the Qwen2-0.5B / SmolLM-class heads of qwen2.rs / smolvlm.rs) on the MFMA
    flash kernel: 128-row blocks on eight waves as two key halves (alternate 32-key
    sub-tiles of 128-key tiles, merged at the end) with the 8-chunk row swizzle, global,
    window 37 and window 1 layers, chunked continuation, f16 and bf16 caches."""
    from gguf_runner_amd import ffi
    fmt = getattr(orc, fmt_name)
    got, ref, kc, vc = _case(orc, dev, m=300, n_heads=14, n_kv=2, d=64, fmt=fmt, seed=640 + window,
                             rope_mode=ffi.ROPE_NEOX, theta=1e6, window=window, norm=window == 37,
                             base_chunks=chunks)
    _assert_close(got, ref)
    _assert_cache(kc, vc, fmt, orc)


def test_prefill_head_dim_64_four_wave_blocks(orc, dev):
    """A 2048-token head_dim-64 chunk with 60 Q / 4 KV heads (kv_mul 15): 240 eight-wave
    items do not fill the CUs and 480 four-wave ones are more than one per CU, so the
    launch takes the four-wave kernel (128-row blocks over 64-key tiles, no key halves)."""
    from gguf_runner_amd import ffi
    got, ref, kc, vc = _case(orc, dev, m=2048, n_heads=60, n_kv=4, d=64, fmt=orc.F16, seed=6460,
                             rope_mode=ffi.ROPE_NEOX, theta=1e6)
    _assert_close(got, ref)
    _assert_cache(kc, vc, orc.F16, orc)


def test_prefill_head_dim_64_eight_wave_blocks(orc, dev):
    """A 2048-token head_dim-64 chunk with 64 Q heads launches the 8-wave workgroups
    (256-row query blocks over 128-key tiles, two workgroups per CU)."""
    from gguf_runner_amd import ffi
    got, ref, kc, vc = _case(orc, dev, m=2048, n_heads=64, n_kv=8, d=64, fmt=orc.F16, seed=6464,
                             rope_mode=ffi.ROPE_ADJACENT, theta=1e4)
    _assert_close(got, ref)
    _assert_cache(kc, vc, orc.F16, orc)


@pytest.mark.parametrize("d,n_heads,n_kv,fmt_name", [(64, 14, 2, "BF16"), (128, 28, 4, "F16"), (128, 8, 2, "BF16")])
def test_prefill_qwen2_attention_biases(orc, dev, d, n_heads, n_kv, fmt_name):
    """Qwen2 q / k / v biases (qkv_bias_and_norm, inference.rs:2545-2559) added on the
    device before RoPE: head_dim 64 (Qwen2-0.5B) through the staging pass, head_dim 128
    (Qwen2-7B) with Q prepared inside the attention kernel, in two chunks."""
    from gguf_runner_amd import ffi
    rng = np.random.default_rng(2545 + d + n_heads)
    bias = tuple((0.5 * rng.standard_normal(h * d)).astype(np.float32) for h in (n_heads, n_kv, n_kv))
    fmt = getattr(orc, fmt_name)
    got, ref, kc, vc = _case(orc, dev, m=260, n_heads=n_heads, n_kv=n_kv, d=d, fmt=fmt, seed=d + n_kv,
                             rope_mode=ffi.ROPE_NEOX, theta=1e6, base_chunks=[100, 160], bias=bias)
    _assert_close(got, ref)
    _assert_cache(kc, vc, fmt, orc)
