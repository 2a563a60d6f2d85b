"""Decode parity: gr_decode_attention (split-K HIP kernels) vs the CPU oracle's
attention_token (reference inference.rs:1970-2530) on identical seeded inputs.

Tolerances (written here, fixed before measuring):
  fp32 KV (config 1):           max |gpu - ref| <= 1e-5
  f16 / bf16 KV (configs 3, 4): |gpu - ref| <= 2e-3 + 1e-2 * |ref| elementwise
"""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-5
ATOL_16, RTOL_16 = 2e-3, 1e-2


def _run_case(orc, dev, *, n_heads, n_kv, d, starts, ends, seq_len, fmt, seed, online=False,
              score_scale=None, split_keys=0):
    from gguf_runner_amd import ops
    rng = np.random.default_rng(seed)
    n_seq = len(ends)
    q = rng.standard_normal((n_seq, n_heads, d), dtype=np.float32)
    kf = rng.standard_normal((n_seq, seq_len, n_kv * d), dtype=np.float32)
    vf = rng.standard_normal((n_seq, seq_len, n_kv * d), dtype=np.float32)
    if fmt == orc.F32:
        kc, vc = kf, vf
        tdt = torch.float32
        kt = torch.from_numpy(kc)
        vt = torch.from_numpy(vc)
    else:
        conv = orc.f16_bits if fmt == orc.F16 else orc.bf16_bits
        kc, vc = conv(kf), conv(vf)
        tdt = torch.float16 if fmt == orc.F16 else torch.bfloat16
        kt = torch.from_numpy(kc.view(np.int16)).view(tdt)
        vt = torch.from_numpy(vc.view(np.int16)).view(tdt)
    kt = kt.reshape(n_seq, seq_len, n_kv, d).to(dev)
    vt = vt.reshape(n_seq, seq_len, n_kv, d).to(dev)
    qt = torch.from_numpy(q).to(dev)
    st = torch.tensor(starts, dtype=torch.int32, device=dev)
    en = torch.tensor(ends, dtype=torch.int32, device=dev)
    scale = (1.0 / np.sqrt(np.float32(d))) if score_scale is None else score_scale
    out = ops.decode_attention(qt, kt, vt, st, en, max_kv_len=max(e - s for s, e in zip(starts, ends)),
                               score_scale=float(scale), split_keys=split_keys)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ref = np.stack([
        orc.attention_token(q[s].reshape(-1), kc[s], vc[s], fmt, n_heads, n_kv, d, starts[s],
                            ends[s], attn_scale=float(scale), apply_attn_scale=True,
                            online=online, n_threads=orc.env_threads()).reshape(n_heads, d)
        for s in range(n_seq)])
    return got, ref


def _assert_close(got, ref, fmt, orc):
    err = np.abs(got - ref)
    if fmt == orc.F32:
        assert float(err.max()) <= TOL_F32, f"max abs {err.max():.3e}"
    else:
        bad = ~(err <= ATOL_16 + RTOL_16 * np.abs(ref))  # NaN counts as out of tolerance
        assert not bad.any(), f"{bad.sum()} elements out of tolerance, max abs {err.max():.3e}"


@pytest.mark.parametrize("online", [False, True])
def test_config1_qwen3_0p6b_decode_f32(orc, dev, online):
    """Config 1: B=1, 16 Q / 8 KV heads, d128, 1024 cached keys, fp32, scale 1/sqrt(128)."""
    got, ref = _run_case(orc, dev, n_heads=16, n_kv=8, d=128, starts=[0], ends=[1024],
                         seq_len=1024, fmt=orc.F32, seed=1001, online=online)
    _assert_close(got, ref, orc.F32, orc)


def test_config3_qwen3_30b_a3b_ragged_f16(orc, dev):
    """Config 3: 16 sequences, ragged lengths U[1024, 32768], 32 Q / 4 KV heads, f16 KV."""
    rng = np.random.default_rng(1003)
    lens = rng.integers(1024, 32768, size=16, endpoint=True).tolist()
    got, ref = _run_case(orc, dev, n_heads=32, n_kv=4, d=128, starts=[0] * 16, ends=lens,
                         seq_len=32768, fmt=orc.F16, seed=2003)
    _assert_close(got, ref, orc.F16, orc)


@pytest.mark.parametrize("window", [1024, 0])
def test_config4_gemma3_decode_bf16(orc, dev, window):
    """Config 4 decode: 8 Q / 4 KV heads, d256, bf16; local window 1024 vs global.
    Gemma3 q is pre-scaled so scores are unscaled (inference.rs:1982)."""
    pos = 8192 + 17
    start, end = orc.visible_keys(window, pos)
    got, ref = _run_case(orc, dev, n_heads=8, n_kv=4, d=256, starts=[start], ends=[end],
                         seq_len=pos + 1, fmt=orc.BF16, seed=1004, score_scale=1.0)
    _assert_close(got, ref, orc.BF16, orc)


@pytest.mark.parametrize("fmt_name", ["F16", "BF16"])
@pytest.mark.parametrize("n_heads,n_kv,ends", [(14, 2, [1, 33, 700, 5000, 20000]), (9, 3, [1024]),
                                               (14, 2, [4096, 300])])
def test_decode_head_dim_64_16bit_mfma(orc, dev, fmt_name, n_heads, n_kv, ends):
    """head_dim 64 over f16 / bf16 caches (Qwen2-0.5B 14 / 2 heads, SmolLM-135M 9 / 3) on
    the MFMA decode kernel: a ragged batch on the stream schedule, and short calls on
    the fixed grid of the small-call plan; the 8-chunk K tile swizzle (r >> 1) & 7."""
    fmt = getattr(orc, fmt_name)
    got, ref = _run_case(orc, dev, n_heads=n_heads, n_kv=n_kv, d=64, starts=[0] * len(ends), ends=ends,
                         seq_len=max(ends), fmt=fmt, seed=6400 + sum(ends) % 97)
    _assert_close(got, ref, fmt, orc)


@pytest.mark.parametrize("L", [1, 2, 63, 64, 65, 1000])
def test_decode_edge_lengths(orc, dev, L):
    """Single key (out == v), lengths around the 64-row block step, f32."""
    got, ref = _run_case(orc, dev, n_heads=4, n_kv=4, d=64, starts=[0], ends=[L], seq_len=L,
                         fmt=orc.F32, seed=L)
    _assert_close(got, ref, orc.F32, orc)


def test_decode_single_key_returns_v(orc, dev):
    """With one visible key softmax is exactly 1 and xb == v (two-pass softmax)."""
    from gguf_runner_amd import ops
    rng = np.random.default_rng(7)
    d, n_kv = 128, 2
    q = torch.from_numpy(rng.standard_normal((1, 4, d), dtype=np.float32)).to(dev)
    kv = rng.standard_normal((1, 5, n_kv, d), dtype=np.float32)
    k = torch.from_numpy(kv).to(dev)
    v = torch.from_numpy(kv * 3).to(dev)
    st = torch.tensor([3], dtype=torch.int32, device=dev)
    en = torch.tensor([4], dtype=torch.int32, device=dev)
    out = ops.decode_attention(q, k, v, st, en, max_kv_len=1).cpu().numpy()
    exp = np.repeat(kv[0, 3] * 3, 2, axis=0)
    assert np.array_equal(out[0], exp)


@pytest.mark.parametrize("split", [64, 128, 4096])
def test_decode_split_sizes_agree(orc, dev, split):
    """Forced split sizes (many partials vs one) give the oracle's answer."""
    got, ref = _run_case(orc, dev, n_heads=16, n_kv=2, d=128, starts=[5, 0, 100],
                         ends=[3000, 1, 2100], seq_len=3000, fmt=orc.F16, seed=split,
                         split_keys=split)
    _assert_close(got, ref, orc.F16, orc)


def test_decode_windowed_ragged_bf16(orc, dev):
    """Sliding-window start offsets per sequence, kv_mul 4, bf16, d128."""
    starts = [0, 7, 1023, 4000]
    ends = [17, 1031, 2047, 5024]
    got, ref = _run_case(orc, dev, n_heads=16, n_kv=4, d=128, starts=starts, ends=ends,
                         seq_len=5024, fmt=orc.BF16, seed=99)
    _assert_close(got, ref, orc.BF16, orc)


@pytest.mark.parametrize("fmt_name", ["f16", "bf16"])
@pytest.mark.parametrize("L,n_heads,n_kv", [(1, 16, 1), (31, 4, 2), (32, 12, 1), (33, 8, 8),
                                             (129, 16, 4), (4097, 32, 4)])
def test_decode_16bit_mfma_shapes(orc, dev, fmt_name, L, n_heads, n_kv):
    """The MFMA split kernel (16-bit caches): tile tails, kv_mul 1..16 (incl. 12),
    head_dim 128."""
    fmt = orc.F16 if fmt_name == "f16" else orc.BF16
    got, ref = _run_case(orc, dev, n_heads=n_heads, n_kv=n_kv, d=128, starts=[0], ends=[L],
                         seq_len=L, fmt=fmt, seed=L + n_heads)
    _assert_close(got, ref, fmt, orc)


@pytest.mark.parametrize("fmt_name", ["f16", "bf16"])
def test_decode_16bit_d256_window(orc, dev, fmt_name):
    fmt = orc.F16 if fmt_name == "f16" else orc.BF16
    got, ref = _run_case(orc, dev, n_heads=8, n_kv=4, d=256, starts=[3, 0], ends=[1500, 77],
                         seq_len=1500, fmt=fmt, seed=256, score_scale=1.0)
    _assert_close(got, ref, fmt, orc)


@pytest.mark.parametrize("fmt_name,n_heads,n_kv", [("f16", 16, 4), ("bf16", 48, 2), ("q8", 16, 4)])
def test_decode_stream_many_short_ragged(orc, dev, fmt_name, n_heads, n_kv):
    """Stream schedule over 40 short ragged sequences, four of them empty and most
    offset: with ~512 virtual keys charged per (sequence, KV head) pair, workgroup
    ranges begin and end inside those virtual keys and cross several pairs each;
    48 / 2 heads put two workgroup columns on each KV head.  An empty range gives
    zeros, as the oracle's loop over no keys does."""
    rng = np.random.default_rng(4242 + n_heads)
    n = 40
    lens = rng.integers(1, 700, size=n)
    lens[[3, 4, 17, 39]] = 0
    starts = rng.integers(0, 100, size=n)
    ends = starts + lens
    kw = dict(n_heads=n_heads, n_kv=n_kv, d=128, starts=starts.tolist(), ends=ends.tolist(),
              seq_len=int(ends.max()), seed=77 + n_heads)
    if fmt_name == "q8":
        from test_gpu_q8 import TOL, _decode_case
        got, ref = _decode_case(orc, dev, block=False, **kw)
        assert float(np.abs(got - ref).max()) <= TOL, np.abs(got - ref).max()
    else:
        fmt = orc.F16 if fmt_name == "f16" else orc.BF16
        got, ref = _run_case(orc, dev, fmt=fmt, **kw)
        _assert_close(got, ref, fmt, orc)
    assert not got[[3, 4, 17, 39]].any()


@pytest.mark.parametrize("n_seq", [1024, 1025])
def test_decode_stream_sequence_limit(orc, dev, n_seq):
    """1024 sequences fill the stream schedule's per-workgroup tables (two per
    thread of the scan); 1025 take the fixed split grid.  Short ragged lengths,
    some empty, f16, 8 / 2 heads."""
    rng = np.random.default_rng(n_seq)
    lens = rng.integers(0, 48, size=n_seq)
    starts = rng.integers(0, 16, size=n_seq)
    ends = starts + lens
    got, ref = _run_case(orc, dev, n_heads=8, n_kv=2, d=128, starts=starts.tolist(), ends=ends.tolist(),
                         seq_len=int(ends.max()), fmt=orc.F16, seed=n_seq)
    _assert_close(got, ref, orc.F16, orc)
    assert not got[lens == 0].any()


def test_decode_stream_length_above_declared_max(orc, dev):
    """A sequence longer than the max_kv_len the caller declared (a contract
    violation the host cannot see) stays contained on the stream schedule: its
    length is capped at what the partial slots cover, the other sequences keep
    the oracle's answer, and its own output is finite.  The cache holds every
    key, so no read leaves it."""
    from gguf_runner_amd import ops
    rng = np.random.default_rng(31337)
    n_heads, n_kv, d = 8, 2, 128
    lens = [300, 5000, 40, 500]
    declared = 512  # only sequence 1 exceeds it
    L = max(lens)
    q = rng.standard_normal((len(lens), n_heads, d), dtype=np.float32)
    kb = orc.f16_bits(rng.standard_normal((len(lens), L, n_kv * d), dtype=np.float32))
    vb = orc.f16_bits(rng.standard_normal((len(lens), L, n_kv * d), dtype=np.float32))
    T16 = lambda a: torch.from_numpy(a.view(np.int16)).view(torch.float16).reshape(len(lens), L, n_kv, d).to(dev)
    st = torch.zeros(len(lens), dtype=torch.int32, device=dev)
    en = torch.tensor(lens, dtype=torch.int32, device=dev)
    out = ops.decode_attention(torch.from_numpy(q).to(dev), T16(kb), T16(vb), st, en, max_kv_len=declared)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    for s in (0, 2, 3):
        ref = orc.attention_token(q[s].reshape(-1), kb[s], vb[s], orc.F16, n_heads, n_kv, d, 0, lens[s],
                                  n_threads=orc.env_threads()).reshape(n_heads, d)
        _assert_close(got[s], ref, orc.F16, orc)
