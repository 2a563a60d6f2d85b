"""Turbo KV cache on the device (KvCacheFormat::Turbo, the reference's default
format, inference.rs:346-1334): the quantising write and attention over the
packed codes, against the CPU oracle.

Tolerances (fixed before measuring):
  codes, sign bits, sigma and gamma the device writes from a given f32 row:
      bit-exact with the oracle's quantize_turboquant_head;
  attention over a Turbo cache (f32 semantics): max |gpu - ref| <= 1e-5 against
      the oracle's attention_token on the same packed rows.
"""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _oracle_cache(orc, rows_k, rows_v, table, layer, n_kv, d):
    c = orc.TurboCache(rows_k.shape[0], n_kv, d)
    for r in range(rows_k.shape[0]):
        orc.kv_write_turbo(c, r, rows_k[r], rows_v[r], table, layer)
    return c


def _decode_case(orc, dev, *, n_heads, n_kv, d, starts, ends, seq_len, seed, online=False, layer=1,
                 n_layers=2):
    from gguf_runner_amd import ops
    rng = np.random.default_rng(seed)
    n_seq = len(ends)
    kv_dim = n_kv * d
    table = orc.turbo_sign_table(n_layers, n_kv, d)
    q = rng.standard_normal((n_seq, n_heads, d), dtype=np.float32)
    caches = []
    for s in range(n_seq):
        kk = rng.standard_normal((seq_len, kv_dim), dtype=np.float32)
        vv = rng.standard_normal((seq_len, kv_dim), dtype=np.float32)
        caches.append(_oracle_cache(orc, kk, vv, table, layer, n_kv, d))
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    stack = lambda name, w: T(np.stack([getattr(c, name).reshape(seq_len, w) for c in caches]))
    out = torch.empty((n_seq, n_heads, d), device=dev)
    call = ops.TurboDecodeCall(T(q), stack("kbase", kv_dim // 4), stack("vbase", kv_dim // 4),
                               stack("ksign", kv_dim // 8), stack("vsign", kv_dim // 8),
                               stack("kscale", n_kv), stack("vscale", n_kv), stack("kres", n_kv),
                               stack("vres", n_kv), T(table), layer,
                               torch.tensor(starts, dtype=torch.int32, device=dev),
                               torch.tensor(ends, dtype=torch.int32, device=dev), out,
                               max_kv_len=max(e - s for s, e in zip(starts, ends)))
    call()
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ref = np.stack([orc.attention_token_turbo(q[s].reshape(-1), caches[s], table, layer, n_heads,
                                              starts[s], ends[s], online=online,
                                              n_threads=orc.env_threads()).reshape(n_heads, d)
                    for s in range(n_seq)])
    return got, ref


@pytest.mark.parametrize("online", [False, True])
def test_config1_turbo_decode(orc, dev, online):
    """Config 1 over the reference's default KV format: 16 Q / 8 KV heads, d128, 1024 keys."""
    got, ref = _decode_case(orc, dev, n_heads=16, n_kv=8, d=128, starts=[0], ends=[1024], seq_len=1024,
                            seed=1201, online=online)
    assert float(np.abs(got - ref).max()) <= TOL, float(np.abs(got - ref).max())


def test_turbo_decode_ragged_gqa8_tails_and_windows(orc, dev):
    """Config-3 shape (32 Q / 4 KV heads) with lengths ending inside a 32-key tile and
    sliding-window starts."""
    ends = [1, 31, 33, 1000, 3000]
    starts = [0, 0, 5, 0, 3000 - 1024]
    got, ref = _decode_case(orc, dev, n_heads=32, n_kv=4, d=128, starts=starts, ends=ends, seq_len=3000,
                            seed=1203)
    assert float(np.abs(got - ref).max()) <= TOL, float(np.abs(got - ref).max())


@pytest.mark.parametrize("d,n_heads,n_kv", [(64, 16, 8), (64, 32, 2), (256, 8, 4), (256, 16, 1), (128, 32, 2)])
def test_turbo_decode_head_dims_and_groups(orc, dev, d, n_heads, n_kv):
    """Every head size the reference's codec takes (inference.rs:363-365, 822-831),
    with GQA groups of 2 and 8 query heads (hi / lo query pieces as MFMA columns) and
    16 (one column per head); lengths ending inside a 32-key tile and a window."""
    ends = [1, 33, 700]
    starts = [0, 2, 700 - 300]
    got, ref = _decode_case(orc, dev, n_heads=n_heads, n_kv=n_kv, d=d, starts=starts, ends=ends,
                            seq_len=700, seed=1300 + d + n_kv)
    assert float(np.abs(got - ref).max()) <= TOL, float(np.abs(got - ref).max())


def _turbo_state(rt, ffi, *, rope=False, n_seq=1, seq_len=256, n_heads=16, n_kv=8, d=128):
    rng = np.random.default_rng(78)
    if rope:
        kw = dict(rope_mode=ffi.ROPE_NEOX, rope_theta=1e6, rms_norm_eps=1e-6,
                  q_norm=(1 + 0.1 * rng.standard_normal((2, d))).astype(np.float32),
                  k_norm=(1 + 0.1 * rng.standard_normal((2, d))).astype(np.float32))
    else:
        kw = dict(rope_mode=ffi.ROPE_NONE)
    p = rt.Config(n_layers=2, n_heads=n_heads, n_kv_heads=n_kv, head_dim=d, seq_len=seq_len, n_seq=n_seq,
                  kv_dtype=ffi.DTYPE_TURBO, **kw)
    return p, rt.malloc_run_state(p)


def _assert_rows_equal(dev_rows, c, row0, n, n_kv, d):
    kv_dim = n_kv * d
    for side, base, sign, sc, rn in (("k", c.kbase, c.ksign, c.kscale, c.kres),
                                     ("v", c.vbase, c.vsign, c.vscale, c.vres)):
        assert np.array_equal(dev_rows[side + "_base"], base.reshape(-1, kv_dim // 4)[row0:row0 + n]), side
        assert np.array_equal(dev_rows[side + "_sign"], sign.reshape(-1, kv_dim // 8)[row0:row0 + n]), side
        assert np.array_equal(dev_rows[side + "_scale"], sc.reshape(-1, n_kv)[row0:row0 + n]), side
        assert np.array_equal(dev_rows[side + "_rnorm"], rn.reshape(-1, n_kv)[row0:row0 + n]), side


@pytest.mark.parametrize("d", [64, 128, 256])
def test_turbo_kv_write_token_bit_exact(orc, dev, d):
    """gr_kv_write_token into a Turbo cache writes the oracle's codes, sign bits, sigma
    and gamma bit for bit: random rows of several magnitudes, an all-zero row (sigma 0)
    and a row with one silent head."""
    from gguf_runner_amd import ffi, runtime as rt
    p, s = _turbo_state(rt, ffi, seq_len=128, d=d)
    rng = np.random.default_rng(9)
    n, layer = 24, 1
    k = (rng.standard_normal((n, p.kv_dim)) * rng.uniform(0.01, 30, size=(n, 1))).astype(np.float32)
    v = rng.standard_normal((n, p.kv_dim)).astype(np.float32)
    k[2] = 0.0
    v[5, :d] = 0.0
    for t in range(n):
        s.k[:], s.v[:] = k[t], v[t]
        rt.kv_write_token(p, s, layer, 60 + t)
    table = orc.turbo_sign_table(2, p.n_kv_heads, d)
    c = orc.TurboCache(60 + n, p.n_kv_heads, d)
    for t in range(n):
        orc.kv_write_turbo(c, 60 + t, k[t], v[t], table, layer)
    _assert_rows_equal(rt.read_turbo_rows(p, s, layer, 60, n), c, 60, n, p.n_kv_heads, d)


@pytest.mark.parametrize("d", [64, 128, 256])
def test_turbo_prefill_chunk_write_batched_bit_exact(orc, dev, d):
    """A 1401-row prefill chunk with 3 KV heads has 8406 K and V units, past the 4096
    from which the write quantises 4 units per wave (lane u running unit u's
    sequential norms): the last wave holds 2 units and one wave holds both K and V
    units (4203 of each).  Codes, sign bits, sigma and gamma equal the oracle's
    quantize_turboquant_head bit for bit, over rows of several magnitudes, an
    all-zero K row (sigma 0) and a silent V head."""
    from gguf_runner_amd import ffi, runtime as rt
    m, layer = 1401, 1
    p, s = _turbo_state(rt, ffi, seq_len=1408, n_heads=6, n_kv=3, d=d)
    rng = np.random.default_rng(31 + d)
    q = rng.standard_normal((m, p.q_dim)).astype(np.float32)
    k = (rng.standard_normal((m, p.kv_dim)) * rng.uniform(0.01, 30, size=(m, 1))).astype(np.float32)
    v = rng.standard_normal((m, p.kv_dim)).astype(np.float32)
    k[2] = 0.0
    v[5, :d] = 0.0
    rt.prefill_attention_chunk(p, s, layer, 0, q, k, v)
    table = orc.turbo_sign_table(2, p.n_kv_heads, d)
    c = orc.TurboCache(m, p.n_kv_heads, d)
    for t in range(m):
        orc.kv_write_turbo(c, t, k[t], v[t], table, layer)
    _assert_rows_equal(rt.read_turbo_rows(p, s, layer, 0, m), c, 0, m, p.n_kv_heads, d)


def test_turbo_layer_token_loop_and_chunked_prefill(orc, dev):
    """Qwen3-0.6B-shaped layer (QK-norm, NeoX theta 1e6) over a Turbo cache: the
    token-serial gr_attention_layer_token loop and 64-token prefill chunks write the
    same rows, those rows are the oracle's encoding of the device's normed and RoPE'd
    k (and of v), bit for bit, and each output equals the oracle's attention over
    them with the device's q (1e-5)."""
    from gguf_runner_amd import ffi, runtime as rt
    p, s_tok = _turbo_state(rt, ffi, rope=True)
    _, s_chk = _turbo_state(rt, ffi, rope=True)
    _, s_aux = _turbo_state(rt, ffi, rope=True)
    rng = np.random.default_rng(10)
    m, layer, d = 130, 1, 128
    q = rng.standard_normal((m, p.q_dim)).astype(np.float32)
    k = rng.standard_normal((m, p.kv_dim)).astype(np.float32)
    v = rng.standard_normal((m, p.kv_dim)).astype(np.float32)
    tok = np.zeros((m, p.q_dim), np.float32)
    for t in range(m):
        s_tok.q[:], s_tok.k[:], s_tok.v[:] = q[t], k[t], v[t]
        rt.attention_layer_token(p, s_tok, layer, t)
        tok[t] = s_tok.xb
    chk = np.concatenate([rt.prefill_attention_chunk(p, s_chk, layer, b, q[b:b + 64], k[b:b + 64],
                                                     v[b:b + 64]) for b in range(0, m, 64)])
    r1 = rt.read_turbo_rows(p, s_tok, layer, 0, m)
    r2 = rt.read_turbo_rows(p, s_chk, layer, 0, m)
    for key in r1:
        assert np.array_equal(r1[key], r2[key]), key
    assert float(np.abs(tok - chk).max()) <= TOL
    table = orc.turbo_sign_table(2, p.n_kv_heads, d)
    c = orc.TurboCache(m, p.n_kv_heads, d)
    qs = []
    for t in range(m):
        s_aux.q[:], s_aux.k[:] = q[t], k[t]
        rt.qkv_bias_and_norm(p, s_aux, layer)
        rt.apply_rope_qk(p, s_aux, layer, t)
        orc.kv_write_turbo(c, t, s_aux.k, v[t], table, layer)
        qs.append(s_aux.q.copy())
    _assert_rows_equal(r1, c, 0, m, p.n_kv_heads, d)
    for t in range(m):
        ref = orc.attention_token_turbo(qs[t], c, table, layer, 16, 0, t + 1)
        assert float(np.abs(tok[t] - ref).max()) <= TOL, (t, float(np.abs(tok[t] - ref).max()))


def test_turbo_decode_layer_batch_slots(orc, dev):
    """gr_decode_layer_batch over three sequence slots of a Turbo cache."""
    from gguf_runner_amd import ffi, runtime as rt
    p, s = _turbo_state(rt, ffi, n_seq=3, seq_len=300, n_heads=32, n_kv=4)
    rng = np.random.default_rng(11)
    lens = [5, 170, 299]
    table = orc.turbo_sign_table(2, 4, 128)
    caches = []
    for sq, L in enumerate(lens):
        kk = rng.standard_normal((L + 1, p.kv_dim)).astype(np.float32)
        vv = rng.standard_normal((L + 1, p.kv_dim)).astype(np.float32)
        for t in range(L):
            s.k[:], s.v[:] = kk[t], vv[t]
            rt.kv_write_token(p, s, 0, t, seq=sq)
        caches.append((kk, vv))
    q = rng.standard_normal((3, p.q_dim)).astype(np.float32)
    order = [2, 0, 1]
    got = rt.decode_layer_batch(p, s, 0, order, [lens[i] for i in order], q[order],
                                np.stack([caches[i][0][lens[i]] for i in order]),
                                np.stack([caches[i][1][lens[i]] for i in order]))
    for b, sq in enumerate(order):
        c = _oracle_cache(orc, caches[sq][0], caches[sq][1], table, 0, 4, 128)
        ref = orc.attention_token_turbo(q[sq], c, table, 0, 32, 0, lens[sq] + 1)
        assert float(np.abs(got[b] - ref).max()) <= TOL, (sq, float(np.abs(got[b] - ref).max()))


@pytest.mark.parametrize("n_heads,n_kv,window,image,d", [
    (16, 8, None, False, 128), (32, 4, 70, False, 128), (16, 1, None, False, 128), (16, 8, 45, True, 128),
    (32, 4, None, True, 128), (8, 4, 50, False, 256), (8, 4, None, True, 256), (16, 8, None, False, 64)])
def test_turbo_prefill_chunk_token_packed(orc, dev, n_heads, n_kv, window, image, d):
    """A 200-row gr_prefill_attention_chunk (or gr_prefill_image_block) over a Turbo
    cache after a 40-token history: the split kernel packs 16 / kv_mul consecutive
    rows into its MFMA columns (kv_mul 2, 8 and 16: 8, 2 and 1 rows; at d256 8 / kv_mul
    rows, each with an f16 hi and a lo query column), each column masked to its own
    visible keys; global or sliding-window layer; head_dim 64, 128 and 256.  Each
    output row == the oracle's attention_token_turbo over the oracle's encoding of
    the same rows, with that row's visible range (1e-5)."""
    from gguf_runner_amd import ffi, runtime as rt
    p = rt.Config(n_layers=2, n_heads=n_heads, n_kv_heads=n_kv, head_dim=d, seq_len=320,
                  kv_dtype=ffi.DTYPE_TURBO, rope_mode=ffi.ROPE_NONE, layer_windows=[window, window])
    s = rt.malloc_run_state(p)
    rng = np.random.default_rng(41 + n_kv + (window or 0))
    hist, m, layer = 40, 200, 1
    n = hist + m
    q = rng.standard_normal((n, p.q_dim)).astype(np.float32)
    k = rng.standard_normal((n, p.kv_dim)).astype(np.float32)
    v = rng.standard_normal((n, p.kv_dim)).astype(np.float32)
    rt.prefill_attention_chunk(p, s, layer, 0, q[:hist], k[:hist], v[:hist])
    call = rt.prefill_image_block if image else rt.prefill_attention_chunk
    got = call(p, s, layer, hist, q[hist:], k[hist:], v[hist:])
    table = orc.turbo_sign_table(2, n_kv, d)
    c = orc.TurboCache(n, n_kv, d)
    for t in range(n):
        orc.kv_write_turbo(c, t, k[t], v[t], table, layer)
    _assert_rows_equal(rt.read_turbo_rows(p, s, layer, 0, n), c, 0, n, n_kv, d)
    worst = 0.0
    for i in range(m):
        pos = hist + i
        start = max(0, pos + 1 - window) if window else 0
        end = pos + 1
        if image:
            start, end = min(start, hist), n
        ref = orc.attention_token_turbo(q[pos], c, table, layer, n_heads, start, end)
        worst = max(worst, float(np.abs(got[i] - ref).max()))
    assert worst <= TOL, worst


@pytest.mark.parametrize("n_heads,n_kv,d,m,window", [(32, 8, 128, 6656, None), (32, 8, 128, 6656, 300),
                                                     (16, 8, 256, 6656, None), (16, 8, 64, 12800, None)])
def test_turbo_prefill_chunk_single_split_finished_in_split_kernel(orc, dev, n_heads, n_kv, d, m, window):
    """A chunk runs as overlapped pieces of 256 rows, six middle pieces and 256 rows;
    a piece with at least 2048 (row group, KV head) workgroups gets one split per
    group (the middle pieces here: 1024 rows in groups of 4 x 8 KV heads = 2048; d64:
    2048 rows in groups of 8), and the split kernel finishes those rows itself (1/l,
    the inverse rotations, the output store) with no partials and no combine launch;
    the 256-row edge pieces take several splits and the combine.  Sampled rows (the
    first two groups, every piece edge, the end and 12 random rows) == the oracle's
    attention_token_turbo with each row's causal or window range (1e-5)."""
    from gguf_runner_amd import ffi, runtime as rt
    p = rt.Config(n_layers=2, n_heads=n_heads, n_kv_heads=n_kv, head_dim=d, seq_len=m + 8,
                  kv_dtype=ffi.DTYPE_TURBO, rope_mode=ffi.ROPE_NONE, layer_windows=[window, window])
    s = rt.malloc_run_state(p)
    rng = np.random.default_rng(7 * d + m + (window or 0))
    layer = 1
    q = rng.standard_normal((m, p.q_dim)).astype(np.float32)
    k = rng.standard_normal((m, p.kv_dim)).astype(np.float32)
    v = rng.standard_normal((m, p.kv_dim)).astype(np.float32)
    got = rt.prefill_attention_chunk(p, s, layer, 0, q, k, v)
    table = orc.turbo_sign_table(2, n_kv, d)
    c = orc.TurboCache(m, n_kv, d)
    for t in range(m):
        orc.kv_write_turbo(c, t, k[t], v[t], table, layer)
    edges = [256 + (m - 512) * i // 6 for i in range(7)]
    rows = sorted(set(range(8)) | {e + o for e in edges for o in (-1, 0)} | {m - 2, m - 1}
                  | set(rng.integers(0, m, 12).tolist()))
    worst = 0.0
    for i in rows:
        start = max(0, i + 1 - window) if window else 0
        ref = orc.attention_token_turbo(q[i], c, table, layer, n_heads, start, i + 1)
        worst = max(worst, float(np.abs(got[i] - ref).max()))
    assert worst <= TOL, worst


@pytest.mark.parametrize("n_kv,m,window,hist", [(8, 3, None, 5), (8, 11, 1, 20), (2, 1, None, 0), (4, 37, 3, 60)])
def test_turbo_prefill_chunk_partial_groups(orc, dev, n_kv, m, window, hist):
    """Token-packed Turbo prefill with partial row groups (16 query heads: kv_mul 2
    packs 8 rows per group, so chunks of 3 and 11 rows end inside a group; kv_mul 4
    packs 4, so 37 rows do), a one-row chunk (kv_mul 8: two rows per group), and
    windows 1 and 3 (rows of one group see different keys)."""
    from gguf_runner_amd import ffi, runtime as rt
    n_heads, d = 16, 128
    p = rt.Config(n_layers=1, n_heads=n_heads, n_kv_heads=n_kv, head_dim=d, seq_len=128,
                  kv_dtype=ffi.DTYPE_TURBO, rope_mode=ffi.ROPE_NONE, layer_windows=[window])
    s = rt.malloc_run_state(p)
    rng = np.random.default_rng(17 + m)
    n = hist + m
    q = rng.standard_normal((n, p.q_dim)).astype(np.float32)
    k = rng.standard_normal((n, p.kv_dim)).astype(np.float32)
    v = rng.standard_normal((n, p.kv_dim)).astype(np.float32)
    if hist:
        rt.prefill_attention_chunk(p, s, 0, 0, q[:hist], k[:hist], v[:hist])
    got = rt.prefill_attention_chunk(p, s, 0, hist, q[hist:], k[hist:], v[hist:])
    table = orc.turbo_sign_table(1, n_kv, d)
    c = orc.TurboCache(n, n_kv, d)
    for t in range(n):
        orc.kv_write_turbo(c, t, k[t], v[t], table, 0)
    for i in range(m):
        pos = hist + i
        start = max(0, pos + 1 - window) if window else 0
        ref = orc.attention_token_turbo(q[pos], c, table, 0, n_heads, start, pos + 1)
        assert float(np.abs(got[i] - ref).max()) <= TOL, (i, float(np.abs(got[i] - ref).max()))


@pytest.mark.parametrize("d,n_heads,n_kv", [(128, 32, 4), (128, 32, 2), (64, 16, 8), (256, 8, 4)])
def test_turbo_decode_stream_many_short_ragged(orc, dev, d, n_heads, n_kv):
    """Stream schedule over 24 short ragged sequences, four of them empty and most
    offset: workgroup ranges begin and end inside the virtual keys charged per
    (sequence, KV head) pair and cross several pairs each; GQA groups of 8 (hi / lo
    query pieces as MFMA columns) and 16 (one column per head).  An empty range
    gives zeros, as the oracle's loop over no keys does."""
    rng = np.random.default_rng(5151 + d + n_kv)
    n = 24
    lens = rng.integers(1, 600, size=n)
    lens[[0, 5, 6, 23]] = 0
    starts = rng.integers(0, 80, size=n)
    ends = starts + lens
    got, ref = _decode_case(orc, dev, n_heads=n_heads, n_kv=n_kv, d=d, starts=starts.tolist(),
                            ends=ends.tolist(), seq_len=int(ends.max()), seed=1400 + d + n_kv)
    assert float(np.abs(got - ref).max()) <= TOL, float(np.abs(got - ref).max())
    assert not got[[0, 5, 6, 23]].any()


@pytest.mark.parametrize("n_seq", [1024, 1025])
def test_turbo_decode_stream_sequence_limit(orc, dev, n_seq):
    """The Turbo split kernel's stream schedule at its 1024-sequence table limit
    (four per thread of the scan) and the fixed grid just past it."""
    rng = np.random.default_rng(n_seq + 7)
    lens = rng.integers(0, 24, size=n_seq)
    starts = rng.integers(0, 8, size=n_seq)
    ends = starts + lens
    got, ref = _decode_case(orc, dev, n_heads=8, n_kv=4, d=64, starts=starts.tolist(), ends=ends.tolist(),
                            seq_len=int(ends.max()), seed=1500 + n_seq)
    assert float(np.abs(got - ref).max()) <= TOL, float(np.abs(got - ref).max())
    assert not got[lens == 0].any()


def test_turbo_large_chunk_runs_in_overlapped_pieces(orc, dev):
    """A 2048-row chunk at the config-2 shape over a Turbo cache, then a 1024-row
    one: overlapped pieces of 256, 512, 512, 512, 256 and of 256, 512, 256 rows,
    each piece's keys written before the next piece's queries read them.  Every
    row's Turbo encoding == the oracle's (bit-exact); sampled output rows of both
    chunks == the oracle's attention_token_turbo (1e-5)."""
    from gguf_runner_amd import ffi, runtime as rt
    n_heads, n_kv, d, layer = 32, 8, 128, 0
    m1, m2 = 2048, 1024
    n = m1 + m2
    p = rt.Config(n_layers=1, n_heads=n_heads, n_kv_heads=n_kv, head_dim=d, seq_len=n,
                  kv_dtype=ffi.DTYPE_TURBO, rope_mode=ffi.ROPE_NONE)
    s = rt.malloc_run_state(p)
    rng = np.random.default_rng(3072)
    q = rng.standard_normal((n, p.q_dim)).astype(np.float32)
    k = rng.standard_normal((n, p.kv_dim)).astype(np.float32)
    v = rng.standard_normal((n, p.kv_dim)).astype(np.float32)
    out1 = rt.prefill_attention_chunk(p, s, layer, 0, q[:m1], k[:m1], v[:m1]).copy()
    out2 = rt.prefill_attention_chunk(p, s, layer, m1, q[m1:], k[m1:], v[m1:]).copy()
    got = np.concatenate([out1, out2])
    table = orc.turbo_sign_table(1, n_kv, d)
    c = orc.TurboCache(n, n_kv, d)
    for t in range(n):
        orc.kv_write_turbo(c, t, k[t], v[t], table, layer)
    _assert_rows_equal(rt.read_turbo_rows(p, s, layer, 0, n), c, 0, n, n_kv, d)
    rows = sorted({0, 1, 255, 256, 767, 768, 1279, 1280, 1791, 1792, 2047, 2048, 2303, 2304, 2815, 2816, n - 1}
                  | set(rng.integers(0, n, 10).tolist()))
    worst = 0.0
    for t in rows:
        ref = orc.attention_token_turbo(q[t], c, table, layer, n_heads, 0, t + 1)
        worst = max(worst, float(np.abs(got[t] - ref).max()))
    assert worst <= TOL, worst
