"""Q8 KV cache on the device (KvCacheFormat::Q8): the write path (kv_write_token's
Q8 branch, reference inference.rs:166-268 and 1886-1917) and attention over int8
rows with row scales or 32-element block scales (GGUF_Q8_BLOCK_SCALES,
inference.rs:1337-1483), against the CPU oracle.

Tolerances (fixed before measuring):
  codes and scales the device writes from a given f32 row: bit-exact with the
      oracle's quantize_row_q8 (integer / byte work);
  attention over a Q8 cache (f32 semantics, config 1's Q8 mode): max |gpu - ref|
      <= 1e-5 against the oracle on the same int8 rows and scales;
  the stress cases whose rows are scaled by up to e^2 per 32-element block (outputs
      ~20, thousands of keys): the reference's own fp32 loops drift from the exact
      result by up to ~6e-4 there, so both are measured against a float64 evaluation
      of the same int8 rows and scales, and the device must be no further from it
      than the oracle is, plus 1e-5.
"""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _assert_vs_f64(got, ref, exact):
    e_gpu = float(np.abs(got - exact).max())
    e_orc = float(np.abs(ref - exact).max())
    assert e_gpu <= e_orc + TOL, f"device {e_gpu:.3e} vs oracle {e_orc:.3e} from float64"


def _quantize_cache(orc, x, block):
    """[n_seq][L][kv_dim] f32 -> (int8 codes, f32 scales [n_seq][L][per_row])."""
    n_seq, L, kv_dim = x.shape
    per = kv_dim // 32 if block else 1
    codes = np.zeros(x.shape, np.int8)
    scales = np.zeros((n_seq, L, per), np.float32)
    for s in range(n_seq):
        for t in range(L):
            codes[s, t], scales[s, t] = orc.kv_quantize_row(x[s, t], block)
    return codes, scales


def _decode_case(orc, dev, *, n_heads, n_kv, d, starts, ends, seq_len, block, seed, online=False,
                 loud_blocks=False):
    from gguf_runner_amd import ops
    rng = np.random.default_rng(seed)
    n_seq = len(ends)
    kv_dim = n_kv * d
    q = rng.standard_normal((n_seq, n_heads, d), dtype=np.float32)
    kf = rng.standard_normal((n_seq, seq_len, kv_dim), dtype=np.float32)
    vf = rng.standard_normal((n_seq, seq_len, kv_dim), dtype=np.float32)
    if loud_blocks:  # block magnitudes spread over e^+-2: a wrong block scale index shows
        mag = np.exp(rng.uniform(-2, 2, size=(n_seq, seq_len, kv_dim // 32))).astype(np.float32)
        kf *= np.repeat(mag, 32, axis=2)
        vf *= np.repeat(mag[:, :, ::-1], 32, axis=2)
    kq, ks = _quantize_cache(orc, kf, block)
    vq, vs = _quantize_cache(orc, vf, block)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    st = torch.tensor(starts, dtype=torch.int32, device=dev)
    en = torch.tensor(ends, dtype=torch.int32, device=dev)
    out = ops.decode_attention(T(q), T(kq.reshape(n_seq, seq_len, n_kv, d)),
                               T(vq.reshape(n_seq, seq_len, n_kv, d)), st, en,
                               max_kv_len=max(e - s for s, e in zip(starts, ends)),
                               k_scale=T(ks), v_scale=T(vs), q8_block=block)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    fmt = orc.Q8B if block else orc.Q8
    ref = np.stack([
        orc.attention_token(q[s].reshape(-1), kq[s], vq[s], fmt, n_heads, n_kv, d, starts[s], ends[s],
                            key_scale=ks[s].reshape(-1), value_scale=vs[s].reshape(-1),
                            online=online, n_threads=orc.env_threads()).reshape(n_heads, d)
        for s in range(n_seq)])
    if not loud_blocks:
        return got, ref
    # float64 closed form over the same dequantised rows
    per = kv_dim // 32 if block else 1
    exact = np.zeros((n_seq, n_heads, d))
    for s in range(n_seq):
        a, b = starts[s], ends[s]
        K = kq[s, a:b].astype(np.float64) * np.repeat(ks[s, a:b], kv_dim // per, axis=1)
        V = vq[s, a:b].astype(np.float64) * np.repeat(vs[s, a:b], kv_dim // per, axis=1)
        for h in range(n_heads):
            g = h // (n_heads // n_kv)
            sc = K[:, g * d:(g + 1) * d] @ q[s, h].astype(np.float64) / np.sqrt(d)
            w = np.exp(sc - sc.max())
            exact[s, h] = (w / w.sum()) @ V[:, g * d:(g + 1) * d]
    return got, ref, exact


@pytest.mark.parametrize("block", [False, True])
@pytest.mark.parametrize("online", [False, True])
def test_config1_q8_decode(orc, dev, block, online):
    """Config 1 in Q8 mode: 16 Q / 8 KV heads, d128, 1024 cached keys."""
    got, ref = _decode_case(orc, dev, n_heads=16, n_kv=8, d=128, starts=[0], ends=[1024],
                            seq_len=1024, block=block, seed=1101, online=online)
    assert float(np.abs(got - ref).max()) <= TOL, float(np.abs(got - ref).max())


@pytest.mark.parametrize("block", [False, True])
def test_q8_decode_ragged_gqa8_tails(orc, dev, block):
    """Config-3 shape (32 Q / 4 KV heads, d128) with ragged lengths that end inside
    a 32-key tile (1, 31, 33, 1000, 4097 keys) and block magnitudes spread out."""
    ends = [1, 31, 33, 1000, 4097]
    got, ref, exact = _decode_case(orc, dev, n_heads=32, n_kv=4, d=128, starts=[0] * 5, ends=ends,
                                   seq_len=4097, block=block, seed=1103, loud_blocks=True)
    _assert_vs_f64(got, ref, exact)


@pytest.mark.parametrize("block", [False, True])
def test_q8_decode_d256_sliding_window(orc, dev, block):
    """Gemma-3 shape (8 Q / 4 KV heads, d256) with sliding-window ranges
    [pos + 1 - W, pos] (attention.rs:74-96), W = 1024, unaligned starts."""
    ends = [1500, 2049, 700]
    starts = [max(0, e - 1024) for e in ends]
    got, ref, exact = _decode_case(orc, dev, n_heads=8, n_kv=4, d=256, starts=starts, ends=ends,
                                   seq_len=2049, block=block, seed=1104, loud_blocks=True)
    _assert_vs_f64(got, ref, exact)


def _q8_state(rt, ffi, block, *, rope=False, n_seq=1, seq_len=512, n_heads=16, n_kv=8, d=128):
    rng = np.random.default_rng(77)
    kw = {}
    if rope:
        kw = dict(rope_mode=ffi.ROPE_NEOX, rope_theta=1e6, rms_norm_eps=1e-6,
                  q_norm=(1 + 0.1 * rng.standard_normal((2, d))).astype(np.float32),
                  k_norm=(1 + 0.1 * rng.standard_normal((2, d))).astype(np.float32))
    else:
        kw = dict(rope_mode=ffi.ROPE_NONE)
    p = rt.Config(n_layers=2, n_heads=n_heads, n_kv_heads=n_kv, head_dim=d, seq_len=seq_len,
                  n_seq=n_seq, kv_dtype=ffi.DTYPE_Q8, q8_block_scales=block, **kw)
    return p, rt.malloc_run_state(p)


@pytest.mark.parametrize("block", [False, True])
def test_q8_kv_write_token_bit_exact(orc, dev, block):
    """gr_kv_write_token into a Q8 cache writes the oracle's codes and scales bit for
    bit: random rows, an all-zero row (scale 1, codes 0), and exact .5 ties that round
    away from zero (Rust f32::round)."""
    from gguf_runner_amd import ffi, runtime as rt
    p, s = _q8_state(rt, ffi, block)
    rng = np.random.default_rng(5)
    n = 40
    rows_k = rng.standard_normal((n, p.kv_dim)).astype(np.float32) * 3
    rows_v = rng.standard_normal((n, p.kv_dim)).astype(np.float32)
    rows_k[3] = 0.0
    ties = np.tile(np.array([127.0, 0.5, -0.5, 1.5, -2.5, 126.5, -126.5, 3.0], np.float32),
                   p.kv_dim // 8)
    rows_v[7] = ties
    rows_k[9, :32] = 0.0  # one silent block inside a live row
    layer = 1
    for t in range(n):
        s.k[:], s.v[:] = rows_k[t], rows_v[t]
        rt.kv_write_token(p, s, layer, 100 + t)
    kq, vq = rt.read_kv_rows(p, s, layer, 100, n)
    ks, vs = rt.read_kv_scales(p, s, layer, 100, n)
    for t in range(n):
        ek, eks = orc.kv_quantize_row(rows_k[t], block)
        ev, evs = orc.kv_quantize_row(rows_v[t], block)
        assert np.array_equal(kq[t], ek) and np.array_equal(vq[t], ev), t
        assert np.array_equal(ks[t], eks) and np.array_equal(vs[t], evs), t
    assert list(vq[7][:8]) == [127, 1, -1, 2, -3, 127, -127, 3]


@pytest.mark.parametrize("block", [False, True])
def test_q8_layer_token_loop_and_chunked_prefill(orc, dev, block):
    """Qwen3-0.6B-shaped layer (QK-norm, NeoX theta 1e6) over a Q8 cache: the
    token-serial gr_attention_layer_token loop and 64-token gr_prefill_attention_chunk
    calls write the same rows; each row holds the oracle's quantize_row_q8 codes of
    the device's normed and RoPE'd k (gr_qkv_norm + gr_apply_rope_qk, which other
    tests pin to the oracle) and of v, bit for bit; and each output equals the
    oracle's attention_token over those rows with the device's q (1e-5)."""
    from gguf_runner_amd import ffi, runtime as rt
    p, s_tok = _q8_state(rt, ffi, block, rope=True, seq_len=256)
    _, s_chk = _q8_state(rt, ffi, block, rope=True, seq_len=256)
    _, s_aux = _q8_state(rt, ffi, block, rope=True, seq_len=256)
    rng = np.random.default_rng(6)
    m, layer, d = 150, 1, 128
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
    kq, vq = rt.read_kv_rows(p, s_tok, layer, 0, m)
    ks, vs = rt.read_kv_scales(p, s_tok, layer, 0, m)
    kq2, vq2 = rt.read_kv_rows(p, s_chk, layer, 0, m)
    ks2, vs2 = rt.read_kv_scales(p, s_chk, layer, 0, m)
    assert np.array_equal(kq, kq2) and np.array_equal(vq, vq2)
    assert np.array_equal(ks, ks2) and np.array_equal(vs, vs2)
    assert float(np.abs(tok - chk).max()) <= TOL
    fmt = orc.Q8B if block else orc.Q8
    for t in range(m):
        s_aux.q[:], s_aux.k[:] = q[t], k[t]
        rt.qkv_bias_and_norm(p, s_aux, layer)
        rt.apply_rope_qk(p, s_aux, layer, t)
        ek, eks = orc.kv_quantize_row(s_aux.k, block)
        ev, evs = orc.kv_quantize_row(v[t], block)
        assert np.array_equal(kq[t], ek) and np.array_equal(ks[t], eks), t
        assert np.array_equal(vq[t], ev) and np.array_equal(vs[t], evs), t
        ref = orc.attention_token(s_aux.q, kq, vq, fmt, 16, 8, d, 0, t + 1,
                                  key_scale=ks.reshape(-1), value_scale=vs.reshape(-1))
        assert float(np.abs(tok[t] - ref).max()) <= TOL, (t, float(np.abs(tok[t] - ref).max()))


@pytest.mark.parametrize("block", [False, True])
def test_q8_decode_layer_batch_slots(orc, dev, block):
    """gr_decode_layer_batch over three sequence slots of a Q8 cache (the batched
    per-sequence layer_attention_token_staged calls) == the oracle per sequence."""
    from gguf_runner_amd import ffi, runtime as rt
    p, s = _q8_state(rt, ffi, block, n_seq=3, seq_len=300, n_heads=32, n_kv=4)
    rng = np.random.default_rng(8)
    lens = [5, 170, 299]
    rows = {}
    for sq, L in enumerate(lens):  # history via kv_write_token
        kk = rng.standard_normal((L, p.kv_dim)).astype(np.float32)
        vv = rng.standard_normal((L, p.kv_dim)).astype(np.float32)
        for t in range(L):
            s.k[:], s.v[:] = kk[t], vv[t]
            rt.kv_write_token(p, s, 0, t, seq=sq)
        rows[sq] = (kk, vv)
    q = rng.standard_normal((3, p.q_dim)).astype(np.float32)
    k = rng.standard_normal((3, p.kv_dim)).astype(np.float32)
    v = rng.standard_normal((3, p.kv_dim)).astype(np.float32)
    got = rt.decode_layer_batch(p, s, 0, [2, 0, 1], [lens[2], lens[0], lens[1]], q[[2, 0, 1]],
                                k[[2, 0, 1]], v[[2, 0, 1]])
    fmt = orc.Q8B if block else orc.Q8
    for b, sq in enumerate([2, 0, 1]):
        L = lens[sq] + 1
        kk = np.concatenate([rows[sq][0], k[sq:sq + 1]])
        vv = np.concatenate([rows[sq][1], v[sq:sq + 1]])
        kq, ks = _quantize_cache(orc, kk[None], block)
        vq, vs = _quantize_cache(orc, vv[None], block)
        ref = orc.attention_token(q[sq], kq[0], vq[0], fmt, 32, 4, 128, 0, L,
                                  key_scale=ks.reshape(-1), value_scale=vs.reshape(-1))
        assert float(np.abs(got[b] - ref).max()) <= TOL, (sq, float(np.abs(got[b] - ref).max()))


@pytest.mark.parametrize("block,d,window,image", [
    (False, 128, None, False), (True, 128, 100, False), (False, 256, None, False),
    (True, 256, 37, False), (False, 128, None, True), (True, 128, 60, True),
    (False, 256, None, True), (True, 256, 60, True), (False, 64, None, False),
    (True, 64, 50, False), (False, 64, 70, True), (True, 64, None, True)])
def test_q8_prefill_chunk_mfma(orc, dev, block, d, window, image):
    """One long gr_prefill_attention_chunk (or gr_prefill_image_block) over a Q8 cache
    after a 40-token history: 300 query rows of the MFMA prefill kernel (d128: 128-row
    query blocks over 128-key tiles; d256: 64-row blocks over 64-key tiles), global or
    sliding-window layer, row or block scales; d64 as d128 with 8-chunk rows.  Each output
    row == the oracle's attention_token over the rows the device wrote, with that row's
    visible range (1e-5)."""
    from gguf_runner_amd import ffi, runtime as rt
    n_heads, n_kv = {64: (12, 4), 128: (16, 8), 256: (8, 2)}[d]
    p = rt.Config(n_layers=2, n_heads=n_heads, n_kv_heads=n_kv, head_dim=d, seq_len=512,
                  kv_dtype=ffi.DTYPE_Q8, q8_block_scales=block, rope_mode=ffi.ROPE_NONE,
                  layer_windows=[window, window])
    s = rt.malloc_run_state(p)
    rng = np.random.default_rng(31 + d + (window or 0))
    hist, m, layer = 40, 300, 1
    n = hist + m
    q = rng.standard_normal((n, p.q_dim)).astype(np.float32)
    k = rng.standard_normal((n, p.kv_dim)).astype(np.float32)
    v = rng.standard_normal((n, p.kv_dim)).astype(np.float32)
    rt.prefill_attention_chunk(p, s, layer, 0, q[:hist], k[:hist], v[:hist])
    call = rt.prefill_image_block if image else rt.prefill_attention_chunk
    got = call(p, s, layer, hist, q[hist:], k[hist:], v[hist:])
    kq, vq = rt.read_kv_rows(p, s, layer, 0, n)
    ks, vs = rt.read_kv_scales(p, s, layer, 0, n)
    fmt = orc.Q8B if block else orc.Q8
    worst = 0.0
    for i in range(m):
        pos = hist + i
        start = max(0, pos + 1 - window) if window else 0
        end = pos + 1
        if image:
            start, end = min(start, hist), n
        ref = orc.attention_token(q[pos], kq, vq, fmt, n_heads, n_kv, d, start, end,
                                  key_scale=ks.reshape(-1), value_scale=vs.reshape(-1))
        worst = max(worst, float(np.abs(got[i] - ref).max()))
    assert worst <= TOL, worst


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("block,m,window,hist", [
    (False, 1, None, 7), (True, 31, 1, 0), (False, 33, 5, 90), (True, 97, None, 415)])
def test_q8_prefill_chunk_edges(orc, dev, block, m, window, hist, d):
    """Q8 prefill edge cases at both tilings: one-row and ragged chunks (1, 31, 33, 97
    rows: partial 32-row groups, inactive row groups and partial query blocks), window 1
    (each row sees only itself, so one key half of a workgroup is empty) and 5, a chunk
    that ends exactly at seq_len (history 415 + 97 = 512)."""
    from gguf_runner_amd import ffi, runtime as rt
    n_heads, n_kv = {64: (12, 4), 128: (16, 8), 256: (8, 2)}[d]
    p = rt.Config(n_layers=1, n_heads=n_heads, n_kv_heads=n_kv, head_dim=d, seq_len=512,
                  kv_dtype=ffi.DTYPE_Q8, q8_block_scales=block, rope_mode=ffi.ROPE_NONE,
                  layer_windows=[window])
    s = rt.malloc_run_state(p)
    rng = np.random.default_rng(7 + m)
    n = hist + m
    q = rng.standard_normal((n, p.q_dim)).astype(np.float32)
    k = rng.standard_normal((n, p.kv_dim)).astype(np.float32)
    v = rng.standard_normal((n, p.kv_dim)).astype(np.float32)
    if hist:
        rt.prefill_attention_chunk(p, s, 0, 0, q[:hist], k[:hist], v[:hist])
    got = rt.prefill_attention_chunk(p, s, 0, hist, q[hist:], k[hist:], v[hist:])
    kq, vq = rt.read_kv_rows(p, s, 0, 0, n)
    ks, vs = rt.read_kv_scales(p, s, 0, 0, n)
    fmt = orc.Q8B if block else orc.Q8
    for i in range(m):
        pos = hist + i
        start = max(0, pos + 1 - window) if window else 0
        ref = orc.attention_token(q[pos], kq, vq, fmt, n_heads, n_kv, d, start, pos + 1,
                                  key_scale=ks.reshape(-1), value_scale=vs.reshape(-1))
        assert float(np.abs(got[i] - ref).max()) <= TOL, (i, float(np.abs(got[i] - ref).max()))


@pytest.mark.parametrize("kv", ["q8", "q8b", "turbo"])
def test_quantised_prefill_into_a_middle_sequence_slot(orc, dev, kv):
    """Q8 (row / block scales) and Turbo prefill into sequence slot 1 of a 3-slot,
    2-layer run state whose slots 0 and 2 hold other rows: the outputs match the
    oracle over slot 1's own rows (cache and scale offsets of slot and layer), and
    the neighbouring slots are left byte-for-byte unchanged."""
    from gguf_runner_amd import ffi, runtime as rt
    n_heads, n_kv, d, L = 16, 4, 128, 160
    turbo = kv == "turbo"
    p = rt.Config(n_layers=2, n_heads=n_heads, n_kv_heads=n_kv, head_dim=d, seq_len=L, n_seq=3,
                  kv_dtype=ffi.DTYPE_TURBO if turbo else ffi.DTYPE_Q8, q8_block_scales=kv == "q8b",
                  rope_mode=ffi.ROPE_NONE)
    s = rt.malloc_run_state(p)
    rng = np.random.default_rng(123)
    rows = {sq: [rng.standard_normal((L, w)).astype(np.float32) for w in (p.q_dim, p.kv_dim, p.kv_dim)]
            for sq in range(3)}
    layer = 1
    for sq in (0, 2):
        q, k, v = rows[sq]
        rt.prefill_attention_chunk(p, s, layer, 0, q[:100], k[:100], v[:100], seq=sq)
    snap = lambda sq: (rt.read_turbo_rows(p, s, layer, 0, 100, seq=sq) if turbo
                       else (rt.read_kv_rows(p, s, layer, 0, 100, seq=sq), rt.read_kv_scales(p, s, layer, 0, 100, seq=sq)))
    before = {sq: snap(sq) for sq in (0, 2)}
    q, k, v = rows[1]
    hist, m = 30, 130
    rt.prefill_attention_chunk(p, s, layer, 0, q[:hist], k[:hist], v[:hist], seq=1)
    got = rt.prefill_attention_chunk(p, s, layer, hist, q[hist:hist + m], k[hist:hist + m], v[hist:hist + m], seq=1)
    n = hist + m
    if turbo:
        table = orc.turbo_sign_table(2, n_kv, d)
        c = orc.TurboCache(n, n_kv, d)
        for t in range(n):
            orc.kv_write_turbo(c, t, k[t], v[t], table, layer)
        refs = [orc.attention_token_turbo(q[hist + i], c, table, layer, n_heads, 0, hist + i + 1) for i in range(m)]
    else:
        kq, vq = rt.read_kv_rows(p, s, layer, 0, n, seq=1)
        ks, vs = rt.read_kv_scales(p, s, layer, 0, n, seq=1)
        fmt = orc.Q8B if kv == "q8b" else orc.Q8
        for t in range(n):  # slot 1's rows are the oracle's quantisation of its own k / v
            ek, eks = orc.kv_quantize_row(k[t], kv == "q8b")
            assert np.array_equal(kq[t], ek) and np.array_equal(ks[t], eks), t
        refs = [orc.attention_token(q[hist + i], kq, vq, fmt, n_heads, n_kv, d, 0, hist + i + 1,
                                    key_scale=ks.reshape(-1), value_scale=vs.reshape(-1)) for i in range(m)]
    worst = max(float(np.abs(got[i] - refs[i]).max()) for i in range(m))
    assert worst <= TOL, worst
    for sq in (0, 2):
        after = snap(sq)
        if turbo:
            for key in after:
                assert np.array_equal(after[key], before[sq][key]), (sq, key)
        else:
            assert np.array_equal(after[0][0], before[sq][0][0]) and np.array_equal(after[0][1], before[sq][0][1])
            assert np.array_equal(after[1][0], before[sq][1][0]) and np.array_equal(after[1][1], before[sq][1][1])


@pytest.mark.parametrize("block,window", [(False, None), (True, 700)])
def test_q8_large_chunks_run_in_overlapped_pieces(orc, dev, block, window):
    """Chunks of 2048 and 1024 rows at the config-2 shape (32 / 8 heads, d128): above
    16 MB of host rows the run-state call cuts its rows into pieces (256, 512, 512, 512,
    256 rows, then 256, 512, 256) whose uploads, kernels and downloads overlap, each piece written to the
    cache before the next one's queries read it.  The K / V codes and scales of every
    row == the oracle's quantize_row_q8 (bit-exact); sampled output rows of both chunks
    (piece edges included) == the oracle's attention_token over those rows (1e-5)."""
    from gguf_runner_amd import ffi, runtime as rt
    n_heads, n_kv, d = 32, 8, 128
    m1, m2 = 2048, 1024
    n = m1 + m2
    p = rt.Config(n_layers=1, n_heads=n_heads, n_kv_heads=n_kv, head_dim=d, seq_len=n,
                  kv_dtype=ffi.DTYPE_Q8, q8_block_scales=block, rope_mode=ffi.ROPE_NONE,
                  layer_windows=[window])
    s = rt.malloc_run_state(p)
    rng = np.random.default_rng(2048 + (window or 0))
    q = rng.standard_normal((n, p.q_dim)).astype(np.float32)
    k = rng.standard_normal((n, p.kv_dim)).astype(np.float32)
    v = rng.standard_normal((n, p.kv_dim)).astype(np.float32)
    out1 = rt.prefill_attention_chunk(p, s, 0, 0, q[:m1], k[:m1], v[:m1]).copy()
    out2 = rt.prefill_attention_chunk(p, s, 0, m1, q[m1:], k[m1:], v[m1:]).copy()
    got = np.concatenate([out1, out2])
    kq, vq = rt.read_kv_rows(p, s, 0, 0, n)
    ks, vs = rt.read_kv_scales(p, s, 0, 0, n)
    ck, sk = _quantize_cache(orc, k[None], block)
    cv, sv = _quantize_cache(orc, v[None], block)
    assert np.array_equal(kq, ck[0]) and np.array_equal(vq, cv[0])
    assert np.array_equal(ks.reshape(sk[0].shape), sk[0]) and np.array_equal(vs.reshape(sv[0].shape), sv[0])
    fmt = orc.Q8B if block else orc.Q8
    rows = sorted({0, 1, 255, 256, 767, 768, 1279, 1280, 1791, 1792, 2047, 2048, 2303, 2304, 2815, 2816, n - 1}
                  | set(rng.integers(0, n, 10).tolist()))
    worst = 0.0
    for t in rows:
        start = max(0, t + 1 - window) if window else 0
        ref = orc.attention_token(q[t], kq, vq, fmt, n_heads, n_kv, d, start, t + 1,
                                  key_scale=ks.reshape(-1), value_scale=vs.reshape(-1))
        worst = max(worst, float(np.abs(got[t] - ref).max()))
    assert worst <= TOL, worst
