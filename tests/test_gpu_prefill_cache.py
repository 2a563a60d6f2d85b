"""Prefill-cache (GPFC v1) export / import of the device run state
(gr_prefill_cache_snapshot / gr_prefill_cache_inject = snapshot, PrefixCache::parse
and inject, src/app/prefill_cache.rs:178-507).

The device blob must equal, byte for byte, the oracle's GPFC writer (oracle/gpfc.py,
pinned by the reference's own prefill-cache tests) over the rows the oracle's codecs
produce for the same inputs (quantize_row_q8 / the Turbo writer, bit-exact) and the
same SSM arrays.  Injection is checked by reading the rows back, by re-snapshotting,
and by the next decode step, which must match the state the blob came from (1e-5,
the fp32 bar).
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

L, NH, NKV, D, K = 3, 4, 2, 128, 29
SSM_H, SSM_K, CONV_K = 2, 1, 4
CONV_DIM = (SSM_H + 2 * SSM_K) * D
FORMATS = [("q8", False), ("q8", True), ("turbo", False)]


def _config(rt, ffi, fmt, block, seq_len, n_seq, ssm=True):
    rng = np.random.default_rng(1)
    kw = {}
    if ssm:
        kw = dict(ssm_n_heads=SSM_H, ssm_head_dim=D, ssm_n_k_heads=SSM_K, ssm_conv_kernel=CONV_K,
                  ssm_conv1d=rng.standard_normal((L, CONV_DIM, CONV_K)).astype(np.float32),
                  ssm_a=rng.standard_normal((L, SSM_H)).astype(np.float32),
                  ssm_dt_bias=rng.standard_normal((L, SSM_H)).astype(np.float32),
                  ssm_norm=np.ones((L, D), np.float32))
    dt = ffi.DTYPE_TURBO if fmt == "turbo" else (ffi.DTYPE_Q8 if fmt == "q8" else ffi.DTYPE_F16)
    p = rt.Config(n_layers=L, n_heads=NH, n_kv_heads=NKV, head_dim=D, seq_len=seq_len, n_seq=n_seq,
                  kv_dtype=dt, q8_block_scales=block, rope_mode=ffi.ROPE_NONE, **kw)
    return p, rt.malloc_run_state(p)


def _fill(rt, p, s, seq, rows, seed):
    """rows K/V rows per layer into slot `seq`, plus random SSM arrays; returns them."""
    rng = np.random.default_rng(seed)
    kr = (rng.standard_normal((L, rows, p.kv_dim)) * rng.uniform(0.05, 20, (L, rows, 1))).astype(np.float32)
    vr = rng.standard_normal((L, rows, p.kv_dim)).astype(np.float32)
    kr[1, min(3, rows - 1)] = 0.0  # one all-zero row (Q8 scale 1, Turbo sigma 0)
    for l in range(L):
        for t in range(rows):
            s.k[:], s.v[:] = kr[l, t], vr[l, t]
            rt.kv_write_token(p, s, l, t, seq=seq)
    if not p.ssm_n_heads:
        return kr, vr, None, None
    conv = rng.standard_normal((L, CONV_K - 1, CONV_DIM)).astype(np.float32)
    state = rng.standard_normal((L, SSM_H, D, D)).astype(np.float32)
    for l in range(L):
        rt.write_ssm_conv_state(p, s, l, conv[l])
        rt.write_ssm_state(p, s, l, state[l])
    return kr, vr, conv, state


def _expected_host_state(orc, fmt, block, seq_len, kr, vr, conv, state):
    g = orc.gpfc
    st = g.HostState(g.TURBO if fmt == "turbo" else g.Q8, block, L, seq_len, NKV, D,
                     0 if conv is None else conv.size, 0 if state is None else state.size)
    kv = NKV * D
    if fmt == "q8":
        spr = kv // 32 if block else 1
        for l in range(L):
            for t in range(kr.shape[1]):
                r = l * seq_len + t
                for side, rows in (("key", kr), ("value", vr)):
                    codes, sc = orc.kv_quantize_row(rows[l, t], block)
                    st.a[side + "_q8"][r * kv:(r + 1) * kv] = codes
                    st.a[side + "_scale"][r * spr:(r + 1) * spr] = sc
    else:
        table = orc.turbo_sign_table(L, NKV, D)
        for l in range(L):
            c = orc.TurboCache(seq_len, NKV, D)
            for t in range(kr.shape[1]):
                orc.kv_write_turbo(c, t, kr[l, t], vr[l, t], table, l)
            for name, arr in (("key_base", c.kbase), ("value_base", c.vbase), ("key_sign", c.ksign),
                              ("value_sign", c.vsign), ("key_scale", c.kscale), ("value_scale", c.vscale),
                              ("key_rnorm", c.kres), ("value_rnorm", c.vres)):
                n = arr.size
                st.a[name][l * n:(l + 1) * n] = arr
    if conv is not None:
        st.a["ssm_conv"][:] = conv.reshape(-1)
        st.a["ssm_state"][:] = state.reshape(-1)
    return st


def _rows(rt, p, s, fmt, seq, n):
    out = []
    for l in range(L):
        if fmt == "turbo":
            out.append(rt.read_turbo_rows(p, s, l, 0, n, seq=seq))
        else:
            out.append((rt.read_kv_rows(p, s, l, 0, n, seq=seq), rt.read_kv_scales(p, s, l, 0, n, seq=seq)))
    return out


def _same_rows(a, b):
    for x, y in zip(a, b):
        if isinstance(x, dict):
            assert x.keys() == y.keys()
            for key in x:
                assert np.array_equal(x[key], y[key]), key
        else:
            for u, v in zip(x, y):
                for uu, vv in zip(u, v):
                    assert np.array_equal(uu, vv)


# (sequence slots, snapshot slot, SSM state): an SSM state has one slot (as one
# reference RunState), so the two-slot cases carry KV sections only.
SLOTS = [(2, 1, False), (1, 0, True)]


@pytest.mark.parametrize("n_seq,slot,ssm", SLOTS)
@pytest.mark.parametrize("fmt,block", FORMATS)
def test_snapshot_matches_oracle_bytes(orc, dev, fmt, block, n_seq, slot, ssm):
    """The last slot of the state (slot 0 of a two-slot state holds other rows): the
    device blob is the oracle's blob of the same rows, codes, scales and SSM arrays,
    byte for byte."""
    from gguf_runner_amd import ffi, runtime as rt
    p, s = _config(rt, ffi, fmt, block, seq_len=48, n_seq=n_seq, ssm=ssm)
    if slot:
        _fill(rt, p, s, 0, 40, seed=10)
    kr, vr, conv, state = _fill(rt, p, s, slot, K, seed=11)
    toks = list(range(1000, 1000 + K))
    blob = rt.snapshot(p, s, toks, 4_000_000_123, 0xFEEDFACECAFEBEEF, seq=slot)
    ref = orc.gpfc.snapshot(_expected_host_state(orc, fmt, block, 48, kr, vr, conv, state),
                            toks, 4_000_000_123, 0xFEEDFACECAFEBEEF)
    assert len(blob) == len(ref)
    assert blob == ref


@pytest.mark.parametrize("n_seq,slot,ssm", SLOTS)
@pytest.mark.parametrize("fmt,block", FORMATS)
def test_inject_restrides_and_decode_continues(orc, dev, fmt, block, n_seq, slot, ssm):
    """The blob of the last slot (context 48) injected into the same slot of a state
    with context 80: the rows and SSM arrays read back equal the source's, slot 0 of
    a two-slot state is untouched, the new state's snapshot differs only in
    seq_len_at_render, and the next token's attention over the injected rows equals
    the source state's."""
    from gguf_runner_amd import ffi, runtime as rt
    pa, sa = _config(rt, ffi, fmt, block, seq_len=48, n_seq=n_seq, ssm=ssm)
    _fill(rt, pa, sa, slot, K, seed=12)
    toks = list(range(7, 7 + K))
    blob = rt.snapshot(pa, sa, toks, 1, 2, seq=slot)
    pb, sb = _config(rt, ffi, fmt, block, seq_len=80, n_seq=n_seq, ssm=ssm)
    if slot:
        _fill(rt, pb, sb, 0, 5, seed=13)
        slot0 = _rows(rt, pb, sb, fmt, 0, 5)
    assert rt.inject(pb, sb, blob, seq=slot) == K
    _same_rows(_rows(rt, pb, sb, fmt, slot, K), _rows(rt, pa, sa, fmt, slot, K))
    if slot:
        _same_rows(_rows(rt, pb, sb, fmt, 0, 5), slot0)
    for l in range(L if ssm else 0):
        assert np.array_equal(rt.read_ssm_state(pb, sb, l), rt.read_ssm_state(pa, sa, l))
        assert np.array_equal(rt.read_ssm_conv_state(pb, sb, l), rt.read_ssm_conv_state(pa, sa, l))
    blob_b = rt.snapshot(pb, sb, toks, 1, 2, seq=slot)
    assert blob_b[:24] + blob_b[28:] == blob[:24] + blob[28:]
    assert int.from_bytes(blob_b[24:28], "little") == 80
    rng = np.random.default_rng(14)
    q = rng.standard_normal(pa.q_dim).astype(np.float32)
    k = rng.standard_normal(pa.kv_dim).astype(np.float32)
    v = rng.standard_normal(pa.kv_dim).astype(np.float32)
    outs = []
    for p, s in ((pa, sa), (pb, sb)):
        s.q[:], s.k[:], s.v[:] = q, k, v
        rt.attention_layer_token(p, s, 2, K, seq=slot)
        outs.append(s.xb.copy())
    assert float(np.abs(outs[0] - outs[1]).max()) <= 1e-5


def test_empty_prefix_and_size_query(orc, dev):
    """k = 0: empty KV sections, the SSM arrays still travel; the size query returns
    the blob length; a short buffer is refused."""
    from gguf_runner_amd import ffi, runtime as rt
    import ctypes
    p, s = _config(rt, ffi, "q8", False, seq_len=16, n_seq=1)
    _, _, conv, state = _fill(rt, p, s, 0, 4, seed=15)
    blob = rt.snapshot(p, s, [], 0, 0)
    g = orc.gpfc
    st = g.HostState(g.Q8, False, L, 16, NKV, D, conv.size, state.size)
    st.a["ssm_conv"][:] = conv.reshape(-1)
    st.a["ssm_state"][:] = state.reshape(-1)
    assert blob == g.snapshot(st, [], 0, 0)
    p2, s2 = _config(rt, ffi, "q8", False, seq_len=16, n_seq=1)
    assert rt.inject(p2, s2, blob) == 0
    assert np.array_equal(rt.read_ssm_state(p2, s2, 2), state[2])
    buf = np.zeros(len(blob) - 1, np.uint8)
    size = ctypes.c_uint64()
    rc = ffi.lib().gr_prefill_cache_snapshot(s.handle, 0, None, 0, 0, 0, buf.ctypes.data, buf.size,
                                             ctypes.byref(size))
    assert rc != 0 and size.value == len(blob)
    assert b"buffer too small" in ffi.lib().gr_last_error()


def test_errors_follow_reference_messages(orc, dev):
    """The reference's parse / inject errors; a rejected blob leaves the state as it was."""
    from gguf_runner_amd import ffi, runtime as rt
    p, s = _config(rt, ffi, "turbo", False, seq_len=48, n_seq=1)
    _fill(rt, p, s, 0, K, seed=16)
    blob = rt.snapshot(p, s, list(range(K)), 0, 0)

    def err(fn, msg):
        with pytest.raises(ffi.GrError, match=msg):
            fn()

    pf, sf = _config(rt, ffi, "f16", False, seq_len=48, n_seq=1)
    err(lambda: rt.snapshot(pf, sf, [1], 0, 0), "requires a Q8 or Turbo KV cache")
    err(lambda: rt.snapshot(p, s, list(range(49)), 0, 0), "prefix longer than context")
    pq, sq = _config(rt, ffi, "q8", False, seq_len=48, n_seq=1)
    err(lambda: rt.inject(pq, sq, blob), "model/config mismatch")
    ps, ss = _config(rt, ffi, "turbo", False, seq_len=20, n_seq=1)
    err(lambda: rt.inject(ps, ss, blob), "prefix longer than context")
    pt, st = _config(rt, ffi, "turbo", False, seq_len=48, n_seq=1)
    _fill(rt, pt, st, 0, 3, seed=17)
    before = _rows(rt, pt, st, "turbo", 0, K)
    err(lambda: rt.inject(pt, st, b"GPFX" + blob[4:]), "bad magic")
    err(lambda: rt.inject(pt, st, blob[:4] + b"\x02\x00" + blob[6:]), "unsupported version 2")
    err(lambda: rt.inject(pt, st, blob[:6] + b"\x05" + blob[7:]), "bad kv format 5")
    err(lambda: rt.inject(pt, st, blob[:-1]), "prefill cache truncated")
    pn, sn = _config(rt, ffi, "turbo", False, seq_len=48, n_seq=1, ssm=False)
    err(lambda: rt.inject(pn, sn, blob), "ssm state size mismatch")
    _same_rows(_rows(rt, pt, st, "turbo", 0, K), before)
