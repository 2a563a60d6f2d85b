"""The GPFC prefill-cache restatement (oracle/gpfc.py) against the reference's own
tests of src/app/prefill_cache.rs (:513-556), the published FNV-1a test vectors,
and the byte layout stated in the format comment (prefill_cache.rs:11-19)."""
from __future__ import annotations

import numpy as np
import pytest


@pytest.fixture(scope="module")
def g(orc):
    return orc.gpfc


def test_writer_reader_roundtrip_primitives(g):
    """writer_reader_roundtrip_primitives (prefill_cache.rs:517-528)."""
    w = g.Writer()
    w.u16(7)
    w.u32(1234)
    w.u64(0xDEADBEEF)
    w.section(bytes([1, 2, 3]))
    r = g.Reader(bytes(w.b))
    assert r.u16() == 7 and r.u32() == 1234 and r.u64() == 0xDEADBEEF
    assert r.section() == bytes([1, 2, 3])
    assert bytes(w.b[:2]) == b"\x07\x00"  # little-endian
    with pytest.raises(g.GpfcError, match="prefill cache truncated"):
        r.take(1)


def test_gather_scatter_roundtrip_restrides(g):
    """gather_scatter_roundtrip_restrides (prefill_cache.rs:530-548): 2 layers, source
    seq_len 4, destination seq_len 6, k = 2 rows of 3 elements."""
    src = np.arange(2 * 4 * 3, dtype=np.int8)
    packed = g.gather_rows(src, 3, 4, 2, 2)
    assert len(packed) == 2 * 2 * 3
    dst = np.zeros(2 * 6 * 3, np.int8)
    g.scatter_rows(dst, packed, 3, 6, 2, 2)
    assert np.array_equal(dst[0:6], src[0:6])
    assert np.array_equal(dst[18:24], src[12:18])
    assert not dst[6:18].any() and not dst[24:].any()
    with pytest.raises(g.GpfcError, match="section size mismatch"):
        g.scatter_rows(dst, packed[:-1], 3, 6, 2, 2)


def test_fnv1a_published_vectors(g):
    """fnv_is_stable (prefill_cache.rs:550-554) and the FNV-1a 64-bit vectors of the
    FNV reference test suite."""
    assert g.fnv1a(b"everlock") == g.fnv1a(b"everlock")
    assert g.fnv1a(b"everlock") != g.fnv1a(b"everloch")
    assert g.fnv1a(b"") == 0xCBF29CE484222325
    assert g.fnv1a(b"a") == 0xAF63DC4C8601EC8C
    assert g.fnv1a(b"foobar") == 0x85944171F73967E8
    blob = bytes(range(256)) * 5000
    assert g.model_fingerprint(blob) == (len(blob), g.fnv1a(blob[: 1 << 20]))


def _filled(g, fmt, block, seq_len, seed, n_layers=2, n_kv=2, d=64, conv=12, ssm=20):
    rng = np.random.default_rng(seed)
    st = g.HostState(fmt, block, n_layers, seq_len, n_kv, d, conv, ssm)
    for name, a in st.a.items():
        if a.dtype == np.float32:
            a[:] = rng.standard_normal(a.size).astype(np.float32)
        else:
            a[:] = rng.integers(0, 256, a.size).astype(np.uint8).view(a.dtype)
    return st


def test_header_layout_by_offset(g):
    """Every header field at the byte offset the format comment gives, and the
    section sizes of a Q8 block-scale snapshot."""
    st = _filled(g, g.Q8, True, 8, 1)
    blob = g.snapshot(st, [5, -1, 70000], 123456789012, 0x0123456789ABCDEF)
    assert blob[0:4] == b"GPFC" and blob[4:6] == b"\x01\x00"
    assert blob[6] == 0 and blob[7] == 1
    u32 = lambda o: int.from_bytes(blob[o:o + 4], "little")
    assert (u32(8), u32(12), u32(16), u32(20), u32(24)) == (2, 128, 2, 3, 8)
    assert int.from_bytes(blob[28:36], "little") == 123456789012
    assert int.from_bytes(blob[36:44], "little") == 0x0123456789ABCDEF
    assert np.array_equal(np.frombuffer(blob[44:56], "<i4"), [5, -1, 70000])
    at, sizes = 56, []
    while at < len(blob):
        n = int.from_bytes(blob[at:at + 8], "little")
        sizes.append(n)
        at += 8 + n
    assert at == len(blob)
    # key/value codes 2 layers x 3 rows x 128, scales x 4 per row x 4 bytes, conv, ssm
    assert sizes == [768, 768, 96, 96, 48, 80]
    # layer 1's rows follow layer 0's first k rows (gather_rows)
    kq = np.frombuffer(blob[64:64 + 768], np.int8)
    assert np.array_equal(kq[384:], st.a["key_q8"][8 * 128:8 * 128 + 384])


@pytest.mark.parametrize("fmt,block", [(0, False), (0, True), (1, False)])
def test_snapshot_parse_inject_restrides(g, fmt, block):
    """snapshot -> parse -> inject into a state with another seq_len copies the first k
    rows of every layer and the SSM arrays and nothing else; the new state's own
    snapshot differs from the first only in seq_len_at_render."""
    a = _filled(g, fmt, block, 10, 2)
    toks = list(range(100, 107))
    blob = g.snapshot(a, toks, 99, 77)
    pc = g.PrefixCache.parse(blob)
    assert pc.tokens == toks and (pc.model_len, pc.model_head_fnv) == (99, 77)
    assert pc.match_len(toks + [1]) == 7 and pc.match_len(toks) is None
    assert pc.match_len([100, 101, 9, 1, 2, 3, 4, 5]) is None
    b = g.HostState(fmt, block, 2, 16, 2, 64, 12, 20)
    pc.inject(b)
    for name, per_row in a.kv_sections():
        for l in range(2):
            src = a.a[name][l * 10 * per_row:(l * 10 + 7) * per_row]
            dst = b.a[name][l * 16 * per_row:(l * 16 + 16) * per_row]
            assert np.array_equal(dst[:7 * per_row], src) and not dst[7 * per_row:].any()
    assert np.array_equal(b.a["ssm_state"], a.a["ssm_state"])
    blob2 = g.snapshot(b, toks, 99, 77)
    assert blob2[:24] + blob2[28:] == blob[:24] + blob[28:]
    assert int.from_bytes(blob2[24:28], "little") == 16


def test_parse_and_inject_errors(g):
    st = _filled(g, g.TURBO, False, 6, 3)
    blob = g.snapshot(st, [1, 2, 3], 0, 0)
    P = g.PrefixCache.parse
    for bad, msg in [(b"GPFX" + blob[4:], "bad magic"), (blob[:4] + b"\x02\x00" + blob[6:], "unsupported version 2"),
                     (blob[:6] + b"\x02" + blob[7:], "bad kv format 2"), (blob[:-1], "truncated")]:
        with pytest.raises(g.GpfcError, match=msg):
            P(bad)
    pc = P(blob)
    for other, msg in [(g.HostState(g.Q8, False, 2, 6, 2, 64, 12, 20), "model/config mismatch"),
                       (g.HostState(g.TURBO, True, 2, 6, 2, 64, 12, 20), "model/config mismatch"),
                       (g.HostState(g.TURBO, False, 2, 2, 2, 64, 12, 20), "prefix longer than context"),
                       (g.HostState(g.TURBO, False, 2, 6, 2, 64, 0, 0), "ssm state size mismatch")]:
        with pytest.raises(g.GpfcError, match=msg):
            pc.inject(other)
    pc.sections[4] = pc.sections[4][:-2]
    with pytest.raises(g.GpfcError, match="bad f32 section length"):
        pc.inject(g.HostState(g.TURBO, False, 2, 6, 2, 64, 12, 20))
