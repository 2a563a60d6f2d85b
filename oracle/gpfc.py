"""GPFC v1 prefill-cache writer and reader -- TEST INFRASTRUCTURE ONLY.

Importable only from tests/ (through oracle.py): it checks the bytes that
libgr_attn's gr_prefill_cache_snapshot writes and the device rows that
gr_prefill_cache_inject restores; it is never part of the product path.

A restatement of src/app/prefill_cache.rs over host arrays laid out like the
reference's RunState: every KV array holds n_layers * seq_len rows, row t of
layer l at (l * seq_len + t) * per_row.

    Writer / Reader           prefill_cache.rs:70-112
    gather_rows / scatter_rows                 :139-175
    snapshot                                   :178-310
    PrefixCache.parse                          :316-364
    PrefixCache.match_len                      :366-377
    PrefixCache.inject                         :380-507
    fnv1a / model_fingerprint                  :56-68
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

MAGIC = b"GPFC"
VERSION = 1
Q8, TURBO = 0, 1
Q8_BLOCK = 32
HEADER_BYTES = 44  # magic 4 + version 2 + format 1 + q8_block 1 + 5 x u32 + 2 x u64


class GpfcError(ValueError):
    """The reference's Err(String) from parse / inject / snapshot."""


def fnv1a(data: bytes) -> int:
    """64-bit FNV-1a (offset basis 0xcbf29ce484222325, prime 0x100000001b3)."""
    h = 0xCBF29CE484222325
    for b in data:
        h ^= b
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def model_fingerprint(model_bytes: bytes):
    return len(model_bytes), fnv1a(model_bytes[: 1 << 20])


class Writer:
    def __init__(self):
        self.b = bytearray()

    def u16(self, v):
        self.b += int(v).to_bytes(2, "little")

    def u32(self, v):
        self.b += int(v).to_bytes(4, "little")

    def u64(self, v):
        self.b += int(v).to_bytes(8, "little")

    def section(self, data: bytes):
        self.u64(len(data))
        self.b += data


class Reader:
    def __init__(self, b: bytes):
        self.b, self.at = b, 0

    def take(self, n):
        if self.at + n > len(self.b):
            raise GpfcError("prefill cache truncated")
        s = self.b[self.at:self.at + n]
        self.at += n
        return s

    def u16(self):
        return int.from_bytes(self.take(2), "little")

    def u32(self):
        return int.from_bytes(self.take(4), "little")

    def u64(self):
        return int.from_bytes(self.take(8), "little")

    def section(self):
        return bytes(self.take(self.u64()))


def gather_rows(src, per_row, seq_len, n_layers, k):
    """The first k rows of each layer of a [n_layers * seq_len]-row array."""
    src = np.asarray(src)
    return np.concatenate([src[l * seq_len * per_row:(l * seq_len + k) * per_row]
                           for l in range(n_layers)]) if n_layers else src[:0]


def scatter_rows(dst, packed, per_row, seq_len, n_layers, k):
    """Inverse of gather_rows with the destination's own seq_len stride."""
    if len(packed) != n_layers * k * per_row:
        raise GpfcError("prefill cache: section size mismatch")
    for l in range(n_layers):
        dst[l * seq_len * per_row:(l * seq_len + k) * per_row] = packed[l * k * per_row:(l + 1) * k * per_row]


def _f32s(b: bytes):
    if len(b) % 4:
        raise GpfcError("prefill cache: bad f32 section length")
    return np.frombuffer(b, "<f4").copy()


@dataclass
class HostState:
    """The RunState fields a snapshot reads (types.rs:745-809)."""

    kv_format: int
    q8_block_scales: bool
    n_layers: int
    seq_len: int
    n_kv_heads: int
    head_dim: int
    conv_len: int = 0     # ssm_conv_state floats (all layers)
    ssm_len: int = 0      # ssm_state floats (all layers)
    a: dict = field(default_factory=dict)

    @property
    def kv_dim(self):
        return self.n_kv_heads * self.head_dim

    def __post_init__(self):
        rows = self.n_layers * self.seq_len
        d, h = self.kv_dim, max(self.n_kv_heads, 1)
        if self.kv_format == Q8:
            spr = max(d // Q8_BLOCK, 1) if self.q8_block_scales else 1
            spec = dict(key_q8=(d, np.int8), value_q8=(d, np.int8),
                        key_scale=(spr, np.float32), value_scale=(spr, np.float32))
        else:
            spec = dict(key_base=(d // 4, np.uint8), value_base=(d // 4, np.uint8),
                        key_sign=(d // 8, np.uint8), value_sign=(d // 8, np.uint8),
                        key_scale=(h, np.float32), value_scale=(h, np.float32),
                        key_rnorm=(h, np.float32), value_rnorm=(h, np.float32))
        for name, (per_row, dt) in spec.items():
            self.a.setdefault(name, np.zeros(rows * per_row, dt))
        self.a.setdefault("ssm_conv", np.zeros(self.conv_len, np.float32))
        self.a.setdefault("ssm_state", np.zeros(self.ssm_len, np.float32))

    def kv_sections(self):
        """(array name, elements per row) in the blob's section order."""
        d, h = self.kv_dim, max(self.n_kv_heads, 1)
        if self.kv_format == Q8:
            spr = max(d // Q8_BLOCK, 1) if self.q8_block_scales else 1
            return [("key_q8", d), ("value_q8", d), ("key_scale", spr), ("value_scale", spr)]
        return [("key_base", d // 4), ("value_base", d // 4), ("key_sign", d // 8),
                ("value_sign", d // 8), ("key_scale", h), ("value_scale", h),
                ("key_rnorm", h), ("value_rnorm", h)]


def snapshot(st: HostState, tokens, model_len: int, model_head_fnv: int) -> bytes:
    k = len(tokens)
    if st.kv_dim % 8:
        raise GpfcError("prefill cache requires kv_dim % 8 == 0")
    w = Writer()
    w.b += MAGIC
    w.u16(VERSION)
    w.b.append(st.kv_format)
    w.b.append(1 if st.q8_block_scales else 0)
    w.u32(st.n_layers)
    w.u32(st.kv_dim)
    w.u32(max(st.n_kv_heads, 1))
    w.u32(k)
    w.u32(st.seq_len)
    w.u64(model_len)
    w.u64(model_head_fnv)
    for t in tokens:
        w.b += int(t).to_bytes(4, "little", signed=True)
    for name, per_row in st.kv_sections():
        arr = gather_rows(st.a[name], per_row, st.seq_len, st.n_layers, k)
        w.section(arr.astype(arr.dtype.newbyteorder("<")).tobytes())
    w.section(st.a["ssm_conv"].astype("<f4").tobytes())
    w.section(st.a["ssm_state"].astype("<f4").tobytes())
    return bytes(w.b)


@dataclass
class PrefixCache:
    tokens: list
    kv_format: int
    q8_block_scales: bool
    n_layers: int
    kv_dim: int
    n_kv_heads: int
    model_len: int
    model_head_fnv: int
    sections: list

    @staticmethod
    def parse(blob: bytes) -> "PrefixCache":
        r = Reader(blob)
        if r.take(4) != MAGIC:
            raise GpfcError("prefill cache: bad magic")
        version = r.u16()
        if version != VERSION:
            raise GpfcError(f"prefill cache: unsupported version {version}")
        fmt = r.take(1)[0]
        if fmt not in (Q8, TURBO):
            raise GpfcError(f"prefill cache: bad kv format {fmt}")
        q8_block = r.take(1)[0] != 0
        n_layers, kv_dim, n_kv, k, _ = (r.u32() for _ in range(5))
        model_len, fnv = r.u64(), r.u64()
        tokens = [int.from_bytes(r.take(4), "little", signed=True) for _ in range(k)]
        sections = [r.section() for _ in range((4 if fmt == Q8 else 8) + 2)]
        return PrefixCache(tokens, fmt, q8_block, n_layers, kv_dim, n_kv, model_len, fnv, sections)

    def match_len(self, prompt_tokens):
        k = len(self.tokens)
        if k == 0 or len(prompt_tokens) <= k:
            return None
        return k if list(prompt_tokens[:k]) == self.tokens else None

    def inject(self, st: HostState) -> None:
        k = len(self.tokens)
        if (self.n_layers != st.n_layers or self.kv_dim != st.kv_dim
                or self.n_kv_heads != max(st.n_kv_heads, 1) or self.kv_format != st.kv_format
                or self.q8_block_scales != st.q8_block_scales):
            raise GpfcError("prefill cache: model/config mismatch")
        if k > st.seq_len:
            raise GpfcError("prefill cache: prefix longer than context")
        specs = st.kv_sections()
        n_bytes = 2 if self.kv_format == Q8 else 4  # byte sections before the f32 ones
        for (name, per_row), sec in zip(specs[:n_bytes], self.sections[:n_bytes]):
            dt = st.a[name].dtype
            scatter_rows(st.a[name], np.frombuffer(sec, dt), per_row, st.seq_len, st.n_layers, k)
        vals = [_f32s(sec) for sec in self.sections[n_bytes:len(specs)]]
        for (name, per_row), v in zip(specs[n_bytes:], vals):
            scatter_rows(st.a[name], v, per_row, st.seq_len, st.n_layers, k)
        conv = _f32s(self.sections[len(specs)])
        ssm = _f32s(self.sections[len(specs) + 1])
        if len(conv) != len(st.a["ssm_conv"]) or len(ssm) != len(st.a["ssm_state"]):
            raise GpfcError("prefill cache: ssm state size mismatch")
        st.a["ssm_conv"][:] = conv
        st.a["ssm_state"][:] = ssm
