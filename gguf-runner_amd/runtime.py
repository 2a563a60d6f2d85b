"""Host-side mirror of the reference's attention interface over libgr_attn's
run-state C ABI.

`Config` carries the fields of Config (src/engine/types.rs:639-697) that the
attention path reads, `RunState` owns the host rows q / k / v / xb like the
reference's RunState (types.rs:745-809) plus the opaque device state (KV cache,
SSM state, stream), and the module functions keep the reference's names and
argument meaning:

    qkv_bias_and_norm(p, s, l)        inference.rs:2535  (QK-norm part)
    apply_rope_qk(p, s, l, pos)       inference.rs:1817
    kv_write_token(p, s, l, pos)      inference.rs:1877
    attention_token(p, s, l, pos)     inference.rs:1970
    qwen3next_state_step(...)         math.rs:890-934 over heads

Errors come back as ffi.GrError carrying the reference's message text.  All
arithmetic runs in the HIP kernels; nothing here computes attention.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import ffi


@dataclass
class Config:
    n_layers: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    seq_len: int
    n_seq: int = 1
    kv_dtype: int = ffi.DTYPE_F32      # raw F32/F16/BF16, or DTYPE_Q8 (KvCacheFormat::Q8)
    rope_mode: int = ffi.ROPE_NEOX
    rope_dim: int = 0
    rope_theta: float = 10_000.0
    rope_theta_swa: float = 0.0
    rope_scale_global: float = 1.0
    rope_scale_local: float = 1.0
    layer_windows: list | None = None   # per layer: 0 / None = global, W = sliding window
    swa_pattern: int = 0
    is_gemma3: bool = False
    online_attn_fusion: bool = False
    rms_norm_eps: float = 1e-6
    q_norm: np.ndarray | None = None    # [n_layers][head_dim]
    k_norm: np.ndarray | None = None
    qk_norm_present: list | None = None
    ssm_n_heads: int = 0
    ssm_head_dim: int = 128
    q8_block_scales: bool = False       # GGUF_Q8_BLOCK_SCALES (inference.rs:1883)
    # Qwen3.5 SSM layer (Qwen3NextLinearAttentionShape, math.rs:549-620)
    ssm_n_k_heads: int = 0              # ssm_group_count
    ssm_conv_kernel: int = 0
    ssm_conv1d: np.ndarray | None = None  # [n_layers][conv_dim][K]
    ssm_a: np.ndarray | None = None       # [n_layers][n_v]
    ssm_dt_bias: np.ndarray | None = None  # [n_layers][n_v]
    ssm_norm: np.ndarray | None = None    # [n_layers][ssm_head_dim]
    _keep: list = field(default_factory=list, repr=False)

    def to_c(self) -> ffi.AttnConfig:
        c = ffi.AttnConfig()
        for name in ("n_layers", "n_heads", "n_kv_heads", "head_dim", "seq_len", "n_seq",
                     "kv_dtype", "rope_mode", "rope_dim", "swa_pattern", "ssm_n_heads",
                     "ssm_head_dim", "ssm_n_k_heads", "ssm_conv_kernel"):
            setattr(c, name, int(getattr(self, name)))
        for name in ("rope_theta", "rope_theta_swa", "rope_scale_global", "rope_scale_local",
                     "rms_norm_eps"):
            setattr(c, name, float(getattr(self, name)))
        c.is_gemma3 = int(bool(self.is_gemma3))
        c.online_attn_fusion = int(bool(self.online_attn_fusion))
        c.q8_block_scales = int(bool(self.q8_block_scales))
        self._keep = []
        if self.layer_windows is not None:
            w = np.ascontiguousarray([0 if x is None else int(x) for x in self.layer_windows],
                                     dtype=np.int32)
            self._keep.append(w)
            c.layer_windows = w.ctypes.data
        for name in ("q_norm", "k_norm", "ssm_conv1d", "ssm_a", "ssm_dt_bias", "ssm_norm"):
            arr = getattr(self, name)
            if arr is not None:
                a = np.ascontiguousarray(arr, dtype=np.float32)
                self._keep.append(a)
                setattr(c, name, a.ctypes.data)
        if self.qk_norm_present is not None:
            a = np.ascontiguousarray(self.qk_norm_present, dtype=np.uint8)
            self._keep.append(a)
            c.qk_norm_present = a.ctypes.data
        return c

    @property
    def q_dim(self) -> int:
        return self.n_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.n_kv_heads * self.head_dim


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


class RunState:
    """malloc_run_state (inference.rs:1529-1748): host rows + device state."""

    def __init__(self, p: Config):
        self.q = np.zeros(p.q_dim, np.float32)
        self.k = np.zeros(p.kv_dim, np.float32)
        self.v = np.zeros(p.kv_dim, np.float32)
        self.xb = np.zeros(p.q_dim, np.float32)
        self._handle = ctypes.c_void_p()
        c = p.to_c()
        ffi.check(ffi.lib().gr_malloc_run_state(ctypes.byref(c), ctypes.byref(self._handle)))

    @property
    def handle(self):
        return self._handle

    def close(self) -> None:
        if self._handle:
            ffi.lib().gr_free_run_state(self._handle)
            self._handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def malloc_run_state(p: Config) -> RunState:
    return RunState(p)


def qkv_bias_and_norm(p: Config, s: RunState, l: int) -> None:
    ffi.check(ffi.lib().gr_qkv_norm(s.handle, l, _p(s.q), _p(s.k)))


def apply_rope_qk(p: Config, s: RunState, l: int, pos: int) -> None:
    ffi.check(ffi.lib().gr_apply_rope_qk(s.handle, l, pos, _p(s.q), _p(s.k)))


def kv_write_token(p: Config, s: RunState, l: int, pos: int, seq: int = 0) -> None:
    ffi.check(ffi.lib().gr_kv_write_token(s.handle, seq, l, pos, _p(s.k), _p(s.v)))


def attention_token(p: Config, s: RunState, l: int, pos: int, seq: int = 0) -> None:
    ffi.check(ffi.lib().gr_attention_token(s.handle, seq, l, pos, _p(s.q), _p(s.xb)))


def attention_layer_token(p: Config, s: RunState, l: int, pos: int, seq: int = 0) -> None:
    """qkv_bias_and_norm -> apply_rope_qk -> kv_write_token -> attention_token in one
    device pass (layer_attention_token_staged, inference.rs:3499-3507); reads the
    pre-norm s.q / s.k / s.v, writes s.xb."""
    ffi.check(ffi.lib().gr_attention_layer_token(s.handle, seq, l, pos, _p(s.q), _p(s.k),
                                                 _p(s.v), _p(s.xb)))


def _out_rows(out, m: int, width: int) -> np.ndarray:
    """The output rows: `out` when given (a reused [m][width] f32 buffer, like the
    reference's run-state xb), else a new zeroed array."""
    if out is None:
        return np.zeros((m, width), np.float32)
    if out.dtype != np.float32 or out.shape != (m, width) or not out.flags.c_contiguous:
        raise ValueError(f"out must be a C-contiguous float32 array of shape {(m, width)}")
    return out


def prefill_attention_chunk(p: Config, s: RunState, l: int, base_pos: int, q, k, v,
                            seq: int = 0, out=None) -> np.ndarray:
    """The attention loop of transformer_prefill_batch (inference.rs:2981-3017) for
    rows q [m][q_dim], k/v [m][kv_dim]; returns xb rows [m][q_dim]."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    m = q.shape[0]
    xb = _out_rows(out, m, p.q_dim)
    ffi.check(ffi.lib().gr_prefill_attention_chunk(s.handle, seq, l, base_pos, m, _p(q), _p(k),
                                                   _p(v), _p(xb)))
    return xb


def prefill_image_block(p: Config, s: RunState, l: int, base_pos: int, q, k, v,
                        seq: int = 0, out=None) -> np.ndarray:
    """The attention of transformer_prefill_image_block (media_prefill.rs:15-124) for
    one complete bidirectional image block at base_pos..base_pos+m-1; returns xb rows."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    m = q.shape[0]
    xb = _out_rows(out, m, p.q_dim)
    ffi.check(ffi.lib().gr_prefill_image_block(s.handle, seq, l, base_pos, m, _p(q), _p(k),
                                               _p(v), _p(xb)))
    return xb


def decode_layer_batch(p: Config, s: RunState, l: int, seqs, pos, q, k, v) -> np.ndarray:
    seqs = np.ascontiguousarray(seqs, np.int32)
    pos = np.ascontiguousarray(pos, np.int64)
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    n = seqs.size
    xb = np.zeros((n, p.q_dim), np.float32)
    ffi.check(ffi.lib().gr_decode_layer_batch(s.handle, l, n, _p(seqs), _p(pos), _p(q), _p(k),
                                              _p(v), _p(xb)))
    return xb


def read_kv_rows(p: Config, s: RunState, l: int, row0: int, n_rows: int, seq: int = 0):
    dt = {ffi.DTYPE_F32: np.float32, ffi.DTYPE_Q8: np.int8, ffi.DTYPE_TURBO: np.uint8}.get(p.kv_dtype,
                                                                                           np.uint16)
    width = p.kv_dim // 4 if p.kv_dtype == ffi.DTYPE_TURBO else p.kv_dim
    k = np.zeros((n_rows, width), dt)
    v = np.zeros((n_rows, width), dt)
    ffi.check(ffi.lib().gr_read_kv_rows(s.handle, l, seq, row0, n_rows, _p(k), _p(v)))
    return k, v


def read_kv_scales(p: Config, s: RunState, l: int, row0: int, n_rows: int, seq: int = 0):
    """key_cache_scale / value_cache_scale of a Q8 cache: [n_rows] (row mode) or
    [n_rows][kv_dim/32] (block mode); Turbo: sigma [n_rows][n_kv_heads]."""
    per = (p.n_kv_heads if p.kv_dtype == ffi.DTYPE_TURBO else
           (p.kv_dim // 32 if p.q8_block_scales else 1))
    ks = np.zeros((n_rows, per), np.float32)
    vs = np.zeros((n_rows, per), np.float32)
    ffi.check(ffi.lib().gr_read_kv_scales(s.handle, l, seq, row0, n_rows, _p(ks), _p(vs)))
    return ks, vs


def read_turbo_rows(p: Config, s: RunState, l: int, row0: int, n_rows: int, seq: int = 0):
    """Turbo cache rows: dict of k/v codes [n_rows][kv_dim/4], signs [n_rows][kv_dim/8],
    sigma and gamma [n_rows][n_kv_heads]."""
    out = {}
    for side in ("k", "v"):
        out[side + "_base"] = np.zeros((n_rows, p.kv_dim // 4), np.uint8)
        out[side + "_sign"] = np.zeros((n_rows, p.kv_dim // 8), np.uint8)
        out[side + "_rnorm"] = np.zeros((n_rows, p.n_kv_heads), np.float32)
    ffi.check(ffi.lib().gr_read_turbo_rows(s.handle, l, seq, row0, n_rows, _p(out["k_base"]),
                                           _p(out["k_sign"]), _p(out["k_rnorm"]), _p(out["v_base"]),
                                           _p(out["v_sign"]), _p(out["v_rnorm"])))
    ks = np.zeros((n_rows, p.n_kv_heads), np.float32)
    vs = np.zeros((n_rows, p.n_kv_heads), np.float32)
    ffi.check(ffi.lib().gr_read_kv_scales(s.handle, l, seq, row0, n_rows, _p(ks), _p(vs)))
    out["k_scale"], out["v_scale"] = ks, vs
    return out


def qwen3next_ssm_layer(p: Config, s: RunState, l: int, qkv, z, gate_a, gate_b=None) -> np.ndarray:
    """qwen3next_linear_attention_step_from_projections (math.rs:715-953) for T
    consecutive tokens: qkv [T][conv_dim], z [T][d_inner], gate_a the fused [T][2 n_v]
    (gate_b None) or alpha [T][n_v] with gate_b = beta [T][n_v].  Returns ssm_proj
    [T][d_inner]."""
    qkv = np.ascontiguousarray(qkv, np.float32)
    z = np.ascontiguousarray(z, np.float32)
    ga = np.ascontiguousarray(gate_a, np.float32)
    gb = np.ascontiguousarray(gate_b, np.float32) if gate_b is not None else None
    T = qkv.shape[0]
    out = np.zeros((T, p.ssm_n_heads * p.ssm_head_dim), np.float32)
    ffi.check(ffi.lib().gr_qwen3next_ssm_layer(s.handle, l, T, _p(qkv), _p(z), _p(ga),
                                               _p(gb) if gb is not None else None, _p(out)))
    return out


def read_ssm_conv_state(p: Config, s: RunState, l: int) -> np.ndarray:
    conv_dim = (p.ssm_n_heads + 2 * p.ssm_n_k_heads) * p.ssm_head_dim
    out = np.zeros((max(p.ssm_conv_kernel - 1, 0), conv_dim), np.float32)
    ffi.check(ffi.lib().gr_read_ssm_conv_state(s.handle, l, _p(out)))
    return out


def qwen3next_state_step(p: Config, s: RunState, l: int, q, k, v, g, beta) -> np.ndarray:
    """qwen3next_state_head_step for every value head (math.rs:890-934); q, k already
    normalised, g = exp(gate) per head, beta per head.  Returns ssm_proj [H*d]."""
    arrs = [np.ascontiguousarray(x, np.float32) for x in (q, k, v, g, beta)]
    out = np.zeros(p.ssm_n_heads * p.ssm_head_dim, np.float32)
    ffi.check(ffi.lib().gr_qwen3next_state_step(s.handle, l, *[_p(a) for a in arrs], _p(out)))
    return out


def qwen3next_prefill(p: Config, s: RunState, l: int, q, k, v, gate, beta) -> np.ndarray:
    arrs = [np.ascontiguousarray(x, np.float32) for x in (q, k, v, gate, beta)]
    T = arrs[0].shape[0]
    out = np.zeros((T, p.ssm_n_heads * p.ssm_head_dim), np.float32)
    ffi.check(ffi.lib().gr_qwen3next_prefill(s.handle, l, T, *[_p(a) for a in arrs], _p(out)))
    return out


def read_ssm_state(p: Config, s: RunState, l: int) -> np.ndarray:
    out = np.zeros((p.ssm_n_heads, p.ssm_head_dim, p.ssm_head_dim), np.float32)
    ffi.check(ffi.lib().gr_read_ssm_state(s.handle, l, _p(out)))
    return out


def write_ssm_state(p: Config, s: RunState, l: int, state) -> None:
    st = np.ascontiguousarray(state, np.float32)
    ffi.check(ffi.lib().gr_write_ssm_state(s.handle, l, _p(st)))


def write_ssm_conv_state(p: Config, s: RunState, l: int, hist) -> None:
    h = np.ascontiguousarray(hist, np.float32)
    ffi.check(ffi.lib().gr_write_ssm_conv_state(s.handle, l, _p(h)))


def snapshot(p: Config, s: RunState, tokens, model_len: int, model_head_fnv: int,
             seq: int = 0) -> bytes:
    """snapshot (src/app/prefill_cache.rs:178-310): the GPFC v1 blob of the first
    len(tokens) cache rows of every layer plus the SSM arrays, read from the device."""
    tok = np.ascontiguousarray(tokens, np.int32)
    L = ffi.lib()
    size = ctypes.c_uint64()
    tp = _p(tok) if tok.size else None
    ffi.check(L.gr_prefill_cache_snapshot(s.handle, seq, tp, tok.size, model_len, model_head_fnv,
                                          None, 0, ctypes.byref(size)))
    buf = np.zeros(size.value, np.uint8)
    ffi.check(L.gr_prefill_cache_snapshot(s.handle, seq, tp, tok.size, model_len, model_head_fnv,
                                          _p(buf), buf.size, ctypes.byref(size)))
    return buf.tobytes()


def inject(p: Config, s: RunState, blob: bytes, seq: int = 0) -> int:
    """PrefixCache::parse + inject (prefill_cache.rs:316-352, 380-507) into the
    device state; returns the number of cached prompt tokens."""
    b = np.frombuffer(blob, np.uint8)
    k = ctypes.c_int32()
    ffi.check(ffi.lib().gr_prefill_cache_inject(s.handle, seq, b.ctypes.data if b.size else None,
                                                b.size, ctypes.byref(k)))
    return k.value
