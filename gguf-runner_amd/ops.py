"""Device-pointer entry points of libgr_attn for torch tensors resident in HBM.

torch is used only for device memory and the stream handle; every computation
is a HIP kernel of libgr_attn.so reached through the C ABI (see ffi.py).
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import ffi

_DT = {torch.float32: ffi.DTYPE_F32, torch.float16: ffi.DTYPE_F16, torch.bfloat16: ffi.DTYPE_BF16,
       torch.int8: ffi.DTYPE_Q8}


def _ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("libgr_attn device entry points take device tensors")
    return t.data_ptr()


def _stream(stream=None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 256) + 256, dtype=torch.uint8, device=device)


def _aligned(ws: torch.Tensor) -> int:
    p = ws.data_ptr()
    return (p + 255) // 256 * 256


def _set_gate(a, gate, row_stride, head_stride) -> None:
    """The optional Qwen3.5 output gate (an f32 device tensor, or None): element
    (row r, head h, i) at r * row_stride + h * head_stride + i of gate's storage."""
    if gate is None:
        return
    assert gate.dtype == torch.float32 and gate.is_cuda
    a.out_gate = _ptr(gate)
    a.out_gate_row_stride = int(row_stride)
    a.out_gate_head_stride = int(head_stride)


class DecodeCall:
    """A prepared gr_decode_attention call (args + workspace), reusable for timing.

    q [n_seq][Hq][d] f32; k_cache/v_cache [n_seq][seq_len][Hkv][d] (f32/f16/bf16, or
    int8 Q8 codes with f32 k_scale/v_scale [n_seq][seq_len] (one per row) or
    [n_seq][seq_len][Hkv*d/32] (q8_block: one per 32 elements));
    kv_start/kv_end int32 [n_seq]; out [n_seq][Hq][d] f32.
    """

    def __init__(self, q, k_cache, v_cache, kv_start, kv_end, out, *, max_kv_len,
                 score_scale=None, split_keys=0, k_scale=None, v_scale=None, q8_block=False,
                 out_gate=None, out_gate_row_stride=0, out_gate_head_stride=0):
        n_seq, n_heads, d = q.shape
        _, seq_len, n_kv, d2 = k_cache.shape
        assert d2 == d and v_cache.shape == k_cache.shape and out.shape == q.shape
        assert q.dtype == torch.float32 and out.dtype == torch.float32
        assert kv_start.dtype == torch.int32 and kv_end.dtype == torch.int32
        assert k_cache.is_contiguous() and v_cache.is_contiguous() and q.is_contiguous()
        self._keep = (q, k_cache, v_cache, kv_start, kv_end, out, k_scale, v_scale)
        a = ffi.DecodeArgs()
        a.n_seq, a.n_heads, a.n_kv_heads, a.head_dim = n_seq, n_heads, n_kv, d
        a.kv_dtype = _DT[k_cache.dtype]
        a.split_keys = split_keys
        a.max_kv_len = int(max_kv_len)
        a.score_scale = 1.0 / math.sqrt(d) if score_scale is None else float(score_scale)
        a.q, a.k_cache, a.v_cache = _ptr(q), _ptr(k_cache), _ptr(v_cache)
        a.seq_stride = seq_len * n_kv * d
        a.row_stride = n_kv * d
        a.kv_start, a.kv_end, a.out = _ptr(kv_start), _ptr(kv_end), _ptr(out)
        if k_cache.dtype == torch.int8:
            per_row = n_kv * d // 32 if q8_block else 1
            for t in (k_scale, v_scale):
                assert t is not None and t.dtype == torch.float32 and t.is_contiguous()
                assert t.numel() == n_seq * seq_len * per_row
            a.k_scale, a.v_scale = _ptr(k_scale), _ptr(v_scale)
            a.scale_seq_stride = seq_len * per_row
            a.scale_row_stride = per_row
            a.q8_block = int(bool(q8_block))
        _set_gate(a, out_gate, out_gate_row_stride, out_gate_head_stride)
        self._keep = self._keep + (out_gate,)
        L = ffi.lib()
        nbytes = L.gr_decode_workspace_size(ctypes.byref(a))
        self.ws = _workspace(nbytes, q.device)
        a.workspace = _aligned(self.ws)
        self.args = a

    def __call__(self, stream=None) -> None:
        ffi.check(ffi.lib().gr_decode_attention(ctypes.byref(self.args), _stream(stream)))


def turbo_sign_table(n_layers: int, n_kv_heads: int, head_size: int):
    """gr_turbo_sign_table: host uint8 [4][n_layers][n_kv_heads][ceil(head_size/8)]."""
    import numpy as np
    t = np.zeros((4, n_layers, n_kv_heads, (head_size + 7) // 8), np.uint8)
    ffi.check(ffi.lib().gr_turbo_sign_table(n_layers, n_kv_heads, head_size, t.ctypes.data))
    return t


class TurboDecodeCall:
    """gr_decode_attention over a Turbo cache (device tensors):
    codes k_base/v_base uint8 [n_seq][seq_len][Hkv*d/4], signs k_sign/v_sign uint8
    [n_seq][seq_len][Hkv*d/8], sigma k_scale/v_scale and gamma k_rnorm/v_rnorm f32
    [n_seq][seq_len][Hkv], signs_dev uint8 [4][n_layers][Hkv][d/8] (the whole table)
    and the layer index; q / out as DecodeCall."""

    def __init__(self, q, k_base, v_base, k_sign, v_sign, k_scale, v_scale, k_rnorm, v_rnorm,
                 signs_dev, layer, kv_start, kv_end, out, *, max_kv_len, score_scale=None,
                 split_keys=0):
        n_seq, n_heads, d = q.shape
        _, seq_len, nb = k_base.shape
        n_kv = nb * 4 // d
        _, n_layers, n_kv2, sb = signs_dev.shape
        assert n_kv2 == n_kv and sb == d // 8 and k_sign.shape == (n_seq, seq_len, n_kv * d // 8)
        for t in (k_scale, v_scale, k_rnorm, v_rnorm):
            assert t.shape == (n_seq, seq_len, n_kv) and t.dtype == torch.float32 and t.is_contiguous()
        self._keep = (q, k_base, v_base, k_sign, v_sign, k_scale, v_scale, k_rnorm, v_rnorm, signs_dev,
                      kv_start, kv_end, out)
        a = ffi.DecodeArgs()
        a.n_seq, a.n_heads, a.n_kv_heads, a.head_dim = n_seq, n_heads, n_kv, d
        a.kv_dtype = ffi.DTYPE_TURBO
        a.split_keys = split_keys
        a.max_kv_len = int(max_kv_len)
        a.score_scale = 1.0 / math.sqrt(d) if score_scale is None else float(score_scale)
        a.q, a.k_cache, a.v_cache = _ptr(q), _ptr(k_base), _ptr(v_base)
        a.seq_stride = seq_len * n_kv * d
        a.row_stride = n_kv * d
        a.kv_start, a.kv_end, a.out = _ptr(kv_start), _ptr(kv_end), _ptr(out)
        a.k_scale, a.v_scale, a.k_rnorm, a.v_rnorm = _ptr(k_scale), _ptr(v_scale), _ptr(k_rnorm), _ptr(v_rnorm)
        a.k_sign, a.v_sign = _ptr(k_sign), _ptr(v_sign)
        a.scale_seq_stride = seq_len * n_kv
        a.scale_row_stride = n_kv
        a.turbo_signs = signs_dev.data_ptr() + layer * n_kv * sb
        a.turbo_slot_stride = n_layers * n_kv * sb
        L = ffi.lib()
        self.ws = _workspace(L.gr_decode_workspace_size(ctypes.byref(a)), q.device)
        a.workspace = _aligned(self.ws)
        self.args = a

    def __call__(self, stream=None) -> None:
        ffi.check(ffi.lib().gr_decode_attention(ctypes.byref(self.args), _stream(stream)))


def decode_attention(q, k_cache, v_cache, kv_start, kv_end, *, max_kv_len=None, score_scale=None,
                     split_keys=0, out=None, k_scale=None, v_scale=None, q8_block=False):
    if out is None:
        out = torch.empty_like(q)
    if max_kv_len is None:
        max_kv_len = int((kv_end - kv_start).max().item())
    DecodeCall(q, k_cache, v_cache, kv_start, kv_end, out, max_kv_len=max_kv_len,
               score_scale=score_scale, split_keys=split_keys, k_scale=k_scale, v_scale=v_scale,
               q8_block=q8_block)()
    return out


def rope_freqs(theta: float, rope_dim: int) -> list[float]:
    """Host-computed RoPE frequency table (gr_rope_freqs, inference.rs:1590-1609)."""
    buf = (ctypes.c_float * (rope_dim // 2))()
    ffi.check(ffi.lib().gr_rope_freqs(float(theta), int(rope_dim), ctypes.cast(buf, ctypes.c_void_p)))
    return list(buf)


class PrefillCall:
    """A prepared gr_prefill_attention call.

    q [m][Hq][d], k/v [m][Hkv][d] (f16 or bf16, pre-norm, pre-RoPE);
    k_cache/v_cache [rows][Hkv][d] of the same dtype (rows >= base_pos + m);
    out [m][Hq][d] f32.  rope_freqs is a device f32 tensor [rope_dim/2].
    """

    def __init__(self, q, k, v, k_cache, v_cache, out, *, base_pos=0, window=0,
                 rope_mode=ffi.ROPE_NONE, rope_dim=0, rope_scale=1.0, rope_freqs=None,
                 q_norm=None, k_norm=None, norm_eps=1e-6, is_gemma3=False, bidirectional=False,
                 out_gate=None, out_gate_row_stride=0, out_gate_head_stride=0, q_bias=None, k_bias=None,
                 v_bias=None):
        m, n_heads, d = q.shape
        _, n_kv, d2 = k.shape
        assert d2 == d and v.shape == k.shape and out.shape == (m, n_heads, d)
        assert q.dtype == k.dtype == v.dtype == k_cache.dtype == v_cache.dtype
        assert out.dtype == torch.float32
        for t in (q, k, v, k_cache, v_cache, out):
            assert t.is_contiguous()
        self._keep = (q, k, v, k_cache, v_cache, out, rope_freqs, q_norm, k_norm, out_gate, q_bias, k_bias, v_bias)
        a = ffi.PrefillArgs()
        a.n_tokens, a.base_pos, a.n_heads, a.n_kv_heads, a.head_dim = m, base_pos, n_heads, n_kv, d
        a.dtype = _DT[q.dtype]
        a.window = int(window)
        a.rope_mode, a.rope_dim, a.rope_scale = int(rope_mode), int(rope_dim), float(rope_scale)
        a.rope_freqs = _ptr(rope_freqs)
        a.q_norm, a.k_norm = _ptr(q_norm), _ptr(k_norm)
        a.q_bias, a.k_bias, a.v_bias = _ptr(q_bias), _ptr(k_bias), _ptr(v_bias)
        a.norm_eps = float(norm_eps)
        a.is_gemma3 = int(bool(is_gemma3))
        a.bidirectional = int(bool(bidirectional))
        a.q, a.k, a.v = _ptr(q), _ptr(k), _ptr(v)
        a.k_cache, a.v_cache = _ptr(k_cache), _ptr(v_cache)
        a.cache_row_stride = n_kv * d
        a.out = _ptr(out)
        _set_gate(a, out_gate, out_gate_row_stride, out_gate_head_stride)
        nbytes = ffi.lib().gr_prefill_workspace_size(ctypes.byref(a))
        self.ws = _workspace(nbytes, q.device)
        a.workspace = _aligned(self.ws)
        self.args = a

    def __call__(self, stream=None) -> None:
        ffi.check(ffi.lib().gr_prefill_attention(ctypes.byref(self.args), _stream(stream)))


def prefill_attention(q, k, v, k_cache, v_cache, **kw):
    out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    PrefillCall(q, k, v, k_cache, v_cache, out, **kw)()
    return out


def encoder_self_attention(q, k, v, *, n_seq, tokens, heads, head_dim, out=None, stream=None):
    """gr_encoder_self_attention (encoder_self_attention, multimodal/mod.rs:145-256):
    f32 device rows [n_seq*tokens][heads*head_dim]; returns out of the same shape."""
    for t in (q, k, v):
        assert t.dtype == torch.float32 and t.is_contiguous()
    if out is None:
        out = torch.empty_like(q)
    ffi.check(ffi.lib().gr_encoder_self_attention(_ptr(out), _ptr(q), _ptr(k), _ptr(v), int(n_seq),
                                                  int(tokens), int(heads), int(head_dim),
                                                  _stream(stream)))
    return out


class DeltaNetCall:
    """A prepared gr_deltanet_attention call.

    q/k/v [T][H][d] (f32/f16/bf16); gate/beta [T][H] f32; state [H][d][d] f32
    (updated in place); out [T][H][d] f32.
    """

    def __init__(self, q, k, v, gate, beta, state, out, *, l2norm=True, eps=1e-6,
                 algo=ffi.DELTANET_AUTO):
        T, H, d = q.shape
        assert k.shape == v.shape == q.shape and q.dtype == k.dtype == v.dtype
        assert gate.shape == beta.shape == (T, H) and gate.dtype == beta.dtype == torch.float32
        assert state.shape == (H, d, d) and state.dtype == torch.float32
        assert out.shape == (T, H, d) and out.dtype == torch.float32
        for t in (q, k, v, gate, beta, state, out):
            assert t.is_contiguous()
        self._keep = (q, k, v, gate, beta, state, out)
        a = ffi.DeltaNetArgs()
        a.n_tokens, a.n_heads, a.head_dim = T, H, d
        a.in_dtype = _DT[q.dtype]
        a.l2norm = int(bool(l2norm))
        a.algo = int(algo)
        a.eps = float(eps)
        a.q, a.k, a.v = _ptr(q), _ptr(k), _ptr(v)
        a.gate, a.beta, a.state, a.out = _ptr(gate), _ptr(beta), _ptr(state), _ptr(out)
        nbytes = ffi.lib().gr_deltanet_workspace_size(ctypes.byref(a))
        self.ws = _workspace(nbytes, q.device) if nbytes else None
        a.workspace = _aligned(self.ws) if nbytes else None
        self.args = a

    def __call__(self, stream=None) -> None:
        ffi.check(ffi.lib().gr_deltanet_attention(ctypes.byref(self.args), _stream(stream)))
