"""ctypes wrapper of the CPU oracle (oracle.c) -- TEST INFRASTRUCTURE ONLY.

Importable only from tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg.  It is the checker, never the thing measured as the product
and never a fallback for the HIP path.
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"

F32, F16, BF16, Q8, Q8B = 0, 1, 2, 3, 4
Q8_BLOCK = 32

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        _declare(_lib)
    return _lib


_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t
_f = ctypes.c_float


def _declare(L: ctypes.CDLL) -> None:
    L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.orc_f16_to_f32.restype = _f
    L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
    L.orc_bf16_to_f32.restype = _f
    L.orc_f32_to_f16.argtypes = [_f]
    L.orc_f32_to_f16.restype = ctypes.c_uint16
    L.orc_f32_to_bf16.argtypes = [_f]
    L.orc_f32_to_bf16.restype = ctypes.c_uint16
    for name in ("orc_f32_to_f16_n", "orc_f32_to_bf16_n", "orc_f16_to_f32_n", "orc_bf16_to_f32_n"):
        getattr(L, name).argtypes = [_p, _p, _sz]
    L.orc_rope_freqs.argtypes = [_f, _i, _p]
    L.orc_rope_cache.argtypes = [_p, _i, _i64, _f, _p, _p]
    L.orc_apply_rope_qk.argtypes = [_p, _p, _i, _i, _i, _i, _p, _p, _i, _i, _f]
    L.orc_rmsnorm_per_head.argtypes = [_p, _p, _i, _i, _f]
    L.orc_quantize_row_q8.argtypes = [_p, _i, _p, _p]
    L.orc_kv_quantize_row.argtypes = [_p, _i, _i, _p, _p]
    L.orc_softmax.argtypes = [_p, _i]
    L.orc_attention_token.argtypes = [_p, _p, _p, _sz, _i, _i, _i, _p, _p, _i, _p, _p, _sz, _sz,
                                      _sz, _f, _i, _i, _i]
    L.orc_visible_keys.argtypes = [_i64, _i64, ctypes.POINTER(_i64), ctypes.POINTER(_i64)]
    L.orc_prefill_layer.argtypes = [_p, _p, _p, _p, _i, _i64, _i, _i, _i, _p, _p, _i, _i, _i, _p,
                                    _f, _i, _i, _i64, _p, _p, _f, _p, _p, _i, _p, _i]
    L.orc_deltanet_head_step.argtypes = [_p, _p, _p, _p, _p, _f, _f, _i]
    L.orc_deltanet_l2norm.argtypes = [_p, _p, _i, _f]
    L.orc_deltanet_scan.argtypes = [_p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _f, _i]
    L.orc_max_threads.restype = _i
    L.orc_encoder_self_attention.argtypes = [_p, _p, _p, _p, _i, _i, _i, _i, _i]
    L.orc_sigmoid_mul.argtypes = [_p, _p, _i]
    L.orc_qwen3next_ssm_token.argtypes = [_p, _p, _p, _p, _i, _i, _i, _i, _p, _p, _p, _p, _f, _p, _p, _p]
    L.orc_splitmix64.argtypes = [ctypes.c_uint64]
    L.orc_splitmix64.restype = ctypes.c_uint64
    L.orc_turbo_sign_table.argtypes = [_i, _i, _i, _p]
    L.orc_turbo_transform.argtypes = [_p, _i, _p, _p]
    L.orc_turbo_quantize_head.argtypes = [_p, _i, _p, _i, _i, _i, _i, _p, _p, _sz, _p, _p]
    L.orc_kv_write_turbo.argtypes = [_p, _p, _i, _i, _p, _i, _i, _sz, _p, _p, _p, _p, _p, _p, _p, _p]
    L.orc_attention_token_turbo.argtypes = [_p, _p, _p, _sz, _i, _i, _i, _p, _p, _p, _p, _p, _p, _p,
                                            _p, _p, _i, _i, _sz, _sz, _sz, _f, _i, _i, _i]


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def max_threads() -> int:
    return int(lib().orc_max_threads())


def rope_freqs(theta: float, rope_dim: int) -> np.ndarray:
    out = np.zeros(rope_dim // 2, np.float32)
    lib().orc_rope_freqs(theta, rope_dim, _ptr(out))
    return out


def rope_cache(freqs: np.ndarray, pos: int, scale: float):
    freqs = _f32(freqs)
    c = np.zeros_like(freqs)
    s = np.zeros_like(freqs)
    lib().orc_rope_cache(_ptr(freqs), freqs.size, pos, scale, _ptr(c), _ptr(s))
    return c, s


def apply_rope_qk(q, k, n_heads, n_kv_heads, head_size, cos_t, sin_t, neox, gemma_q_scale=False,
                  attn_scale=None):
    """In-place on copies; returns (q, k)."""
    q = _f32(q).copy()
    k = _f32(k).copy()
    cos_t = _f32(cos_t)
    sin_t = _f32(sin_t)
    if attn_scale is None:
        attn_scale = float(np.float32(1.0) / np.sqrt(np.float32(head_size)))
    lib().orc_apply_rope_qk(_ptr(q), _ptr(k), n_heads, n_kv_heads, head_size, cos_t.size,
                            _ptr(cos_t), _ptr(sin_t), int(neox), int(gemma_q_scale), attn_scale)
    return q, k


def rmsnorm_per_head(x, w, n_heads, head_size, eps):
    x = _f32(x).copy()
    w = _f32(w)
    lib().orc_rmsnorm_per_head(_ptr(x), _ptr(w), n_heads, head_size, eps)
    return x


def quantize_row_q8(src):
    src = _f32(src)
    dst = np.zeros(src.size, np.int8)
    scale = np.zeros(1, np.float32)
    lib().orc_quantize_row_q8(_ptr(src), src.size, _ptr(dst), _ptr(scale))
    return dst, float(scale[0])


def kv_quantize_row(src, block: bool):
    """kv_write_token's Q8 branch for one kv_dim row: (int8 row, scales) with one
    scale (row mode) or kv_dim/32 scales (block mode)."""
    src = _f32(src)
    dst = np.zeros(src.size, np.int8)
    scales = np.zeros(src.size // Q8_BLOCK if block else 1, np.float32)
    lib().orc_kv_quantize_row(_ptr(src), src.size, int(block), _ptr(dst), _ptr(scales))
    return dst, scales


def softmax(x):
    x = _f32(x).copy()
    lib().orc_softmax(_ptr(x), x.size)
    return x


def visible_keys(window: int, query: int):
    s = _i64()
    e = _i64()
    lib().orc_visible_keys(window, query, ctypes.byref(s), ctypes.byref(e))
    return s.value, e.value


def attention_token(q, key_cache, value_cache, fmt, n_heads, n_kv_heads, head_size, vis_start,
                    vis_end, *, layer_row_base=0, key_scale=None, value_scale=None,
                    attn_scale=None, apply_attn_scale=True, online=False, n_threads=1):
    """attention_token for one query position; caches are flat row-major
    [rows][n_kv_heads*head_size] arrays of f32 / uint16 (f16|bf16 bits) / int8."""
    q = _f32(q)
    xb = np.zeros(n_heads * head_size, np.float32)
    att_stride = max(vis_end - vis_start, 1)
    att = np.zeros(n_heads * att_stride, np.float32)
    if attn_scale is None:
        attn_scale = float(np.float32(1.0) / np.sqrt(np.float32(head_size)))
    key_cache = np.ascontiguousarray(key_cache)
    value_cache = np.ascontiguousarray(value_cache)
    ks = _f32(key_scale) if key_scale is not None else None
    vs = _f32(value_scale) if value_scale is not None else None
    lib().orc_attention_token(_ptr(q), _ptr(xb), _ptr(att), att_stride, n_heads, n_kv_heads,
                              head_size, _ptr(key_cache), _ptr(value_cache), fmt, _ptr(ks),
                              _ptr(vs), layer_row_base, vis_start, vis_end, attn_scale,
                              int(apply_attn_scale), int(online), n_threads)
    return xb


def prefill_layer(q, k, v, *, n_heads, n_kv_heads, head_size, seq_len, fmt, rope_dim, neox,
                  rope_freqs_tab, rope_scale, is_gemma3=False, online=False, window=0,
                  q_norm=None, k_norm=None, eps=1e-6, base_pos=0, key_cache=None,
                  value_cache=None, n_threads=1, attend_rows=None, image_block=False):
    """Token-serial prefill of one layer (inference.rs:2981-3017), raw or Q8 KV.
    q [m][n_heads*d], k/v [m][n_kv_heads*d] f32.  Returns (xb [m][q_dim], kcache, vcache);
    for fmt Q8 / Q8B the caches are (int8 rows, scales) pairs.  attend_rows (indices into
    the m rows) limits the attention to those rows; every row is still normed, rotated and
    written to the cache in order, and the other xb rows stay 0.  image_block: the m rows
    are one bidirectional image block (transformer_prefill_image_block, media_prefill.rs:
    84-121): all rows are staged first, then row pos attends to [min(start, base_pos),
    base_pos + m) (attention.rs:87-94)."""
    q = _f32(q)
    k = _f32(k)
    v = _f32(v)
    m = q.shape[0]
    kv_dim = n_kv_heads * head_size
    q8 = fmt in (Q8, Q8B)
    cdt = np.float32 if fmt == F32 else (np.int8 if q8 else np.uint16)
    ks = vs = None
    if q8 and key_cache is not None:
        key_cache, ks = key_cache
        value_cache, vs = value_cache
    if key_cache is None:
        key_cache = np.zeros((seq_len, kv_dim), cdt)
        value_cache = np.zeros((seq_len, kv_dim), cdt)
    if q8 and ks is None:
        nsc = seq_len * (kv_dim // Q8_BLOCK if fmt == Q8B else 1)
        ks = np.zeros(nsc, np.float32)
        vs = np.zeros(nsc, np.float32)
    xb = np.zeros((m, n_heads * head_size), np.float32)
    freqs = _f32(rope_freqs_tab) if rope_freqs_tab is not None else None
    qn = _f32(q_norm) if q_norm is not None else None
    kn = _f32(k_norm) if k_norm is not None else None
    att = None
    if attend_rows is not None:
        att = np.zeros(m, np.uint8)
        att[np.asarray(attend_rows, dtype=np.int64)] = 1
    lib().orc_prefill_layer(_ptr(q), _ptr(k), _ptr(v), _ptr(xb), m, base_pos, n_heads, n_kv_heads,
                            head_size, _ptr(key_cache), _ptr(value_cache), fmt, rope_dim,
                            int(neox), _ptr(freqs), rope_scale, int(is_gemma3), int(online),
                            window, _ptr(qn), _ptr(kn), eps, _ptr(ks), _ptr(vs), n_threads,
                            _ptr(att), int(bool(image_block)))
    if q8:
        return xb, (key_cache, ks), (value_cache, vs)
    return xb, key_cache, value_cache


def deltanet_head_step(state, q, k, v, g, beta):
    state = _f32(state).copy()
    d = q.size
    out = np.zeros(d, np.float32)
    lib().orc_deltanet_head_step(_ptr(state), _ptr(out), _ptr(_f32(q)), _ptr(_f32(k)),
                                 _ptr(_f32(v)), g, beta, d)
    return state, out


def deltanet_scan(q, k, v, gate, beta, state, *, l2norm=True, eps=1e-6, n_threads=1):
    """q,k,v [T][H][d]; gate, beta [T][H]; state [H][d][d].  Returns (out, state)."""
    q = _f32(q)
    k = _f32(k)
    v = _f32(v)
    gate = _f32(gate)
    beta = _f32(beta)
    state = _f32(state).copy()
    T, H, d = q.shape
    out = np.zeros((T, H, d), np.float32)
    lib().orc_deltanet_scan(_ptr(q), _ptr(k), _ptr(v), _ptr(gate), _ptr(beta), _ptr(state),
                            _ptr(out), T, H, d, int(l2norm), eps, n_threads)
    return out, state


# ---- Turbo KV codec ----------------------------------------------------------

TQ_ROT_PRE, TQ_ROT_POST, TQ_RES_PRE, TQ_RES_POST = 0, 1, 2, 3


def encoder_self_attention(q, k, v, *, n_seq, tokens, heads, head_dim, n_threads=1):
    """encoder_self_attention (multimodal/mod.rs:145-256): rows [n_seq*tokens][heads*head_dim]
    f32; every token attends to all tokens of its own sequence."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.zeros((n_seq * tokens, heads * head_dim), np.float32)
    lib().orc_encoder_self_attention(_ptr(out), _ptr(q), _ptr(k), _ptr(v), n_seq, tokens, heads,
                                     head_dim, n_threads)
    return out


def splitmix64(x: int) -> int:
    return int(lib().orc_splitmix64(x & 0xFFFFFFFFFFFFFFFF))


def turbo_sign_table(n_layers, n_kv_heads, head_size) -> np.ndarray:
    """[4 slots][n_layers][n_kv_heads][ceil(head_size/8)] sign bits (bit set = negate)."""
    nb = (head_size + 7) // 8
    t = np.zeros((4, n_layers, n_kv_heads, nb), np.uint8)
    lib().orc_turbo_sign_table(n_layers, n_kv_heads, head_size, _ptr(t))
    return t


def turbo_transform(v, first_bits, second_bits) -> np.ndarray:
    v = _f32(v).copy()
    a = np.ascontiguousarray(first_bits, np.uint8)
    b = np.ascontiguousarray(second_bits, np.uint8)
    lib().orc_turbo_transform(_ptr(v), v.size, _ptr(a), _ptr(b))
    return v


def turbo_quantize_head(src, table, layer, kv_head):
    """quantize_turboquant_head for one head: (base bytes [n/4], sign bytes [n/8], sigma, gamma)."""
    src = _f32(src)
    n = src.size
    _, n_layers, n_kv, _ = table.shape
    base = np.zeros((n + 3) // 4, np.uint8)
    sign = np.zeros((n + 7) // 8, np.uint8)
    sc = np.zeros(1, np.float32)
    gm = np.zeros(1, np.float32)
    lib().orc_turbo_quantize_head(_ptr(src), n, _ptr(np.ascontiguousarray(table)), layer, kv_head,
                                  n_layers, n_kv, _ptr(base), _ptr(sign), 0, _ptr(sc), _ptr(gm))
    return base, sign, float(sc[0]), float(gm[0])


class TurboCache:
    """Host Turbo KV storage of `rows` rows (RunState's key/value_cache_turbo_base,
    _sign, key/value_cache_scale and _residual_norm)."""

    def __init__(self, rows, n_kv_heads, head_size):
        kv_dim = n_kv_heads * head_size
        self.n_kv_heads, self.head_size = n_kv_heads, head_size
        self.kbase = np.zeros(rows * kv_dim // 4, np.uint8)
        self.vbase = np.zeros(rows * kv_dim // 4, np.uint8)
        self.ksign = np.zeros(rows * kv_dim // 8, np.uint8)
        self.vsign = np.zeros(rows * kv_dim // 8, np.uint8)
        self.kscale = np.zeros(rows * n_kv_heads, np.float32)
        self.vscale = np.zeros(rows * n_kv_heads, np.float32)
        self.kres = np.zeros(rows * n_kv_heads, np.float32)
        self.vres = np.zeros(rows * n_kv_heads, np.float32)


def kv_write_turbo(cache: TurboCache, row, k, v, table, layer):
    k = _f32(k)
    v = _f32(v)
    n_layers = table.shape[1]
    lib().orc_kv_write_turbo(_ptr(k), _ptr(v), cache.n_kv_heads, cache.head_size,
                             _ptr(np.ascontiguousarray(table)), layer, n_layers, row,
                             _ptr(cache.kbase), _ptr(cache.ksign), _ptr(cache.kscale),
                             _ptr(cache.kres), _ptr(cache.vbase), _ptr(cache.vsign),
                             _ptr(cache.vscale), _ptr(cache.vres))


def attention_token_turbo(q, cache: TurboCache, table, layer, n_heads, vis_start, vis_end, *,
                          layer_row_base=0, attn_scale=None, apply_attn_scale=True, online=False,
                          n_threads=1):
    q = _f32(q)
    d = cache.head_size
    xb = np.zeros(n_heads * d, np.float32)
    att_stride = max(vis_end - vis_start, 1)
    att = np.zeros(n_heads * att_stride, np.float32)
    if attn_scale is None:
        attn_scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    n_layers = table.shape[1]
    c = cache
    lib().orc_attention_token_turbo(_ptr(q), _ptr(xb), _ptr(att), att_stride, n_heads, c.n_kv_heads, d,
                                    _ptr(c.kbase), _ptr(c.ksign), _ptr(c.kscale), _ptr(c.kres),
                                    _ptr(c.vbase), _ptr(c.vsign), _ptr(c.vscale), _ptr(c.vres),
                                    _ptr(np.ascontiguousarray(table)), layer, n_layers,
                                    layer_row_base, vis_start, vis_end, attn_scale,
                                    int(apply_attn_scale), int(online), n_threads)
    return xb


def qwen3next_ssm_tokens(qkv, z, gate_a, gate_b, *, n_k_heads, n_v_heads, head_dim, conv_kernel,
                         conv_w, dt_bias, ssm_a, ssm_norm, eps, conv_hist=None, state=None):
    """The per-token SSM layer (math.rs:766-953) over T tokens in order (the serial
    prefill loop, inference.rs:2866-2885).  gate_b None = fused [b | a] gates.
    Returns (out [T][n_v*d], conv_hist [(K-1)][conv_dim], state [n_v][d][d])."""
    qkv = _f32(qkv)
    z = _f32(z)
    ga = _f32(gate_a)
    gb = _f32(gate_b) if gate_b is not None else None
    T = qkv.shape[0]
    d_inner = n_v_heads * head_dim
    conv_dim = d_inner + 2 * n_k_heads * head_dim
    hist = np.zeros((max(conv_kernel - 1, 0), conv_dim), np.float32) if conv_hist is None else _f32(conv_hist).copy()
    st = np.zeros((n_v_heads, head_dim, head_dim), np.float32) if state is None else _f32(state).copy()
    out = np.zeros((T, d_inner), np.float32)
    cw, db, sa, sn = _f32(conv_w), _f32(dt_bias), _f32(ssm_a), _f32(ssm_norm)
    for t in range(T):
        lib().orc_qwen3next_ssm_token(_ptr(qkv[t]), _ptr(z[t]), _ptr(ga[t]),
                                      _ptr(gb[t]) if gb is not None else None, n_k_heads, n_v_heads,
                                      head_dim, conv_kernel, _ptr(cw), _ptr(db), _ptr(sa), _ptr(sn), eps,
                                      _ptr(hist), _ptr(st), _ptr(out[t]))
    return out, hist, st


def qwen3next_ssm_tokens_f64(qkv, z, gate_a, gate_b, *, n_k_heads, n_v_heads, head_dim, conv_kernel,
                             conv_w, dt_bias, ssm_a, ssm_norm, eps, conv_hist=None, state=None):
    """The same layer as qwen3next_ssm_tokens evaluated in float64 (numpy), stage by
    stage from the reference's formulas (math.rs:766-953): depthwise causal conv over
    the K - 1 history rows + the token (776-812) and SiLU; periodic K -> V head tiling
    (824-826); q / |q| / sqrt(d), k / |k| (833-846); beta = sigmoid, decay
    exp(softplus(alpha + dt_bias) * a) (848-874); the delta rule (math.rs:492-546);
    gated RMSNorm with SiLU(z) (936-951).  All values are assumed finite (no guards).
    A reference point for fp32 evaluations: returns (out [T][n_v*d] f64,
    conv_hist [(K-1)][conv_dim] f32, state [n_v][d][d] f64)."""
    qkv = np.asarray(qkv, np.float32)
    T = qkv.shape[0]
    nk, nv, d, K = n_k_heads, n_v_heads, head_dim, conv_kernel
    d_inner = nv * d
    conv_dim = d_inner + 2 * nk * d
    hist = (np.zeros((K - 1, conv_dim), np.float32) if conv_hist is None
            else np.asarray(conv_hist, np.float32))
    x = np.concatenate([hist, qkv]).astype(np.float64)
    cw = np.asarray(conv_w, np.float64).reshape(conv_dim, K)
    db, sa = np.asarray(dt_bias, np.float64), np.asarray(ssm_a, np.float64)
    sn = np.asarray(ssm_norm, np.float64)
    ga = np.asarray(gate_a, np.float64)
    gb = None if gate_b is None else np.asarray(gate_b, np.float64)
    zz = np.asarray(z, np.float64).reshape(T, nv, d)
    S = (np.zeros((nv, d, d)) if state is None else np.asarray(state, np.float64)).copy()
    sig = lambda v: 1.0 / (1.0 + np.exp(-v))
    softplus = lambda v: np.where(v > 20, v, np.where(v < -20, np.exp(np.minimum(v, 20)),
                                                     np.log1p(np.exp(np.minimum(v, 20)))))
    heads = np.arange(nv)
    src = heads % nk
    hpg = nv // nk
    out = np.zeros((T, nv, d))
    for t in range(T):
        acc = (x[t:t + K] * cw.T).sum(axis=0)            # window oldest first, token last
        conv = acc * sig(acc)
        q = conv[:nk * d].reshape(nk, d)[src]
        k = conv[nk * d:2 * nk * d].reshape(nk, d)[src]
        v = conv[2 * nk * d:].reshape(nv, d)
        q = q / np.sqrt((q * q).sum(-1, keepdims=True) + eps) / np.sqrt(d)
        k = k / np.sqrt((k * k).sum(-1, keepdims=True) + eps)
        if gb is None:
            base = (heads // hpg) * 2 * hpg + heads % hpg
            beta, alpha = sig(ga[t, base]), ga[t, base + hpg] + db
        else:
            beta, alpha = sig(gb[t]), ga[t] + db
        g = np.exp(softplus(alpha) * sa)
        S *= g[:, None, None]
        delta = beta[:, None] * (v - np.einsum("hji,hj->hi", S, k))
        S += k[:, :, None] * delta[:, None, :]
        o = np.einsum("hji,hj->hi", S, q)
        inv = 1.0 / np.sqrt((o * o).mean(-1, keepdims=True) + eps)
        out[t] = sn * (o * inv) * (zz[t] * sig(zz[t]))
    new_hist = np.concatenate([hist, qkv])[T:T + K - 1] if K > 1 else hist
    return out.reshape(T, d_inner), np.ascontiguousarray(new_hist, np.float32), S


def sigmoid_mul(d, g) -> np.ndarray:
    """orc_sigmoid_mul on a copy of d (the Qwen3.5 output gate, math.rs:396-403)."""
    d = _f32(d).copy()
    g = _f32(g)
    assert d.shape == g.shape
    lib().orc_sigmoid_mul(_ptr(d), _ptr(g), d.size)
    return d


def f16_bits(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, np.float32).astype(np.float16)).view(np.uint16)


def bf16_bits(x) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit pattern (gguf.rs fp32_to_bf16 semantics)."""
    a = np.ascontiguousarray(np.asarray(x, np.float32)).view(np.uint32)
    nan = (a & 0x7FFFFFFF) > 0x7F800000
    r = ((a + 0x7FFF + ((a >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((a[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def c_f32_to_f16(x) -> np.ndarray:
    """orc_f32_to_f16 element-wise (the raw f16 cache rounding, gguf.rs:72-106)."""
    x = _f32(x).reshape(-1)
    out = np.empty(x.size, np.uint16)
    lib().orc_f32_to_f16_n(_ptr(x), _ptr(out), x.size)
    return out


def c_f32_to_bf16(x) -> np.ndarray:
    """orc_f32_to_bf16 element-wise (gguf.rs:108-117)."""
    x = _f32(x).reshape(-1)
    out = np.empty(x.size, np.uint16)
    lib().orc_f32_to_bf16_n(_ptr(x), _ptr(out), x.size)
    return out


def c_f16_to_f32(bits) -> np.ndarray:
    """orc_f16_to_f32 element-wise (gguf.rs:26-53)."""
    b = np.ascontiguousarray(np.asarray(bits, np.uint16)).reshape(-1)
    out = np.empty(b.size, np.float32)
    lib().orc_f16_to_f32_n(_ptr(b), _ptr(out), b.size)
    return out


def c_bf16_to_f32(bits) -> np.ndarray:
    """orc_bf16_to_f32 element-wise (gguf.rs:55-58)."""
    b = np.ascontiguousarray(np.asarray(bits, np.uint16)).reshape(-1)
    out = np.empty(b.size, np.float32)
    lib().orc_bf16_to_f32_n(_ptr(b), _ptr(out), b.size)
    return out


def bf16_to_f32(bits) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f16_to_f32(bits) -> np.ndarray:
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def upcast(bits, fmt) -> np.ndarray:
    if fmt == F16:
        return f16_to_f32(bits)
    if fmt == BF16:
        return bf16_to_f32(bits)
    return np.asarray(bits, np.float32)


def env_threads() -> int:
    return int(os.environ.get("ORACLE_THREADS", "0")) or max_threads()


def _load_gpfc():
    """oracle/gpfc.py (the GPFC prefill-cache restatement) as `gpfc`."""
    import importlib.util
    import sys
    name = "gr_oracle_gpfc"
    if name not in sys.modules:
        spec = importlib.util.spec_from_file_location(name, HERE / "gpfc.py")
        mod = importlib.util.module_from_spec(spec)
        sys.modules[name] = mod
        spec.loader.exec_module(mod)
    return sys.modules[name]


gpfc = _load_gpfc()
