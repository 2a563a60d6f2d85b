"""Config 4 at full size: Gemma-3-4B-shaped attention with 5 local : 1 global layers,
an 8192-token prefill then 256 decode steps through the run-state entry points
(gr_prefill_attention_chunk = the prefill loop of inference.rs:2981-3017,
gr_attention_layer_token = the decode driver's calls at inference.rs:3499-3507).

Shape: 8 Q / 4 KV heads, head_dim 256, bf16 KV cache, Q/K/V ~N(0,1) rounded to bf16,
QK RMSNorm eps 1e-6 with weights ~N(1, 0.1) per layer, NeoX RoPE (local layers theta 1e4,
global layer theta 1e6 x 0.125), Gemma q pre-scale 1/sqrt(256) and unscaled scores,
window 1024 on the local layers (layer_windows [1024]*5 + [global]).

Oracle: each layer's token-serial prefill over all 8448 rows (norm -> RoPE -> bf16 cache
write), with the attention evaluated on a sample of the 8192 prefill rows and on every
one of the 256 decode rows.  Tolerance of the bf16 MFMA path (fixed before measuring):
|gpu - ref| <= 2e-3 + 1e-2 |ref| elementwise.
"""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
N_PREFILL, N_DECODE = 8192, 256
N_HEADS, N_KV, D = 8, 4, 256
WINDOW = 1024
LAYERS = [WINDOW] * 5 + [0]


def _close(got, ref, what):
    err = np.abs(got - ref)
    bad = ~(err <= ATOL + RTOL * np.abs(ref))  # NaN counts as out of tolerance
    assert not bad.any(), f"{what}: {bad.sum()} / {bad.size} out of tolerance; max abs {err.max():.3e}"


def test_config4_gemma3_5to1_prefill_8192_then_256_decode(dev, orc):
    from gguf_runner_amd import ffi, runtime as rt
    rng = np.random.default_rng(1004)
    n_tok = N_PREFILL + N_DECODE
    qn = (1.0 + 0.1 * rng.standard_normal((len(LAYERS), D))).astype(np.float32)
    kn = (1.0 + 0.1 * rng.standard_normal((len(LAYERS), D))).astype(np.float32)
    p = rt.Config(n_layers=len(LAYERS), n_heads=N_HEADS, n_kv_heads=N_KV, head_dim=D,
                  seq_len=n_tok, kv_dtype=ffi.DTYPE_BF16, rope_mode=ffi.ROPE_NEOX,
                  rope_theta=1e6, rope_theta_swa=1e4, rope_scale_global=0.125,
                  rope_scale_local=1.0, layer_windows=LAYERS, is_gemma3=True,
                  rms_norm_eps=1e-6, q_norm=qn, k_norm=kn)
    s = rt.malloc_run_state(p)
    sample = np.unique(np.concatenate([
        [0, 1, 2, 31, 32, 63, 64, 127, 128, 255, 256, 1022, 1023, 1024, 1025, 2047, 2048,
         4095, 4096, 6143, 6144, 8190, 8191],
        rng.integers(0, N_PREFILL, 24)]))
    for layer, window in enumerate(LAYERS):
        bf = lambda shape: orc.bf16_to_f32(orc.bf16_bits(rng.standard_normal(shape, dtype=np.float32)))
        q, k, v = bf((n_tok, p.q_dim)), bf((n_tok, p.kv_dim)), bf((n_tok, p.kv_dim))
        # GPU: the prefill in 4 chunks of 2048 (continuation over the device cache) ...
        got = np.concatenate([rt.prefill_attention_chunk(p, s, layer, b, q[b:b + 2048],
                                                         k[b:b + 2048], v[b:b + 2048])
                              for b in range(0, N_PREFILL, 2048)])
        # ... then one token at a time
        dec = np.zeros((N_DECODE, p.q_dim), np.float32)
        for i in range(N_DECODE):
            t = N_PREFILL + i
            s.q[:], s.k[:], s.v[:] = q[t], k[t], v[t]
            rt.attention_layer_token(p, s, layer, t)
            dec[i] = s.xb
        # oracle over all rows, attention on the sampled prefill rows and every decode row
        local = window > 0
        rows = np.concatenate([sample, np.arange(N_PREFILL, n_tok)])
        ref, kc, vc = orc.prefill_layer(
            q, k, v, n_heads=N_HEADS, n_kv_heads=N_KV, head_size=D, seq_len=n_tok, fmt=orc.BF16,
            rope_dim=D, neox=True, rope_freqs_tab=orc.rope_freqs(1e4 if local else 1e6, D),
            rope_scale=1.0 if local else 0.125, is_gemma3=True, window=window,
            q_norm=qn[layer], k_norm=kn[layer], eps=1e-6, n_threads=orc.env_threads(),
            attend_rows=rows)
        _close(got[sample], ref[sample], f"layer {layer} prefill")
        _close(dec, ref[N_PREFILL:], f"layer {layer} decode")
        # the cache rows the device wrote: V exact, post-RoPE K within 2 bf16 ulp
        kd, vd = rt.read_kv_rows(p, s, layer, 0, n_tok)
        assert np.array_equal(vd, vc), f"layer {layer}: V cache rows differ"
        a, b = orc.upcast(kd, orc.BF16), orc.upcast(kc, orc.BF16)
        assert np.all(np.abs(a - b) <= 2 * 2.0 ** -7 * np.maximum(np.abs(b), 2.0 ** -14)), \
            f"layer {layer}: K cache max diff {np.abs(a - b).max():.3e}"
