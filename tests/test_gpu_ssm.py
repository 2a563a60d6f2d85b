"""The Qwen3.5 SSM layer around the DeltaNet recurrence (conv1d + SiLU, K -> V
head tiling, L2 norms, beta / decay gates, gated RMSNorm with SiLU(z); reference
math.rs:766-953) through gr_qwen3next_ssm_layer, against the oracle's token-serial
restatement (the loop of inference.rs:2866-2885).

Tolerances (fp32 path):
  recurrent state: max |gpu - ref| <= 1e-5 (the DeltaNet bar);
  layer output, against the float64 statement of the layer (oracle.py
      qwen3next_ssm_tokens_f64, pinned against the oracle on the CPU): elementwise
      |gpu - f64| <= |oracle - f64| + 1e-5, i.e. the device is no further from the
      exact value than the reference's own fp32 token loop plus the fp32 bar.  (The
      gated RMSNorm rescales o to unit RMS and multiplies it by SiLU(z) * w, so
      outputs reach ~20, where a few ulps of any fp32 order exceed 1e-5.);
  conv history: bit-exact (a copy of the last K - 1 raw inputs).
"""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _weights(rng, n_layers, nk, nv, d, K):
    conv_dim = (nv + 2 * nk) * d
    return dict(
        ssm_conv1d=(0.3 * rng.standard_normal((n_layers, conv_dim, K))).astype(np.float32),
        ssm_a=-rng.uniform(0.2, 1.2, (n_layers, nv)).astype(np.float32),
        ssm_dt_bias=(0.1 * rng.standard_normal((n_layers, nv))).astype(np.float32),
        ssm_norm=(1 + 0.1 * rng.standard_normal((n_layers, d))).astype(np.float32))


@pytest.mark.parametrize("nk,fused,chunks,d", [(8, True, (300, 37), 128), (16, False, (37, 130), 128),
                                                (4, True, (90, 20), 64), (2, False, (70, 3), 256),
                                                (8, True, (1500, 1100), 128)])
def test_qwen3next_ssm_layer_matches_token_loop(orc, dev, nk, fused, chunks, d):
    """Config-5 shape (16 value heads, d128, conv kernel 4): two consecutive calls
    (chunked and recurrent DeltaNet paths) carry the conv history and the state; state
    sizes 64 and 256 (ssm_state_size, math.rs:566) on the token recurrence.  Calls of
    1500 and 1100 tokens (over 16 MB of host rows) run as overlapped pieces cut at
    multiples of 64 tokens (256, 448, 512, 284 and 256, 576, 268), each piece's
    launches carrying the conv history and the state to the next."""
    from gguf_runner_amd import runtime as rt
    rng = np.random.default_rng(500 + nk + d)
    nv, K, layer, eps = 16, 4, 1, 1e-6
    W = _weights(rng, 2, nk, nv, d, K)
    p = rt.Config(n_layers=2, n_heads=2, n_kv_heads=1, head_dim=128, seq_len=16, ssm_n_heads=nv,
                  ssm_head_dim=d, ssm_n_k_heads=nk, ssm_conv_kernel=K, rms_norm_eps=eps, **W)
    s = rt.malloc_run_state(p)
    conv_dim = (nv + 2 * nk) * d
    hist = None
    state = None
    state64 = None
    for T in chunks:
        qkv = rng.standard_normal((T, conv_dim)).astype(np.float32)
        z = rng.standard_normal((T, nv * d)).astype(np.float32)
        ga = rng.standard_normal((T, 2 * nv if fused else nv)).astype(np.float32)
        gb = None if fused else rng.standard_normal((T, nv)).astype(np.float32)
        got = rt.qwen3next_ssm_layer(p, s, layer, qkv, z, ga, gb)
        lw = dict(n_k_heads=nk, n_v_heads=nv, head_dim=d, conv_kernel=K,
                  conv_w=W["ssm_conv1d"][layer], dt_bias=W["ssm_dt_bias"][layer],
                  ssm_a=W["ssm_a"][layer], ssm_norm=W["ssm_norm"][layer], eps=eps)
        ex, _, state64 = orc.qwen3next_ssm_tokens_f64(qkv, z, ga, gb, **lw, conv_hist=hist,
                                                      state=state64)
        ref, hist, state = orc.qwen3next_ssm_tokens(qkv, z, ga, gb, **lw, conv_hist=hist, state=state)
        excess = np.abs(got - ex) - (np.abs(ref - ex) + TOL)
        assert float(excess.max()) <= 0.0, (T, float(excess.max()), float(np.abs(got - ref).max()))
        assert np.array_equal(rt.read_ssm_conv_state(p, s, layer), hist)
        dev_state = np.zeros((nv, d, d), np.float32)
        from gguf_runner_amd import ffi
        ffi.check(ffi.lib().gr_read_ssm_state(s.handle, layer, dev_state.ctypes.data))
        assert float(np.abs(dev_state - state).max()) <= TOL
    # layer 0 untouched
    assert not rt.read_ssm_conv_state(p, s, 0).any()


def test_qwen3next_ssm_layer_errors(dev):
    from gguf_runner_amd import ffi, runtime as rt
    p = rt.Config(n_layers=1, n_heads=2, n_kv_heads=1, head_dim=128, seq_len=16, ssm_n_heads=4,
                  ssm_head_dim=128)
    s = rt.malloc_run_state(p)
    with pytest.raises(ffi.GrError, match="missing qwen3next SSM tensors"):
        rt.qwen3next_ssm_layer(p, s, 0, np.zeros((1, 4 * 128 * 3), np.float32),
                               np.zeros((1, 512), np.float32), np.zeros((1, 8), np.float32))
