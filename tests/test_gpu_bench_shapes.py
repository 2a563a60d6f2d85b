"""Decode parity at the full sizes the benchmark times: 16 sequences x 32768 cached
keys, 32 Q / 4 KV heads, d128 (config 3's head shape at its maximum length), over
the f16 cache, the Q8 cache (row and 32-element block scales) and the Turbo cache,
against the CPU oracle's attention_token / attention_token_turbo (reference
inference.rs:1970-2530 and 1246-1334).

The Q8 and Turbo caches hold random codes, signs and scales (every bit pattern is
a valid row of those formats; the write paths have their own tests), so the
caches need no host-side encoding.  The oracle evaluates every sequence of the
f16 case and a sample of sequences of the others; the kernels run all 16.

Tolerances (fixed before measuring):
  f16 cache: |gpu - ref| <= 2e-3 + 1e-2 |ref| elementwise (the f16 MFMA path);
  Q8 cache: measured against a float64 evaluation of the same int8 rows and
      scales, the device no further from it than the oracle is, plus 1e-5;
  Turbo cache: max |gpu - ref| <= 1e-5.
"""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

N_SEQ, L, HQ, HKV, D = 16, 32768, 32, 4, 128


def test_decode_32k_f16_all_sequences(orc, dev):
    from test_gpu_decode import _assert_close, _run_case
    got, ref = _run_case(orc, dev, n_heads=HQ, n_kv=HKV, d=D, starts=[0] * N_SEQ, ends=[L] * N_SEQ,
                         seq_len=L, fmt=orc.F16, seed=3232)
    _assert_close(got, ref, orc.F16, orc)


def _f64_attention(q, codes_k, scale_k, codes_v, scale_v):
    """Exact attention of one sequence over dequantised int8 rows, in float64."""
    # row mode: one scale per row; block mode: one per 32 consecutive elements
    widen = lambda sc: np.repeat(sc.astype(np.float64).reshape(L, -1), (HKV * D) // sc.reshape(L, -1).shape[1], axis=1)
    sk, sv = widen(scale_k), widen(scale_v)
    k = (codes_k.astype(np.float64) * sk).reshape(L, HKV, D)
    v = (codes_v.astype(np.float64) * sv).reshape(L, HKV, D)
    out = np.zeros((HQ, D))
    for h in range(HQ):
        g = h // (HQ // HKV)
        s = k[:, g, :] @ q[h].astype(np.float64) / np.sqrt(D)
        p = np.exp(s - s.max())
        out[h] = (p @ v[:, g, :]) / p.sum()
    return out


@pytest.mark.parametrize("block", [False, True])
def test_decode_32k_q8_sampled_sequences(orc, dev, block):
    from gguf_runner_amd import ops
    from test_gpu_q8 import _assert_vs_f64
    rng = np.random.default_rng(3308 + block)
    per = HKV * D // 32 if block else 1
    q = rng.standard_normal((N_SEQ, HQ, D), dtype=np.float32)
    kc = rng.integers(-127, 128, (N_SEQ, L, HKV * D), dtype=np.int8)
    vc = rng.integers(-127, 128, (N_SEQ, L, HKV * D), dtype=np.int8)
    ks = rng.uniform(0.004, 0.02, (N_SEQ, L, per)).astype(np.float32)
    vs = rng.uniform(0.004, 0.02, (N_SEQ, L, per)).astype(np.float32)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    st = torch.zeros(N_SEQ, dtype=torch.int32, device=dev)
    en = torch.full((N_SEQ,), L, dtype=torch.int32, device=dev)
    out = ops.decode_attention(T(q), T(kc.reshape(N_SEQ, L, HKV, D)), T(vc.reshape(N_SEQ, L, HKV, D)),
                               st, en, max_kv_len=L, k_scale=T(ks), v_scale=T(vs), q8_block=block)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    fmt = orc.Q8B if block else orc.Q8
    for s in (0, 5, 10, 15):
        ref = orc.attention_token(q[s].reshape(-1), kc[s], vc[s], fmt, HQ, HKV, D, 0, L,
                                  key_scale=ks[s].reshape(-1), value_scale=vs[s].reshape(-1),
                                  n_threads=orc.env_threads()).reshape(HQ, D)
        exact = _f64_attention(q[s], kc[s], ks[s], vc[s], vs[s])
        _assert_vs_f64(got[s], ref, exact)


def test_decode_32k_turbo_sampled_sequences(orc, dev):
    from gguf_runner_amd import ops
    rng = np.random.default_rng(3309)
    layer, n_layers = 0, 1
    table = orc.turbo_sign_table(n_layers, HKV, D)
    kv_dim = HKV * D
    q = rng.standard_normal((N_SEQ, HQ, D), dtype=np.float32)
    # two distinct caches, alternating over the 16 sequences (each with its own query)
    caches = []
    for _ in range(2):
        c = orc.TurboCache(L, HKV, D)
        c.kbase[:] = rng.integers(0, 256, c.kbase.size, dtype=np.uint8)
        c.vbase[:] = rng.integers(0, 256, c.vbase.size, dtype=np.uint8)
        c.ksign[:] = rng.integers(0, 256, c.ksign.size, dtype=np.uint8)
        c.vsign[:] = rng.integers(0, 256, c.vsign.size, dtype=np.uint8)
        for name in ("kscale", "vscale", "kres", "vres"):
            getattr(c, name)[:] = rng.uniform(0.5, 1.5, getattr(c, name).size).astype(np.float32)
        caches.append(c)
    seq_cache = [caches[s % 2] for s in range(N_SEQ)]
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    stack = lambda name, w: T(np.stack([getattr(c, name).reshape(L, w) for c in seq_cache]))
    out = torch.empty((N_SEQ, HQ, D), device=dev)
    ops.TurboDecodeCall(T(q), stack("kbase", kv_dim // 4), stack("vbase", kv_dim // 4),
                        stack("ksign", kv_dim // 8), stack("vsign", kv_dim // 8),
                        stack("kscale", HKV), stack("vscale", HKV), stack("kres", HKV),
                        stack("vres", HKV), T(table), layer,
                        torch.zeros(N_SEQ, dtype=torch.int32, device=dev),
                        torch.full((N_SEQ,), L, dtype=torch.int32, device=dev), out,
                        max_kv_len=L)()
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for s in (0, 7, 14):
        ref = orc.attention_token_turbo(q[s].reshape(-1), seq_cache[s], table, layer, HQ, 0, L,
                                        n_threads=orc.env_threads()).reshape(HQ, D)
        err = float(np.abs(got[s] - ref).max())
        assert err <= 1e-5, f"sequence {s}: max abs {err:.3e}"
