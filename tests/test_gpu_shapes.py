"""GQA shapes the reference's attention_token accepts for any kv_mul = Hq / Hkv and
every head size (inference.rs:1970-2530, kv_head = h / kv_mul at 2019): groups that
are not a power of two or exceed one workgroup's query columns (16 MFMA columns,
8 VALU heads: the group is split over several workgroup columns per KV head), and
a Q8 cache at head_dim 64.  Same bars as the per-format tests: f32 and Q8 max abs
1e-5 against the oracle; f16 / bf16 2e-3 + 1e-2 |ref|; Turbo 1e-5.
"""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n_heads,n_kv,d", [(6, 2, 128), (21, 3, 64), (24, 2, 128), (32, 1, 64),
                                            (40, 1, 128), (12, 4, 256)])
def test_f32_decode_any_group_size(orc, dev, n_heads, n_kv, d):
    """VALU split kernel: groups of 3, 7, 12, 32, 40 and 3 query heads."""
    from test_gpu_decode import _assert_close, _run_case
    got, ref = _run_case(orc, dev, n_heads=n_heads, n_kv=n_kv, d=d, starts=[0, 5], ends=[300, 777],
                         seq_len=800, fmt=orc.F32, seed=600 + n_heads)
    _assert_close(got, ref, orc.F32, orc)


@pytest.mark.parametrize("fmt_name", ["F16", "BF16"])
@pytest.mark.parametrize("n_heads,n_kv,d,split", [(24, 1, 128, 0), (48, 2, 128, 0), (32, 1, 256, 0),
                                                  (40, 2, 128, 128), (21, 3, 64, 0), (12, 1, 64, 0)])
def test_16bit_decode_groups_above_16(orc, dev, fmt_name, n_heads, n_kv, d, split):
    """MFMA kernel with 2-3 workgroup columns per KV head (stream schedule and the
    fixed split grid), and the VALU kernel at head_dim 64 with groups of 7 and 12."""
    from test_gpu_decode import _assert_close, _run_case
    fmt = getattr(orc, fmt_name)
    got, ref = _run_case(orc, dev, n_heads=n_heads, n_kv=n_kv, d=d, starts=[0, 100, 0],
                         ends=[1500, 900, 40], seq_len=1500, fmt=fmt, seed=700 + n_heads + d,
                         split_keys=split)
    _assert_close(got, ref, fmt, orc)


@pytest.mark.parametrize("n_heads,n_kv,d", [(20, 1, 128), (32, 2, 64), (48, 2, 256)])
def test_turbo_decode_groups_above_16(orc, dev, n_heads, n_kv, d):
    from test_gpu_turbo import _decode_case
    got, ref = _decode_case(orc, dev, n_heads=n_heads, n_kv=n_kv, d=d, starts=[0, 30], ends=[400, 256],
                            seq_len=400, seed=800 + n_heads)
    assert float(np.abs(got - ref).max()) <= 1e-5, np.abs(got - ref).max()


@pytest.mark.parametrize("block", [False, True])
@pytest.mark.parametrize("n_heads,n_kv", [(8, 4), (12, 4), (32, 1)])
def test_q8_decode_head_dim_64(orc, dev, block, n_heads, n_kv):
    """Q8 rows (row or 32-element block scales) at head_dim 64 on the MFMA kernel,
    including a group of 32 (two columns per KV head)."""
    from test_gpu_q8 import TOL, _decode_case
    got, ref = _decode_case(orc, dev, n_heads=n_heads, n_kv=n_kv, d=64, starts=[0, 3, 0],
                            ends=[1000, 517, 1], seq_len=1000, block=block, seed=900 + n_heads)
    assert float(np.abs(got - ref).max()) <= TOL, np.abs(got - ref).max()


@pytest.mark.parametrize("kv", ["q8", "turbo"])
def test_runstate_prefill_and_decode_at_new_shapes(orc, dev, kv):
    """Run-state entry points at shapes they now accept: a Q8 cache at head_dim 64
    (the chunk goes through the decode kernels) and a Turbo cache with 32 query
    heads per KV head (unpacked rows); a chunked prefill then token steps equal the
    token-by-token loop (gr_attention_layer_token per token, inference.rs:3499-3507)."""
    from gguf_runner_amd import ffi, runtime as rt
    d, n_heads, n_kv = (64, 8, 2) if kv == "q8" else (128, 32, 1)
    dt = ffi.DTYPE_Q8 if kv == "q8" else ffi.DTYPE_TURBO
    mk = lambda: rt.Config(n_layers=1, n_heads=n_heads, n_kv_heads=n_kv, head_dim=d, seq_len=128,
                           kv_dtype=dt, rope_mode=ffi.ROPE_NEOX, rope_theta=1e4)
    rng = np.random.default_rng(31)
    T = 70
    q = rng.standard_normal((T, n_heads * d)).astype(np.float32)
    k = rng.standard_normal((T, n_kv * d)).astype(np.float32)
    v = rng.standard_normal((T, n_kv * d)).astype(np.float32)
    # reference: token by token
    p1 = mk()
    s1 = rt.malloc_run_state(p1)
    want = np.zeros((T, n_heads * d), np.float32)
    def step(p, s, t):
        s.q[:], s.k[:], s.v[:] = q[t], k[t], v[t]
        rt.attention_layer_token(p, s, 0, t)
        return s.xb.copy()
    for t in range(T):
        want[t] = step(p1, s1, t)
    # chunked prefill of 60 rows, then 10 single-token steps
    p2 = mk()
    s2 = rt.malloc_run_state(p2)
    got = np.zeros_like(want)
    got[:60] = rt.prefill_attention_chunk(p2, s2, 0, 0, q[:60], k[:60], v[:60])
    for t in range(60, T):
        got[t] = step(p2, s2, t)
    assert float(np.abs(got - want).max()) <= 1e-5, np.abs(got - want).max()
