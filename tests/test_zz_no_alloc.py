"""gr_decode_attention_noalloc (the decode entry point that allocates nothing) against
gr_decode_attention on the same inputs, over two calls in a row, the second smaller
than the first, so the second call runs over the first call's partials left in the
built-in scratch array.

Bar: the decode path's own (f16 cache: |d| <= 2e-3 + 1e-2 |ref|; Q8 and Turbo caches:
1e-5, the fp32 bar).  The two entry points run the same kernels, but the d128 decode's waves
claim key tiles dynamically, so the f16 rounding of P (relative to a running maximum)
differs from run to run; the test prints that run-to-run difference of the
workspace entry point beside the no-alloc difference."""
from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _case(torch, dev, rng, n_seq, n_heads, n_kv, d, lens, dtype, q8_block=False):
    from gguf_runner_amd import ops
    seq_len = int(max(lens))
    q = torch.from_numpy(rng.standard_normal((n_seq, n_heads, d), dtype=np.float32)).to(dev)
    shape = (n_seq, seq_len, n_kv, d)
    ks = vs = None
    if dtype == torch.int8:
        kc = torch.from_numpy(rng.integers(-127, 128, shape, dtype=np.int8)).to(dev)
        vc = torch.from_numpy(rng.integers(-127, 128, shape, dtype=np.int8)).to(dev)
        per_row = n_kv * d // 32 if q8_block else 1
        ks = torch.from_numpy(rng.uniform(0.001, 0.05, (n_seq, seq_len, per_row)).astype(np.float32)).to(dev)
        vs = torch.from_numpy(rng.uniform(0.001, 0.05, (n_seq, seq_len, per_row)).astype(np.float32)).to(dev)
    else:
        kc = torch.from_numpy(rng.standard_normal(shape, dtype=np.float32)).to(dev).to(dtype)
        vc = torch.from_numpy(rng.standard_normal(shape, dtype=np.float32)).to(dev).to(dtype)
    ends = np.asarray(lens, np.int32)
    starts = np.zeros(n_seq, np.int32)
    kv_start = torch.from_numpy(starts).to(dev)
    kv_end = torch.from_numpy(ends).to(dev)
    out_ref = torch.full((n_seq, n_heads, d), float("nan"), device=dev)
    out_na = torch.full((n_seq, n_heads, d), float("nan"), device=dev)
    call = ops.DecodeCall(q, kc, vc, kv_start, kv_end, out_ref, max_kv_len=seq_len,
                          k_scale=ks, v_scale=vs, q8_block=q8_block)
    return call, out_ref, out_na, (q, kc, vc, ks, vs, kv_start, kv_end)


def _turbo_case(torch, dev, rng, n_seq, n_heads, n_kv, d, lens):
    """A Turbo cache of random codes / signs and sigma, gamma ~U[0.5, 1.5]."""
    from gguf_runner_amd import ops
    L = int(max(lens))
    kv_dim = n_kv * d
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    u8 = lambda w: T(rng.integers(0, 256, (n_seq, L, w), dtype=np.uint8))
    aux = lambda: T(rng.uniform(0.5, 1.5, (n_seq, L, n_kv)).astype(np.float32))
    q = T(rng.standard_normal((n_seq, n_heads, d), dtype=np.float32))
    table = T(ops.turbo_sign_table(1, n_kv, d))
    kv_start = T(np.zeros(n_seq, np.int32))
    kv_end = T(np.asarray(lens, np.int32))
    out_ref = torch.full((n_seq, n_heads, d), float("nan"), device=dev)
    out_na = torch.full((n_seq, n_heads, d), float("nan"), device=dev)
    kb, vb, ks, vs = u8(kv_dim // 4), u8(kv_dim // 4), u8(kv_dim // 8), u8(kv_dim // 8)
    sk, sv, gk, gv = aux(), aux(), aux(), aux()
    call = ops.TurboDecodeCall(q, kb, vb, ks, vs, sk, sv, gk, gv, table, 0, kv_start, kv_end, out_ref,
                               max_kv_len=L)
    return call, out_ref, out_na, (q, kb, vb, ks, vs, sk, sv, gk, gv, table, kv_start, kv_end)


def _run_noalloc(call, out_na):
    from gguf_runner_amd import ffi, ops
    a = ffi.DecodeArgs.from_buffer_copy(call.args)
    a.workspace = None  # ignored by the no-alloc entry point
    a.out = out_na.data_ptr()
    ffi.check(ffi.lib().gr_decode_attention_noalloc(ctypes.byref(a), ops._stream(None)))


@pytest.mark.parametrize("kind", ["f16", "q8", "turbo"])
def test_noalloc_decode_matches_workspace_decode_twice(dev, kind):
    import torch
    rng = np.random.default_rng(4242)
    dt = torch.float16 if kind == "f16" else torch.int8
    # First call: config-3 shaped (32 / 4 heads, d128), 8 ragged sequences up to 16k
    # keys; second call: 3 shorter sequences with other heads.
    cases = [dict(n_seq=8, n_heads=32, n_kv=4, d=128, lens=rng.integers(1024, 16385, 8)),
             dict(n_seq=3, n_heads=16, n_kv=8, d=128, lens=[1, 300, 2049])]
    for i, c in enumerate(cases):
        print(f"noalloc case {i} {kind}: {c['n_seq']} seqs, lens {list(map(int, c['lens']))}", flush=True)
        if kind == "turbo":
            call, out_ref, out_na, keep = _turbo_case(torch, dev, rng, c["n_seq"], c["n_heads"], c["n_kv"],
                                                      c["d"], c["lens"])
        else:
            call, out_ref, out_na, keep = _case(torch, dev, rng, c["n_seq"], c["n_heads"], c["n_kv"], c["d"],
                                                c["lens"], dt)
        call()
        torch.cuda.synchronize()
        ref0 = out_ref.cpu().numpy()
        call()
        _run_noalloc(call, out_na)
        torch.cuda.synchronize()
        ref = out_ref.cpu().numpy()
        got = out_na.cpu().numpy()
        assert np.isfinite(ref).all() and np.isfinite(got).all()
        err = np.abs(got - ref)
        print(f"  max |noalloc - workspace| {err.max():.3e}, workspace run to run "
              f"{np.abs(ref - ref0).max():.3e}", flush=True)
        if kind == "f16":
            assert np.all(err <= 2e-3 + 1e-2 * np.abs(ref)), float(err.max())
        else:
            assert float(err.max()) <= 1e-5


def test_noalloc_rejects_oversize_before_launch(dev):
    """A call whose partials exceed the built-in array fails with the limit in the
    message and launches nothing (the output stays untouched)."""
    import torch
    from gguf_runner_amd import ffi
    n_seq, n_heads, n_kv, d, L = 64, 32, 4, 128, 65536
    a = ffi.DecodeArgs()
    a.n_seq, a.n_heads, a.n_kv_heads, a.head_dim = n_seq, n_heads, n_kv, d
    a.kv_dtype, a.max_kv_len, a.score_scale = ffi.DTYPE_F16, L, 1.0 / math.sqrt(d)
    out = torch.zeros((n_seq, n_heads, d), device=dev)
    dummy = torch.zeros(1024, dtype=torch.int32, device=dev)
    a.q = a.k_cache = a.v_cache = a.kv_start = a.kv_end = dummy.data_ptr()
    a.out = out.data_ptr()
    a.seq_stride, a.row_stride = L * n_kv * d, n_kv * d
    assert ffi.lib().gr_decode_workspace_size(ctypes.byref(a)) > (64 << 20)
    rc = ffi.lib().gr_decode_attention_noalloc(ctypes.byref(a), None)
    assert rc == ffi.GR_ERR_ARG
    assert b"built-in scratch" in ffi.lib().gr_last_error()
    torch.cuda.synchronize()
    assert float(out.abs().max()) == 0.0


def test_noalloc_decode_replays_under_graph_capture(dev):
    """The first no-alloc call on a device resolves the scratch address and the launch
    occupancy (host queries, outside any capture); after it the call records into a
    HIP graph as kernel nodes only.  Each replay, with new kv_end contents written
    between replays and eager work and synchronisations around them, matches
    gr_decode_attention on the same contents (Q8 cache: the 1e-5 bar)."""
    import torch
    from gguf_runner_amd import ffi, ops
    rng = np.random.default_rng(99)
    lens = [3000, 17, 1200, 4096]
    call, out_ref, out_na, keep = _case(torch, dev, rng, 4, 32, 4, 128, lens, torch.int8)
    kv_end = keep[6]
    _run_noalloc(call, out_na)  # first call on the device: before the capture
    torch.cuda.synchronize()
    a = ffi.DecodeArgs.from_buffer_copy(call.args)
    a.workspace = None
    a.out = out_na.data_ptr()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(g, stream=s):
        ffi.check(ffi.lib().gr_decode_attention_noalloc(ctypes.byref(a), ops._stream(s)))
    torch.cuda.synchronize()
    for i, ends in enumerate(([3000, 17, 1200, 4096], [5, 4096, 1, 2000], [4096] * 4)):
        print(f"graph replay {i}: kv_end {ends}", flush=True)
        kv_end.copy_(torch.tensor(ends, dtype=torch.int32))
        out_na.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = out_na.cpu().numpy()
        out_ref.fill_(float("nan"))
        call()
        torch.cuda.synchronize()
        ref = out_ref.cpu().numpy()
        assert np.isfinite(ref).all() and np.isfinite(got).all()
        err = float(np.abs(got - ref).max())
        print(f"  max |replay - workspace| {err:.3e}", flush=True)
        assert err <= 1e-5
