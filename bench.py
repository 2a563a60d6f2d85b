"""Benchmark of the attention hot path on one MI355X (prints ONE JSON line).

Headline (`value`): split-K decode attention, configuration 3 of the benchmark set
(Qwen3-30B-A3B-shaped: 16 sequences with ragged cached lengths U[1024, 32768],
32 Q / 4 KV heads, head_dim 128, f16 KV cache), in GB/s of algorithmic KV bytes
  bytes/step = sum_b L_b * Hkv * d * 2 (K and V) * 2 B
with every input already resident in HBM.  A step is one gr_decode_attention
call (split kernel + combine kernel) over the whole batch.  Consecutive steps
read different copies of the workload (at least 768 MB of other inputs between
two reads of one copy), so no step is served from the 256 MB Infinity Cache.

Also reported in the same line:
  decode_32k   -- the decode target run (all 16 sequences at 32768 keys)
  decode_32k_q8 -- the same over a Q8 cache (int8 rows + one f32 scale per row)
  decode_32k_turbo -- the same over a Turbo cache (2-bit codes + residual signs + 2
                  f32 per kv head and row; compute-bound, so also given as the f16
                  cache bytes per second it replaces)
  prefill      -- the 8k prefill target run (config 2's shape at 8192 tokens:
                  Llama-3-8B-shaped causal prefill, f16, RoPE fused), in TFLOP/s
                  with flops = 4 * Hq * d * sum_q visible(q), with its roofline
                  block; also flat as prefill_tflops / prefill_frac_of_mfma_peak
  prefill_config2_s2048 -- config 2 itself (2048 tokens)
  deltanet     -- config 5 (gated DeltaNet, 16 heads, d128): 4096-token chunked
                  prefill and one recurrent decode step
  prefill_2048_quantised_cache -- run-state prefill of a 2048-token chunk over a
                  Q8 and a Turbo cache, wall time per call with host buffers
  encoder_siglip -- encoder self-attention at the Gemma 3 SigLIP shape (4096
                  patches, 16 heads, d72, f32)
  config1_decode -- config 1 (Qwen3-0.6B-shaped decode, f32 KV, 1024 keys)
  runstate_token_us -- the drop-in per-token call (gr_attention_layer_token: QK
                  norm, RoPE, KV write and attention over 1024 keys with host rows),
                  config 1's heads over f32 / f16 / Q8 / Turbo caches, us per call
  config4      -- config 4 (Gemma-3-4B-shaped, d256, bf16): the 8192-token prefill
                  of a sliding-window (1024) and the global layer, the 5 : 1 stack
                  of six layers, and one decode step over the six layers after it
  roofline     -- the dominant kernel (decode) against 8 TB/s HBM; prefill.roofline
                  the 8k prefill against the dense f16 MFMA peak
  cpu_baseline -- the CPU oracle (a C restatement of the reference's loops,
                  oracle/oracle.c) timed on this host's cores.  `value` is the
                  config-3 decode over the reference's Q8 storage (headline unit);
                  the legs add the Turbo storage (the reference's default), f16 raw
                  KV (the GPU headline's format, which the reference never stores),
                  token-serial prefill and the serial DeltaNet scan (median of 3
                  runs after one warm-up each).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X published dense f16 / bf16 MFMA peak
METRIC = "decode attn GB/s (% of 8 TB/s) + prefill attn TFLOP/s (% MFMA), 1×MI355X"


def _timed(fn, steps, warmup, stream):
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    # settle clocks and TLBs on freshly allocated buffers: at least ~0.2 s of work
    t_end = time.perf_counter() + 0.2
    while time.perf_counter() < t_end:
        fn()
        torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(steps):
        fn()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return ev0.elapsed_time(ev1) / steps, wall * 1e3 / steps  # ms per step (events, wall)


# MI355X has a 256 MB Infinity Cache (MALL) in front of HBM.  Calling one
# single-layer decode over and over would let it serve part of the KV cache
# from the previous call, which a real decode step never sees (every other
# layer's KV is read before the same layer comes round again).  Decode
# workloads therefore cycle through enough independent copies that at least
# ROTATE_BYTES of other inputs are read between two calls on the same copy.
ROTATE_BYTES = 768 << 20


def rotating(build, seed):
    """build(seed) -> (call, bytes, keep); returns a call that cycles through
    1 + ceil(ROTATE_BYTES / bytes) copies, the bytes of one call, and the copies."""
    first = build(seed)
    n = 1 + -(-ROTATE_BYTES // first[1])
    copies = [first] + [build(seed + 1000 * i) for i in range(1, n)]
    state = {"i": 0}

    def call():
        copies[state["i"]][0]()
        state["i"] = (state["i"] + 1) % n

    call.copies = n
    return call, first[1], copies


def measured_traffic(name="decode_mfma_f16_d128_config3.md"):
    """HBM bytes per decode call from the committed rocprofv3 PMC summary (FETCH_SIZE +
    WRITE_SIZE of both kernels, calibrated against a plain copy), or None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", name)
    try:
        with open(path) as f:
            for ln in f:
                if ln.startswith("traffic_bytes_per_call:"):
                    return int(float(ln.split(":")[1]))
    except OSError:
        pass
    return None


def decode_workload(dev, lens, seed, n_heads=32, n_kv=4, d=128, kv_dtype=None, starts=None):
    import torch
    from gguf_runner_amd import ops
    kv_dtype = kv_dtype or torch.float16
    n_seq = len(lens)
    max_len = int(max(lens))
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    q = torch.randn((n_seq, n_heads, d), generator=g, device=dev, dtype=torch.float32)
    kc = torch.randn((n_seq, max_len, n_kv, d), generator=g, device=dev, dtype=kv_dtype)
    vc = torch.randn((n_seq, max_len, n_kv, d), generator=g, device=dev, dtype=kv_dtype)
    st = torch.tensor(starts or [0] * n_seq, dtype=torch.int32, device=dev)
    en = torch.tensor(lens, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    call = ops.DecodeCall(q, kc, vc, st, en, out, max_kv_len=max(e - b for e, b in zip(lens, starts or [0] * n_seq)))
    esz = torch.finfo(kv_dtype).bits // 8
    nbytes = int(sum(e - b for e, b in zip(lens, starts or [0] * n_seq))) * n_kv * d * 2 * esz
    return call, nbytes, (q, kc, vc, st, en, out)


def decode_q8_workload(dev, lens, seed, n_heads=32, n_kv=4, d=128, block=False):
    """Config-3 shape over a Q8 cache (int8 codes ~U[-127, 127], f32 scales)."""
    import torch
    from gguf_runner_amd import ops
    n_seq = len(lens)
    max_len = int(max(lens))
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    q = torch.randn((n_seq, n_heads, d), generator=g, device=dev, dtype=torch.float32)
    kc = torch.randint(-127, 128, (n_seq, max_len, n_kv, d), generator=g, device=dev,
                       dtype=torch.int8)
    vc = torch.randint(-127, 128, (n_seq, max_len, n_kv, d), generator=g, device=dev,
                       dtype=torch.int8)
    per = n_kv * d // 32 if block else 1
    ks = torch.rand((n_seq, max_len, per), generator=g, device=dev) * 0.02 + 0.01
    vs = torch.rand((n_seq, max_len, per), generator=g, device=dev) * 0.02 + 0.01
    st = torch.zeros(n_seq, dtype=torch.int32, device=dev)
    en = torch.tensor(lens, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    call = ops.DecodeCall(q, kc, vc, st, en, out, max_kv_len=max_len, k_scale=ks, v_scale=vs,
                          q8_block=block)
    nbytes = int(sum(lens)) * (n_kv * d * 2 + 2 * per * 4)
    return call, nbytes, (q, kc, vc, ks, vs, st, en, out)


def decode_turbo_workload(dev, lens, seed, n_heads=32, n_kv=4, d=128):
    """Config-3 shape over a Turbo cache: random code and sign bytes, sigma / gamma
    ~U[0.5, 1.5] (the decode's cost does not depend on the values)."""
    import torch
    from gguf_runner_amd import ops
    n_seq = len(lens)
    L = int(max(lens))
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    kv_dim = n_kv * d
    rnd8 = lambda w: torch.randint(0, 256, (n_seq, L, w), generator=g, device=dev, dtype=torch.uint8)
    aux = lambda: torch.rand((n_seq, L, n_kv), generator=g, device=dev) + 0.5
    q = torch.randn((n_seq, n_heads, d), generator=g, device=dev)
    kb, vb, ks_, vs_ = rnd8(kv_dim // 4), rnd8(kv_dim // 4), rnd8(kv_dim // 8), rnd8(kv_dim // 8)
    sig_k, sig_v, gam_k, gam_v = aux(), aux(), aux(), aux()
    table = torch.from_numpy(ops.turbo_sign_table(1, n_kv, d)).to(dev)
    st = torch.zeros(n_seq, dtype=torch.int32, device=dev)
    en = torch.tensor(lens, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    call = ops.TurboDecodeCall(q, kb, vb, ks_, vs_, sig_k, sig_v, gam_k, gam_v, table, 0, st, en, out,
                               max_kv_len=L)
    nbytes = int(sum(lens)) * n_kv * 2 * (d // 4 + d // 8 + 8)
    return call, nbytes, (q, kb, vb, ks_, vs_, sig_k, sig_v, gam_k, gam_v, table, st, en, out)


def prefill_workload(dev, S, seed, n_heads=32, n_kv=8, d=128, dtype=None):
    import torch
    from gguf_runner_amd import ffi, ops
    dtype = dtype or torch.float16
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    q = torch.randn((S, n_heads, d), generator=g, device=dev, dtype=dtype)
    k = torch.randn((S, n_kv, d), generator=g, device=dev, dtype=dtype)
    v = torch.randn((S, n_kv, d), generator=g, device=dev, dtype=dtype)
    kc = torch.empty((S, n_kv, d), device=dev, dtype=dtype)
    vc = torch.empty_like(kc)
    out = torch.empty((S, n_heads, d), device=dev, dtype=torch.float32)
    fr = torch.tensor(ops.rope_freqs(5e5, d), dtype=torch.float32, device=dev)
    call = ops.PrefillCall(q, k, v, kc, vc, out, rope_mode=ffi.ROPE_ADJACENT, rope_dim=d,
                           rope_freqs=fr)
    flops = 4 * n_heads * d * S * (S + 1) // 2
    return call, flops, (q, k, v, kc, vc, out, fr)


def prefill_d64_workload(dev, S, seed, n_heads=14, n_kv=2, d=64, dtype=None):
    """head_dim-64 causal prefill at the Qwen2-0.5B shape (14 Q / 2 KV heads, f16 (or
    `dtype`) Q/K/V, NeoX RoPE theta 1e6 fused on load)."""
    import torch
    from gguf_runner_amd import ffi, ops
    dtype = dtype or torch.float16
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    q = torch.randn((S, n_heads, d), generator=g, device=dev, dtype=dtype)
    k = torch.randn((S, n_kv, d), generator=g, device=dev, dtype=dtype)
    v = torch.randn((S, n_kv, d), generator=g, device=dev, dtype=dtype)
    kc, vc = torch.empty_like(k), torch.empty_like(v)
    out = torch.empty((S, n_heads, d), device=dev, dtype=torch.float32)
    fr = torch.tensor(ops.rope_freqs(1e6, d), dtype=torch.float32, device=dev)
    call = ops.PrefillCall(q, k, v, kc, vc, out, rope_mode=ffi.ROPE_NEOX, rope_dim=d, rope_freqs=fr)
    return call, 4 * n_heads * d * S * (S + 1) // 2, (q, k, v, kc, vc, out, fr)


def prefill_q8_workload(S, seed, block, n_heads=32, n_kv=8, d=128, turbo=False):
    """Run-state prefill of one S-token chunk over a Q8 KV cache (row or 32-element
    block scales) or a Turbo cache: gr_prefill_attention_chunk with host q / k / v
    rows, i.e. upload, QK prep, the cache write, the attention (Q8: the MFMA flash
    pass; Turbo: query rotation, token-packed split kernel, merge + inverse
    rotations) and the download of the outputs."""
    from gguf_runner_amd import ffi, runtime as rt
    p = rt.Config(n_layers=1, n_heads=n_heads, n_kv_heads=n_kv, head_dim=d, seq_len=S,
                  kv_dtype=ffi.DTYPE_TURBO if turbo else ffi.DTYPE_Q8, q8_block_scales=block,
                  rope_mode=ffi.ROPE_NONE)
    s = rt.malloc_run_state(p)
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((S, p.q_dim)).astype(np.float32)
    k = rng.standard_normal((S, p.kv_dim)).astype(np.float32)
    v = rng.standard_normal((S, p.kv_dim)).astype(np.float32)
    xb = np.zeros((S, p.q_dim), np.float32)  # reused, as the caller's run-state rows are
    flops = 4 * n_heads * d * S * (S + 1) // 2
    return (lambda: rt.prefill_attention_chunk(p, s, 0, 0, q, k, v, out=xb)), flops, (p, s, xb)


def config4_prefill_workload(dev, W, S=8192, seed=4):
    """Config 4 (Gemma-3-4B-shaped attention layer): 8 Q / 4 KV heads, d256, bf16 q/k/v,
    QK RMSNorm (eps 1e-6, weights ~N(1, 0.1)), NeoX RoPE, Gemma q scale, an 8192-token
    prefill; W = 1024 for the sliding-window layers, 0 for the global one."""
    import torch
    from gguf_runner_amd import ffi, ops
    Hq, Hk, d = 8, 4, 256
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    q = torch.randn((S, Hq, d), generator=g, device=dev, dtype=torch.bfloat16)
    k = torch.randn((S, Hk, d), generator=g, device=dev, dtype=torch.bfloat16)
    v = torch.randn((S, Hk, d), generator=g, device=dev, dtype=torch.bfloat16)
    kc, vc = torch.empty_like(k), torch.empty_like(v)
    out = torch.empty((S, Hq, d), device=dev, dtype=torch.float32)
    qn = (1 + 0.1 * torch.randn(d, generator=g, device=dev)).float()
    kn = (1 + 0.1 * torch.randn(d, generator=g, device=dev)).float()
    theta, scale = (1e4, 1.0) if W else (1e6, 0.125)
    fr = torch.tensor(ops.rope_freqs(theta, d), dtype=torch.float32, device=dev)
    call = ops.PrefillCall(q, k, v, kc, vc, out, window=W, rope_mode=ffi.ROPE_NEOX, rope_dim=d,
                           rope_freqs=fr, rope_scale=scale, q_norm=qn, k_norm=kn, is_gemma3=True)
    flops = 4 * Hq * d * sum(min(i + 1, W) if W else i + 1 for i in range(S))
    return call, flops, (q, k, v, kc, vc, out, qn, kn, fr)


def encoder_workload(dev, stream):
    """Gemma 3 SigLIP vision attention: one noncausal sequence of 4096 patches, 16
    heads of dim 72, f32 rows (gr_encoder_self_attention)."""
    import torch
    from gguf_runner_amd import ops
    g = torch.Generator(device=dev)
    g.manual_seed(9)
    q, k, v = (torch.randn((4096, 16 * 72), generator=g, device=dev) for _ in range(3))
    out = torch.empty_like(q)
    call = lambda: ops.encoder_self_attention(q, k, v, n_seq=1, tokens=4096, heads=16, head_dim=72,
                                              out=out, stream=stream)
    return call, 4 * 16 * 72 * 4096 * 4096, (q, k, v, out)


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_runs(run, n=3):
    """One untimed warm-up, then the median of n timed runs of run() -> (units, seconds)."""
    run()
    rates, secs = [], []
    for _ in range(n):
        t0 = time.perf_counter()
        units = run()
        dt = time.perf_counter() - t0
        rates.append(units / dt)
        secs.append(dt)
    return float(np.median(rates)), float(sum(secs))


def cpu_baseline(lens, n_heads=32, n_kv=4, d=128):
    """The CPU oracle (oracle/oracle.c, a C restatement of the reference's x86 loops)
    on this host's cores, each leg a bounded sample of a benchmark configuration, the
    median of 3 runs after one warm-up.  The decode legs run the 16 config-3
    sequences whole, in batch order, one sequence at a time and parallel over heads
    (as the reference's rayon pool runs attention_token):
      value (decode_q8) -- the reference's Q8 storage (int8 rows + one f32 scale per
          row, dot_q8_row / axpy_q8_row, inference.rs:1337-1366);
      decode_turbo -- the reference's default storage (switches.rs:233-235): 2-bit
          codes + residual signs + sigma / gamma per (row, KV head), the query
          rotations and dot_ / axpy_turboquant_head* (inference.rs:954-968,
          1246-1334); the cost does not depend on the code values, which are random;
      decode_f16_raw -- f16 raw KV rows, the GPU headline's storage.  The reference
          stores only Q8 or Turbo rows (KvCacheFormat, types.rs:811-814): this leg
          is the oracle's raw-row mode, not a reference configuration;
      prefill_token_serial -- transformer_prefill_batch's per-token loop
          (inference.rs:2981-3017: QK-norm, RoPE, KV write, attention_token) over the
          first 1024 tokens of config 2 (32 / 8 heads, d128, adjacent RoPE theta 5e5);
      deltanet_scan -- the serial gated-delta-rule scan of the SSM prefill
          (inference.rs:2866-2885, qwen3next_state_head_step per head) over the 4096
          tokens of config 5 (16 heads, d128), parallel over heads."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import __graft_entry__ as ge
    orc = ge.load_oracle()
    threads = orc.max_threads()
    rng = np.random.default_rng(1003)
    seqs = list(lens)
    Lmax = max(seqs)
    kf = rng.standard_normal((Lmax, n_kv * d), dtype=np.float32)
    vf = rng.standard_normal((Lmax, n_kv * d), dtype=np.float32)
    q = rng.standard_normal(n_heads * d, dtype=np.float32)
    k8 = [orc.kv_quantize_row(r, False) for r in kf]
    v8 = [orc.kv_quantize_row(r, False) for r in vf]
    kq = np.stack([c for c, _ in k8]); ks = np.concatenate([sc for _, sc in k8]).astype(np.float32)
    vq = np.stack([c for c, _ in v8]); vs = np.concatenate([sc for _, sc in v8]).astype(np.float32)

    def dec_q8():
        for L in seqs:
            orc.attention_token(q, kq, vq, orc.Q8, n_heads, n_kv, d, 0, L, key_scale=ks, value_scale=vs,
                                n_threads=threads)
        return sum(seqs) * (n_kv * d * 2 + 2 * 4)
    q8_rate, q8_s = _median_runs(dec_q8)
    del k8, v8

    tc = orc.TurboCache(Lmax, n_kv, d)
    for arr in (tc.kbase, tc.vbase, tc.ksign, tc.vsign):
        arr[:] = rng.integers(0, 256, arr.size, dtype=np.uint8)
    for arr in (tc.kscale, tc.vscale, tc.kres, tc.vres):
        arr[:] = (rng.random(arr.size) + 0.5).astype(np.float32)
    table = orc.turbo_sign_table(1, n_kv, d)

    def dec_turbo():
        for L in seqs:
            orc.attention_token_turbo(q, tc, table, 0, n_heads, 0, L, n_threads=threads)
        return sum(seqs) * n_kv * 2 * (d // 4 + d // 8 + 8)
    tb_rate, tb_s = _median_runs(dec_turbo)
    del tc

    kc, vc = orc.f16_bits(kf), orc.f16_bits(vf)

    def dec_f16():
        for L in seqs:
            orc.attention_token(q, kc, vc, orc.F16, n_heads, n_kv, d, 0, L, n_threads=threads)
        return sum(seqs) * n_kv * d * 2 * 2
    f16_rate, f16_s = _median_runs(dec_f16)
    del kc, vc, kf, vf
    # token-serial prefill: first M tokens of config 2
    M, Hq2, Hk2 = 1024, 32, 8
    qp = rng.standard_normal((M, Hq2 * d), dtype=np.float32)
    kp = rng.standard_normal((M, Hk2 * d), dtype=np.float32)
    vp = rng.standard_normal((M, Hk2 * d), dtype=np.float32)
    freqs = orc.rope_freqs(5e5, d)
    pairs = M * (M + 1) // 2

    def prefill():
        orc.prefill_layer(qp, kp, vp, n_heads=Hq2, n_kv_heads=Hk2, head_size=d, seq_len=M, fmt=orc.F16,
                          rope_dim=d, neox=False, rope_freqs_tab=freqs, rope_scale=1.0, n_threads=threads)
        return pairs
    pf_rate, pf_s = _median_runs(prefill)
    # serial DeltaNet scan: first T tokens of config 5
    T, H = 4096, 16
    qd = rng.standard_normal((T, H, d), dtype=np.float32)
    kd = rng.standard_normal((T, H, d), dtype=np.float32)
    vd = rng.standard_normal((T, H, d), dtype=np.float32)
    gate = (-0.1 * rng.random((T, H))).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((T, H))))).astype(np.float32)
    st0 = np.zeros((H, d, d), np.float32)

    def scan():
        orc.deltanet_scan(qd, kd, vd, gate, beta, st0, n_threads=threads)
        return T
    dn_rate, dn_s = _median_runs(scan)
    return {"value": round(q8_rate / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "cpu_model": _cpu_model(),
            "sample": f"oracle attention_token over the reference's Q8 KV storage (int8 rows + row scales, "
                      f"two-pass softmax, parallel over heads) on the {len(seqs)} config-3 sequences "
                      f"({sum(seqs)} keys), median of 3 runs after one warm-up ({q8_s:.2f} s timed)",
            "legs": {
                "decode_turbo": {"gbs": round(tb_rate / 1e9, 3),
                                 "f16_equivalent_gbs": round(tb_rate / 1e9 * (d * 2 * 2) / (2 * (d // 4 + d // 8 + 8)), 3),
                                 "sample": f"the same sequences over the Turbo storage, the reference's default "
                                           f"({tb_s:.2f} s timed)"},
                "decode_f16_raw": {"gbs": round(f16_rate / 1e9, 3),
                                   "sample": f"the same sequences over f16 raw KV rows: the GPU headline's format, "
                                             f"not a reference storage mode ({f16_s:.2f} s timed)"},
                "prefill_token_serial": {
                    "visible_pairs_per_s": round(pf_rate), "tflops": round(pf_rate * 4 * Hq2 * d / 1e12, 5),
                    "sample": f"first {M} tokens of config 2 (f16 KV, {pairs} (query, key) pairs per "
                              f"head, {pf_s:.2f} s timed)"},
                "deltanet_scan": {"tok_s": round(dn_rate, 1),
                                  "sample": f"the {T} tokens of config 5, 16 heads ({dn_s:.2f} s timed)"},
            }}


def deltanet_workload(dev, T, seed, H=16, d=128):
    """Config 5: bf16 q/k/v ~N(0,1) (L2-normed in-kernel), beta = sigmoid(N(0,1)),
    log-decay ~U(-0.1, 0), fp32 state; chunk-64 prefill."""
    import torch
    from gguf_runner_amd import ffi, ops
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    q = torch.randn((T, H, d), generator=g, device=dev, dtype=torch.bfloat16)
    k = torch.randn((T, H, d), generator=g, device=dev, dtype=torch.bfloat16)
    v = torch.randn((T, H, d), generator=g, device=dev, dtype=torch.bfloat16)
    beta = torch.sigmoid(torch.randn((T, H), generator=g, device=dev))
    gate = -0.1 * torch.rand((T, H), generator=g, device=dev)
    state = torch.zeros((H, d, d), device=dev)
    out = torch.empty((T, H, d), device=dev)
    algo = ffi.DELTANET_CHUNKED if T >= 64 else ffi.DELTANET_RECURRENT
    call = ops.DeltaNetCall(q, k, v, gate, beta, state, out, algo=algo)
    return call, (q, k, v, beta, gate, state, out)


def ssm_runstate_workload(T, seed, H=16, d=128, K=4):
    """Config 5's heads through the run-state DeltaNet calls with host rows, T tokens
    per call: gr_qwen3next_ssm_layer (conv + SiLU, q / k normalisation, gates, the
    chunked scan, gated RMSNorm; host qkv / z / gate rows in, ssm_proj rows out) and
    gr_qwen3next_prefill (host q / k / v / gate / beta rows in, outputs out)."""
    from gguf_runner_amd import runtime as rt
    rng = np.random.default_rng(seed)
    conv_dim = 3 * H * d
    p = rt.Config(n_layers=1, n_heads=1, n_kv_heads=1, head_dim=128, seq_len=8, ssm_n_heads=H,
                  ssm_head_dim=d, ssm_n_k_heads=H, ssm_conv_kernel=K, rms_norm_eps=1e-6,
                  ssm_conv1d=(0.3 * rng.standard_normal((1, conv_dim, K))).astype(np.float32),
                  ssm_a=-rng.uniform(0.2, 1.2, (1, H)).astype(np.float32),
                  ssm_dt_bias=(0.1 * rng.standard_normal((1, H))).astype(np.float32),
                  ssm_norm=(1 + 0.1 * rng.standard_normal((1, d))).astype(np.float32))
    s = rt.malloc_run_state(p)
    qkv = rng.standard_normal((T, conv_dim)).astype(np.float32)
    z = rng.standard_normal((T, H * d)).astype(np.float32)
    ga = rng.standard_normal((T, 2 * H)).astype(np.float32)
    q, k, v = (rng.standard_normal((T, H * d)).astype(np.float32) for _ in range(3))
    gate = rng.uniform(-0.1, 0, (T, H)).astype(np.float32)
    beta = rng.uniform(0, 1, (T, H)).astype(np.float32)
    layer = lambda: rt.qwen3next_ssm_layer(p, s, 0, qkv, z, ga)
    prefill = lambda: rt.qwen3next_prefill(p, s, 0, q, k, v, gate, beta)
    return layer, prefill, (p, s)


def runstate_token_us(steps):
    """The drop-in per-token call gr_attention_layer_token (QK norm, RoPE, KV write and
    attention of one token over 1024 cached keys; host q / k / v rows in, xb out) at
    config 1's heads (16 / 8, d128) over each cache format: us per call, host wall
    clock of synchronous calls (the best of three runs of `steps` calls)."""
    from gguf_runner_amd import ffi, runtime as rt
    out = {}
    for name, kv in (("f32", ffi.DTYPE_F32), ("f16", ffi.DTYPE_F16), ("q8", ffi.DTYPE_Q8),
                     ("turbo", ffi.DTYPE_TURBO)):
        p = rt.Config(n_layers=1, n_heads=16, n_kv_heads=8, head_dim=128, seq_len=2048, kv_dtype=kv,
                      rope_mode=ffi.ROPE_NEOX, rope_dim=128, rope_theta=1e6)
        s = rt.malloc_run_state(p)
        rng = np.random.default_rng(1)
        for a in (s.q, s.k, s.v):
            a[:] = rng.standard_normal(a.shape).astype(np.float32)
        for pos in range(1024):
            rt.attention_layer_token(p, s, 0, pos)
        best = None
        for _ in range(3):
            t0 = time.perf_counter()
            for _ in range(steps):
                rt.attention_layer_token(p, s, 0, 1023)
            us = (time.perf_counter() - t0) / steps * 1e6
            best = us if best is None else min(best, us)
        out[name] = round(best, 1)
        del s
    return out


def run_one(args, dev, stream, lens) -> int:
    """A single workload, for rocprofv3 runs; prints one short JSON line."""
    import torch
    res = {"only": args.only, "steps": args.steps}
    if args.only in ("decode3", "decode32k"):
        ls = lens if args.only == "decode3" else [32768] * 16
        call, nbytes, keep = rotating(lambda sd: decode_workload(dev, ls, sd), 3)
        ms, _ = _timed(call, args.steps, args.warmup, stream)
        res.update(ms=ms, gbs=nbytes / (ms * 1e-3) / 1e9, bytes=nbytes)
    elif args.only == "decode32k_turbo":
        call, nbytes, keep = rotating(lambda sd: decode_turbo_workload(dev, [32768] * 16, sd), 35)
        ms, _ = _timed(call, args.steps, args.warmup, stream)
        res.update(ms=ms, gbs=nbytes / (ms * 1e-3) / 1e9, bytes=nbytes,
                   f16_equiv_gbs=16 * 32768 * 4 * 128 * 4 / (ms * 1e-3) / 1e9)
    elif args.only in ("decode32k_q8", "decode32k_q8b"):
        blk = args.only.endswith("b")
        call, nbytes, keep = rotating(lambda sd: decode_q8_workload(dev, [32768] * 16, sd, block=blk), 34)
        ms, _ = _timed(call, args.steps, args.warmup, stream)
        res.update(ms=ms, gbs=nbytes / (ms * 1e-3) / 1e9, bytes=nbytes)
    elif args.only in ("prefill2k", "prefill8k"):
        S = 2048 if args.only == "prefill2k" else 8192
        call, flops, keep = prefill_workload(dev, S, 8)
        ms, _ = _timed(call, args.steps, args.warmup, stream)
        res.update(ms=ms, tflops=flops / (ms * 1e-3) / 1e12, gflop=flops / 1e9)
    elif args.only == "decode_c1":
        # config 1: Qwen3-0.6B-shaped single-layer decode, f32 KV, 1024 keys
        call, nbytes, keep = rotating(
            lambda sd: decode_workload(dev, [1024], sd, n_heads=16, n_kv=8, kv_dtype=torch.float32), 41)
        ms, _ = _timed(call, args.steps, args.warmup, stream)
        res.update(ms=ms, gbs=nbytes / (ms * 1e-3) / 1e9, bytes=nbytes)
    elif args.only == "decode_c4":
        # config 4: one decode step after the 8192-token prefill, 5 local + 1 global layer
        for key, (b, e) in (("local", (8193 - 1024, 8193)), ("global", (0, 8193))):
            call, nbytes, keep = rotating(
                lambda sd: decode_workload(dev, [e], sd, n_heads=8, n_kv=4, d=256, kv_dtype=torch.bfloat16,
                                           starts=[b]), 43)
            ms, _ = _timed(call, args.steps, args.warmup, stream)
            res[key] = {"ms": ms, "gbs": nbytes / (ms * 1e-3) / 1e9, "bytes": nbytes}
            del keep, call
        res["step_ms"] = 5 * res["local"]["ms"] + res["global"]["ms"]
    elif args.only == "decode_small":
        # small 16-bit decode calls (the fixed-grid plan for short contexts): us per call
        shapes = (("1x1024 bf16 8/4 d256", [1024], 8, 4, 256, torch.bfloat16),
                  ("2x1024 bf16 16/8 d128", [1024] * 2, 16, 8, 128, torch.bfloat16),
                  ("1x512 f16 16/8 d128", [512], 16, 8, 128, torch.float16),
                  ("8x1024 f16 32/8 d128", [1024] * 8, 32, 8, 128, torch.float16),
                  ("1x4096 f16 32/8 d128", [4096], 32, 8, 128, torch.float16),
                  ("4x2048 f16 32/4 d128", [2048] * 4, 32, 4, 128, torch.float16))
        for name, ls, H, G, d, dt in shapes:
            call, nbytes, keep = rotating(
                lambda sd: decode_workload(dev, ls, sd, n_heads=H, n_kv=G, d=d, kv_dtype=dt), 5)
            ms, _ = _timed(call, args.steps, args.warmup, stream)
            res[name] = round(ms * 1e3, 2)
            del keep, call
    elif args.only == "decode_small_turbo":
        # small decode calls over a Turbo cache (the reference's default format): us per call
        shapes = (("1x512 16/8", [512], 16, 8), ("1x1024 16/8", [1024], 16, 8), ("1x4096 16/8", [4096], 16, 8),
                  ("1x8192 32/8", [8192], 32, 8), ("4x2048 32/4", [2048] * 4, 32, 4),
                  ("16x1024 32/4", [1024] * 16, 32, 4), ("1x8192 64/4", [8192], 64, 4))
        for name, ls, H, G in shapes:
            call, nbytes, keep = rotating(lambda sd: decode_turbo_workload(dev, ls, sd, n_heads=H, n_kv=G), 7)
            ms, _ = _timed(call, args.steps, args.warmup, stream)
            res[name] = round(ms * 1e3, 2)
            del keep, call
    elif args.only in ("decode_small_q8", "decode_small_q8b"):
        # small decode calls over a Q8 cache (row or block scales): us per call
        blk = args.only.endswith("b")
        shapes = (("1x1024 16/8", [1024], 16, 8, 128), ("1x4096 16/8", [4096], 16, 8, 128),
                  ("1x8192 32/8", [8192], 32, 8, 128), ("4x2048 32/4", [2048] * 4, 32, 4, 128),
                  ("1x1024 8/4 d256", [1024], 8, 4, 256))
        for name, ls, H, G, d in shapes:
            call, nbytes, keep = rotating(
                lambda sd: decode_q8_workload(dev, ls, sd, n_heads=H, n_kv=G, d=d, block=blk), 3)
            ms, _ = _timed(call, args.steps, args.warmup, stream)
            res[name] = round(ms * 1e3, 2)
            del keep, call
    elif args.only == "runstate_token":
        res.update(runstate_token_us(args.steps))
    elif args.only == "runstate_chunk":
        # gr_prefill_attention_chunk with the reference's short chunks (16 and 64 rows at
        # base_pos 1024, host rows in and out), 16 / 8 and 32 / 8 heads, d128: us per call
        from gguf_runner_amd import ffi, runtime as rt
        for name, kv in (("f16", ffi.DTYPE_F16), ("q8", ffi.DTYPE_Q8), ("turbo", ffi.DTYPE_TURBO)):
            for H, G in ((16, 8), (32, 8)):
                p = rt.Config(n_layers=1, n_heads=H, n_kv_heads=G, head_dim=128, seq_len=2048, kv_dtype=kv,
                              rope_mode=ffi.ROPE_NEOX, rope_dim=128, rope_theta=1e6)
                s = rt.malloc_run_state(p)
                rng = np.random.default_rng(1)
                for m in (16, 64):
                    q = rng.standard_normal((m, p.q_dim)).astype(np.float32)
                    k = rng.standard_normal((m, p.kv_dim)).astype(np.float32)
                    v = rng.standard_normal((m, p.kv_dim)).astype(np.float32)
                    xb = np.zeros((m, p.q_dim), np.float32)
                    for _ in range(3):
                        rt.prefill_attention_chunk(p, s, 0, 1024, q, k, v, out=xb)
                    best = None
                    for _ in range(3):
                        t0 = time.perf_counter()
                        for _ in range(args.steps):
                            rt.prefill_attention_chunk(p, s, 0, 1024, q, k, v, out=xb)
                        us = (time.perf_counter() - t0) / args.steps * 1e6
                        best = us if best is None else min(best, us)
                    res[f"{name} {H}/{G} m{m}"] = round(best, 1)
                del s
    elif args.only in ("prefill8k_bf16", "prefill8k_d64_bf16"):
        # bf16 caches (the f16 MFMA path on an exact f16 copy of the rows)
        if args.only == "prefill8k_bf16":
            call, flops, keep = prefill_workload(dev, 8192, 8, dtype=torch.bfloat16)
        else:
            call, flops, keep = prefill_d64_workload(dev, 8192, 64, dtype=torch.bfloat16)
        ms, _ = _timed(call, args.steps, args.warmup, stream)
        res.update(ms=ms, tflops=flops / (ms * 1e-3) / 1e12, gflop=flops / 1e9)
    elif args.only in ("prefill2k_d64", "prefill8k_d64"):
        S = 2048 if args.only == "prefill2k_d64" else 8192
        call, flops, keep = prefill_d64_workload(dev, S, 64)
        ms, _ = _timed(call, args.steps, args.warmup, stream)
        res.update(ms=ms, tflops=flops / (ms * 1e-3) / 1e12, gflop=flops / 1e9)
    elif args.only in ("prefill2k_q8", "prefill2k_q8b", "prefill2k_turbo"):
        # synchronous host-buffer calls: the wall time per call includes the PCIe
        # copies; the kernels' own times come from a kernel trace of this run
        call, flops, keep = prefill_q8_workload(2048, 8, args.only.endswith("b"),
                                                turbo=args.only.endswith("turbo"))
        _, wall = _timed(call, args.steps, args.warmup, stream)
        res.update(call_ms=wall, call_tflops=flops / (wall * 1e-3) / 1e12, gflop=flops / 1e9)
    elif args.only == "ssm_token":
        # per-token run-state DeltaNet calls (config 5 heads): the SSM layer with one
        # token (conv, gates, the state step, gated RMSNorm) and the bare state step;
        # us per call (host wall clock, synchronous calls)
        from gguf_runner_amd import runtime as rt
        layer, _, keep = ssm_runstate_workload(1, 9)
        p, s = keep
        rng = np.random.default_rng(3)
        H, d = p.ssm_n_heads, p.ssm_head_dim
        q, k, v = (rng.standard_normal(H * d).astype(np.float32) for _ in range(3))
        gq = rng.uniform(0.9, 1.0, H).astype(np.float32)
        bq = rng.uniform(0, 1, H).astype(np.float32)
        step = lambda: rt.qwen3next_state_step(p, s, 0, q, k, v, gq, bq)
        for name, fn in (("ssm_layer_T1", layer), ("state_step", step)):
            for _ in range(5):
                fn()
            best = None
            for _ in range(3):
                t0 = time.perf_counter()
                for _ in range(args.steps):
                    fn()
                us = (time.perf_counter() - t0) / args.steps * 1e6
                best = us if best is None else min(best, us)
            res[name] = round(best, 1)
    elif args.only == "ssm2k":
        # synchronous host-buffer calls, 2048 tokens each (wall time incl. PCIe copies)
        layer, prefill, keep = ssm_runstate_workload(2048, 9)
        _, lw = _timed(layer, args.steps, args.warmup, stream)
        _, pw = _timed(prefill, args.steps, args.warmup, stream)
        res.update(ssm_layer_call_ms=lw, prefill_call_ms=pw, tokens=2048)
    elif args.only == "prefill8k_d256":
        # config 4 shape (Gemma-3-4B): the sliding-window (1024) and the global layer
        for W, key in ((1024, "local"), (0, "global")):
            call, flops, keep = config4_prefill_workload(dev, W)
            ms, _ = _timed(call, args.steps, args.warmup, stream)
            res[key] = {"ms": ms, "tflops": flops / (ms * 1e-3) / 1e12, "gflop": flops / 1e9}
            del keep, call
    elif args.only == "encoder":
        call, flops, keep = encoder_workload(dev, stream)
        ms, _ = _timed(call, args.steps, args.warmup, stream)
        res.update(ms=ms, tflops=flops / (ms * 1e-3) / 1e12, gflop=flops / 1e9)
    elif args.only == "deltanet":
        pcall, keep = deltanet_workload(dev, 4096, 5)
        ms, _ = _timed(pcall, args.steps, args.warmup, stream)
        dcall, keep2 = deltanet_workload(dev, 1, 6)
        dms, _ = _timed(dcall, args.steps, args.warmup, stream)
        res.update(prefill_ms=ms, prefill_tok_s=4096 / (ms * 1e-3), decode_step_ms=dms,
                   decode_state_gbs=2 * 16 * 128 * 128 * 4 / (dms * 1e-3) / 1e9)
    else:  # copy: calibration of the HBM byte counters with a plain 1 GiB device copy
        a = torch.empty(1 << 28, dtype=torch.float32, device=dev)
        b = torch.empty_like(a)
        a.fill_(1.0)
        ms, _ = _timed(lambda: b.copy_(a), args.steps, args.warmup, stream)
        res.update(ms=ms, bytes_read=a.numel() * 4, bytes_written=b.numel() * 4,
                   gbs=2 * a.numel() * 4 / (ms * 1e-3) / 1e9)
    print(json.dumps(res), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only", default="all",
                    choices=["all", "decode3", "decode32k", "decode_c1", "decode_c4", "decode_small", "decode_small_turbo", "decode_small_q8", "decode_small_q8b", "runstate_token", "runstate_chunk", "decode32k_q8", "decode32k_q8b", "decode32k_turbo",
                             "prefill2k", "prefill8k", "prefill8k_bf16", "prefill2k_d64", "prefill8k_d64", "prefill8k_d64_bf16", "prefill2k_q8", "prefill2k_q8b", "prefill2k_turbo", "prefill8k_d256", "encoder", "deltanet", "ssm2k", "ssm_token",
                             "copy"],
                    help="run one workload (for profiling); prints a short JSON line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "the attention path shards over heads and sequences without communication, "
              "so no multi-GPU figure is produced", file=sys.stderr)
        return 2

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import __graft_entry__ as ge
    ge.load_package()
    import torch
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()

    rng = np.random.default_rng(1003)
    lens = rng.integers(1024, 32768, size=16, endpoint=True).tolist()

    if args.only != "all":
        return run_one(args, dev, stream, lens)

    # headline: config 3 decode (ragged)
    dcall, dbytes, _keep_d = rotating(lambda sd: decode_workload(dev, lens, sd), 3)
    dec_ms, dec_wall = _timed(dcall, args.steps, args.warmup, stream)
    dec_gbs = dbytes / (dec_ms * 1e-3) / 1e9
    del _keep_d, dcall

    # decode target run: all sequences at 32768 keys
    tcall, tbytes, _keep_t = rotating(lambda sd: decode_workload(dev, [32768] * 16, sd), 33)
    t_ms, _ = _timed(tcall, args.steps, args.warmup, stream)
    t_gbs = tbytes / (t_ms * 1e-3) / 1e9
    del _keep_t, tcall

    # the same target run over a Q8 cache (row scales, the reference's Q8 format)
    qcall, qbytes, _keep_q = rotating(lambda sd: decode_q8_workload(dev, [32768] * 16, sd), 34)
    q_ms, _ = _timed(qcall, args.steps, args.warmup, stream)
    q_gbs = qbytes / (q_ms * 1e-3) / 1e9
    del _keep_q, qcall

    # and over a Turbo cache (the reference's default KV format)
    ucall, ubytes, _keep_u = rotating(lambda sd: decode_turbo_workload(dev, [32768] * 16, sd), 35)
    u_ms, _ = _timed(ucall, args.steps, args.warmup, stream)
    u_gbs = ubytes / (u_ms * 1e-3) / 1e9
    del _keep_u, ucall

    pre = {}
    for S, seed in ((2048, 2), (8192, 8)):
        pcall, flops, _keep_p = prefill_workload(dev, S, seed)
        p_ms, _ = _timed(pcall, max(5, args.steps // 5), 2, stream)
        tf = flops / (p_ms * 1e-3) / 1e12
        pre[S] = {"tflops": round(tf, 2), "ms": round(p_ms, 4),
                  "frac_of_mfma_peak": round(tf / MFMA_F16_PEAK_TFLOPS, 4), "gflop": round(flops / 1e9, 3)}
        del _keep_p, pcall
    tf8 = pre[8192]["tflops"]
    # the prefill half of the metric: the 8k target run, flat, with its roofline block
    prefill_line = dict(pre[8192])
    prefill_line.update({
        "value": tf8, "unit": "TFLOP/s",
        "workload": "config 2 shape at S = 8192: causal GQA prefill, 32 Q / 8 KV heads, d128, f16 Q/K/V, "
                    "adjacent RoPE theta 5e5 fused on load",
        "roofline": {"bound": "mfma", "achieved": tf8, "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tf8 / MFMA_F16_PEAK_TFLOPS, 4),
                     "kernel": "gr_prefill_attention, S = 8192, 32 / 8 heads, d128, f16: qkv_prep_kernel + "
                               "prefill_kernel<f16, 128, 8>, hipEvent-timed (4 * Hq * d * sum visible FLOP)"}})

    # config 1: Qwen3-0.6B-shaped single-layer decode, f32 KV, 1024 keys (latency-bound)
    c1call, c1bytes, _keep_c1 = rotating(
        lambda sd: decode_workload(dev, [1024], sd, n_heads=16, n_kv=8, kv_dtype=torch.float32), 41)
    c1_ms, _ = _timed(c1call, args.steps, args.warmup, stream)
    del _keep_c1, c1call

    # config 4: Gemma-3-4B-shaped, 5 local (W = 1024) : 1 global layers, bf16, d256
    c4 = {}
    for key, W in (("local", 1024), ("global", 0)):
        ccall, cflops, _keep_c = config4_prefill_workload(dev, W)
        c_ms, _ = _timed(ccall, max(5, args.steps // 5), 2, stream)
        c4[f"prefill_{key}_layer"] = {"ms": round(c_ms, 4), "tflops": round(cflops / (c_ms * 1e-3) / 1e12, 2),
                                      "gflop": round(cflops / 1e9, 3)}
        del _keep_c, ccall
    six = 5 * c4["prefill_local_layer"]["ms"] + c4["prefill_global_layer"]["ms"]
    six_flops = 1e9 * (5 * c4["prefill_local_layer"]["gflop"] + c4["prefill_global_layer"]["gflop"])
    c4["prefill_6_layers"] = {"ms": round(six, 4), "tflops": round(six_flops / (six * 1e-3) / 1e12, 2),
                              "frac_of_mfma_peak": round(six_flops / (six * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)}
    # one decode step after the 8192-token prefill: position 8192 sees 1024 keys in a
    # local layer and 8193 in the global one
    dsteps = {}
    for key, (b, e) in (("local", (8193 - 1024, 8193)), ("global", (0, 8193))):
        dcall4, dbytes4, _keep_d4 = rotating(
            lambda sd: decode_workload(dev, [e], sd, n_heads=8, n_kv=4, d=256, kv_dtype=torch.bfloat16,
                                       starts=[b]), 43)
        d4_ms, _ = _timed(dcall4, args.steps, args.warmup, stream)
        dsteps[key] = (d4_ms, dbytes4)
        del _keep_d4, dcall4
    step_ms = 5 * dsteps["local"][0] + dsteps["global"][0]
    step_bytes = 5 * dsteps["local"][1] + dsteps["global"][1]
    c4["decode_step_6_layers"] = {"ms": round(step_ms, 5), "gbs": round(step_bytes / (step_ms * 1e-3) / 1e9, 2),
                                  "bytes": step_bytes,
                                  "local_layer_ms": round(dsteps["local"][0], 5),
                                  "global_layer_ms": round(dsteps["global"][0], 5)}

    line = {
        "metric": METRIC,
        "value": round(dec_gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1) Q/K/V, no checkpoint)",
        "config": {"workload": "config 3: Qwen3-30B-A3B-shaped split-K decode, 16 seqs, ragged "
                               "L~U[1024,32768] (seed 1003), 32 Q / 4 KV heads, d128, f16 KV",
                   "seq_lens_sum": int(sum(lens)), "bytes_per_step": dbytes},
        "roofline": {"bound": "hbm", "achieved": round(dec_gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(dec_gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(),
                     "kernel": "gr_decode_attention (split kernel + combine), hipEvent-timed"},
        "decode_32k": {"gbs": round(t_gbs, 2), "ms": round(t_ms, 5),
                       "frac_of_hbm": round(t_gbs / HBM_PEAK_GBS, 4), "bytes": tbytes},
        "decode_32k_q8": {"gbs": round(q_gbs, 2), "ms": round(q_ms, 5),
                          "frac_of_hbm": round(q_gbs / HBM_PEAK_GBS, 4), "bytes": qbytes},
        "decode_32k_turbo": {"gbs": round(u_gbs, 2), "ms": round(u_ms, 5), "bytes": ubytes,
                             "f16_equivalent_gbs": round(tbytes / (u_ms * 1e-3) / 1e9, 2)},
        "prefill": prefill_line,
        "prefill_tflops": tf8,
        "prefill_frac_of_mfma_peak": round(tf8 / MFMA_F16_PEAK_TFLOPS, 4),
        "prefill_config2_s2048": pre[2048],
        "config1_decode": {"ms": round(c1_ms, 5), "gbs": round(c1bytes / (c1_ms * 1e-3) / 1e9, 2),
                           "bytes": c1bytes, "shape": "1 seq, 16 Q / 8 KV heads, d128, 1024 keys, f32 KV"},
        "config4": c4,
        "wall_ms_per_step": round(dec_wall, 5),
    }

    # config 5: gated DeltaNet, 4096-token chunked prefill and one recurrent step
    pcall, _keep_d = deltanet_workload(dev, 4096, 5)
    d_ms, _ = _timed(pcall, max(5, args.steps // 5), 2, stream)
    scall, _keep_s = deltanet_workload(dev, 1, 6)
    s_ms, _ = _timed(scall, args.steps, args.warmup, stream)
    line["deltanet"] = {"prefill_ms": round(d_ms, 4), "prefill_tok_s": round(4096 / (d_ms * 1e-3)),
                        "decode_step_ms": round(s_ms, 5)}
    del _keep_d, _keep_s, pcall, scall

    # prefill of a 2048-token chunk over Q8 and Turbo run-state caches (host q / k / v
    # rows: the wall time includes their upload and the download of the outputs)
    qpre = {}
    for key, blk, tb in (("q8", False, False), ("turbo", False, True)):
        qcall, flops, _keep_q = prefill_q8_workload(2048, 8, blk, turbo=tb)
        _, w_ms = _timed(qcall, max(5, args.steps // 5), 2, stream)
        qpre[key] = {"call_ms": round(w_ms, 4), "gflop": round(flops / 1e9, 3)}
        del _keep_q, qcall
    line["prefill_2048_quantised_cache"] = qpre

    ecall, eflops, _keep_e = encoder_workload(dev, stream)
    e_ms, _ = _timed(ecall, max(5, args.steps // 5), 2, stream)
    line["encoder_siglip"] = {"ms": round(e_ms, 4), "tflops": round(eflops / (e_ms * 1e-3) / 1e12, 2)}
    del _keep_e, ecall

    line["runstate_token_us"] = runstate_token_us(max(50, args.steps))

    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(lens)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
