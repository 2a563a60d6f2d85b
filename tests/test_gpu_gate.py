"""The Qwen3.5 packed-q output gate (qwen3next_packed_q_gate: inference.rs:3509-3519
after attention_token in decode, 3003-3016 in the batched prefill) fused into the
kernels that write the attention output: out = finite_or_zero(out * sigmoid(g))
(sigmoid_mul_inplace, math.rs:396-403, restated as oracle sigmoid_mul and pinned on
the CPU).  The gate rows are the reference's packed [q_h | gate_h] projection rows:
head stride 2 * head_dim, row stride 2 * n_heads * head_dim.

Tolerances (written here, fixed before measuring):
  f32 decode against the oracle's attention_token + sigmoid_mul: max abs 1e-5;
  16-bit and Turbo paths against the oracle's gate applied to the same kernel's
  ungated output (the gate multiply is the only difference): relative 1e-6
  (the device expf and the host libm exp may differ by an ulp or two).
"""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def _packed_gate(rng, rows, n_heads, d, dev):
    """Packed [q | gate] rows; returns (device tensor, host gate [rows][n_heads][d])."""
    packed = rng.standard_normal((rows, n_heads, 2 * d)).astype(np.float32) * 3
    packed[0, 0, d + 5] = np.nan   # a NaN gate: the element becomes 0
    packed[-1, -1, d + 7] = 200.0  # saturated: the element passes unchanged
    return torch.from_numpy(packed).to(dev), packed[:, :, d:]


def _gate_kw(packed_dev, n_heads, d):
    return dict(out_gate=packed_dev[:, :, d:], out_gate_row_stride=2 * n_heads * d,
                out_gate_head_stride=2 * d)


def _assert_gated(got, ungated, gate, orc, rel=1e-6):
    exp = orc.sigmoid_mul(ungated, gate)
    err = np.abs(got - exp)
    assert np.all(err <= rel * np.abs(exp) + 1e-30), float(err.max())


def _caches(rng, n_seq, seq_len, n_kv, d, fmt, orc, dev):
    kf = rng.standard_normal((n_seq, seq_len, n_kv * d), dtype=np.float32)
    vf = rng.standard_normal((n_seq, seq_len, n_kv * d), dtype=np.float32)
    if fmt == orc.F32:
        kc, vc = kf, vf
        kt, vt = torch.from_numpy(kc), torch.from_numpy(vc)
    else:
        conv = orc.f16_bits if fmt == orc.F16 else orc.bf16_bits
        tdt = torch.float16 if fmt == orc.F16 else torch.bfloat16
        kc, vc = conv(kf), conv(vf)
        kt = torch.from_numpy(kc.view(np.int16)).view(tdt)
        vt = torch.from_numpy(vc.view(np.int16)).view(tdt)
    return kc, vc, kt.reshape(n_seq, seq_len, n_kv, d).to(dev), vt.reshape(n_seq, seq_len, n_kv, d).to(dev)


@pytest.mark.parametrize("fmt_name", ["F32", "F16", "BF16"])
def test_decode_output_gate(orc, dev, fmt_name):
    """Three sequences (16 Q / 8 KV heads, d128) through the VALU (f32) and MFMA
    (16-bit) split kernels; the gate is applied in the combine kernel."""
    from gguf_runner_amd import ops
    fmt = getattr(orc, fmt_name)
    rng = np.random.default_rng(77)
    n_seq, n_heads, n_kv, d, seq_len = 3, 16, 8, 128, 700
    starts, ends = [0, 100, 0], [700, 650, 33]
    kc, vc, kt, vt = _caches(rng, n_seq, seq_len, n_kv, d, fmt, orc, dev)
    q = rng.standard_normal((n_seq, n_heads, d), dtype=np.float32)
    packed, gate = _packed_gate(rng, n_seq, n_heads, d, dev)
    qt = torch.from_numpy(q).to(dev)
    st = torch.tensor(starts, dtype=torch.int32, device=dev)
    en = torch.tensor(ends, dtype=torch.int32, device=dev)
    outs = []
    for kw in ({}, _gate_kw(packed, n_heads, d)):
        out = torch.empty_like(qt)
        ops.DecodeCall(qt, kt, vt, st, en, out, max_kv_len=700, **kw)()
        outs.append(out)
    torch.cuda.synchronize()
    ungated, got = (o.cpu().numpy() for o in outs)
    _assert_gated(got, ungated, gate, orc)
    assert got[0, 0, 5] == 0.0 and got[-1, -1, 7] == ungated[-1, -1, 7]
    if fmt == orc.F32:  # the reference's order: attention_token, then sigmoid_mul
        ref = np.stack([orc.attention_token(q[s].reshape(-1), kc[s], vc[s], fmt, n_heads, n_kv, d,
                                            starts[s], ends[s], n_threads=orc.env_threads())
                        .reshape(n_heads, d) for s in range(n_seq)])
        assert float(np.abs(got - orc.sigmoid_mul(ref, gate)).max()) <= 1e-5


def test_turbo_decode_output_gate(orc, dev):
    """Turbo cache (the reference's default KV format): the gate in the Turbo combine."""
    from gguf_runner_amd import ops
    from test_gpu_turbo import _oracle_cache
    rng = np.random.default_rng(78)
    n_seq, n_heads, n_kv, d, seq_len, layer = 2, 16, 8, 128, 300, 1
    kv_dim = n_kv * d
    table = orc.turbo_sign_table(2, n_kv, d)
    caches = [_oracle_cache(orc, rng.standard_normal((seq_len, kv_dim), dtype=np.float32),
                            rng.standard_normal((seq_len, kv_dim), dtype=np.float32), table, layer, n_kv, d)
              for _ in range(n_seq)]
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    stack = lambda name, w: T(np.stack([getattr(c, name).reshape(seq_len, w) for c in caches]))
    q = T(rng.standard_normal((n_seq, n_heads, d), dtype=np.float32))
    packed, gate = _packed_gate(rng, n_seq, n_heads, d, dev)
    outs = []
    for gated in (False, True):
        out = torch.empty((n_seq, n_heads, d), device=dev)
        call = ops.TurboDecodeCall(q, stack("kbase", kv_dim // 4), stack("vbase", kv_dim // 4),
                                   stack("ksign", kv_dim // 8), stack("vsign", kv_dim // 8),
                                   stack("kscale", n_kv), stack("vscale", n_kv), stack("kres", n_kv),
                                   stack("vres", n_kv), T(table), layer,
                                   torch.tensor([0, 17], dtype=torch.int32, device=dev),
                                   torch.tensor([300, 250], dtype=torch.int32, device=dev), out,
                                   max_kv_len=300)
        if gated:
            ops._set_gate(call.args, packed[:, :, d:], 2 * n_heads * d, 2 * d)
        call()
        outs.append(out)
    torch.cuda.synchronize()
    ungated, got = (o.cpu().numpy() for o in outs)
    _assert_gated(got, ungated, gate, orc)


@pytest.mark.parametrize("fmt_name,d", [("F16", 128), ("BF16", 128), ("BF16", 256)])
def test_prefill_output_gate(orc, dev, fmt_name, d):
    """gr_prefill_attention with the gate of every token row in the kernel's epilogue
    (the batched prefill's per-token gate, inference.rs:3003-3016)."""
    from gguf_runner_amd import ops
    fmt = getattr(orc, fmt_name)
    tdt = torch.float16 if fmt == orc.F16 else torch.bfloat16
    rng = np.random.default_rng(79 + d)
    m, n_heads, n_kv = 300, 8, 2
    mk = lambda *s: torch.from_numpy(rng.standard_normal(s).astype(np.float32)).to(dev).to(tdt)
    q, k, v = mk(m, n_heads, d), mk(m, n_kv, d), mk(m, n_kv, d)
    packed, gate = _packed_gate(rng, m, n_heads, d, dev)
    outs = []
    for kw in ({}, _gate_kw(packed, n_heads, d)):
        kc = torch.zeros((m, n_kv, d), dtype=tdt, device=dev)
        vc = torch.zeros_like(kc)
        out = torch.empty((m, n_heads, d), device=dev)
        ops.PrefillCall(q, k, v, kc, vc, out, **kw)()
        outs.append(out)
    torch.cuda.synchronize()
    ungated, got = (o.cpu().numpy() for o in outs)
    _assert_gated(got, ungated, gate, orc)
