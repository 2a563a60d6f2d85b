"""Gated DeltaNet parity: gr_deltanet_attention (recurrent and chunk-64 HIP paths)
vs the CPU oracle's token-serial recurrence (qwen3next_state_head_step,
reference math.rs:492-546, per token as inference.rs:2866-2885).

Tolerance (fp32 state path, fixed before measuring): max |gpu - ref| <= 1e-5 for
outputs and final state."""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _inputs(orc, T, H, d, seed, fmt):
    rng = np.random.default_rng(seed)
    conv = {orc.F32: lambda x: x, orc.F16: orc.f16_bits, orc.BF16: orc.bf16_bits}[fmt]
    q = conv(rng.standard_normal((T, H, d), dtype=np.float32))
    k = conv(rng.standard_normal((T, H, d), dtype=np.float32))
    v = conv(rng.standard_normal((T, H, d), dtype=np.float32))
    beta = (1.0 / (1.0 + np.exp(-rng.standard_normal((T, H))))).astype(np.float32)
    gate = rng.uniform(-0.1, 0.0, (T, H)).astype(np.float32)
    return q, k, v, gate, beta


def _to_dev(x, fmt, orc, dev):
    if fmt == orc.F32:
        return torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    dt = torch.float16 if fmt == orc.F16 else torch.bfloat16
    return torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).view(dt).to(dev)


def _run(orc, dev, T, H, d, seed, fmt, algo, state0=None, chunks=None):
    from gguf_runner_amd import ops
    q, k, v, gate, beta = _inputs(orc, T, H, d, seed, fmt)
    S0 = np.zeros((H, d, d), np.float32) if state0 is None else state0
    ref, Sref = orc.deltanet_scan(orc.upcast(q, fmt), orc.upcast(k, fmt), orc.upcast(v, fmt),
                                  gate, beta, S0, eps=1e-6, n_threads=orc.env_threads())
    st = torch.from_numpy(S0.copy()).to(dev)
    qd, kd, vd = (_to_dev(x, fmt, orc, dev) for x in (q, k, v))
    gd = torch.from_numpy(gate).to(dev)
    bd = torch.from_numpy(beta).to(dev)
    out = torch.empty((T, H, d), dtype=torch.float32, device=dev)
    b = 0
    for c in (chunks or [T]):
        o = torch.empty((c, H, d), dtype=torch.float32, device=dev)
        ops.DeltaNetCall(qd[b:b + c].contiguous(), kd[b:b + c].contiguous(),
                         vd[b:b + c].contiguous(), gd[b:b + c].contiguous(),
                         bd[b:b + c].contiguous(), st, o, algo=algo)()
        out[b:b + c] = o
        b += c
    torch.cuda.synchronize()
    return out.cpu().numpy(), ref, st.cpu().numpy(), Sref


@pytest.mark.parametrize("algo", [1, 2])
def test_config5_deltanet_prefill_4096(orc, dev, algo):
    """Config 5: 16 heads, d128, fp32 state, 4096-token prefill (chunk 64), bf16 inputs,
    q/k L2-normed in-kernel, beta = sigmoid(N(0,1)), log-decay ~U(-0.1, 0)."""
    got, ref, S, Sref = _run(orc, dev, 4096, 16, 128, 1005, orc.BF16, algo)
    assert float(np.abs(got - ref).max()) <= TOL, np.abs(got - ref).max()
    assert float(np.abs(S - Sref).max()) <= TOL, np.abs(S - Sref).max()


def test_config5_deltanet_decode_steps_after_prefill(orc, dev):
    """Config 5 as one sequence: the 4096-token chunked prefill, then 512 single-token
    recurrent decode steps on the state it leaves, against one token-serial scan
    over all 4608 tokens."""
    got, ref, S, Sref = _run(orc, dev, 4096 + 512, 16, 128, 1015, orc.BF16, 0,
                             chunks=[4096] + [1] * 512)
    assert float(np.abs(got - ref).max()) <= TOL, np.abs(got - ref).max()
    assert float(np.abs(S - Sref).max()) <= TOL, np.abs(S - Sref).max()


@pytest.mark.parametrize("T", [1, 5, 63, 64, 65, 200])
@pytest.mark.parametrize("algo", [1, 2])
def test_deltanet_ragged_lengths(orc, dev, T, algo):
    """Partial chunks (padded with beta = 0, gate = 0) and short sequences, f32 inputs,
    non-zero initial state."""
    rng = np.random.default_rng(T)
    S0 = (0.1 * rng.standard_normal((4, 128, 128))).astype(np.float32)
    got, ref, S, Sref = _run(orc, dev, T, 4, 128, 77 + T, orc.F32, algo, state0=S0)
    assert float(np.abs(got - ref).max()) <= TOL, np.abs(got - ref).max()
    assert float(np.abs(S - Sref).max()) <= TOL, np.abs(S - Sref).max()


def test_deltanet_nonfinite_inputs_follow_reference_guards(orc, dev):
    """Non-finite inputs take the reference's per-token guards (math.rs:523-545 and
    833-874: finite_or_zero on the normalised q / k, on v, on exp(gate), on beta, on
    kv, delta and o) on the chunked path too: the scan stops before a chunk with a
    non-finite value and the step kernel continues from its first token.  One event
    per head: NaN v element, inf k element, NaN q element, NaN gate, inf beta,
    gate +100 (exp overflows, g = 0 zeroes the state), one in the ragged last chunk."""
    T, H, d = 1000, 16, 128
    q, k, v, gate, beta = _inputs(orc, T, H, d, 4242, orc.F32)
    v[100, 3, 7] = np.nan
    k[300, 5, 11] = np.inf
    q[450, 7, 0] = np.nan
    gate[500, 9] = np.nan
    beta[700, 11] = np.inf
    gate[400, 1] = 100.0
    beta[990, 13] = np.nan
    S0 = (0.05 * np.random.default_rng(1).standard_normal((H, d, d))).astype(np.float32)
    ref, Sref = orc.deltanet_scan(q, k, v, gate, beta, S0, eps=1e-6, n_threads=orc.env_threads())
    assert np.isfinite(ref).all() and np.isfinite(Sref).all()
    from gguf_runner_amd import ops
    st = torch.from_numpy(S0.copy()).to(dev)
    out = torch.empty((T, H, d), dtype=torch.float32, device=dev)
    ops.DeltaNetCall(*(torch.from_numpy(x).to(dev) for x in (q, k, v, gate, beta)), st, out,
                     algo=2)()
    torch.cuda.synchronize()
    got, S = out.cpu().numpy(), st.cpu().numpy()
    assert np.isfinite(got).all() and np.isfinite(S).all()
    assert float(np.abs(got - ref).max()) <= TOL, np.abs(got - ref).max()
    assert float(np.abs(S - Sref).max()) <= TOL, np.abs(S - Sref).max()
    # the events matter: the state of head 1 restarts from zero at token 400
    assert float(np.abs(Sref[1]).max()) < float(np.abs(Sref[0]).max())


@pytest.mark.parametrize("fmt", ["F16", "BF16"])
@pytest.mark.parametrize("l2norm", [True, False])
def test_deltanet_16bit_inputs_chunked(orc, dev, fmt, l2norm):
    """16-bit q/k/v on the chunked path (exact 16-bit Gram products, raw-row MFMA
    operands), a ragged last chunk, non-zero initial state, with and without the
    fused normalisation (without it the oracle gets rows of norm ~1 so the
    recurrence stays in range)."""
    f = getattr(orc, fmt)
    T, H, d = 200, 4, 128
    q, k, v, gate, beta = _inputs(orc, T, H, d, 300 + int(l2norm), f)
    if not l2norm:  # unit-norm-ish rows stored in the 16-bit format
        conv = orc.f16_bits if f == orc.F16 else orc.bf16_bits
        rng = np.random.default_rng(9)
        qq = rng.standard_normal((T, H, d)).astype(np.float32)
        kk = rng.standard_normal((T, H, d)).astype(np.float32)
        q = conv(qq / np.linalg.norm(qq, axis=-1, keepdims=True) / np.sqrt(d))
        k = conv(kk / np.linalg.norm(kk, axis=-1, keepdims=True))
    S0 = (0.1 * np.random.default_rng(3).standard_normal((H, d, d))).astype(np.float32)
    ref, Sref = orc.deltanet_scan(orc.upcast(q, f), orc.upcast(k, f), orc.upcast(v, f), gate, beta, S0,
                                  l2norm=l2norm, eps=1e-6, n_threads=orc.env_threads())
    from gguf_runner_amd import ops
    st = torch.from_numpy(S0.copy()).to(dev)
    out = torch.empty((T, H, d), dtype=torch.float32, device=dev)
    ops.DeltaNetCall(_to_dev(q, f, orc, dev), _to_dev(k, f, orc, dev), _to_dev(v, f, orc, dev),
                     torch.from_numpy(gate).to(dev), torch.from_numpy(beta).to(dev), st, out,
                     l2norm=l2norm, algo=2)()
    torch.cuda.synchronize()
    got, S = out.cpu().numpy(), st.cpu().numpy()
    assert float(np.abs(got - ref).max()) <= TOL, np.abs(got - ref).max()
    assert float(np.abs(S - Sref).max()) <= TOL, np.abs(S - Sref).max()


@pytest.mark.parametrize("d,algo,fmt_name", [(64, 1, "F32"), (64, 0, "BF16"), (256, 1, "F32"), (256, 2, "F16")])
def test_deltanet_state_sizes_64_and_256(orc, dev, d, algo, fmt_name):
    """State sizes other than 128 (the reference takes any ssm_state_size, math.rs:566):
    the token recurrence at d = 64 and 256, also when the chunked or automatic algorithm
    is asked for (the chunked kernels are built for 128), in two calls that carry the
    state."""
    fmt = getattr(orc, fmt_name)
    got, ref, S, Sref = _run(orc, dev, 150, 3, d, 900 + d + algo, fmt, algo, chunks=[70, 80])
    assert float(np.abs(got - ref).max()) <= TOL
    assert float(np.abs(S - Sref).max()) <= TOL
