"""The C-ABI library loads on a CPU-only host and exports every entry point that
include/gr_attn.h declares (no compute calls: there is no GPU here)."""
from __future__ import annotations

import ctypes
import subprocess


def test_header_symbols_exported(pkg):
    from gguf_runner_amd import ffi
    names = ffi.header_symbols()
    assert "gr_decode_attention" in names and "gr_last_error" in names
    L = ffi.lib()
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_no_unexpected_exports(pkg):
    """Every exported gr_* function is declared in the header (no hidden ABI)."""
    from gguf_runner_amd import ffi
    out = subprocess.run(["nm", "-D", "--defined-only", str(ffi.LIB_PATH)], check=True,
                         capture_output=True, text=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T gr_" in ln}
    assert exported <= set(ffi.header_symbols()), exported - set(ffi.header_symbols())


def test_abi_version_and_error_path(pkg):
    from gguf_runner_amd import ffi
    L = ffi.lib()
    assert L.gr_abi_version() == 5
    a = ffi.DecodeArgs()
    a.n_seq, a.n_heads, a.n_kv_heads, a.head_dim = 1, 6, 4, 128
    rc = L.gr_decode_attention(ctypes.byref(a), None)
    assert rc == ffi.GR_ERR_ARG
    assert b"multiple" in L.gr_last_error()


def test_decode_rejects_bad_q8_args(pkg):
    """Q8 decode argument checks run before any launch (no GPU needed)."""
    from gguf_runner_amd import ffi
    L = ffi.lib()
    a = ffi.DecodeArgs()
    a.n_seq, a.n_heads, a.n_kv_heads, a.head_dim, a.kv_dtype, a.max_kv_len = 1, 8, 4, 96, ffi.DTYPE_Q8, 16
    assert L.gr_decode_attention(ctypes.byref(a), None) == ffi.GR_ERR_ARG
    assert b"head_dim 96 unsupported" in L.gr_last_error()
    a.head_dim = 64
    assert L.gr_decode_attention(ctypes.byref(a), None) == ffi.GR_ERR_ARG
    assert b"k_scale and v_scale" in L.gr_last_error()
    a.k_scale = a.v_scale = 4
    a.q8_block, a.scale_row_stride = 1, 7  # block mode needs kv_dim / 32 = 8 scales a row
    assert L.gr_decode_attention(ctypes.byref(a), None) == ffi.GR_ERR_ARG
    assert b"scale_row_stride >= kv_dim/32" in L.gr_last_error()


def test_malloc_run_state_rejects_invalid_rope_scales(pkg):
    """inference.rs:4120-4131 (rope_scaling_rejects_invalid_runtime_policies): scales
    0, -1, NaN, inf are refused before any device allocation (runs without a GPU)."""
    from gguf_runner_amd import ffi, runtime
    for scale in (0.0, -1.0, float("nan"), float("inf")):
        for glob in (True, False):
            p = runtime.Config(n_layers=1, n_heads=1, n_kv_heads=1, head_dim=64, seq_len=8,
                               rope_scale_global=scale if glob else 1.0,
                               rope_scale_local=1.0 if glob else scale)
            try:
                runtime.malloc_run_state(p)
            except ffi.GrError as e:
                assert e.code == ffi.GR_ERR_ARG
                assert "RoPE frequency scales must be finite and positive" in str(e)
            else:
                raise AssertionError("invalid scale accepted")


def test_malloc_run_state_rejects_bad_windows_and_shapes(pkg):
    from gguf_runner_amd import ffi, runtime
    bad = [dict(layer_windows=[1024, -1]), dict(n_kv_heads=3), dict(head_dim=96),
           dict(kv_dtype=ffi.DTYPE_Q8, head_dim=96), dict(kv_dtype=7),
           dict(rope_mode=ffi.ROPE_ADJACENT, rope_dim=32)]
    for kw in bad:
        base = dict(n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64, seq_len=8)
        base.update(kw)
        try:
            runtime.malloc_run_state(runtime.Config(**base))
        except ffi.GrError as e:
            assert e.code == ffi.GR_ERR_ARG
        else:
            raise AssertionError(f"accepted {kw}")


def test_rope_freqs_match_oracle_bitwise(pkg, orc):
    """gr_rope_freqs and the oracle both restate inference.rs:1590-1609 with host powf."""
    import numpy as np
    from gguf_runner_amd import ops
    for theta, dim in ((5e5, 128), (1e4, 256), (1e6, 64)):
        a = np.array(ops.rope_freqs(theta, dim), np.float32)
        assert np.array_equal(a, orc.rope_freqs(theta, dim))


def test_turbo_sign_table_matches_oracle_bitwise(pkg, orc):
    """gr_turbo_sign_table (host) == the oracle's turboquant_build_sign_table restatement."""
    import numpy as np
    from gguf_runner_amd import ops
    for L, G, d in ((2, 8, 128), (3, 4, 64), (1, 1, 40)):
        assert np.array_equal(ops.turbo_sign_table(L, G, d), orc.turbo_sign_table(L, G, d))


def test_ssm_config_validation(pkg):
    """Qwen3NextLinearAttentionShape checks (math.rs:571-584) at allocation, before any
    device work: n_v % n_k, missing tensors."""
    import numpy as np
    from gguf_runner_amd import ffi, runtime as rt
    base = dict(n_layers=1, n_heads=2, n_kv_heads=1, head_dim=128, seq_len=8, ssm_n_heads=6,
                ssm_head_dim=128, ssm_n_k_heads=4, ssm_conv_kernel=4,
                ssm_conv1d=np.zeros((1, 14 * 128, 4), np.float32), ssm_a=np.zeros((1, 6), np.float32),
                ssm_dt_bias=np.zeros((1, 6), np.float32), ssm_norm=np.ones((1, 128), np.float32))
    try:
        rt.malloc_run_state(rt.Config(**base))
    except ffi.GrError as e:
        assert "not divisible by n_k_heads" in str(e)
    else:
        raise AssertionError("accepted n_v % n_k != 0")
    base.update(ssm_n_k_heads=3, ssm_a=None)
    try:
        rt.malloc_run_state(rt.Config(**base))
    except ffi.GrError as e:
        assert "missing qwen3next SSM tensors" in str(e)
    else:
        raise AssertionError("accepted missing ssm_a")


def test_ssm_state_needs_one_sequence_slot(pkg):
    """The SSM state and conv history exist once per layer, as in one reference
    RunState (types.rs:745-809); a multi-slot state with an SSM is refused before any
    device work."""
    from gguf_runner_amd import ffi, runtime as rt
    try:
        rt.malloc_run_state(rt.Config(n_layers=1, n_heads=2, n_kv_heads=1, head_dim=128, seq_len=8,
                                      n_seq=2, ssm_n_heads=2, ssm_head_dim=128))
    except ffi.GrError as e:
        assert e.code == ffi.GR_ERR_ARG and "n_seq == 1" in str(e)
    else:
        raise AssertionError("accepted an SSM state with two sequence slots")


def test_decode_rejects_misaligned_q(pkg):
    """q is read as 16-byte vectors: a q pointer off a 16-byte boundary is an
    argument error, reported before any launch (no GPU needed)."""
    from gguf_runner_amd import ffi
    L = ffi.lib()
    a = ffi.DecodeArgs()
    a.n_seq, a.n_heads, a.n_kv_heads, a.head_dim, a.kv_dtype, a.max_kv_len = 1, 8, 4, 128, ffi.DTYPE_F16, 16
    a.row_stride, a.seq_stride = 4 * 128, 16 * 4 * 128
    a.k_cache = a.v_cache = a.kv_start = a.kv_end = a.out = 1 << 20
    a.workspace = 1 << 21
    a.q = (1 << 22) + 4
    assert L.gr_decode_attention(ctypes.byref(a), None) == ffi.GR_ERR_ARG
    assert b"q must be 16-byte aligned" in L.gr_last_error()


def test_prefill_rejects_misaligned_norm_weights(pkg):
    """The QK-norm weights are read as 16-byte vectors: a weight pointer off a
    16-byte boundary is an argument error, reported before any launch."""
    from gguf_runner_amd import ffi
    L = ffi.lib()
    a = ffi.PrefillArgs()
    a.n_tokens, a.n_heads, a.n_kv_heads, a.head_dim, a.dtype = 16, 8, 4, 256, ffi.DTYPE_BF16
    a.q_norm, a.k_norm = (1 << 20) + 8, 1 << 21
    assert L.gr_prefill_attention(ctypes.byref(a), None) == ffi.GR_ERR_ARG
    assert b"q_norm and k_norm must be 16-byte aligned" in L.gr_last_error()
