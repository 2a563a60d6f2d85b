"""ctypes bindings of libgr_attn.so (include/gr_attn.h).

The structs below mirror the header field for field.  Nothing here computes
attention: every call goes to the HIP kernels, and loading fails loudly when the
library has not been built.
"""
from __future__ import annotations

import ctypes
import os
import pathlib

PKG_DIR = pathlib.Path(__file__).resolve().parent
LIB_PATH = pathlib.Path(os.environ.get("GR_ATTN_LIB") or PKG_DIR / "_build" / "libgr_attn.so")
HEADER = PKG_DIR.parent / "include" / "gr_attn.h"

GR_OK = 0
GR_ERR_ARG = -1
GR_ERR_HIP = -2
GR_ERR_RANGE = -3
GR_ERR_OOM = -4

DTYPE_F32, DTYPE_F16, DTYPE_BF16, DTYPE_Q8, DTYPE_TURBO = 0, 1, 2, 3, 4
ROPE_NONE, ROPE_ADJACENT, ROPE_NEOX = 0, 1, 2

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_f = ctypes.c_float


class GrError(RuntimeError):
    """A libgr_attn call returned a negative status; .code holds it."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"gr_attn error {code}: {msg}")
        self.code = code


class DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("n_seq", _i32), ("n_heads", _i32), ("n_kv_heads", _i32), ("head_dim", _i32),
        ("kv_dtype", _i32), ("split_keys", _i32), ("max_kv_len", _i32), ("score_scale", _f),
        ("q", _p), ("k_cache", _p), ("v_cache", _p), ("seq_stride", _i64), ("row_stride", _i64),
        ("kv_start", _p), ("kv_end", _p), ("out", _p), ("workspace", _p),
        ("k_scale", _p), ("v_scale", _p), ("scale_seq_stride", _i64), ("scale_row_stride", _i64),
        ("q8_block", _i32), ("k_sign", _p), ("v_sign", _p), ("k_rnorm", _p), ("v_rnorm", _p),
        ("turbo_signs", _p), ("turbo_slot_stride", _i64),
        ("out_gate", _p), ("out_gate_row_stride", _i64), ("out_gate_head_stride", _i32),
    ]


class PrefillArgs(ctypes.Structure):
    _fields_ = [
        ("n_tokens", _i32), ("base_pos", _i32), ("n_heads", _i32), ("n_kv_heads", _i32),
        ("head_dim", _i32), ("dtype", _i32), ("window", _i32), ("rope_mode", _i32),
        ("rope_dim", _i32), ("rope_scale", _f), ("rope_freqs", _p), ("q_norm", _p),
        ("k_norm", _p), ("norm_eps", _f), ("is_gemma3", _i32), ("q", _p), ("k", _p), ("v", _p),
        ("k_cache", _p), ("v_cache", _p), ("cache_row_stride", _i64), ("out", _p),
        ("workspace", _p), ("bidirectional", _i32),
        ("out_gate", _p), ("out_gate_row_stride", _i64), ("out_gate_head_stride", _i32),
        ("q_bias", _p), ("k_bias", _p), ("v_bias", _p),
    ]


class DeltaNetArgs(ctypes.Structure):
    _fields_ = [
        ("n_tokens", _i32), ("n_heads", _i32), ("head_dim", _i32), ("in_dtype", _i32),
        ("l2norm", _i32), ("algo", _i32), ("eps", _f), ("q", _p), ("k", _p), ("v", _p),
        ("gate", _p), ("beta", _p), ("state", _p), ("out", _p), ("workspace", _p),
    ]


DELTANET_AUTO, DELTANET_RECURRENT, DELTANET_CHUNKED = 0, 1, 2


class AttnConfig(ctypes.Structure):
    _fields_ = [
        ("n_layers", _i32), ("n_heads", _i32), ("n_kv_heads", _i32), ("head_dim", _i32),
        ("seq_len", _i32), ("n_seq", _i32), ("kv_dtype", _i32), ("rope_mode", _i32),
        ("rope_dim", _i32), ("rope_theta", _f), ("rope_theta_swa", _f),
        ("rope_scale_global", _f), ("rope_scale_local", _f), ("layer_windows", _p),
        ("swa_pattern", _i32), ("is_gemma3", _i32), ("online_attn_fusion", _i32),
        ("rms_norm_eps", _f), ("q_norm", _p), ("k_norm", _p), ("qk_norm_present", _p),
        ("ssm_n_heads", _i32), ("ssm_head_dim", _i32), ("q8_block_scales", _i32),
        ("ssm_n_k_heads", _i32), ("ssm_conv_kernel", _i32), ("ssm_conv1d", _p), ("ssm_a", _p),
        ("ssm_dt_bias", _p), ("ssm_norm", _p),
    ]

_lib = None


def lib() -> ctypes.CDLL:
    """Load libgr_attn.so (raises if it was not built: there is no fallback)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `make -C gguf-runner_amd` "
                "(or __graft_entry__.build()); the HIP path has no CPU fallback")
        L = ctypes.CDLL(str(LIB_PATH))
        _declare(L)
        _lib = L
    return _lib


def _declare(L: ctypes.CDLL) -> None:
    L.gr_last_error.restype = ctypes.c_char_p
    L.gr_abi_version.restype = ctypes.c_int
    L.gr_decode_workspace_size.argtypes = [ctypes.POINTER(DecodeArgs)]
    L.gr_decode_workspace_size.restype = ctypes.c_size_t
    L.gr_decode_attention.argtypes = [ctypes.POINTER(DecodeArgs), _p]
    L.gr_decode_attention.restype = ctypes.c_int
    L.gr_decode_attention_noalloc.argtypes = [ctypes.POINTER(DecodeArgs), _p]
    L.gr_decode_attention_noalloc.restype = ctypes.c_int
    L.gr_prefill_workspace_size.argtypes = [ctypes.POINTER(PrefillArgs)]
    L.gr_prefill_workspace_size.restype = ctypes.c_size_t
    L.gr_prefill_attention.argtypes = [ctypes.POINTER(PrefillArgs), _p]
    L.gr_prefill_attention.restype = ctypes.c_int
    L.gr_rope_freqs.argtypes = [_f, _i32, _p]
    L.gr_rope_freqs.restype = ctypes.c_int
    L.gr_turbo_sign_table.argtypes = [_i32, _i32, _i32, _p]
    L.gr_turbo_sign_table.restype = ctypes.c_int
    L.gr_deltanet_workspace_size.argtypes = [ctypes.POINTER(DeltaNetArgs)]
    L.gr_deltanet_workspace_size.restype = ctypes.c_size_t
    L.gr_deltanet_attention.argtypes = [ctypes.POINTER(DeltaNetArgs), _p]
    L.gr_deltanet_attention.restype = ctypes.c_int
    ip = ctypes.c_int
    L.gr_malloc_run_state.argtypes = [ctypes.POINTER(AttnConfig), ctypes.POINTER(_p)]
    L.gr_malloc_run_state.restype = ip
    L.gr_free_run_state.argtypes = [_p]
    L.gr_free_run_state.restype = None
    L.gr_qkv_norm.argtypes = [_p, _i32, _p, _p]
    L.gr_apply_rope_qk.argtypes = [_p, _i32, _i64, _p, _p]
    L.gr_kv_write_token.argtypes = [_p, _i32, _i32, _i64, _p, _p]
    L.gr_attention_token.argtypes = [_p, _i32, _i32, _i64, _p, _p]
    L.gr_attention_layer_token.argtypes = [_p, _i32, _i32, _i64, _p, _p, _p, _p]
    L.gr_prefill_attention_chunk.argtypes = [_p, _i32, _i32, _i64, _i32, _p, _p, _p, _p]
    L.gr_encoder_self_attention.argtypes = [_p, _p, _p, _p, _i32, _i32, _i32, _i32, _p]
    L.gr_prefill_image_block.argtypes = [_p, _i32, _i32, _i64, _i32, _p, _p, _p, _p]
    L.gr_decode_layer_batch.argtypes = [_p, _i32, _i32, _p, _p, _p, _p, _p, _p]
    L.gr_qwen3next_state_step.argtypes = [_p, _i32, _p, _p, _p, _p, _p, _p]
    L.gr_qwen3next_prefill.argtypes = [_p, _i32, _i32, _p, _p, _p, _p, _p, _p]
    L.gr_read_kv_rows.argtypes = [_p, _i32, _i32, _i64, _i64, _p, _p]
    L.gr_read_kv_scales.argtypes = [_p, _i32, _i32, _i64, _i64, _p, _p]
    L.gr_read_turbo_rows.argtypes = [_p, _i32, _i32, _i64, _i64, _p, _p, _p, _p, _p, _p]
    L.gr_read_ssm_state.argtypes = [_p, _i32, _p]
    L.gr_qwen3next_ssm_layer.argtypes = [_p, _i32, _i32, _p, _p, _p, _p, _p]
    L.gr_read_ssm_conv_state.argtypes = [_p, _i32, _p]
    L.gr_write_ssm_conv_state.argtypes = [_p, _i32, _p]
    L.gr_write_ssm_state.argtypes = [_p, _i32, _p]
    L.gr_prefill_cache_snapshot.argtypes = [_p, _i32, _p, _i32, _u64, _u64, _p, _u64, _p]
    L.gr_prefill_cache_inject.argtypes = [_p, _i32, _p, _u64, _p]
    for n in ("gr_qkv_norm", "gr_apply_rope_qk", "gr_kv_write_token", "gr_attention_token",
              "gr_attention_layer_token", "gr_prefill_attention_chunk", "gr_prefill_image_block",
              "gr_decode_layer_batch",
              "gr_qwen3next_state_step", "gr_qwen3next_prefill", "gr_read_kv_rows",
              "gr_read_kv_scales", "gr_read_turbo_rows",
              "gr_read_ssm_state", "gr_write_ssm_state", "gr_qwen3next_ssm_layer",
              "gr_read_ssm_conv_state", "gr_prefill_cache_snapshot", "gr_prefill_cache_inject", "gr_write_ssm_conv_state"):
        getattr(L, n).restype = ip


def check(rc: int) -> None:
    if rc != GR_OK:
        raise GrError(rc, lib().gr_last_error().decode())


def header_symbols() -> list[str]:
    """Function names declared in include/gr_attn.h."""
    import re
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gr_[a-z0-9_]+)\s*\(", text)))
