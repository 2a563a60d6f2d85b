"""ctypes bindings of libgr_attn.so (include/gr_attn.h).

The structs below mirror the header field for field.  Nothing here computes
attention: every call goes to the HIP kernels, and loading fails loudly when the
library has not been built.
"""
from __future__ import annotations

import ctypes
import pathlib

PKG_DIR = pathlib.Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "_build" / "libgr_attn.so"
HEADER = PKG_DIR.parent / "include" / "gr_attn.h"

GR_OK = 0
GR_ERR_ARG = -1
GR_ERR_HIP = -2
GR_ERR_RANGE = -3
GR_ERR_OOM = -4

DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
ROPE_NONE, ROPE_ADJACENT, ROPE_NEOX = 0, 1, 2

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
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
    ]


class PrefillArgs(ctypes.Structure):
    _fields_ = [
        ("n_tokens", _i32), ("base_pos", _i32), ("n_heads", _i32), ("n_kv_heads", _i32),
        ("head_dim", _i32), ("dtype", _i32), ("window", _i32), ("rope_mode", _i32),
        ("rope_dim", _i32), ("rope_scale", _f), ("rope_freqs", _p), ("q_norm", _p),
        ("k_norm", _p), ("norm_eps", _f), ("is_gemma3", _i32), ("q", _p), ("k", _p), ("v", _p),
        ("k_cache", _p), ("v_cache", _p), ("cache_row_stride", _i64), ("out", _p),
        ("workspace", _p),
    ]


class DeltaNetArgs(ctypes.Structure):
    _fields_ = [
        ("n_tokens", _i32), ("n_heads", _i32), ("head_dim", _i32), ("in_dtype", _i32),
        ("l2norm", _i32), ("algo", _i32), ("eps", _f), ("q", _p), ("k", _p), ("v", _p),
        ("gate", _p), ("beta", _p), ("state", _p), ("out", _p), ("workspace", _p),
    ]


DELTANET_AUTO, DELTANET_RECURRENT, DELTANET_CHUNKED = 0, 1, 2

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
    L.gr_prefill_workspace_size.argtypes = [ctypes.POINTER(PrefillArgs)]
    L.gr_prefill_workspace_size.restype = ctypes.c_size_t
    L.gr_prefill_attention.argtypes = [ctypes.POINTER(PrefillArgs), _p]
    L.gr_prefill_attention.restype = ctypes.c_int
    L.gr_rope_freqs.argtypes = [_f, _i32, _p]
    L.gr_rope_freqs.restype = ctypes.c_int
    L.gr_deltanet_workspace_size.argtypes = [ctypes.POINTER(DeltaNetArgs)]
    L.gr_deltanet_workspace_size.restype = ctypes.c_size_t
    L.gr_deltanet_attention.argtypes = [ctypes.POINTER(DeltaNetArgs), _p]
    L.gr_deltanet_attention.restype = ctypes.c_int


def check(rc: int) -> None:
    if rc != GR_OK:
        raise GrError(rc, lib().gr_last_error().decode())


def header_symbols() -> list[str]:
    """Function names declared in include/gr_attn.h."""
    import re
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gr_[a-z0-9_]+)\s*\(", text)))
