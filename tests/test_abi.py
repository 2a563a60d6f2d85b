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
    assert L.gr_abi_version() == 1
    a = ffi.DecodeArgs()
    a.n_seq, a.n_heads, a.n_kv_heads, a.head_dim = 1, 6, 4, 128
    rc = L.gr_decode_attention(ctypes.byref(a), None)
    assert rc == ffi.GR_ERR_ARG
    assert b"multiple" in L.gr_last_error()
