"""gguf-runner attention hot path for MI355X (gfx950).

Python host side of libgr_attn.so.  `ffi` holds the raw ctypes bindings of the
C ABI (include/gr_attn.h); `ops` wraps the device-pointer entry points for
torch tensors that already live in HBM.  The directory name is not a Python
identifier: __graft_entry__.load_package() registers it in sys.modules as
`gguf_runner_amd`.
"""
from . import ffi  # noqa: F401

__all__ = ["ffi", "ops", "runtime"]
