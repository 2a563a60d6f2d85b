"""The Rust side a gguf-runner maintainer adds (rust/ffi.rs, rust/build.rs) against
include/gr_attn.h, without a Rust toolchain: every #[repr(C)] struct lists the
header struct's fields in order with the matching Rust types, every extern "C"
function of the header is declared with the same parameter and return types, and
the ABI version and enum constants agree.  The ctypes binding (ffi.py) is held to
the same field lists.  CPU only."""
from __future__ import annotations

import functools
import pathlib
import re

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


@functools.lru_cache(maxsize=None)
def _text(*parts: str) -> str:
    path = ROOT.joinpath(*parts)
    if not path.exists():
        pytest.skip(f"{path} is not in this checkout")
    return path.read_text()


def _header() -> str:
    return _text("include", "gr_attn.h")


def _rust() -> str:
    return _text("rust", "ffi.rs")

# C type -> Rust type (parameters and fields)
C2R = {
    "int32_t": "i32", "int64_t": "i64", "uint64_t": "u64", "float": "f32", "size_t": "usize",
    "int": "i32", "void": "()",
    "const float*": "*const f32", "float*": "*mut f32", "const void*": "*const c_void",
    "void*": "*mut c_void", "const int32_t*": "*const i32", "int32_t*": "*mut i32",
    "const int64_t*": "*const i64", "const uint8_t*": "*const u8", "uint8_t*": "*mut u8",
    "uint64_t*": "*mut u64", "const char*": "*const c_char",
    "const gr_decode_args*": "*const GrDecodeArgs", "const gr_prefill_args*": "*const GrPrefillArgs",
    "const gr_deltanet_args*": "*const GrDeltaNetArgs", "const gr_attn_config*": "*const GrAttnConfig",
    "gr_run_state*": "*mut GrRunState", "gr_run_state**": "*mut *mut GrRunState",
}
STRUCTS = {"gr_decode_args": "GrDecodeArgs", "gr_prefill_args": "GrPrefillArgs",
           "gr_deltanet_args": "GrDeltaNetArgs", "gr_attn_config": "GrAttnConfig"}


def _strip_c_comments(s: str) -> str:
    return re.sub(r"/\*.*?\*/", " ", s, flags=re.S)


def _norm_ctype(t: str) -> str:
    t = re.sub(r"\s+", " ", t.strip())
    return re.sub(r"\s*\*", "*", t)


def header_structs() -> dict[str, list[tuple[str, str]]]:
    body = _strip_c_comments(_header())
    out = {}
    for name in STRUCTS:
        m = re.search(r"typedef struct %s \{(.*?)\} %s;" % (name, name), body, re.S)
        assert m, name
        fields = []
        for decl in m.group(1).split(";"):
            decl = decl.strip()
            if not decl:
                continue
            fm = re.match(r"(.*?[\s\*])(\w+)$", decl, re.S)
            fields.append((fm.group(2), _norm_ctype(fm.group(1))))
        out[name] = fields
    return out


def header_functions() -> dict[str, tuple[str, list[str]]]:
    body = _strip_c_comments(_header())
    out = {}
    for m in re.finditer(r"^\s*((?:const )?\w+\s*\**)\s*(gr_\w+)\(([^)]*)\);", body, re.M | re.S):
        ret, name, params = _norm_ctype(m.group(1)), m.group(2), m.group(3)
        types = []
        if params.strip() != "void":
            for p in params.split(","):
                pm = re.match(r"(.*?[\s\*])(\w+)$", p.strip(), re.S)
                types.append(_norm_ctype(pm.group(1)))
        out[name] = (ret, types)
    return out


def rust_structs() -> dict[str, list[tuple[str, str]]]:
    out = {}
    for m in re.finditer(r"#\[repr\(C\)\]\s*pub struct (\w+) \{(.*?)\n\}", _rust(), re.S):
        fields = re.findall(r"pub (\w+): ([^,]+),", m.group(2))
        out[m.group(1)] = [(n, re.sub(r"\s+", " ", t.strip())) for n, t in fields]
    return out


def rust_functions() -> dict[str, tuple[str, list[str]]]:
    rust = _rust()
    block = rust[rust.index('unsafe extern "C" {'):]
    out = {}
    for m in re.finditer(r"pub fn (gr_\w+)\((.*?)\)(?:\s*->\s*([^;]+))?;", block, re.S):
        params = [re.sub(r"\s+", " ", p.split(":", 1)[1].strip()) for p in m.group(2).split(",") if p.strip()]
        out[m.group(1)] = ((m.group(3) or "()").strip(), params)
    return out


def test_rust_structs_match_header_field_for_field():
    hs, rs = header_structs(), rust_structs()
    assert len(hs["gr_decode_args"]) > 20
    for cname, rname in STRUCTS.items():
        want = [(n, C2R[t]) for n, t in hs[cname]]
        assert rs[rname] == want, (cname, [x for x in zip(rs[rname], want) if x[0] != x[1]][:3])


def test_rust_functions_match_header_signatures():
    hf, rf = header_functions(), rust_functions()
    assert "gr_decode_attention_noalloc" in hf and "gr_prefill_cache_inject" in hf
    assert set(rf) == set(hf), (set(hf) ^ set(rf))
    for name, (ret, params) in hf.items():
        rret, rparams = rf[name]
        assert rret == C2R[ret], (name, ret, rret)
        assert rparams == [C2R[t] for t in params], (name, params, rparams)


def test_rust_constants_match_header():
    header, rust = _header(), _rust()
    ver = int(re.search(r"#define GR_ATTN_ABI_VERSION (\d+)", header).group(1))
    assert f"pub const GR_ATTN_ABI_VERSION: i32 = {ver};" in rust
    for name in ("GR_DTYPE_F32", "GR_DTYPE_F16", "GR_DTYPE_BF16", "GR_DTYPE_Q8", "GR_DTYPE_TURBO",
                 "GR_DELTANET_AUTO", "GR_DELTANET_RECURRENT", "GR_DELTANET_CHUNKED"):
        v = int(re.search(name + r"\s*=\s*(\d+)", header).group(1))
        assert f"pub const {name}: i32 = {v};" in rust, name


def test_build_rs_builds_the_gfx950_library():
    b = _text("rust", "build.rs")
    assert '"-C", &src' in b and "libgr_attn.so" in b and "rustc-link-lib=dylib=gr_attn" in b
    mk = _text("gguf-runner_amd", "Makefile")
    assert "--offload-arch=$(ARCH)" in mk and "ARCH ?= gfx950" in mk


def test_ctypes_binding_matches_header_field_lists():
    from gguf_runner_amd import ffi
    hs = header_structs()
    for cname, cls in (("gr_decode_args", ffi.DecodeArgs), ("gr_prefill_args", ffi.PrefillArgs),
                       ("gr_deltanet_args", ffi.DeltaNetArgs), ("gr_attn_config", ffi.AttnConfig)):
        assert [f[0] for f in cls._fields_] == [n for n, _ in hs[cname]], cname
