// build.rs for gguf-runner (repository root), behind a `rocm` cargo feature:
// builds libgr_attn.so for gfx950 with hipcc (gguf-runner_amd/Makefile) and links
// it.  GR_ATTN_DIR points at the gguf-runner_amd directory of this project.
fn main() {
    if std::env::var("CARGO_FEATURE_ROCM").is_err() {
        return;
    }
    let out = std::path::PathBuf::from(std::env::var("OUT_DIR").unwrap());
    let src = std::env::var("GR_ATTN_DIR").unwrap_or_else(|_| "gguf-runner_amd".to_string());
    let status = std::process::Command::new("make")
        .args(["-C", &src, "-j16"]) // hipcc --offload-arch=gfx950 -O3 -fPIC, then -shared
        .status()
        .expect("make / hipcc");
    assert!(status.success(), "building libgr_attn.so failed");
    std::fs::copy(format!("{src}/_build/libgr_attn.so"), out.join("libgr_attn.so")).unwrap();
    println!("cargo:rustc-link-search=native={}", out.display());
    println!("cargo:rustc-link-search=native=/opt/rocm/lib");
    println!("cargo:rustc-link-lib=dylib=gr_attn");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    println!("cargo:rerun-if-changed={src}/csrc");
    println!("cargo:rerun-if-changed={src}/../include/gr_attn.h");
    println!("cargo:rerun-if-env-changed=GR_ATTN_DIR");
}
