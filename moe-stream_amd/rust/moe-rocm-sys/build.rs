//! Link step of moe-rocm-sys: libmoe_rocm.so (built by `python __graft_entry__.py`, hipcc for
//! gfx950) and the HIP runtime it depends on.
//!
//! MOE_ROCM_LIB_DIR: directory holding libmoe_rocm.so (default: the in-tree build output,
//! moe-stream_amd/moe_rocm, two levels above this crate). ROCM_PATH: ROCm install (default
//! /opt/rocm), whose lib/ holds libamdhip64.so.
use std::env;
use std::path::PathBuf;

fn main() {
    println!("cargo:rerun-if-env-changed=MOE_ROCM_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").expect("cargo sets CARGO_MANIFEST_DIR"));
    let lib_dir = env::var("MOE_ROCM_LIB_DIR")
        .map(PathBuf::from)
        .unwrap_or_else(|_| manifest.join("..").join("..").join("moe_rocm"));
    if !lib_dir.join("libmoe_rocm.so").exists() {
        panic!(
            "libmoe_rocm.so not found in {} (build it with `python __graft_entry__.py`, or set MOE_ROCM_LIB_DIR)",
            lib_dir.display()
        );
    }
    let rocm = env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    println!("cargo:rustc-link-search=native={}", lib_dir.display());
    println!("cargo:rustc-link-search=native={}/lib", rocm);
    println!("cargo:rustc-link-lib=dylib=moe_rocm");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    // dependents read DEP_MOE_ROCM_LIB_DIR (the `links` key) to set an rpath if they want one
    println!("cargo:lib_dir={}", lib_dir.display());
    println!("cargo:rerun-if-changed={}", lib_dir.join("libmoe_rocm.so").display());
}
