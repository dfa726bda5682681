//! Builds libstrata_hip (the gfx950 kernels and the C ABI of
//! include/strata_hip.h) with its own Makefile and links it.
//!
//! The library sources are found at `$STRATA_HIP_DIR`, or at
//! `../../strata-rs_amd` from this crate (the layout of this repository).
//! hipcc (ROCm) must be on the build host; the code objects are for gfx950.

use std::env;
use std::path::PathBuf;
use std::process::Command;

fn main() {
    println!("cargo:rerun-if-env-changed=STRATA_HIP_DIR");
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").expect("CARGO_MANIFEST_DIR"));
    let src = env::var_os("STRATA_HIP_DIR")
        .map(PathBuf::from)
        .unwrap_or_else(|| manifest.join("../../strata-rs_amd"));
    let src = src.canonicalize().unwrap_or_else(|e| panic!("library sources at {}: {e}", src.display()));

    let jobs = env::var("NUM_JOBS").unwrap_or_else(|_| "8".to_string());
    let status = Command::new("make")
        .arg("-C")
        .arg(&src)
        .arg(format!("-j{jobs}"))
        .status()
        .expect("running make (hipcc) for libstrata_hip");
    assert!(status.success(), "building libstrata_hip failed");

    let lib = src.join("lib");
    println!("cargo:rustc-link-search=native={}", lib.display());
    println!("cargo:rustc-link-lib=dylib=strata_hip");
    // tests and binaries find the library where it was built
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", lib.display());
    println!("cargo:rerun-if-changed={}", src.join("csrc").display());
    println!("cargo:rerun-if-changed={}", src.join("Makefile").display());
    println!("cargo:rerun-if-changed={}", manifest.join("../../include/strata_hip.h").display());
}
