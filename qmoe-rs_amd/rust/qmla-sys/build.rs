// Builds libqmla.so with hipcc for gfx950 (the package Makefile) and links
// it with the HIP runtime and rocBLAS, which the layer's f32 projections use.
//
// QMLA_ROOT (optional) points at the repository root; by default it is two
// levels above this crate (qmoe-rs_amd/rust/qmla-sys -> repository root).
// ROCM_PATH (optional, default /opt/rocm) locates hipcc and the libraries.
use std::{env, path::PathBuf, process::Command};

fn main() {
    let crate_dir = PathBuf::from(env::var("CARGO_MANIFEST_DIR").expect("CARGO_MANIFEST_DIR"));
    let root = env::var("QMLA_ROOT")
        .map(PathBuf::from)
        .unwrap_or_else(|_| crate_dir.join("../../.."));
    let pkg = root.join("qmoe-rs_amd");
    let rocm = PathBuf::from(env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".into()));
    let jobs = env::var("NUM_JOBS").unwrap_or_else(|_| "8".into());
    let status = Command::new("make")
        .arg("-C")
        .arg(&pkg)
        .arg("-j")
        .arg(&jobs)
        .env("HIPCC", rocm.join("bin/hipcc"))
        .status()
        .expect("running make for libqmla.so");
    assert!(status.success(), "building libqmla.so (hipcc --offload-arch=gfx950) failed");
    println!("cargo:rustc-link-search=native={}", pkg.display());
    println!("cargo:rustc-link-lib=dylib=qmla");
    println!("cargo:rustc-link-search=native={}", rocm.join("lib").display());
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    println!("cargo:rustc-link-lib=dylib=rocblas");
    // libqmla.so is loaded from the package directory at run time
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", pkg.display());
    println!("cargo:rerun-if-changed={}", pkg.join("csrc").display());
    println!("cargo:rerun-if-changed={}", root.join("include/qmla.h").display());
    println!("cargo:rerun-if-env-changed=QMLA_ROOT");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
}
