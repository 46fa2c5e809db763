//! Build script of darkforest-hip: builds libdfattn with hipcc for gfx950 through the library's own
//! Makefile (dark-forest_amd/csrc/Makefile, the role darkforest-cuda/build.rs:102-225 plays for
//! nvcc) and links it and the HIP runtime.
//!
//! Environment: ROCM_PATH (default /opt/rocm) locates hipcc and libamdhip64; HIPCC and ARCH, when
//! set, are passed to make (the Makefile's defaults are $ROCM_PATH/bin/hipcc and gfx950).

use std::env;
use std::path::PathBuf;
use std::process::Command;

fn main() {
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").expect("CARGO_MANIFEST_DIR"));
    let repo = manifest.join("..").join("..");
    let csrc = repo.join("dark-forest_amd").join("csrc");
    let lib_dir = repo.join("dark-forest_amd").join("lib");
    let rocm = PathBuf::from(env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string()));

    let mut make = Command::new("make");
    make.arg("-C").arg(&csrc).arg("-j8");
    if let Ok(hipcc) = env::var("HIPCC") {
        make.arg(format!("HIPCC={hipcc}"));
    } else {
        make.arg(format!("HIPCC={}", rocm.join("bin").join("hipcc").display()));
    }
    if let Ok(arch) = env::var("ARCH") {
        make.arg(format!("ARCH={arch}"));
    }
    let status = make.status().expect("running make (hipcc) failed");
    assert!(status.success(), "building libdfattn with hipcc failed");

    println!("cargo:rustc-link-search=native={}", lib_dir.display());
    println!("cargo:rustc-link-lib=dylib=dfattn");
    println!("cargo:rustc-link-search=native={}", rocm.join("lib").display());
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    // The library is found at run time next to the crate's output as well as through the rpath.
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", lib_dir.display());
    println!("cargo:rerun-if-changed={}", csrc.display());
    println!("cargo:rerun-if-changed={}", repo.join("include").display());
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
    println!("cargo:rerun-if-env-changed=HIPCC");
    println!("cargo:rerun-if-env-changed=ARCH");
}
