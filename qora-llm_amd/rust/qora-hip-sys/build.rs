//! Builds libqora_hip.so (the gfx950 kernels and the C ABI of
//! include/qora_hip.h) with the package's Makefile (hipcc
//! --offload-arch=gfx950) and links the crate against it.
//!
//! QORA_HIP_DIR overrides the directory holding the Makefile; by default it
//! is the package directory two levels above this crate
//! (qora-llm_amd/rust/qora-hip-sys -> qora-llm_amd). QORA_HIP_NO_BUILD=1 links
//! a library that is already built without running make.

use std::env;
use std::path::PathBuf;
use std::process::Command;

fn main() {
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").expect("cargo sets CARGO_MANIFEST_DIR"));
    let dir = match env::var_os("QORA_HIP_DIR") {
        Some(d) => PathBuf::from(d),
        None => manifest.join("..").join(".."),
    };
    let dir = dir.canonicalize().unwrap_or_else(|e| panic!("QORA_HIP_DIR {}: {e}", dir.display()));
    if env::var_os("QORA_HIP_NO_BUILD").is_none() {
        let status = Command::new("make")
            .arg("-C")
            .arg(&dir)
            .status()
            .unwrap_or_else(|e| panic!("running make in {}: {e}", dir.display()));
        assert!(status.success(), "building libqora_hip.so in {} failed", dir.display());
    }
    let lib = dir.join("libqora_hip.so");
    assert!(lib.exists(), "{} is not built", lib.display());
    println!("cargo:rustc-link-search=native={}", dir.display());
    println!("cargo:rustc-link-lib=dylib=qora_hip");
    // the library is loaded from where it was built (no install step)
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", dir.display());
    for f in ["Makefile", "csrc", "../include/qora_hip.h"] {
        println!("cargo:rerun-if-changed={}", dir.join(f).display());
    }
    println!("cargo:rerun-if-env-changed=QORA_HIP_DIR");
    println!("cargo:rerun-if-env-changed=QORA_HIP_NO_BUILD");
}
