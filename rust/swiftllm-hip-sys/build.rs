//! Links libswiftllm_hip.so and the HIP runtime. Replaces the CUDA probe of
//! crates/swiftllm-cuda/build.rs:3-23 (which only looked for a CUDA install
//! and never compiled the kernels).
//!
//! SWIFTLLM_HIP_LIB_DIR names the directory of libswiftllm_hip.so (built by
//! `python -m swiftllm_amd.build`); by default the package directory of this
//! repository, two levels up. ROCM_PATH defaults to /opt/rocm.

use std::path::PathBuf;

fn main() {
    let lib_dir = std::env::var("SWIFTLLM_HIP_LIB_DIR").map(PathBuf::from).unwrap_or_else(|_| {
        let manifest = PathBuf::from(std::env::var("CARGO_MANIFEST_DIR").unwrap());
        manifest.join("../../swiftllm_amd")
    });
    let rocm = std::env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    println!("cargo:rerun-if-env-changed=SWIFTLLM_HIP_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
    println!("cargo:rustc-link-search=native={}", lib_dir.display());
    println!("cargo:rustc-link-lib=dylib=swiftllm_hip");
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    // The library's rpath already names the ROCm lib directory; this one lets
    // test binaries find libswiftllm_hip.so itself without LD_LIBRARY_PATH.
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", lib_dir.display());
}
