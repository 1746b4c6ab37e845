//! Build script of vestra-kernels with the `hip` feature: links the MI355X
//! backend (`libvestra_hip.so`, built by `make -C vestra-kernels_amd`) and
//! the HIP runtime.  Without the feature it does nothing, so CPU-only and
//! `cuda` builds are unchanged.
//!
//! VESTRA_HIP_LIB_DIR: directory holding libvestra_hip.so (required with `hip`).
//! ROCM_PATH: ROCm installation (default /opt/rocm), for libamdhip64.

fn main() {
    println!("cargo:rerun-if-env-changed=VESTRA_HIP_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
    if std::env::var_os("CARGO_FEATURE_HIP").is_none() {
        return;
    }
    if std::env::var_os("CARGO_FEATURE_CUDA").is_some() {
        panic!("features `cuda` and `hip` are exclusive: `hip` replaces the CUDA driver/cuBLAS path");
    }
    let lib_dir = std::env::var("VESTRA_HIP_LIB_DIR")
        .expect("feature `hip`: set VESTRA_HIP_LIB_DIR to the directory of libvestra_hip.so");
    let rocm = std::env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    println!("cargo:rustc-link-search=native={lib_dir}");
    println!("cargo:rustc-link-lib=dylib=vestra_hip");
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    // The library is found at run time through the same directory.
    println!("cargo:rustc-link-arg=-Wl,-rpath,{lib_dir}");
}
