//! Links the prebuilt libullm_hip.so (built by `python -m ullm_amd.build`
//! in the ullm_amd repository) and the HIP runtime.
fn main() {
    let dir = std::env::var("ULLM_HIP_LIB_DIR")
        .expect("set ULLM_HIP_LIB_DIR to the directory holding libullm_hip.so");
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=ullm_hip");
    let rocm = std::env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".into());
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    println!("cargo:rerun-if-env-changed=ULLM_HIP_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
}
