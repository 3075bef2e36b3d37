//! Links librailgun_hip.so (built by `python -c "import __graft_entry__ as g; g.build()"` in
//! the MI355X repository, which leaves it in railgun_amd/) and the HIP runtime.
//!
//! RAILGUN_HIP_LIB_DIR: directory holding librailgun_hip.so (required).
//! ROCM_PATH: ROCm installation (default /opt/rocm) for libamdhip64.so.

fn main() {
    println!("cargo:rerun-if-env-changed=RAILGUN_HIP_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
    let lib_dir = std::env::var("RAILGUN_HIP_LIB_DIR")
        .expect("set RAILGUN_HIP_LIB_DIR to the directory holding librailgun_hip.so");
    let rocm = std::env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    println!("cargo:rustc-link-search=native={lib_dir}");
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=railgun_hip");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    // Let binaries find the library next to where it was built.
    println!("cargo:rustc-link-arg=-Wl,-rpath,{lib_dir}");
}
