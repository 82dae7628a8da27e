// Links libairkv.so: AIRKV_LIB_DIR names the directory that holds it (for
// this repository, air.rs_amd/airkv after `make -C air.rs_amd`), and the
// ROCm runtime it depends on is found through ROCM_PATH (default /opt/rocm).
fn main() {
    println!("cargo:rerun-if-env-changed=AIRKV_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
    if let Ok(dir) = std::env::var("AIRKV_LIB_DIR") {
        println!("cargo:rustc-link-search=native={dir}");
        println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
    }
    let rocm = std::env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=airkv");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
}
