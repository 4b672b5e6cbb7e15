// Links libatlas_hip_ops.so (built by atlas_amd/Makefile: `make -C atlas_amd`).
// ATLAS_HIP_OPS_DIR names the directory that holds it; without it the linker's
// default search path is used.  The library's own dependency on the HIP
// runtime (libamdhip64) is resolved through its DT_NEEDED entry.
fn main() {
    println!("cargo:rerun-if-env-changed=ATLAS_HIP_OPS_DIR");
    if let Ok(dir) = std::env::var("ATLAS_HIP_OPS_DIR") {
        println!("cargo:rustc-link-search=native={dir}");
        println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
    }
    println!("cargo:rustc-link-lib=dylib=atlas_hip_ops");
}
