//! Links libyaxus_hip.so (built by `python -m yaxus_amd.build` in the yaxus_amd
//! repository: hipcc for gfx950). YAXUS_HIP_LIB_DIR names its directory; the rpath lets
//! the binaries find it there at run time.
fn main() {
    println!("cargo:rerun-if-env-changed=YAXUS_HIP_LIB_DIR");
    let dir = std::env::var("YAXUS_HIP_LIB_DIR")
        .expect("set YAXUS_HIP_LIB_DIR to the directory holding libyaxus_hip.so");
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=yaxus_hip");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
}
