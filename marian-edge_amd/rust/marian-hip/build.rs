//! Links libmarian_hip.so.  MARIAN_HIP_LIB_DIR names the directory that holds
//! it (the marian-edge_amd/ folder of the HIP repository, or an install
//! prefix); the library's own dependencies (the HIP runtime) are resolved by
//! the dynamic loader.

fn main() {
    println!("cargo:rerun-if-env-changed=MARIAN_HIP_LIB_DIR");
    let dir = std::env::var("MARIAN_HIP_LIB_DIR")
        .expect("set MARIAN_HIP_LIB_DIR to the directory holding libmarian_hip.so");
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=marian_hip");
    // Let binaries find the library next to where it was linked from.
    println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
}
