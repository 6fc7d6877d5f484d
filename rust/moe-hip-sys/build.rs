// Links libmoe_hip.so (built in-tree by oxidizr_amd/build.py with hipcc for
// gfx950). MOE_HIP_LIB_DIR overrides the directory; the default is the
// repository's oxidizr_amd/ next to this crate.
use std::env;
use std::path::PathBuf;

fn main() {
    let dir = env::var("MOE_HIP_LIB_DIR").map(PathBuf::from).unwrap_or_else(|_| {
        PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap()).join("../../oxidizr_amd")
    });
    println!("cargo:rustc-link-search=native={}", dir.display());
    println!("cargo:rustc-link-lib=dylib=moe_hip");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", dir.display());
    println!("cargo:rerun-if-env-changed=MOE_HIP_LIB_DIR");
}
