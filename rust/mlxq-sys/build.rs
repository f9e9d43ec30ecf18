// Links libmlxq.so.  MLXQ_LIB_DIR names the directory holding it (default:
// the in-tree build, ../../mlxcel_amd relative to this crate).
use std::env;
use std::path::PathBuf;

fn main() {
    let dir = env::var("MLXQ_LIB_DIR").map(PathBuf::from).unwrap_or_else(|_| {
        PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap()).join("../../mlxcel_amd")
    });
    println!("cargo:rerun-if-env-changed=MLXQ_LIB_DIR");
    println!("cargo:rustc-link-search=native={}", dir.display());
    println!("cargo:rustc-link-lib=dylib=mlxq");
    // let binaries find the library at run time without LD_LIBRARY_PATH
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", dir.display());
}
