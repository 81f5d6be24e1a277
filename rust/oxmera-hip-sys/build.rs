//! Link liboxm.so.  Where it lives: $OXM_LIB_DIR, else the in-tree build of
//! this repository (oxmera_amd/liboxm.so, two directories up from this
//! crate).  The library itself depends on the ROCm runtime in /opt/rocm/lib.
use std::env;
use std::path::PathBuf;

fn main() {
    println!("cargo:rerun-if-env-changed=OXM_LIB_DIR");
    let dir = match env::var_os("OXM_LIB_DIR") {
        Some(d) => PathBuf::from(d),
        None => PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap()).join("../../oxmera_amd"),
    };
    if !dir.join("liboxm.so").exists() {
        panic!(
            "liboxm.so not found in {} (build it with `python -m oxmera_amd.build` or set OXM_LIB_DIR)",
            dir.display()
        );
    }
    println!("cargo:rustc-link-search=native={}", dir.display());
    println!("cargo:rustc-link-lib=dylib=oxm");
    println!("cargo:rustc-link-search=native=/opt/rocm/lib");
    // let binaries find the library at run time without LD_LIBRARY_PATH
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", dir.display());
    println!("cargo:rerun-if-changed={}", dir.join("liboxm.so").display());
}
