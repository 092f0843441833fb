//! Links libhip_bridge.so. The library is built from rustane_amd/csrc with
//! `make -C rustane_amd/csrc` and lands in rustane_amd/; HIP_BRIDGE_LIB_DIR
//! points elsewhere (an installed copy). The library itself links the ROCm
//! runtime (libamdhip64) with an rpath to /opt/rocm/lib.
use std::env;
use std::path::PathBuf;

fn main() {
    println!("cargo:rerun-if-env-changed=HIP_BRIDGE_LIB_DIR");
    println!("cargo:rerun-if-changed=../../include/hip_bridge.h");
    let dir = match env::var("HIP_BRIDGE_LIB_DIR") {
        Ok(d) => PathBuf::from(d),
        Err(_) => PathBuf::from(env::var("CARGO_MANIFEST_DIR").expect("cargo sets CARGO_MANIFEST_DIR"))
            .join("..")
            .join("..")
            .join("rustane_amd"),
    };
    println!("cargo:rustc-link-search=native={}", dir.display());
    println!("cargo:rustc-link-lib=dylib=hip_bridge");
    // tests, examples and binaries of this package find the library at run
    // time; dependents set LD_LIBRARY_PATH or their own rpath
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", dir.display());
    // lets dependents' build scripts read DEP_HIP_BRIDGE_LIB_DIR
    println!("cargo:lib_dir={}", dir.display());
}
