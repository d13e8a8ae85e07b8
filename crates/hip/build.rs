//! Links liblinalg_hip.so, the C ABI declared in include/linalg_hip.h.
//!
//! The library is found in LINALG_HIP_LIB_DIR when set, else in the package directory of this
//! repository (pipeline-parallelism-deep-learning-library_amd/, where its build.py writes it).

use std::env;
use std::path::PathBuf;

fn main() {
    println!("cargo:rerun-if-env-changed=LINALG_HIP_LIB_DIR");
    let dir = match env::var("LINALG_HIP_LIB_DIR") {
        Ok(d) => PathBuf::from(d),
        Err(_) => PathBuf::from(env::var("CARGO_MANIFEST_DIR").expect("cargo sets CARGO_MANIFEST_DIR"))
            .join("../../pipeline-parallelism-deep-learning-library_amd"),
    };
    println!("cargo:rustc-link-search=native={}", dir.display());
    println!("cargo:rustc-link-lib=dylib=linalg_hip");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", dir.display());
}
