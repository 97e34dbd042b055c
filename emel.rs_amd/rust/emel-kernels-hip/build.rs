//! Links `libemel_hip.so`, the C-ABI library built by `hipcc` from
//! `emel.rs_amd/csrc` (`python -c "import __graft_entry__ as g; g.build()"`).
//!
//! `EMEL_HIP_LIB_DIR` names the directory that holds the library; without it
//! the loader's search path is used.  The HIP runtime (`libamdhip64`) is a
//! dependency of the library itself and is found through its own run path.

use std::env;

fn main() {
    println!("cargo:rerun-if-env-changed=EMEL_HIP_LIB_DIR");
    if let Ok(dir) = env::var("EMEL_HIP_LIB_DIR") {
        println!("cargo:rustc-link-search=native={dir}");
        // Let test binaries and examples find the library without LD_LIBRARY_PATH.
        println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
    }
    println!("cargo:rustc-link-lib=dylib=emel_hip");
}
