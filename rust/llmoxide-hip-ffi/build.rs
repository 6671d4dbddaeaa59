//! Links libllmoxide_amd.so, built by `python -m llmoxide_amd.build` (the same
//! build `__graft_entry__.build()` runs).  LMX_LIB_DIR names the directory
//! holding the library; by default the `llmoxide_amd/` package directory two
//! levels above this crate.  The library needs libamdhip64 at run time.
use std::env;
use std::path::PathBuf;

fn main() {
    println!("cargo:rerun-if-env-changed=LMX_LIB_DIR");
    let dir = match env::var("LMX_LIB_DIR") {
        Ok(d) => PathBuf::from(d),
        Err(_) => PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap()).join("../../llmoxide_amd"),
    };
    println!("cargo:rustc-link-search=native={}", dir.display());
    println!("cargo:rustc-link-lib=dylib=llmoxide_amd");
}
