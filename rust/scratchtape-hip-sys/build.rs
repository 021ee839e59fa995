// Links libscratchtape_hip.so.  The library is built beforehand by hipcc
// (`python -m scratchtape_amd.build` at the repository root); this script only
// points the linker at it.  SCRATCHTAPE_HIP_DIR overrides the directory, which
// defaults to the in-tree build next to this crate.
use std::path::PathBuf;

fn main() {
    let dir = match std::env::var("SCRATCHTAPE_HIP_DIR") {
        Ok(d) => PathBuf::from(d),
        Err(_) => {
            let manifest = PathBuf::from(std::env::var("CARGO_MANIFEST_DIR").expect("cargo sets CARGO_MANIFEST_DIR"));
            manifest.join("..").join("..").join("scratchtape_amd")
        }
    };
    let lib = dir.join("libscratchtape_hip.so");
    if !lib.exists() {
        panic!(
            "{} not found: build it with `python -m scratchtape_amd.build`, or set SCRATCHTAPE_HIP_DIR",
            lib.display()
        );
    }
    println!("cargo:rustc-link-search=native={}", dir.display());
    println!("cargo:rustc-link-lib=dylib=scratchtape_hip");
    // This crate's own tests and examples find the library at run time without LD_LIBRARY_PATH;
    // a dependent binary sets its own rpath or LD_LIBRARY_PATH.
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", dir.display());
    println!("cargo:rerun-if-env-changed=SCRATCHTAPE_HIP_DIR");
    println!("cargo:rerun-if-changed={}", lib.display());
}
