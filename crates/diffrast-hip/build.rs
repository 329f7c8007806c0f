//! Links libdiffrast_hip.so. The library is built by the Python package's
//! build step (`python -c "import __graft_entry__ as g; g.build()"` at the
//! repository root), which leaves it in `differentiable-rasterizer_amd/`.
//! `DIFFRAST_HIP_LIB_DIR` names another directory; the path is also written
//! into the binaries' run path so no `LD_LIBRARY_PATH` is needed.

use std::path::PathBuf;

fn main() {
    println!("cargo:rerun-if-env-changed=DIFFRAST_HIP_LIB_DIR");
    let dir = match std::env::var_os("DIFFRAST_HIP_LIB_DIR") {
        Some(d) => PathBuf::from(d),
        None => {
            let manifest = PathBuf::from(std::env::var_os("CARGO_MANIFEST_DIR").expect("cargo sets CARGO_MANIFEST_DIR"));
            manifest.join("../../differentiable-rasterizer_amd")
        }
    };
    let lib = dir.join("libdiffrast_hip.so");
    if !lib.exists() {
        panic!(
            "{} not found: build the HIP library first, or set DIFFRAST_HIP_LIB_DIR to the directory that holds it",
            lib.display()
        );
    }
    println!("cargo:rerun-if-changed={}", lib.display());
    println!("cargo:rustc-link-search=native={}", dir.display());
    println!("cargo:rustc-link-lib=dylib=diffrast_hip");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", dir.display());
}
