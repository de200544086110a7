//! Link search path for libtang_hip.so: $TANG_HIP_LIB_DIR, else the
//! directory the library is built into (tang_amd/, next to this crate).
fn main() {
    let dir = std::env::var("TANG_HIP_LIB_DIR").unwrap_or_else(|_| {
        let here = std::env::var("CARGO_MANIFEST_DIR").expect("CARGO_MANIFEST_DIR");
        format!("{}/..", here)
    });
    println!("cargo:rustc-link-search=native={}", dir);
    println!("cargo:rustc-link-lib=dylib=tang_hip");
    println!("cargo:rerun-if-env-changed=TANG_HIP_LIB_DIR");
}
