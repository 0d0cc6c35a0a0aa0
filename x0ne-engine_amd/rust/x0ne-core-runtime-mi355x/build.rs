//! Links libx0ne_core.so: from X0NE_MI355X_LIB_DIR when set, else from the in-tree build
//! (x0ne-engine_amd/x0ne_core/, two directories up from this crate).
use std::path::PathBuf;

fn main() {
    let dir = match std::env::var("X0NE_MI355X_LIB_DIR") {
        Ok(d) => PathBuf::from(d),
        Err(_) => PathBuf::from(std::env::var("CARGO_MANIFEST_DIR").expect("cargo sets CARGO_MANIFEST_DIR"))
            .join("../../x0ne_core"),
    };
    println!("cargo:rustc-link-search=native={}", dir.display());
    println!("cargo:rustc-link-lib=dylib=x0ne_core");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", dir.display());
    println!("cargo:rerun-if-env-changed=X0NE_MI355X_LIB_DIR");
}
