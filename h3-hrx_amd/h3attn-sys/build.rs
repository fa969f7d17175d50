//! Links libh3attn.so. The library is built by `python h3-hrx_amd/build.py` into `h3-hrx_amd/`
//! (this crate's parent directory); `H3ATTN_LIB_DIR` overrides the search directory. The HIP
//! runtime (`libamdhip64`) is a dependency of libh3attn itself and is found through its rpath or
//! the loader path of the ROCm install.
use std::env;
use std::path::PathBuf;

fn main() {
    println!("cargo:rerun-if-env-changed=H3ATTN_LIB_DIR");
    let dir = match env::var_os("H3ATTN_LIB_DIR") {
        Some(d) => PathBuf::from(d),
        None => PathBuf::from(env::var_os("CARGO_MANIFEST_DIR").expect("cargo sets this"))
            .join(".."),
    };
    println!("cargo:rustc-link-search=native={}", dir.display());
    println!("cargo:rustc-link-lib=dylib=h3attn");
    println!("cargo:rerun-if-changed={}", dir.join("libh3attn.so").display());
}
