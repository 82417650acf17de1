//! Link script of the `-sys` crate: the manifest declares `links = "mrun_moe"`, which Cargo accepts
//! only together with a build script that names the native library.
//!
//! `MRUN_MOE_LIB_DIR` is the directory holding `libmrun_moe.so` (built by `python -m
//! mrun_amd.build` into `mrun_amd/lib/`). When it is unset, the dynamic linker's default search
//! path is used.

fn main() {
    println!("cargo:rerun-if-env-changed=MRUN_MOE_LIB_DIR");
    if let Ok(dir) = std::env::var("MRUN_MOE_LIB_DIR") {
        println!("cargo:rustc-link-search=native={dir}");
    }
    println!("cargo:rustc-link-lib=dylib=mrun_moe");
}
