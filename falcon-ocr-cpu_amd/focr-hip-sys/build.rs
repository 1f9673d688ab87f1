//! Links libfocr_hip.so. The library is built by `make -C falcon-ocr-cpu_amd`
//! (hipcc, gfx950) into `falcon-ocr-cpu_amd/lib`; `FOCR_HIP_LIB_DIR` points
//! elsewhere, e.g. to an installed copy.
use std::env;
use std::path::PathBuf;

fn main() {
    let dir = match env::var("FOCR_HIP_LIB_DIR") {
        Ok(dir) => PathBuf::from(dir),
        Err(_) => PathBuf::from(env::var("CARGO_MANIFEST_DIR").expect("cargo sets CARGO_MANIFEST_DIR"))
            .join("..")
            .join("lib"),
    };
    println!("cargo:rerun-if-env-changed=FOCR_HIP_LIB_DIR");
    println!("cargo:rerun-if-changed=../../include/focr_hip.h");
    println!("cargo:rustc-link-search=native={}", dir.display());
    println!("cargo:rustc-link-lib=dylib=focr_hip");
    // The HIP runtime the library itself links against.
    println!("cargo:rustc-link-search=native=/opt/rocm/lib");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
}
