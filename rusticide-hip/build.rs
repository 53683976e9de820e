//! Links librusticide_hip.so, built by `__graft_entry__.build()` in the HIP
//! repository (hipcc --offload-arch=gfx950); RUSTICIDE_HIP_LIB_DIR names the
//! directory that holds it.

fn main() {
    println!("cargo:rerun-if-env-changed=RUSTICIDE_HIP_LIB_DIR");
    match std::env::var("RUSTICIDE_HIP_LIB_DIR") {
        Ok(dir) => {
            println!("cargo:rustc-link-search=native={dir}");
            println!("cargo:rustc-link-lib=dylib=rusticide_hip");
        }
        Err(_) => println!(
            "cargo:warning=RUSTICIDE_HIP_LIB_DIR is not set: set it to the directory of librusticide_hip.so"
        ),
    }
}
