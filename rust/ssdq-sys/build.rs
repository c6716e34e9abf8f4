// Links libssdq.so from SSDQ_LIB_DIR (the directory `make -C ssd-llm_amd` builds it in).
// libssdq.so depends on the HIP runtime (libamdhip64) itself, so nothing else is linked here.
fn main() {
    println!("cargo:rerun-if-env-changed=SSDQ_LIB_DIR");
    if let Ok(dir) = std::env::var("SSDQ_LIB_DIR") {
        println!("cargo:rustc-link-search=native={dir}");
    }
    println!("cargo:rustc-link-lib=dylib=ssdq");
}
